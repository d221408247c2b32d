"""Raw (pre-RoPE) key hand-off between the model's rotary call and the attention layer.

The reference captures raw K by wrapping the model's rotary module (vllm_ttkv/patch.py:229-309)
and pops it in the attention layer (patch.py:123-137, 312-323). Only the stash is kept here: the
model-class patching needs vLLM and is outside this package's scope; whatever calls the rotary
embedding stashes raw K with `stash_raw_k` before attention runs.
"""
from __future__ import annotations

_STASH: dict = {}


def stash_raw_k(layer_name: str, raw_k, positions=None, cos_sin_cache=None) -> None:
    _STASH[layer_name] = dict(raw_k=raw_k, positions=positions, cos_sin_cache=cos_sin_cache)


def take_raw_k(layer_name: str) -> dict:
    """Pop this layer's stash. A missing or double-consumed stash is an error, not a stale read."""
    try:
        return _STASH.pop(layer_name)
    except KeyError:
        raise RuntimeError(
            f"vllm_ttkv: no raw (pre-RoPE) key was stashed for layer {layer_name!r}. The store "
            f"holds keys before rotation, so the attention layer needs the model's raw K; the "
            f"rotary call has to stash it with patch.stash_raw_k for this layer and step.") from None

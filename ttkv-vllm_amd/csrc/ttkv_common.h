// Shared device helpers for the compressed-KV kernels (gfx950 / CDNA4).
//
// Slot format (reference: vllm_ttkv/layout.py:56-261, codec/ttkv_packed_cache.py:50-271):
//   token blob = [K slot | V slot], each zero-padded to 16 bytes
//   K slot = r1 int8 coefficients, fp16 coefficient ruler (LE), H rows of
//            [bitmap d/8 B | MSB-first code stream ceil(k*bits/8) B | fp16 ruler (LE)]
//   V slot = H rows of the same shape
// Two more coefficient fields, selected by the layout's qbits, are this library's own storage
// modes (the reference writes only qbits = 8, layout.py:179):
//   qbits 16: r1 fp16 coefficients (LE), no ruler
//   qbits 4 : 4-bit two's complement coefficients in [-7, 7], 4 * ceil(r1/8) bytes of
//             little-endian words: word w holds rank 8w + 2m at bits 4m .. 4m+3 and rank
//             8w + 2m + 1 at bits 16 + 4m .. 16 + 4m + 3 (m = 0..3; pad nibbles 0), then one fp16
//             scale per group of 32 ranks (ceil(r1/32) of them, LE). A scale has at most 8
//             significant bits and lies in [2^-14, 9344] (or is 0 for an all-zero group), so
//             q * scale is exact in fp16. The coefficient value is q * scale.
// Bitmap: lane j <-> byte j>>3, bit 7-(j&7). The stream holds the kept lanes in increasing lane
// order, `bits` bits each, MSB first; the stored code is q + 2^(bits-1). Decoded value
// (code - 2^(bits-1)) * float(ruler) on kept lanes, 0 elsewhere.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ttkv_hip.h"

namespace ttkv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

constexpr int kD = 128;           // head dim the kernels are built for
constexpr int kBitmapBytes = kD / 8;

// Byte geometry of one layer, derived exactly as layout.py:98-157.
// Coefficient storage modes, by the layout's qbits (8, 16, 4 above).
enum CoefMode { kCoefI8 = 0, kCoefF16 = 1, kCoefI4G32 = 2 };

struct Geom {
  int H, d, r1, qbits, res_k, res_bits, v_lanes, v_bits;
  int coef_mode;     // CoefMode
  int coeff_bytes;   // coefficient values: r1 (int8), 2 * r1 (fp16), 4 * ceil(r1 / 8) (4-bit)
  int coef_groups;   // 4-bit mode: scales (groups of 32 ranks) after the values; else 0
  int k_pb, v_pb;    // packed code bytes per row
  int k_row, v_row;  // bytes per head row
  int k_field;       // offset of head 0's K row in the slot
  int k_slot, v_slot, blob;
};

__host__ inline int align_up16(int n) { return (n + 15) / 16 * 16; }

// Decoder pool (the codec's int8 decoder, ttkv_packed_cache.py:284-293, laid out for the kernels):
//   dec_q     [slots, H*d, R] int8: column j = h*d + dim holds its R rank values contiguously
//   dec_scale [slots, R] fp32: the rank's ruler
// R = 64 for r1 <= 64, 128 for r1 <= 128, else r1 rounded up to 64: every kernel's rank window
// lies inside it (K1: 16-rank units up to 16 KU; K2: 32-rank steps; K3: whole 64-rank chunks of a
// column per lane). Ranks >= r1 hold 0 with ruler 0. A decoder value is float(dec_q) *
// dec_scale, exact in fp32 (8 bits times the codec's 11-bit fp16 ruler).
__host__ __device__ inline int dec_ranks(int r1) {
  return r1 <= 64 ? 64 : r1 <= 128 ? 128 : (r1 + 63) & ~63;
}

// Decoder values of ranks 4m .. 4m+3 from their dword of int8 codes and their rulers: float(q) *
// ruler, exactly, as u * ruler - 128 * ruler with u = q + 128 (a byte convert and an fma per
// value: the fma's exact result is float(q) * ruler, which is representable, so nothing rounds).
__device__ __forceinline__ void dec_values4(uint32_t q4, float4v ruler, float out[4]) {
  const uint32_t u = q4 ^ 0x80808080u;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    out[k] = fmaf((float)((u >> (8 * k)) & 0xffu), ruler[k], -128.0f * ruler[k]);
}

__host__ inline bool make_geom(const ttkv_layout* l, Geom* g) {
  if (!l) return false;
  g->H = l->H; g->d = l->d; g->r1 = l->r1; g->qbits = l->qbits;
  g->res_k = l->res_k; g->res_bits = l->res_bits; g->v_lanes = l->v_lanes; g->v_bits = l->v_bits;
  if (g->d <= 0 || g->d % 8 || g->H <= 0 || g->r1 <= 0) return false;
  if (g->res_k < 0 || g->res_k > g->d || g->v_lanes < 1 || g->v_lanes > g->d) return false;
  int scale_bytes = 2;
  g->coef_groups = 0;
  if (g->qbits == 8) {
    g->coef_mode = kCoefI8;
    g->coeff_bytes = g->r1;
  } else if (g->qbits == 16) {
    g->coef_mode = kCoefF16;
    g->coeff_bytes = 2 * g->r1;
    scale_bytes = 0;
  } else if (g->qbits == 4) {
    g->coef_mode = kCoefI4G32;
    g->coeff_bytes = 4 * ((g->r1 + 7) / 8);
    g->coef_groups = (g->r1 + 31) / 32;
    scale_bytes = 2 * g->coef_groups;
  } else {
    return false;
  }
  g->k_pb = (g->res_k * g->res_bits + 7) / 8;
  g->v_pb = (g->v_lanes * g->v_bits + 7) / 8;
  g->k_row = g->d / 8 + g->k_pb + 2;
  g->v_row = g->d / 8 + g->v_pb + 2;
  g->k_field = g->coeff_bytes + scale_bytes;
  g->k_slot = align_up16(g->k_field + g->H * g->k_row);
  g->v_slot = align_up16(g->H * g->v_row);
  g->blob = g->k_slot + g->v_slot;
  return true;
}

// The read kernels fetch each head row through the 16-byte-aligned 64-byte window that starts at
// the row's first byte rounded down: every row must lie inside its window (misalignment + row
// bytes <= 64). All shipped allocations satisfy it (safe 49 B rows at offsets = h mod 16,
// campaign4x 50 B at 2h mod 16, tight 30/35 B).
__host__ inline bool rows_in_windows(const Geom& g) {
  for (int h = 0; h < g.H; ++h)
    if (((g.k_field + h * g.k_row) & 15) + g.k_row > 64 ||
        ((g.k_slot + h * g.v_row) & 15) + g.v_row > 64)
      return false;
  return true;
}

// A pointer known to be in global memory, so loads through it are global_load_* (vector memory
// counter only). Loads through a generic pointer become flat_load_*, which also count against the
// LDS counter, so every later LDS wait would also wait for them.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gbl(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

// The same for stores: global_store_* instead of flat_store_*.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gblw(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// 16 bytes from global memory (16-byte aligned) as uint4, through a global pointer.
__device__ __forceinline__ uint4 ld_global16(const void* p) {
  const u32x4 v = *gbl((const u32x4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// A streamed 16-byte load (non-temporal hint: read once, not kept in the caches). A plain
// streaming read measured 6.8 TB/s with the hint against 6.3 TB/s without on this GPU.
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(gbl((const u32x4*)p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Load element `i` of a q/out-style tensor of dtype `dt` as fp32.
__device__ __forceinline__ float load_act(const void* p, int dt, int64_t i) {
  if (dt == TTKV_DTYPE_F32) return ((const float*)p)[i];
  uint32_t b = ((const uint16_t*)p)[i];
  return dt == TTKV_DTYPE_F16 ? f16_bits_to_float(b) : bf16_bits_to_float(b);
}

// N (4 or 8) consecutive activations from element i0 of p, as floats, with every load issued
// before any conversion (one memory round trip instead of one per element). `vec`: element i0
// is aligned to the group (N * element bytes, 16 at most), so each group is one or two wide loads.
template <int N>
__device__ __forceinline__ void load_act_n(const void* p, int dt, int64_t i0, bool vec,
                                           float v[N]) {
  static_assert(N == 4 || N == 8, "groups of 4 or 8");
  if (dt == TTKV_DTYPE_F32) {
    const float* q = (const float*)p + i0;
    if (vec) {
#pragma unroll
      for (int k = 0; k < N / 4; ++k) {
        const float4v x = *gbl((const float4v*)q + k);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[4 * k + j] = x[j];
      }
    } else {
#pragma unroll
      for (int k = 0; k < N; ++k) v[k] = *gbl(q + k);
    }
    return;
  }
  const uint16_t* q = (const uint16_t*)p + i0;
  uint32_t bits[N];
  if (vec) {
    if constexpr (N == 8) {
      const u32x4 x = *gbl((const u32x4*)q);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bits[2 * k] = x[k] & 0xffffu;
        bits[2 * k + 1] = x[k] >> 16;
      }
    } else {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 x = *gbl((const u32x2*)q);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        bits[2 * k] = x[k] & 0xffffu;
        bits[2 * k + 1] = x[k] >> 16;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) bits[k] = *gbl(q + k);
  }
#pragma unroll
  for (int k = 0; k < N; ++k)
    v[k] = dt == TTKV_DTYPE_F16 ? f16_bits_to_float(bits[k]) : bf16_bits_to_float(bits[k]);
}

// Whether element offsets that are multiples of 8 (fp32: 4) are 16-byte aligned in an
// activation tensor with this base and row stride (elements).
__device__ __forceinline__ bool act_rows_aligned(const void* p, int dt, int64_t row_stride) {
  const int64_t eb = dt == TTKV_DTYPE_F32 ? 4 : 2;
  return ((uintptr_t)p % 16 == 0) && ((row_stride * eb) % 16 == 0);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// 16 bytes stored write-through to the device-coherent level (the cache policy of an agent-scope
// atomic store, `sc1`), so that another CU, on any XCD, reads them after an agent-scope acquire
// with no L2 writeback on this side. A vector-memory store; p must be 16-byte aligned.
__device__ __forceinline__ void store_agent16(float* p, float4v v) {
  __asm__ volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_agent8(float* p, float2v v) {
  __asm__ volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Split-K hand-off, read side. The partials were stored write-through at agent scope (above, or
// agent-scope atomic stores) and completed (s_waitcnt vmcnt(0)) before their workgroup's
// arrival-counter RMW, so once the last workgroup sees the count complete it reads them with
// agent-scope loads, which are coherent across the XCDs' L2 caches. Neither side needs a
// cache-wide operation: an acquire-release RMW writes back the XCD's whole L2 before the RMW and
// invalidates it after, which measured ~2.7 us per workgroup on the release side and 7-14 us of
// the combining workgroup's tail on the acquire side (K1 headline: 136 -> 125 us per launch).
// K1 and K3 use this; the continuation kernels keep the acquire-release counter and plain loads
// after the acquire, which their combine loops batch better (agent-scope loads there measured
// 280 against 254 us per config-4 launch).
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4v ld_agent4(const float* p) {
  return float4v{ld_agent(p), ld_agent(p + 1), ld_agent(p + 2), ld_agent(p + 3)};
}
// The arrival counter: relaxed (the ordering comes from the completed write-through stores).
__device__ __forceinline__ int arrive(int* cnt) {
  return __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four consecutive activations from element i (a multiple of 4) with one store, where `vec` says
// the tensor's rows are aligned for it; element stores otherwise.
__device__ __forceinline__ void store_act4(void* p, int dt, int64_t i, float4v v, bool vec);

__device__ __forceinline__ void store_act(void* p, int dt, int64_t i, float v) {
  if (dt == TTKV_DTYPE_F32) {
    ((float*)p)[i] = v;
  } else if (dt == TTKV_DTYPE_F16) {
    ((_Float16*)p)[i] = (_Float16)v;
  } else {
    ((uint16_t*)p)[i] = float_to_bf16_bits(v);
  }
}

__device__ __forceinline__ void store_act4(void* p, int dt, int64_t i, float4v v, bool vec) {
  if (!vec) {
#pragma unroll
    for (int j = 0; j < 4; ++j) store_act(p, dt, i + j, v[j]);
    return;
  }
  if (dt == TTKV_DTYPE_F32) {
    *gblw((float4v*)((float*)p + i)) = v;
  } else if (dt == TTKV_DTYPE_F16) {
    const half4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *gblw((half4*)((_Float16*)p + i)) = h;
  } else {
    const u32x2v b = {(uint32_t)float_to_bf16_bits(v[0]) | ((uint32_t)float_to_bf16_bits(v[1]) << 16),
                      (uint32_t)float_to_bf16_bits(v[2]) | ((uint32_t)float_to_bf16_bits(v[3]) << 16)};
    *gblw((u32x2v*)((uint16_t*)p + i)) = b;
  }
}

}  // namespace ttkv


// K1: fused paged decode read over compressed (pre-RoPE, tensor-train) KV slots, one launch per
// layer for the whole decode batch. gfx950 / CDNA4.
//
// Work item = (request r, KV head h, token chunk c). A 256-thread workgroup (4 waves) walks its
// chunk in 64-token tiles:
//   stage   : coefficient bytes -> fp16 MFMA B-fragments in LDS (int8 exact in fp16); this head's
//             K and V rows -> LDS, realigned to 4 bytes.
//   decode  : one thread per half row (64 lanes): bitmap + MSB-first code stream -> dense values.
//             K: (code - 2^(b-1)) * ruler as fp32; V: (code - 2^(b-1)) as fp16 (+ fp32 ruler).
//   recon   : K_pre^T[128 x 16 tokens] = Dec^T[128 x r1] * coeff^T[r1 x 16] on MFMA 16x16x32 f16.
//             The decoder is split hi + lo in fp16 and both halves are applied; decoder_f values
//             are int8 * fp16 row rulers (<= 19 significant bits), so hi + lo is exact and the
//             products are exact in the fp32 accumulator. Wave w owns dims {16w..16w+15} and
//             {64+16w..64+16w+15}, so each RoPE pair (j, j+64) sits in one lane and the decoder
//             fragments stay in registers for the whole chunk.
//   rope+qk : k = cs * acc + residual; rotate by the row's own absolute position; fp32 dot with
//             the G query heads of this KV head; partial dots reduced across lanes and waves.
//   softmax : online (running max / sum), base-2 exponent with scale*log2(e) folded in.
//   P.V     : o[p] += P[p,t] * ruler_v[t] * vcode[t] in fp32 (v_fma_mix with fp16 codes).
// Chunks of one (r, h) are combined in the same launch by the last workgroup to finish
// (device-scope fence + counter), which also resets the counter to zero.
//
// Reference semantics: vllm_ttkv/reference.py:63-163 (dense K, per-row RoPE, scores, softmax,
// V readout), vllm_ttkv/impl.py:511-540 (scale then softmax), decode.py:54-122 (vLLM cos/sin
// half layout), decode.py:307-339 (slot = block_table[r, t/bs]*bs + t%bs).
#include <math.h>

#include <type_traits>

#include "ttkv_common.h"

namespace ttkv {

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kKresStride = 132;   // fp32 per K-residual row in LDS (bank stagger)
constexpr int kVStride = 136;      // fp16 per V row in LDS
constexpr int kRawDw = 15;         // dwords per raw head row in LDS (row + window slack)

struct DecodeArgs {
  Geom g;
  int HQ, G;
  float scale_log2;
  const void* q;
  int q_dtype;
  int64_t q_row_stride;
  const uint8_t* page;
  int64_t n_slots, slot_stride;
  int block_size;
  const int32_t* bt;
  int64_t bt_row_stride;
  int max_blocks;
  const int32_t* seq_lens;
  const int32_t* qsl;
  int num_reqs;
  const int32_t* dec_map;
  int64_t num_blocks;
  const float* dec_pool;
  int64_t n_dec_slots;
  const float* cs_cache;
  int64_t max_pos;
  void* out;
  int out_dtype;
  int64_t out_row_stride;
  float* ws_part;
  int* ws_cnt;
  int* err;
  int chunk, max_chunks, nwork, max_seq;
};

template <int KSTEPS>
struct DecodeSmem {
  static constexpr int kCoefStride = KSTEPS * 32 + 8;  // fp16 per token row
  _Float16 coef[kTile][kCoefStride];
  float kres[kTile][kKresStride];
  _Float16 vval[kTile][kVStride];
  union {
    struct {
      uint32_t rawk[kTile][kRawDw];
      uint32_t rawv[kTile][kRawDw];
    } raw;
    struct {
      float spart[kWaves][kTile][8];
      float pw[8][kTile];
      float alpha[8];
      float m[8], l[8];
    } sm;
  } u;
  float cs[kTile];
  float vrul[kTile];
  int is_last;
};

// int8 x4 (little-endian in a dword) -> two packed fp16 pairs, exact.
__device__ __forceinline__ void i8x4_to_f16(uint32_t x, uint32_t& p01, uint32_t& p23) {
  const uint32_t u = x ^ 0x80808080u;  // b + 128 as unsigned bytes
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  p01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, lo) - bias);
  p23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, hi) - bias);
}

// Decode dims [64*half, 64*half+64) of one head row held in LDS (bitmap at byte 0, code stream
// at byte 16, fp16 ruler after the stream). Calls emit(dim_base, codes[8]) per bitmap byte with
// the raw code of every lane (2^(BITS-1) for lanes not in the bitmap, so value 0).
template <int BITS, typename Emit>
__device__ __forceinline__ void decode_half_row(const uint8_t* row, int half, Emit emit) {
  constexpr uint32_t OFF = 1u << (BITS - 1);
  int rank = 0;
  if (half) {
    const uint32_t* bw = (const uint32_t*)row;
    rank = __builtin_popcount(bw[0]) + __builtin_popcount(bw[1]);
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const uint32_t B = row[8 * half + m];
    const int bp = rank * BITS;
    const uint8_t* s = row + 16 + (bp >> 3);
    // Up to 8 codes (8*BITS bits) starting (bp & 7) bits into the first byte: 31 bits for
    // 3-bit codes fit a 32-bit window, 39 bits for 4-bit codes need a 64-bit one.
    typedef typename std::conditional<(8 * BITS + 7 > 32), uint64_t, uint32_t>::type win_t;
    constexpr int WB = 8 * (int)sizeof(win_t);
    win_t w = 0;
#pragma unroll
    for (int b = 0; b < (int)sizeof(win_t); ++b) w |= (win_t)s[b] << (WB - 8 - 8 * b);
    w <<= (bp & 7);
    uint32_t codes[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool present = (B >> (7 - k)) & 1u;
      const uint32_t c = (uint32_t)(w >> (WB - BITS));
      codes[k] = present ? c : OFF;
      w = present ? (win_t)(w << BITS) : w;
    }
    emit(64 * half + 8 * m, codes);
    rank += __builtin_popcount(B);
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int G, int RB, int VB, int KSTEPS>
__global__ __launch_bounds__(kThreads, 2) void decode_paged_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  DecodeSmem<KSTEPS>& S = *reinterpret_cast<DecodeSmem<KSTEPS>*>(smem_raw);
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // XCD-aware work order: blocks are dealt round-robin to the 8 XCDs, so consecutive work items
  // (the H heads of one token chunk, which read the same coefficient bytes) go to one XCD.
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= a.nwork) return;
  const int h = w % g.H;
  const int rc = w / g.H;
  const int r = rc / a.max_chunks;
  const int c = rc % a.max_chunks;
  if (r >= a.num_reqs) return;
  int seq = a.seq_lens[r];
  if (seq > a.max_seq) {  // the host sized the grid, workspace and table checks from max_seq
    if (tid == 0 && c == 0) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    seq = a.max_seq;
  }
  const int n_chunks = (seq + a.chunk - 1) / a.chunk;
  const int64_t qrow = a.qsl[r];
  if (c >= n_chunks) {
    if (seq <= 0 && c == 0) {  // empty context: the reference's einsum over zero rows is 0
      for (int i = tid; i < G * kD; i += kThreads)
        store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G) * kD + i, 0.f);
    }
    return;
  }
  const int t0 = c * a.chunk;
  const int t1 = min(seq, t0 + a.chunk);

  // Decoder slot via the device registry keyed by the request's first block.
  const int blk0 = a.bt[(int64_t)r * a.bt_row_stride];
  int dslot = -1;
  if (blk0 >= 0 && blk0 < a.num_blocks) dslot = a.dec_map[blk0];
  if (dslot < 0 || dslot >= a.n_dec_slots) {
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    if (c == 0)
      for (int i = tid; i < G * kD; i += kThreads)
        store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G) * kD + i, NAN);
    return;
  }

  // ---- decoder fragments (A operand, M = dims, K = r1), hi/lo fp16, resident in registers.
  const int HD = g.H * kD;
  const float* dec = a.dec_pool + (int64_t)dslot * g.r1 * HD + h * kD;
  half8 ahi[2][KSTEPS], alo[2][KSTEPS];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int dim = 16 * (wv + 4 * mi) + n;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ar = 32 * s + 8 * gq + j;
        const float f = ar < g.r1 ? dec[(int64_t)ar * HD + dim] : 0.f;
        const _Float16 hi = (_Float16)f;
        ahi[mi][s][j] = hi;
        alo[mi][s][j] = (_Float16)(f - (float)hi);
      }
    }
  }

  // ---- query: this lane's 8 dims for each of the G heads of KV head h.
  const int dl = 16 * wv + 4 * gq;
  float ql[G][4], qh[G][4];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const int64_t qb = qrow * a.q_row_stride + (int64_t)(h * G + p) * kD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ql[p][i] = load_act(a.q, a.q_dtype, qb + dl + i);
      qh[p][i] = load_act(a.q, a.q_dtype, qb + 64 + dl + i);
    }
  }

  float o[G][8];
#pragma unroll
  for (int p = 0; p < G; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) o[p][i] = 0.f;
  float m_run[G], l_run[G];  // meaningful in wave 0
#pragma unroll
  for (int p = 0; p < G; ++p) {
    m_run[p] = -INFINITY;
    l_run[p] = 0.f;
  }

  constexpr int kCoefPerPart = KSTEPS * 8;  // coefficients staged per thread (4 threads/token)
  const int k_row_off = g.k_field + h * g.k_row;
  const int v_row_off = g.k_slot + h * g.v_row;

  for (int tt = t0; tt < t1; tt += kTile) {
    const int ntile = min(kTile, t1 - tt);
    // ---------------------------------------------------------------- stage
    {
      const int tok = tid >> 2;
      const int part = tid & 3;
      const uint8_t* base = nullptr;
      if (tok < ntile) {
        const int pos = tt + tok;
        const int bi = pos / a.block_size;
        const int blk = a.bt[(int64_t)r * a.bt_row_stride + bi];
        const int64_t slot = (int64_t)blk * a.block_size + (pos - bi * a.block_size);
        if (blk < 0 || blk >= a.num_blocks || slot >= a.n_slots) {
          if (part == 0) atomicOr(a.err, TTKV_ERR_BAD_BLOCK);
        } else {
          base = a.page + slot * a.slot_stride;
        }
      }
      uint32_t* cdst = (uint32_t*)&S.coef[tok][part * kCoefPerPart];
      if (base) {
        const uint32_t* csrc = (const uint32_t*)(base + part * kCoefPerPart);
#pragma unroll
        for (int dw = 0; dw < kCoefPerPart / 4; ++dw) {
          const int b0 = part * kCoefPerPart + dw * 4;
          uint32_t x = csrc[dw];
          const int keep = g.r1 - b0;  // bytes of this dword that are coefficients
          if (keep <= 0) x = 0;
          else if (keep < 4) x &= (1u << (8 * keep)) - 1u;
          uint32_t p01, p23;
          i8x4_to_f16(x, p01, p23);
          cdst[2 * dw] = p01;
          cdst[2 * dw + 1] = p23;
        }
        if (part == 0) {
          const uint32_t lo = base[g.coeff_bytes], hi = base[g.coeff_bytes + 1];
          S.cs[tok] = f16_bits_to_float(lo | (hi << 8));
        }
        copy_row_realign(base + k_row_off, g.k_row, S.u.raw.rawk[tok], part, 4);
        copy_row_realign(base + v_row_off, g.v_row, S.u.raw.rawv[tok], part, 4);
      } else {
#pragma unroll
        for (int dw = 0; dw < kCoefPerPart / 2; ++dw) cdst[dw] = 0u;
        if (part == 0) S.cs[tok] = 0.f;
        for (int dw = part; dw < kRawDw; dw += 4) {
          S.u.raw.rawk[tok][dw] = 0u;
          S.u.raw.rawv[tok][dw] = 0u;
        }
      }
    }
    __syncthreads();
    // ---------------------------------------------------------------- decode (thread = half row)
    {
      const int kind = tid >> 7;          // waves 0,1: K rows; waves 2,3: V rows
      const int tok = (tid >> 1) & 63;
      const int half = tid & 1;
      if (kind == 0) {
        const uint8_t* row = (const uint8_t*)S.u.raw.rawk[tok];
        const int rb = 16 + g.k_pb;
        const float ruler = f16_bits_to_float((uint32_t)row[rb] | ((uint32_t)row[rb + 1] << 8));
        decode_half_row<RB>(row, half, [&](int d0, const uint32_t* cd) {
          float4v v0, v1;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            v0[k] = (float)((int)cd[k] - (1 << (RB - 1))) * ruler;
            v1[k] = (float)((int)cd[4 + k] - (1 << (RB - 1))) * ruler;
          }
          *(float4v*)&S.kres[tok][d0] = v0;
          *(float4v*)&S.kres[tok][d0 + 4] = v1;
        });
      } else {
        const uint8_t* row = (const uint8_t*)S.u.raw.rawv[tok];
        const int rb = 16 + g.v_pb;
        if (half == 0)
          S.vrul[tok] = f16_bits_to_float((uint32_t)row[rb] | ((uint32_t)row[rb + 1] << 8));
        decode_half_row<VB>(row, half, [&](int d0, const uint32_t* cd) {
          half8 v;
#pragma unroll
          for (int k = 0; k < 8; ++k) v[k] = (_Float16)(float)((int)cd[k] - (1 << (VB - 1)));
          *(half8*)&S.vval[tok][d0] = v;
        });
      }
    }
    __syncthreads();
    // ---------------------------------------------------------------- recon + rope + q.k
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int tok = 16 * nb + n;
      float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const half8 b = *(const half8*)&S.coef[tok][32 * s + 8 * gq];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0][s], b, acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0][s], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1][s], b, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1][s], b, acc1, 0, 0, 0);
      }
      const float cs = S.cs[tok];
      const float4v rl = *(const float4v*)&S.kres[tok][dl];
      const float4v rh = *(const float4v*)&S.kres[tok][64 + dl];
      const int pos = tok < ntile ? tt + tok : tt;
      const float4v cv = *(const float4v*)&a.cs_cache[(int64_t)pos * kD + dl];
      const float4v sv = *(const float4v*)&a.cs_cache[(int64_t)pos * kD + 64 + dl];
      float yl[4], yh[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float kl = fmaf(cs, acc0[i], rl[i]);
        const float kh = fmaf(cs, acc1[i], rh[i]);
        yl[i] = kl * cv[i] - kh * sv[i];
        yh[i] = kh * cv[i] + kl * sv[i];
      }
#pragma unroll
      for (int p = 0; p < G; ++p) {
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          part = fmaf(ql[p][i], yl[i], part);
          part = fmaf(qh[p][i], yh[i], part);
        }
        part += __shfl_xor(part, 16);
        part += __shfl_xor(part, 32);
        if (gq == 0) S.u.sm.spart[wv][tok][p] = part;
      }
    }
    __syncthreads();
    // ---------------------------------------------------------------- online softmax (wave 0)
    if (wv == 0) {
      const int tok = lane;
      const bool valid = tok < ntile;
#pragma unroll
      for (int p = 0; p < G; ++p) {
        float s = S.u.sm.spart[0][tok][p] + S.u.sm.spart[1][tok][p] + S.u.sm.spart[2][tok][p] +
                  S.u.sm.spart[3][tok][p];
        s = valid ? s * a.scale_log2 : -INFINITY;
        const float mt = wave_max(s);
        const float mn = fmaxf(m_run[p], mt);
        const float alpha = exp2f(m_run[p] - mn);
        const float pr = valid ? exp2f(s - mn) : 0.f;
        l_run[p] = l_run[p] * alpha + wave_sum(pr);
        m_run[p] = mn;
        S.u.sm.pw[p][tok] = pr * S.vrul[tok];
        if (lane == 0) S.u.sm.alpha[p] = alpha;
      }
    }
    __syncthreads();
    // ---------------------------------------------------------------- P.V
    {
      float al[G];
#pragma unroll
      for (int p = 0; p < G; ++p) al[p] = S.u.sm.alpha[p];
#pragma unroll
      for (int p = 0; p < G; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[p][i] *= al[p];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int tok = 16 * nb + n;
        _Float16 v[8];
        __builtin_memcpy(&v[0], &S.vval[tok][dl], 8);
        __builtin_memcpy(&v[4], &S.vval[tok][64 + dl], 8);
#pragma unroll
        for (int p = 0; p < G; ++p) {
          const float pw = S.u.sm.pw[p][tok];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[p][i] = fmaf(pw, (float)v[i], o[p][i]);
        }
      }
    }
    __syncthreads();
  }

  // ---- reduce o over the 16 token lanes of each lane group
#pragma unroll
  for (int p = 0; p < G; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = o[p][i];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      v += __shfl_xor(v, 8);
      o[p][i] = v;
    }
  if (wv == 0 && lane == 0) {
#pragma unroll
    for (int p = 0; p < G; ++p) {
      S.u.sm.m[p] = m_run[p];
      S.u.sm.l[p] = l_run[p];
    }
  }
  __syncthreads();

  if (n_chunks == 1) {
    if (n == 0) {
#pragma unroll
      for (int p = 0; p < G; ++p) {
        const float inv = 1.f / S.u.sm.l[p];
        const int64_t ob = qrow * a.out_row_stride + (int64_t)(h * G + p) * kD;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          store_act(a.out, a.out_dtype, ob + dl + i, o[p][i] * inv);
          store_act(a.out, a.out_dtype, ob + 64 + dl + i, o[p][4 + i] * inv);
        }
      }
    }
    return;
  }

  // ---- split-K partial: [G][kD + 2] per (r, h, c): unnormalised o, running max, running sum
  const int64_t pstride = (int64_t)G * (kD + 2);
  float* part = a.ws_part + ((int64_t)(r * g.H + h) * a.max_chunks + c) * pstride;
  if (n == 0) {
#pragma unroll
    for (int p = 0; p < G; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        part[p * (kD + 2) + dl + i] = o[p][i];
        part[p * (kD + 2) + 64 + dl + i] = o[p][4 + i];
      }
  }
  if (tid < G) {
    part[tid * (kD + 2) + kD] = S.u.sm.m[tid];
    part[tid * (kD + 2) + kD + 1] = S.u.sm.l[tid];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&a.ws_cnt[r * g.H + h], 1);
    S.is_last = (prev == n_chunks - 1);
  }
  __syncthreads();
  if (!S.is_last) return;
  __threadfence();
  const float* pbase = a.ws_part + (int64_t)(r * g.H + h) * a.max_chunks * pstride;
  for (int it = tid; it < G * kD; it += kThreads) {
    const int p = it / kD;
    const int dim = it - p * kD;
    float M = -INFINITY;
    for (int cc = 0; cc < n_chunks; ++cc) M = fmaxf(M, pbase[cc * pstride + p * (kD + 2) + kD]);
    float L = 0.f, O = 0.f;
    for (int cc = 0; cc < n_chunks; ++cc) {
      const float* pc = pbase + cc * pstride + p * (kD + 2);
      const float f = exp2f(pc[kD] - M);
      L = fmaf(pc[kD + 1], f, L);
      O = fmaf(pc[dim], f, O);
    }
    store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G + p) * kD + dim,
              O / L);
  }
  if (tid == 0) a.ws_cnt[r * g.H + h] = 0;
}

}  // namespace ttkv

// ------------------------------------------------------------------------------------ host side
#include "ttkv_host.h"

namespace ttkv {

template <int G, int RB, int VB, int KSTEPS>
static int launch_decode_t(const DecodeArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(DecodeSmem<KSTEPS>);
  auto kfn = decode_paged_kernel<G, RB, VB, KSTEPS>;
  static bool attr_set = false;  // per instantiation; benign race (idempotent)
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kfn, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)smem) != hipSuccess)
      return host_fail(TTKV_E_LAUNCH, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
    attr_set = true;
  }
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host_fail(TTKV_E_LAUNCH, std::string("decode launch: ") +
                                                           hipGetErrorString(e));
  return TTKV_OK;
}

template <int RB, int VB, int KSTEPS>
static int dispatch_g(const DecodeArgs& a, int grid, hipStream_t st) {
  switch (a.G) {
    case 1: return launch_decode_t<1, RB, VB, KSTEPS>(a, grid, st);
    case 2: return launch_decode_t<2, RB, VB, KSTEPS>(a, grid, st);
    case 3: return launch_decode_t<3, RB, VB, KSTEPS>(a, grid, st);
    case 4: return launch_decode_t<4, RB, VB, KSTEPS>(a, grid, st);
    case 8: return launch_decode_t<8, RB, VB, KSTEPS>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "num_heads / H = " + std::to_string(a.G) +
                                           " query heads per KV head is not built (1,2,3,4,8)");
}

template <int RB, int VB>
static int dispatch_k(const DecodeArgs& a, int ksteps, int grid, hipStream_t st) {
  switch (ksteps) {
    case 2: return dispatch_g<RB, VB, 2>(a, grid, st);
    case 4: return dispatch_g<RB, VB, 4>(a, grid, st);
    case 5: return dispatch_g<RB, VB, 5>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
}

int decode_chunk_for(int num_reqs, int H, int max_seq_len) {
  const int64_t work = (int64_t)num_reqs * H * std::max(max_seq_len, 1);
  const int64_t target = 4LL * device_cu_count();
  int64_t chunk = (work + target - 1) / target;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  return (int)std::min<int64_t>(std::max<int64_t>(chunk, kTile), 4096);
}

int64_t decode_workspace_bytes(const Geom& g, int G, int num_reqs, int max_seq_len) {
  const int chunk = decode_chunk_for(num_reqs, g.H, max_seq_len);
  const int max_chunks = std::max(1, (max_seq_len + chunk - 1) / chunk);
  const int64_t cnt = ((int64_t)num_reqs * g.H * 4 + 255) / 256 * 256;
  return cnt + (int64_t)num_reqs * g.H * max_chunks * G * (kD + 2) * 4;
}

int decode_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                 int64_t q_row_stride, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                 int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                 const int32_t* seq_lens, const int32_t* qsl, int num_reqs, int max_seq_len,
                 const int32_t* dec_map, int64_t num_blocks, const float* dec_pool,
                 int64_t n_dec_slots, const float* cs_cache, int64_t max_pos, void* out,
                 int out_dtype, int64_t out_row_stride, void* ws, int64_t ws_bytes, int32_t* err,
                 hipStream_t st) {
  if (g.d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (g.qbits != 8) return host_fail(TTKV_E_UNSUPPORTED, "coefficient width must be 8 bits");
  if (!((g.res_bits == 3 && g.v_bits == 3) || (g.res_bits == 4 && g.v_bits == 4)))
    return host_fail(TTKV_E_UNSUPPORTED, "res_bits/v_bits must be 3/3 or 4/4");
  if (HQ <= 0 || HQ % g.H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  const int G = HQ / g.H;
  const int ksteps = g.r1 <= 64 ? 2 : g.r1 <= 128 ? 4 : g.r1 <= 160 ? 5 : 0;
  if (!ksteps) return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
  if (ksteps * 32 > g.k_slot)
    return host_fail(TTKV_E_UNSUPPORTED, "padded coefficient block exceeds the K slot");
  if (!q || !page || !bt || !seq_lens || !qsl || !dec_map || !dec_pool || !cs_cache || !out || !err)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if ((uintptr_t)page % 16 || slot_stride % 16 || slot_stride < g.blob)
    return host_fail(TTKV_E_INVALID,
                     "page must be 16-byte aligned with a slot stride that is a multiple of 16 and "
                     ">= the blob (" + std::to_string(g.blob) + " bytes)");
  if ((uintptr_t)cs_cache % 16) return host_fail(TTKV_E_INVALID, "cos_sin_cache not 16-aligned");
  if (q_dtype < 0 || q_dtype > 2 || out_dtype < 0 || out_dtype > 2)
    return host_fail(TTKV_E_INVALID, "dtype code");
  if (block_size <= 0) return host_fail(TTKV_E_INVALID, "block_size");
  if (num_reqs < 0 || max_seq_len < 0) return host_fail(TTKV_E_INVALID, "negative batch size");
  if (num_reqs == 0) return TTKV_OK;
  if ((int64_t)max_blocks * block_size < max_seq_len)
    return host_fail(TTKV_E_INVALID, "max_seq_len=" + std::to_string(max_seq_len) +
                                         " needs more blocks than the block table row holds");
  if (max_seq_len > max_pos)
    return host_fail(TTKV_E_INVALID, "position " + std::to_string(max_seq_len - 1) +
                                         " is past the model's cos_sin_cache (" +
                                         std::to_string(max_pos) + " entries)");
  DecodeArgs a{};
  a.g = g;
  a.HQ = HQ;
  a.G = G;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_row_stride = q_row_stride;
  a.page = page;
  a.n_slots = n_slots;
  a.slot_stride = slot_stride;
  a.block_size = block_size;
  a.bt = bt;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.qsl = qsl;
  a.num_reqs = num_reqs;
  a.dec_map = dec_map;
  a.num_blocks = num_blocks;
  a.dec_pool = dec_pool;
  a.n_dec_slots = n_dec_slots;
  a.cs_cache = cs_cache;
  a.max_pos = max_pos;
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_row_stride = out_row_stride;
  a.err = err;
  a.chunk = decode_chunk_for(num_reqs, g.H, max_seq_len);
  a.max_chunks = std::max(1, (max_seq_len + a.chunk - 1) / a.chunk);
  if (a.max_chunks > 1) {
    const int64_t need = decode_workspace_bytes(g, G, num_reqs, max_seq_len);
    if (!ws || ws_bytes < need)
      return host_fail(TTKV_E_WORKSPACE, "decode workspace needs " + std::to_string(need) +
                                             " bytes, got " + std::to_string(ws_bytes));
    if ((uintptr_t)ws % 256) return host_fail(TTKV_E_INVALID, "workspace not 256-byte aligned");
    const int64_t cnt = ((int64_t)num_reqs * g.H * 4 + 255) / 256 * 256;
    a.ws_cnt = (int*)ws;
    a.ws_part = (float*)((char*)ws + cnt);
  }
  a.max_seq = max_seq_len;
  a.nwork = num_reqs * a.max_chunks * g.H;
  const int grid = (a.nwork + 7) / 8 * 8;
  if (g.res_bits == 3) return dispatch_k<3, 3>(a, ksteps, grid, st);
  return dispatch_k<4, 4>(a, ksteps, grid, st);
}

}  // namespace ttkv

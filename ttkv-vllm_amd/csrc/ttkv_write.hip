// K3: write/encode of new tokens into compressed slots, one launch for all tokens of a layer.
// gfx950 / CDNA4.
//
// Two launches of 256-thread workgroups, so a decode batch of B tokens spreads its B x 450 KB of
// pinv and B x 113 KB of decoder reads over many CUs:
//   K3a project  one workgroup per (token, 4 ranks): c[a] for its ranks over all H*d
//             dims, complete in the workgroup (wave sums, fixed order), left in the workspace
//                                                                  -- skipped when a fit gives (cq, cs)
//   K3b pack     one workgroup per (token, KV head): every head's workgroup quantises c alike,
//             then the rest for its head:
//   project   c[a] = sum_m M[m] * pinv[m][a], M = the token's raw key flattened m = h*d + j
//             (encode.py:322-324), fp32 in a fixed order          -- or take (cq, cs) from a fit
//   quantise  cs = max|c| * fp32(1/127) (1 if 0); cq = clamp(rint(c / cs), -128, 127)
//             (encode.py:328-332; the fp32 reciprocal multiply is torch-CUDA's scalar division,
//             select_triton.py:76-84; c/cs is a correctly rounded division)
//   residual  R[h][j] = K[h][j] - sum_a (cq[a]*cs) * decoder_f[a][h*d+j]   (encode.py:334-336)
//   rows      for every head: K residual row from R, V row from the value; each row picks exactly
//             k lanes by magnitude (ties -> lowest lane, select_triton.py:181-193), ruler =
//             rowmax * fp32(1/(2^(b-1)-1)) (1 * that if rowmax == 0), q = clamp(rint(x / ruler)),
//             bitmap MSB-first, codes MSB-first in lane order, fp16 ruler LE
//             (ttkv_packed_cache.py:203-231, select_triton.py:195-232)
//   store     coefficients, fp16 coefficient ruler, H K rows, H V rows, zero padding: the
//             bytes layout.pack_k_slots/pack_v_slots produce (layout.py:161-239), written at
//             slot_mapping[i] (encode.py:471-508).
// Selection, quantisation and packing are bit-exact functions of their float inputs (R and the
// value); the projection and reconstruction sums are fp32 with an implementation-defined order,
// as in the reference. Optional outputs expose c and R so tests can pin the bytes from there.
#include <math.h>

#include "ttkv_host.h"

namespace ttkv {

constexpr int kWThreads = 256;

struct WriteArgs {
  Geom g;
  const void* key;
  int k_dtype;
  int64_t k_row_stride;
  const void* val;
  int v_dtype;
  int64_t v_row_stride;
  const int64_t* slot_mapping;
  int num_tokens;
  const int32_t* qsl;
  int num_reqs;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* dec_map;
  int64_t num_blocks;
  const int8_t* dec_q;  // decoder pool (see dec_ranks)
  const float* dec_scale;
  const float* pinv_pool;
  int64_t n_dec_slots;
  int32_t* dec_used;  // [n_dec_slots] or null: set to 1 for every decoder slot a token uses
  const int8_t* cq_in;
  const float* cs_in;
  uint8_t* page;
  int64_t n_slots, slot_stride;
  float* c_out;
  float* r_out;
  int* err;
  int tok0;         // first token of this launch (tokens tok0 .. tok0 + num_tokens - 1)
  float* ws_c;      // [num_tokens][r1] each token's projection c, from K3a for K3b
  int* ws_ds;       // [num_tokens] each token's decoder slot (or -1), from K3a for K3b
  float inv127, inv_rk, inv_rv;
};

// Request of token i (qsl[r] <= i < qsl[r+1]; qsl is non-decreasing) and its decoder slot, or
// -1. Decode tokens come first in a step, one per request, so token i is usually request i: that
// guess, its first block id and the general count (r + 1 = the number of qsl[0..num_reqs) <= i,
// 64 per lane with one load each) are requested in one round trip; a confirmed guess leaves only
// the decoder map's round trip (two in all instead of three). Every lane of the wave must call
// it; all get the same answer.
__device__ int token_decoder(const WriteArgs& a, int i) {
  const int lane = threadIdx.x & 63;
  const bool guess = i < a.num_reqs;
  const int glo = guess ? a.qsl[i] : 0, ghi = guess ? a.qsl[i + 1] : 0;
  const int gblk = guess ? a.bt[(int64_t)i * a.bt_row_stride] : -1;
  int cnt = 0;
  for (int j0 = 0; j0 < a.num_reqs; j0 += 64) {
    const int j = j0 + lane;
    cnt += __builtin_popcountll(__ballot(j < a.num_reqs && a.qsl[j] <= i));
  }
  int blk0 = -1;
  if (guess && glo <= i && i < ghi) {
    blk0 = gblk;
  } else {
    const int r = cnt - 1;
    if (r >= 0 && i < a.qsl[r + 1]) blk0 = a.bt[(int64_t)r * a.bt_row_stride];
  }
  const int ds = blk0 >= 0 && blk0 < a.num_blocks ? a.dec_map[blk0] : -1;
  return (ds < 0 || ds >= a.n_dec_slots) ? -1 : ds;
}

// Exact top-k select + quantise + pack of one 128-lane row held as lane l: x0 = dim l,
// x1 = dim l+64. Writes bitmap, codes and fp16 ruler at dst (any alignment). `codes` is this
// wave's LDS scratch. Every lane of the wave must call it.
template <int BITS>
__device__ void pack_row(float x0, float x1, int k, float inv_ruler, uint8_t* dst,
                         uint8_t* codes) {
  constexpr int OFF = 1 << (BITS - 1);
  const int lane = threadIdx.x & 63;
  const uint32_t u0 = __builtin_bit_cast(uint32_t, fabsf(x0));
  const uint32_t u1 = __builtin_bit_cast(uint32_t, fabsf(x1));
  // k-th largest magnitude by bit construction on the (monotone) magnitude bit pattern.
  uint32_t t = 0;
  for (int b = 30; b >= 0; --b) {
    const uint32_t cand = t | (1u << b);
    const int cnt = __builtin_popcountll(__ballot(u0 >= cand)) +
                    __builtin_popcountll(__ballot(u1 >= cand));
    if (cnt >= k) t = cand;
  }
  const uint64_t above0 = __ballot(u0 > t), above1 = __ballot(u1 > t);
  const int need = k - (__builtin_popcountll(above0) + __builtin_popcountll(above1));
  const uint64_t tie0 = __ballot(u0 == t), tie1 = __ballot(u1 == t);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int tr0 = __builtin_popcountll(tie0 & below);
  const int tr1 = __builtin_popcountll(tie0) + __builtin_popcountll(tie1 & below);
  const bool s0 = (u0 > t) || (u0 == t && tr0 < need);
  const bool s1 = (u1 > t) || (u1 == t && tr1 < need);
  const uint64_t sel0 = __ballot(s0), sel1 = __ballot(s1);
  // Row max (always kept when k >= 1), as bits: non-negative floats order like their bits.
  uint32_t mx = u0 > u1 ? u0 : u1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t other = __shfl_xor(mx, o);
    mx = other > mx ? other : mx;
  }
  const float rmax = __builtin_bit_cast(float, mx);
  const float sc = (rmax == 0.f ? 1.f : rmax) * inv_ruler;
  // Codes, by rank (lane order).
  const int rank0 = __builtin_popcountll(sel0 & below);
  const int rank1 = __builtin_popcountll(sel0) + __builtin_popcountll(sel1 & below);
  if (s0) {
    const float q = fminf(fmaxf(rintf(__fdiv_rn(x0, sc)), (float)-OFF), (float)(OFF - 1));
    codes[rank0] = (uint8_t)((int)q + OFF);
  }
  if (s1) {
    const float q = fminf(fmaxf(rintf(__fdiv_rn(x1, sc)), (float)-OFF), (float)(OFF - 1));
    codes[rank1] = (uint8_t)((int)q + OFF);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int pb = (k * BITS + 7) / 8;
  // Bitmap: byte m holds dims 8m..8m+7, dim 8m at bit 7.
  if (lane < 16) {
    const uint64_t sel = lane < 8 ? sel0 : sel1;
    const uint32_t byte = (uint32_t)(sel >> (8 * (lane & 7))) & 0xffu;
    dst[lane] = (uint8_t)(__builtin_bitreverse32(byte) >> 24);
  }
  // Code stream: byte b = stream bits [8b, 8b+8), MSB first, zero beyond k codes.
  if (lane < pb) {
    uint32_t byte = 0;
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const int p = 8 * lane + bit;
      const int ci = p / BITS;
      const uint32_t code = ci < k ? codes[ci] : 0u;
      byte |= ((code >> (BITS - 1 - (p - ci * BITS))) & 1u) << (7 - bit);
    }
    dst[16 + lane] = (uint8_t)byte;
  }
  if (lane == 0) {
    const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)sc);
    dst[16 + pb] = (uint8_t)(hb & 0xff);
    dst[16 + pb + 1] = (uint8_t)(hb >> 8);
  }
}

// Scale of a 4-bit coefficient group whose largest magnitude is m: m / 7 (IEEE) rounded up to 8
// significant bits, then held within [2^-14, 9344], so that every q * scale (|q| <= 7) is an
// exact fp16 normal; 0 for an all-zero group.
__device__ inline float coef_group_scale(float m) {
  if (!(m > 0.f)) return 0.f;
  uint32_t u = __builtin_bit_cast(uint32_t, __fdiv_rn(m, 7.f));
  if (u & 0xffffu) u = (u & ~0xffffu) + 0x10000u;
  return fminf(fmaxf(__builtin_bit_cast(float, u), 0x1p-14f), 9344.f);
}

// K3a: the projection c = M_i . pinv of token i, one workgroup per (token, slice of kSliceRanks
// ranks). The pool holds each decoder's pseudo-inverse by rank (pinv_pool [slot][r1][H*d], row a
// = rank a's projection vector), so each wave reads whole rows: kWaveRanks ranks from a0 +
// kWaveRanks * w, each lane 16 of the H*d dims (four 16-byte loads per rank, 1 KB per wave
// instruction). Slices of 16 / 8 / 4 ranks measured 4.8 / 4.7 / 4.6 us per 8-token launch (more,
// smaller workgroups spread the pinv reads over more CUs). The wave sums each
// rank over its lanes with an xor butterfly, so every rank's sum is complete inside one workgroup
// and nothing is handed between workgroups; K3b quantises.
constexpr int kSliceRanks = 4;
constexpr int kWaveRanks = kSliceRanks / 4;  // ranks per wave

__host__ __device__ inline int project_slices(const Geom& g) {
  return (g.r1 + kSliceRanks - 1) / kSliceRanks;
}

__global__ __launch_bounds__(kWThreads) void write_project_kernel(WriteArgs a) {
  const Geom& g = a.g;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int ns = project_slices(g);
  const int il = blockIdx.x / ns;  // token within this launch: its workspace row
  const int i = a.tok0 + il;
  const int sl = blockIdx.x % ns;
  const int HD = g.H * kD;
  const int64_t slot = a.slot_mapping[i];
  // this lane's key dims 256j + 4 lane .. + 3, requested before the decoder lookup's round trips
  const int64_t kb = (int64_t)i * a.k_row_stride;
  const bool kvec = act_rows_aligned(a.key, a.k_dtype, a.k_row_stride);
  float kx[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int d0 = 256 * j + 4 * lane;
    if (d0 < HD) {
      load_act_n<4>(a.key, a.k_dtype, kb + d0, kvec, kx[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) kx[j][e] = 0.f;
    }
  }
  const int ds = token_decoder(a, i);
  if (sl == 0 && tid == 0) a.ws_ds[il] = ds;
  if (ds < 0 || slot < 0 || slot >= a.n_slots) return;  // K3b reports it
  const int a0 = sl * kSliceRanks + kWaveRanks * wv;
  if (a0 >= g.r1) return;
  const float* prow = a.pinv_pool + (int64_t)ds * g.r1 * HD;
  float4v pv[kWaveRanks][4];
#pragma unroll
  for (int r = 0; r < kWaveRanks; ++r)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = 256 * j + 4 * lane;
      pv[r][j] = (a0 + r < g.r1 && d0 < HD)
                     ? *gbl((const float4v*)(prow + (int64_t)(a0 + r) * HD + d0))
                     : float4v{0.f, 0.f, 0.f, 0.f};
    }
  float acc[kWaveRanks];
#pragma unroll
  for (int r = 0; r < kWaveRanks; ++r) {
    acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r] = fmaf(kx[j][e], pv[r][j][e], acc[r]);
  }
  // butterfly: the same tree in every lane (operands only commuted), so every lane holds the sum
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int r = 0; r < kWaveRanks; ++r) acc[r] += __shfl_xor(acc[r], o);
  if (lane < kWaveRanks && a0 + lane < g.r1) {
    float c = acc[0];
#pragma unroll
    for (int r = 1; r < kWaveRanks; ++r) c = lane == r ? acc[r] : c;
    a.ws_c[(int64_t)il * g.r1 + a0 + lane] = c;
    if (a.c_out) a.c_out[(int64_t)i * g.r1 + a0 + lane] = c;
  }
}

// K3b: residual of head h, then its K row and V row; head 0 also writes the coefficients.
template <int RB, int VB>
__global__ __launch_bounds__(kWThreads) void write_pack_kernel(WriteArgs a) {
  __shared__ __align__(16) float cqs[256];  // c * cs by rank (0 past r1)
  __shared__ __align__(16) float rul[256];  // decoder rank rulers (0 past r1)
  __shared__ float rp[kD];    // sum_a cqs[a] * dec[a][h*d + j]
  __shared__ uint8_t codes[2][kD];
  __shared__ float gsc[8];  // 4-bit mode: group scales
  const Geom& g = a.g;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int il = blockIdx.x / g.H;  // token within this launch: its workspace rows
  const int i = a.tok0 + il;
  const int h = blockIdx.x % g.H;
  const int HD = g.H * kD;
  const int64_t slot = a.slot_mapping[i];
  // Everything up to the decoder lookup depends only on the token index, so it is requested in
  // the same round trip as the slot id (before the PAD test below, which would otherwise wait
  // for the slot id first). The rows wave 0 (key) and wave 1 (value) pack:
  float xr0 = 0.f, xr1 = 0.f;
  if (wv == 0) {
    const int64_t kb = (int64_t)i * a.k_row_stride + h * kD;
    xr0 = load_act(a.key, a.k_dtype, kb + lane);
    xr1 = load_act(a.key, a.k_dtype, kb + 64 + lane);
  } else if (wv == 1) {
    const int64_t vb = (int64_t)i * a.v_row_stride + h * kD;
    xr0 = load_act(a.val, a.v_dtype, vb + lane);
    xr1 = load_act(a.val, a.v_dtype, vb + 64 + lane);
  }
  // the decoder slot from K3a's lookup when it ran; K3a's projection or the fit's coefficients
  const int ds_k3a = a.cq_in ? -1 : a.ws_ds[il];
  // K3a's projection: lane l loads ranks l, l + 64, l + 128, l + 192, so that every wave sees all
  // of them (the int8 ruler's max needs no barrier); thread t's own rank t is among them
  float cw[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = lane + 64 * k;
    cw[k] = (!a.cq_in && r < g.r1) ? a.ws_c[(int64_t)il * g.r1 + r] : 0.f;
  }
  const float cv = wv == 0 ? cw[0] : wv == 1 ? cw[1] : wv == 2 ? cw[2] : cw[3];
  float cs = a.cq_in ? a.cs_in[i] : 1.f;
  float qv = (a.cq_in && tid < g.r1) ? (float)a.cq_in[(int64_t)i * g.r1 + tid] : 0.f;
  // A negative slot id is vLLM's PAD_SLOT_ID (the padded tokens of a replayed graph): nothing
  // is written and nothing is refused, as vLLM's own cache writers skip them. Ids past the
  // cache are refused.
  if (slot < 0) return;
  const bool slot_ok = slot < a.n_slots;
  const int ds = a.cq_in ? token_decoder(a, i) : ds_k3a;
  if (h == 0 && tid == 0) {
    if (!slot_ok) atomicOr(a.err, TTKV_ERR_BAD_SLOT);
    if (ds < 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    // the decoder registry's use flag (its eviction follows the last use, read by the host)
    if (ds >= 0 && a.dec_used) a.dec_used[ds] = 1;
  }
  if (ds < 0 || !slot_ok) return;
  // this head's decoder: wave w owns dims 32w .. 32w + 31; lane l reads column h*d + 32w + l/2,
  // ranks 64 (l & 1) .. + 63 of each 128-rank block (a lane pair reads one whole 128-byte column
  // line), requested before the coefficients are needed. The rank rulers are staged in LDS beside
  // the coefficients (thread t: rank t; r1 <= 256 threads, host-checked).
  const int R = dec_ranks(g.r1);
  const int cdim = 32 * wv + (lane >> 1);
  const int half = lane & 1;
  const int8_t* dcol = a.dec_q + ((int64_t)ds * HD + h * kD + cdim) * R + 64 * half;
  u32x4 dqv[4];
  auto load_ranks = [&](int b0) {
    if (b0 + 64 * half < R) {  // R = 64 (or 192): the second half has no ranks in the last block
#pragma unroll
      for (int c = 0; c < 4; ++c) dqv[c] = *gbl((const u32x4*)(dcol + b0 + 16 * c));
    }
  };
  load_ranks(0);
  if (!a.cq_in) {
    // Quantise the projection (every head's workgroup alike, so all agree): thread t holds rank t
    if (g.coef_mode == kCoefI8) {  // cs = max|c| * fp32(1/127), cq = clamp(rint(c / cs))
      float mx = fmaxf(fmaxf(fabsf(cw[0]), fabsf(cw[1])), fmaxf(fabsf(cw[2]), fabsf(cw[3])));
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      cs = mx * a.inv127;
      if (cs == 0.f) cs = 1.f;
      if (tid < g.r1) qv = fminf(fmaxf(rintf(__fdiv_rn(cv, cs)), -128.f), 127.f);
    } else if (g.coef_mode == kCoefF16) {
      qv = (float)(_Float16)cv;  // round to nearest even
    } else {  // group k = ranks 32k .. 32k+31 = threads 32k .. 32k+31 (half a wave)
      float gm = fabsf(cv);
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) gm = fmaxf(gm, __shfl_xor(gm, o));
      const float sc = coef_group_scale(gm);
      if (tid < g.r1) qv = sc > 0.f ? fminf(fmaxf(rintf(__fdiv_rn(cv, sc)), -7.f), 7.f) * sc : 0.f;
      if ((tid & 31) == 0 && tid < g.r1) gsc[tid >> 5] = sc;
    }
  }
  if (tid < R) {
    rul[tid] = tid < g.r1 ? a.dec_scale[(int64_t)ds * R + tid] : 0.f;
    cqs[tid] = qv * cs;  // qv = 0 past r1
  }
  uint8_t* base = a.page + slot * a.slot_stride;
  if (h == 0) {
    if (g.coef_mode == kCoefI8) {
      if (tid < g.r1) base[tid] = (uint8_t)(int8_t)(int)qv;
      if (tid == 0) {
        const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)cs);
        base[g.coeff_bytes] = (uint8_t)(hb & 0xff);
        base[g.coeff_bytes + 1] = (uint8_t)(hb >> 8);
      }
    } else if (g.coef_mode == kCoefF16) {
      if (tid < g.r1) {  // qv is an fp16 value: the conversion is exact
        const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)qv);
        base[2 * tid] = (uint8_t)(hb & 0xff);
        base[2 * tid + 1] = (uint8_t)(hb >> 8);
      }
    }
    for (int b = g.k_field + g.H * g.k_row + tid; b < g.k_slot; b += kWThreads) base[b] = 0;
    for (int b = g.k_slot + g.H * g.v_row + tid; b < g.blob; b += kWThreads) base[b] = 0;
  }
  __syncthreads();
  if (g.coef_mode == kCoefI4G32 && h == 0 && tid < g.coef_groups) {  // the group scales (exact)
    const uint16_t hb = __builtin_bit_cast(uint16_t, (_Float16)gsc[tid]);
    base[g.coeff_bytes + 2 * tid] = (uint8_t)(hb & 0xff);
    base[g.coeff_bytes + 2 * tid + 1] = (uint8_t)(hb >> 8);
  }
  if (g.coef_mode == kCoefI4G32 && h == 0 && tid < g.coeff_bytes) {
    // byte b of word w = b / 4 holds the nibbles of ranks lo (bits 0-3) and lo + 2 (bits 4-7):
    // lo = 8w + 4j for byte j < 2 of the word, 8w + 4j - 7 for j >= 2; q = value / scale exactly
    const int j = tid & 3;
    const int lo = 8 * (tid >> 2) + (j < 2 ? 4 * j : 4 * j - 7);
    uint32_t byte = 0;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = lo + 2 * e;
      if (r < g.r1) {
        const float sc = gsc[r >> 5];
        const int q = sc > 0.f ? (int)rintf(__fdiv_rn(cqs[r], sc)) : 0;
        byte |= ((uint32_t)q & 15u) << (4 * e);
      }
    }
    base[tid] = (uint8_t)byte;
  }
  // R[j] = K[h*d+j] - sum_a cqs[a] * dec[a][h*d+j], dec = float(q) * ruler exactly: each lane sums
  // its ranks in increasing order, then the two halves of the column are added
  float acc = 0.f;
  for (int b0 = 0; b0 < R; b0 += 128) {
    if (b0) load_ranks(b0);
    const int r0 = b0 + 64 * half;
    if (r0 < R) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int r = r0 + 16 * c + 4 * m;
          const float4v c4 = *(const float4v*)&cqs[r];
          float d[4];
          dec_values4(dqv[c][m], *(const float4v*)&rul[r], d);
#pragma unroll
          for (int k = 0; k < 4; ++k) acc = fmaf(c4[k], d[k], acc);
        }
    }
  }
  acc += __shfl_xor(acc, 1);
  if (half == 0) rp[cdim] = acc;
  __syncthreads();
  if (wv == 0) {
    const float r0 = xr0 - rp[lane];
    const float r1v = xr1 - rp[64 + lane];
    if (a.r_out) {
      a.r_out[(int64_t)i * HD + h * kD + lane] = r0;
      a.r_out[(int64_t)i * HD + h * kD + 64 + lane] = r1v;
    }
    pack_row<RB>(r0, r1v, g.res_k, a.inv_rk, base + g.k_field + h * g.k_row, codes[0]);
  } else if (wv == 1) {
    pack_row<VB>(xr0, xr1, g.v_lanes, a.inv_rv, base + g.k_slot + h * g.v_row, codes[1]);
  }
}

static float inv_ruler_f32(int bits) { return (float)(1.0 / (double)((1 << (bits - 1)) - 1)); }

// Workspace: the shared 64 KiB counter region (unused here; kept so that one buffer can serve
// every entry point), then per token of a launch its projection (r1 floats) and decoder slot.
// Launches take at most kMaxCounters tokens each.
int64_t write_workspace_bytes(const Geom& g, int num_tokens) {
  const int64_t nt = std::min(std::max(num_tokens, 0), kMaxCounters);
  return kCounterBytes + nt * (g.r1 + 1) * 4;
}

int write_paged(const Geom& g, const void* key, int k_dtype, int64_t k_row_stride, const void* val,
                int v_dtype, int64_t v_row_stride, const int64_t* slot_mapping, int num_tokens,
                const int32_t* qsl, int num_reqs, const int32_t* bt, int64_t bt_row_stride,
                const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                const float* dec_scale, const float* pinv_pool, int64_t n_dec_slots,
                int32_t* dec_used, const int8_t* cq_in, const float* cs_in, uint8_t* page,
                int64_t n_slots, int64_t slot_stride, float* c_out, float* r_out, void* ws,
                int64_t ws_bytes, int32_t* err, hipStream_t st) {
  if (g.d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (g.H > 8) return host_fail(TTKV_E_UNSUPPORTED, "H > 8 KV heads is not built");
  if (g.r1 > 256) return host_fail(TTKV_E_UNSUPPORTED, "r1 > 256 is not built");
  if (g.res_k < 1) return host_fail(TTKV_E_UNSUPPORTED, "res_k must be >= 1");
  if (!((g.res_bits == 3 && g.v_bits == 3) || (g.res_bits == 4 && g.v_bits == 4)))
    return host_fail(TTKV_E_UNSUPPORTED, "res_bits/v_bits must be 3/3 or 4/4");
  if (!key || !val || !slot_mapping || !qsl || !bt || !dec_map || !page || !err)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (!cq_in && !pinv_pool) return host_fail(TTKV_E_INVALID, "need pinv_pool or coeff_q_in");
  if (cq_in && !cs_in) return host_fail(TTKV_E_INVALID, "coeff_q_in needs coeff_scale_in");
  if (cq_in && g.coef_mode != kCoefI8)
    return host_fail(TTKV_E_INVALID, "coeff_q_in is int8: the fp16 and 4-bit coefficient modes "
                                     "quantise the projection themselves (pass pinv_pool)");
  if (slot_stride < g.blob) return host_fail(TTKV_E_INVALID, "slot stride smaller than the blob");
  if (k_dtype < 0 || k_dtype > 2 || v_dtype < 0 || v_dtype > 2)
    return host_fail(TTKV_E_INVALID, "dtype code");
  if (num_tokens < 0 || num_reqs < 0) return host_fail(TTKV_E_INVALID, "negative size");
  if (num_tokens == 0) return TTKV_OK;
  if (!cq_in) {
    const int64_t need = write_workspace_bytes(g, num_tokens);
    if (!ws || ws_bytes < need || (uintptr_t)ws % 256)
      return host_fail(TTKV_E_WORKSPACE, "write workspace needs " + std::to_string(need) +
                                             " bytes (256-aligned), got " +
                                             std::to_string(ws_bytes));
  }
  if (int rc = check_dec_pool(dec_q, dec_scale)) return rc;
  WriteArgs a{};
  a.g = g;
  a.key = key;
  a.k_dtype = k_dtype;
  a.k_row_stride = k_row_stride;
  a.val = val;
  a.v_dtype = v_dtype;
  a.v_row_stride = v_row_stride;
  a.slot_mapping = slot_mapping;
  a.num_tokens = num_tokens;
  a.qsl = qsl;
  a.num_reqs = num_reqs;
  a.bt = bt;
  a.bt_row_stride = bt_row_stride;
  a.dec_map = dec_map;
  a.num_blocks = num_blocks;
  a.dec_q = dec_q;
  a.dec_scale = dec_scale;
  a.pinv_pool = pinv_pool;
  a.n_dec_slots = n_dec_slots;
  a.dec_used = dec_used;
  a.cq_in = cq_in;
  a.cs_in = cs_in;
  a.page = page;
  a.n_slots = n_slots;
  a.slot_stride = slot_stride;
  a.c_out = c_out;
  a.r_out = r_out;
  a.err = err;
  a.inv127 = inv_ruler_f32(8);
  a.inv_rk = inv_ruler_f32(g.res_bits);
  a.inv_rv = inv_ruler_f32(g.v_bits);
  for (int t0 = 0; t0 < num_tokens; t0 += kMaxCounters) {
    WriteArgs b = a;
    b.tok0 = t0;
    b.num_tokens = std::min(kMaxCounters, num_tokens - t0);
    if (!cq_in) {
      b.ws_c = (float*)((char*)ws + kCounterBytes);
      b.ws_ds = (int*)(b.ws_c + (int64_t)b.num_tokens * g.r1);
    }
    const int grid = b.num_tokens * g.H;
    if (!cq_in)
      hipLaunchKernelGGL(write_project_kernel, dim3(b.num_tokens * project_slices(g)),
                         dim3(kWThreads), 0, st, b);
    if (g.res_bits == 3)
      hipLaunchKernelGGL((write_pack_kernel<3, 3>), dim3(grid), dim3(kWThreads), 0, st, b);
    else
      hipLaunchKernelGGL((write_pack_kernel<4, 4>), dim3(grid), dim3(kWThreads), 0, st, b);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host_fail(TTKV_E_LAUNCH, std::string("write launch: ") +
                                                          hipGetErrorString(e));
  return TTKV_OK;
}

}  // namespace ttkv

// Reads of the codec's pooled CONTAINER layout (not slots): the drop-in for the codec's fused
// container kernels `ttkv_krt` and `ttkv_v_out` (codec/ttkv_kernels.cu; launched by
// codec/ttkv_cuda.py:144-257). gfx950 / CDNA4.
//
// Container (codec/ttkv_packed_cache.py:337-385, pooled over B sequences of n tokens each):
//   coefficients  coeff_q [B*n, r1] int8, coeff_scale [B*n]           row = b*n + i
//   decoder       decoder_f [r1, H*d] fp32 (shared) or [B, r1, H*d]    = dec_q * dec_scale
//   residual rows bitmap [B*H*n, d/8], packed [B*H*n, PB], scale [B*H*n]  row = b*H*n + h*n + i
//   V rows        the same three arrays for V.
// Semantics (vllm_ttkv/reference.py:47-109, per row its own absolute position i):
//   krt   : s[b, p, i] = q[b, p] . RoPE_i( (cq[i] * cs[i]) @ decoder_f[:, h(p)*d:(h(p)+1)*d]
//                                          + residual[h(p), i] )            (unscaled, fp32)
//   v_out : o[b, p, :] = sum_i p[b, p, i] * V[b, h(p), i, :]
//
// Both reuse the decode read's machinery. A 256-thread workgroup walks a run of token tiles of one
// (KV head, sequence), building its decode tables and register fragments once. krt (64-token
// tiles): coefficients become exact fp16 MFMA B-fragments in LDS, the residual rows are staged
// big-endian and table-decoded (as the slot read does), the decoder is split hi + lo into resident
// A-fragments, and the rotated key is split hi + lo against a hi + lo query, so every score is the
// fp32 dot product up to fp32 rounding. v_out (128-token tiles): decodes its V rows, accumulates
// in registers and adds its partial sums into `out` with fp32 atomic adds, as the codec kernel
// does (its caller zero-fills `out`).
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kCTile = 64;       // tokens per krt tile
constexpr int kCVTile = 128;     // tokens per v_out tile
constexpr int kCThreads = 256;
constexpr int kCRawDw = 17;      // staged row: bitmap (4 dwords) + code stream (<= 12) + slack
constexpr int kCCode = 144;      // bytes per decoded code row

struct ContainerArgs {
  int n, r1, H, G, B, PB, dec_per_seq, has_res;
  int tiles_per_wg;  // consecutive token tiles one workgroup walks
  const int8_t* cq;
  const float* cs;
  const float* dec;
  const uint8_t* bm;
  const uint8_t* pk;
  const float* rs;
  const float* cosv;
  const float* sinv;
  const float* q;
  float* s;
  const float* p;
  int64_t p_head_stride, p_batch_stride;
  float* o;
};

// One quarter of a token's residual / V row in registers, unaligned: part 0 the 16 bitmap bytes,
// parts 1..3 the five source dwords c0 .. c0 + 4 (c0 = 4 * (part - 1)) of its code stream. Loads
// stay inside the row's dwords (bytes past the row are never decoded). Zero for an invalid row.
// `commit_row_quarter` writes it in the staged format the table decoder reads: dwords 0..3 the
// bitmap as stored, dwords 4.. the code stream realigned with each dword byte-reversed.
__device__ __forceinline__ void load_row_quarter(const ContainerArgs& a, int64_t row, bool valid,
                                                 int part, uint32_t x[5], int& sh) {
  sh = 0;
#pragma unroll
  for (int i = 0; i < 5; ++i) x[i] = 0u;
  if (!valid) return;
  if (part == 0) {
    const uint4 b = ld_global16(a.bm + row * kBitmapBytes);
    x[0] = b.x;
    x[1] = b.y;
    x[2] = b.z;
    x[3] = b.w;
  } else {
    const uintptr_t A = (uintptr_t)(a.pk + row * a.PB);
    const auto* w = gbl((const uint32_t*)(A & ~(uintptr_t)3));
    sh = (int)(A & 3);
    const int nsrc = (sh + a.PB + 3) >> 2;
    const int c0 = 4 * (part - 1);
#pragma unroll
    for (int i = 0; i < 5; ++i) x[i] = w[min(c0 + i, nsrc - 1)];
  }
}

__device__ __forceinline__ void commit_row_quarter(int part, int sh, const uint32_t x[5],
                                                   uint32_t* dst) {
  if (part == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = x[i];
  } else {
    const uint32_t sel = stage_selector(sh, true);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[4 * part + i] = __builtin_amdgcn_perm(x[i + 1], x[i], sel);
  }
  if (part == 3) dst[16] = 0u;
}

template <int KS>
struct KrtSmem {
  _Float16 coef[kCTile][KS * 32 + 8];
  uint32_t raw[kCTile][kCRawDw];
  uint8_t code[kCTile][kCCode];
  float spart[4][kCTile][8];
  uint2 lut[256];
  float cs[kCTile], kr[kCTile];
};

// ---------------------------------------------------------------------------- krt
template <int G, int BITS, int KS>
__global__ __launch_bounds__(kCThreads, 2) void container_krt_kernel(ContainerArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint16_t lut3s[kLut3Entries];  // static: its address folds into the loads
  KrtSmem<KS>& S = *reinterpret_cast<KrtSmem<KS>*>(smem_raw);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;
  const int dl = 16 * wv + 4 * gq;
  const int hv = blockIdx.y;
  const int bz = blockIdx.z;
  const int HD = a.H * kD;
  const int ntiles = (a.n + kCTile - 1) / kCTile;
  const int tile0 = blockIdx.x * a.tiles_per_wg;
  const int tile1 = min(ntiles, tile0 + a.tiles_per_wg);
  if (tile0 >= tile1) return;

  build_luts(S.lut, BITS == 3 ? lut3s : nullptr, tid, kCThreads);
  // ---- decoder fragments (A operand, M = dims, K = r1), hi + lo fp16, resident in registers
  const float* dec = a.dec + (a.dec_per_seq ? (int64_t)bz * a.r1 * HD : 0) + (int64_t)hv * kD;
  half8 ahi[2][KS], alo[2][KS];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int dim = 16 * (wv + 4 * mi) + n;
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ar = 32 * st + 8 * gq + j;
        const float f = ar < a.r1 ? dec[(int64_t)ar * HD + dim] : 0.f;
        const _Float16 hi = (_Float16)f;
        ahi[mi][st][j] = hi;
        alo[mi][st][j] = (_Float16)(f - (float)hi);
      }
  }
  // ---- query fragments (A operand of q.k, M = heads, K = this wave's 32 dims in the order of
  // the rotated-key fragments), hi + lo fp16; rows >= G are zero
  // (rows n >= G load head G - 1 and discard it: no branch around the loads, one round trip)
  half8 qhi, qlo;
  {
    const float* qr = a.q + ((int64_t)bz * a.H * G + hv * G + min(n, G - 1)) * kD;
    const float4v x0 = *gbl((const float4v*)(qr + dl));
    const float4v x1 = *gbl((const float4v*)(qr + 64 + dl));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = n < G ? (j < 4 ? x0[j] : x1[j - 4]) : 0.f;
      const _Float16 hi = (_Float16)x;
      qhi[j] = hi;
      qlo[j] = (_Float16)(x - (float)hi);
    }
  }

  // ---- the next tile's bytes in registers while the current one computes: this thread's share
  // of a token's coefficient row (KS / 2 rounded up groups of 5 unaligned source dwords), one
  // quarter of its residual row, and its rulers
  const int ptok = tid >> 2, part = tid & 3;
  constexpr int kCG = (KS + 1) / 2;
  uint32_t cx[kCG][5], rx[5];
  int csh = 0, rsh = 0;
  float csv = 0.f, rsv = 0.f;
  auto fetch = [&](int tile) {
    const int i = tile * kCTile + ptok;
    const bool valid = i < a.n;
    const int64_t crow = (int64_t)bz * a.n + i;
    const uintptr_t A = (uintptr_t)(a.cq + crow * a.r1);
    const auto* w = gbl((const uint32_t*)(A & ~(uintptr_t)3));
    csh = (int)(A & 3);
    const int nsrc = (csh + a.r1 + 3) >> 2;
#pragma unroll
    for (int gi = 0; gi < kCG; ++gi)
#pragma unroll
      for (int j = 0; j < 5; ++j)
        cx[gi][j] = valid ? w[min(2 * KS * part + 4 * gi + j, nsrc - 1)] : 0u;
    const int64_t rrow = ((int64_t)bz * a.H + hv) * a.n + i;
    load_row_quarter(a, rrow, valid && a.has_res, part, rx, rsh);
    csv = valid && part == 0 ? a.cs[crow] : 0.f;
    rsv = valid && part == 0 && a.has_res ? a.rs[rrow] : 0.f;
  };
  fetch(tile0);
  // 3-bit codes decode as fp8 (c - 4) * unit: the ruler takes the 1 / unit
  const float rscale = BITS == 3 ? 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0] : 1.0f;

  for (int tile = tile0; tile < tile1; ++tile) {
    const int i0 = tile * kCTile;
    // ---- commit: coefficients as exact fp16, the residual row staged big-endian, rulers
    {
      uint32_t* cdst = (uint32_t*)&S.coef[ptok][part * (8 * KS)];
      const uint32_t sel = stage_selector(csh, false);
#pragma unroll
      for (int gi = 0; gi < kCG; ++gi) {
        const int nd = KS - 2 * gi >= 2 ? 4 : 2;  // dwords of this group that belong to the part
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (j < nd) {
            uint32_t p01, p23;
            i8x4_to_f16(__builtin_amdgcn_perm(cx[gi][j + 1], cx[gi][j], sel), p01, p23);
            cdst[2 * (4 * gi + j)] = p01;
            cdst[2 * (4 * gi + j) + 1] = p23;
          }
        }
      }
      commit_row_quarter(part, rsh, rx, S.raw[ptok]);
      if (part == 0) {
        S.cs[ptok] = csv;
        S.kr[ptok] = rsv * rscale;
      }
    }
    // No barrier: a token's four quarter-row threads commit and decode it, all in one wave, and
    // LDS accesses of one wave complete in order (the fences only keep the compiler from moving
    // them). coef / cs / kr / code were last read by the previous tile's reconstruction, before
    // its final barrier (8 x 14,402: 139.6 -> 137.9 us per call, three alternating runs each).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the next tile's bytes, requested as soon as the commit has freed their registers: they
    // arrive during the decode and reconstruction (kernel 159-161 -> 157-158 us at 8 x 14,402;
    // the angle loads then queue behind them, a decode later)
    if (tile + 1 < tile1) fetch(tile + 1);

    // ---- decode the residual rows (thread = token tid/4, quarter tid&3). The decode and
    // reconstruction run at raised wave priority: the co-resident workgroup's commit and
    // read-out fill the issue slots they leave.
    __builtin_amdgcn_s_setprio(1);
    decode_quarter_row_be<BITS>(S.raw[ptok], part, S.lut, lut3s, &S.code[ptok][32 * part]);
    __syncthreads();

    // ---- reconstruct + residual + RoPE + scores, 16 tokens at a time. The pair (j, j + 64)
    // rotates by one angle: the tables duplicate their d/2 ramp, so only the first half of each
    // row is read, as the codec kernel does. The rows (L2 resident) are requested one block ahead.
    auto angle_row = [&](int nb, float4v r[2]) {
      const int64_t pos = min(i0 + 16 * nb + n, a.n - 1);
      r[0] = *(const float4v*)&a.cosv[pos * kD + dl];
      r[1] = *(const float4v*)&a.sinv[pos * kD + dl];
    };
    float4v ang_next[2];
    angle_row(0, ang_next);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int tok = 16 * nb + n;
      const float4v cv = ang_next[0], sv = ang_next[1];
      if (nb < 3) angle_row(nb + 1, ang_next);
      float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const half8 b = *(const half8*)&S.coef[tok][32 * st + 8 * gq];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0][st], b, acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0][st], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1][st], b, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1][st], b, acc1, 0, 0, 0);
      }
      const float cs = S.cs[tok], kr = S.kr[tok];
      const float kb = BITS == 4 ? -8.f * kr : 0.f;  // 4-bit codes arrive as c
      float vl[4], vh[4];
      codes4<BITS>(*(const uint32_t*)&S.code[tok][dl], vl);
      codes4<BITS>(*(const uint32_t*)&S.code[tok][64 + dl], vh);
      float y[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float xl = fmaf(cs, acc0[i], fmaf(kr, vl[i], kb));
        const float xh = fmaf(cs, acc1[i], fmaf(kr, vh[i], kb));
        y[i] = xl * cv[i] - xh * sv[i];
        y[4 + i] = xh * cv[i] + xl * sv[i];
      }
      half8 yhi, ylo;
      split8(y, yhi, ylo);
      float4v sacc = {0.f, 0.f, 0.f, 0.f};
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi, yhi, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi, ylo, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo, yhi, sacc, 0, 0, 0);
      // lane (n, gq) holds heads 4*gq .. 4*gq+3 of token n, over this wave's 32 dims
      if (4 * gq < G) *(float4v*)&S.spart[wv][tok][4 * gq] = sacc;
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    // the partial scores are next written past the following tile's decode barrier, which every
    // wave reaches only after its read-out, so no barrier follows this read-out
    for (int idx = tid; idx < G * kCTile; idx += kCThreads) {
      const int tok = idx & (kCTile - 1), p = idx / kCTile;
      if (i0 + tok < a.n) {
        const float v = (S.spart[0][tok][p] + S.spart[1][tok][p]) + (S.spart[2][tok][p] + S.spart[3][tok][p]);
        a.s[((int64_t)bz * a.H * G + hv * G + p) * a.n + i0 + tok] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------- v_out
struct VoutSmem {
  uint32_t raw[kCVTile][kCRawDw];
  uint8_t code[kCVTile][kCCode];
  // p * ruler split hi + lo in fp16 (22 significant bits), [parity][head][token], double-buffered
  // by tile parity: the P.V MFMA's B operand
  _Float16 pwh[2][8][kCVTile];
  _Float16 pwl[2][8][kCVTile];
  uint2 lut[256];
  int wexp;  // the weight exponent the workgroup runs at (only grows)
};

// 128-token tiles. The next tile's rows, rulers and weights are in registers while the current
// tile decodes and accumulates. Accumulation on MFMA, as K1's P.V: O^T[dims, heads] +=
// V^T[dims, tokens] * W^T[tokens, heads] with the codes as exact fp16 integers (c - 2^(b-1)), read
// transposed from the decoded rows (ds_read_tr8_b64), and the weights w = p * ruler split hi + lo
// in fp16 (two products) after an exact 2^(8 - we) scaling, so the sum keeps fp32-level accuracy:
// at we = 0 the 2^8 keeps small weights out of the fp16 subnormals, and we grows (the workgroup
// agrees on it through LDS at the tile's first barrier) when a weight of 2^(7 + we) or more
// arrives, so every scaled weight stays below 2^15. Wave w owns dims 16w.. and 64 + 16w.. for all
// heads.
template <int G, int BITS>
__global__ __launch_bounds__(kCThreads, 2) void container_v_out_kernel(ContainerArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint16_t lut3s[kLut3Entries];  // static: its address folds into the loads
  VoutSmem& S = *reinterpret_cast<VoutSmem*>(smem_raw);
  constexpr int kPw = (G * kCVTile + kCThreads - 1) / kCThreads;  // weights per thread per tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int hv = blockIdx.y;
  const int bz = blockIdx.z;
  const int ntiles = (a.n + kCVTile - 1) / kCVTile;
  const int tile0 = blockIdx.x * a.tiles_per_wg;
  const int tile1 = min(ntiles, tile0 + a.tiles_per_wg);
  if (tile0 >= tile1) return;
  const int ptok = tid >> 2, part = tid & 3;  // staging: tokens ptok and 64 + ptok, one quarter
  const int n = lane & 15, gq = lane >> 4;
  const int64_t row0 = ((int64_t)bz * a.H + hv) * a.n;
  const float* pb = a.p + (int64_t)bz * a.p_batch_stride + (int64_t)hv * G * a.p_head_stride;

  uint32_t x[2][5];
  int sh[2];
  // weights and their token's row ruler: the product p * ruler is what the accumulation uses
  float pwv[kPw], rwv[kPw];
  auto fetch = [&](int tile) {
    const int i0 = tile * kCVTile;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int tok = ptok + 64 * pass;
      load_row_quarter(a, row0 + i0 + tok, i0 + tok < a.n, part, x[pass], sh[pass]);
    }
#pragma unroll
    for (int k = 0; k < kPw; ++k) {
      const int idx = tid + kCThreads * k, tok = idx & (kCVTile - 1), g = idx / kCVTile;
      const bool ok = g < G && i0 + tok < a.n;
      pwv[k] = ok ? pb[(int64_t)g * a.p_head_stride + i0 + tok] : 0.f;
      rwv[k] = ok ? a.rs[row0 + i0 + tok] : 0.f;
    }
  };
  fetch(tile0);
  build_luts(S.lut, BITS == 3 ? lut3s : nullptr, tid, kCThreads);
  if (tid == 0) S.wexp = 0;
  __syncthreads();  // wexp
  int we = 0;                 // weights are scaled by 2^(8 - we); the accumulators likewise
  float w_thr = 128.f;        // |w| >= 2^(7 + we) needs a larger exponent
  float wsc = 256.f;          // 2^(8 - we)
  float wreg[kPw];
  // 3-bit codes: fp8 bytes of (c - 4) scaled back by 1 / unit to exact integers
  const float inv_unit = 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
  float4v oacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // O^T[dims][head n]
  // transposed code reads: in each 16-lane group, lanes 2j, 2j+1 address the two 8-byte halves of
  // row (token) 8gq + j of a 16-dim tile; lane n receives dim n of those 8 tokens
  const int tr_tok = 8 * gq + (n >> 1);
  const int tr_col = 8 * (n & 1);

  for (int tile = tile0; tile < tile1; ++tile) {
    // ---- commit the prefetched tile, then request the next one. The scaled weights are
    // double-buffered: a thread still accumulating the previous tile reads the other buffer, and
    // the staged rows and codes are only rewritten past a barrier that follows its reads.
    const int buf = (tile - tile0) & 1;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass)
      commit_row_quarter(part, sh[pass], x[pass], S.raw[ptok + 64 * pass]);
#pragma unroll
    for (int k = 0; k < kPw; ++k) {
      wreg[k] = pwv[k] * rwv[k];
      const float aw = fabsf(wreg[k]);
      if (aw >= w_thr) atomicMax(&S.wexp, (int)(__float_as_uint(aw) >> 23) - 127 - 6);
    }
    if (tile + 1 < tile1) fetch(tile + 1);
    __syncthreads();
    {
      // the workgroup's exponent for this tile (every atomicMax above precedes the barrier; the
      // next ones follow the tile's second barrier)
      const int we_new = S.wexp;
      if (we_new != we) {
        const float f = ldexpf(1.f, we - we_new);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) oacc[mi] *= f;
        we = we_new;
        w_thr = ldexpf(1.f, 7 + we);
        wsc = ldexpf(1.f, 8 - we);
      }
    }
#pragma unroll
    for (int k = 0; k < kPw; ++k) {
      const int idx = tid + kCThreads * k;
      if (idx < G * kCVTile) {
        // scaled by 2^(8 - we) (exact): weights down to ~1e-6 stay fp16 normals at we = 0, and
        // every scaled weight stays below 2^15; the sums are scaled back at the end
        const float w = wreg[k] * wsc;
        const _Float16 hi = (_Float16)w;
        S.pwh[buf][idx / kCVTile][idx & (kCVTile - 1)] = hi;
        S.pwl[buf][idx / kCVTile][idx & (kCVTile - 1)] = (_Float16)(w - (float)hi);
      }
    }
    // ---- decode (thread = token tid/2, half tid&1), at raised wave priority
    __builtin_amdgcn_s_setprio(1);
    decode_half_row_be<BITS>(S.raw[tid >> 1], tid & 1, S.lut, lut3s,
                             &S.code[tid >> 1][64 * (tid & 1)]);
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    // ---- O^T += V^T W^T over the tile's 128 tokens, 32 per k-step
#pragma unroll
    for (int kk = 0; kk < kCVTile / 32; ++kk) {
      half8 bh = {}, bl = {};
      if (n < G) {
        bh = *(const half8*)&S.pwh[buf][n][32 * kk + 8 * gq];
        bl = *(const half8*)&S.pwl[buf][n][32 * kk + 8 * gq];
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const uint8_t* src = &S.code[32 * kk + tr_tok][16 * (wv + 4 * mi) + tr_col];
        typedef int v2i __attribute__((ext_vector_type(2)));
        const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) v2i*)(src));
        half8 av;
        if constexpr (BITS == 3) {
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const half2v lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[w], inv_unit, false);
            const half2v hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw[w], inv_unit, true);
            av[4 * w] = lo[0];
            av[4 * w + 1] = lo[1];
            av[4 * w + 2] = hi[0];
            av[4 * w + 3] = hi[1];
          }
        } else {
          // offset-binary code bytes c -> fp16 (c - 8), exact: 1024 + c from the byte placed
          // under the fp16 exponent of 1024, minus 1032
          const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, (uint32_t)raw[w], 0x04010400u);
            const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, (uint32_t)raw[w], 0x04030402u);
            const half2v x0 = __builtin_bit_cast(half2v, lo) - bias;
            const half2v x1 = __builtin_bit_cast(half2v, hi) - bias;
            av[4 * w] = x0[0];
            av[4 * w + 1] = x0[1];
            av[4 * w + 2] = x1[0];
            av[4 * w + 3] = x1[1];
          }
        }
        oacc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh, oacc[mi], 0, 0, 0);
        oacc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl, oacc[mi], 0, 0, 0);
      }
    }
  }
  // ---- this workgroup's sums for its token range: lane (head n, gq) holds dims 4gq.. of each of
  // the wave's two 16-dim tiles
  if (n < G) {
    float* ob = &a.o[((int64_t)bz * a.H * G + hv * G + n) * kD];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        atomicAdd(&ob[16 * (wv + 4 * mi) + 4 * gq + i], oacc[mi][i] * ldexpf(1.f, we - 8));
  }
}

}  // namespace ttkv

// ------------------------------------------------------------------------------------ host side
#include "ttkv_host.h"

namespace ttkv {

// Token tiles per workgroup: about one round of `per_cu` resident workgroups per CU over the
// (sequence, head) pairs, so each workgroup builds its tables and decoder fragments once. krt
// holds three per CU up to r1 = 128 (41 KB of LDS, <= 164 VGPRs; 8 x 14,402 at r1 = 110:
// 158 -> 138 us against two), two above; v_out (37 KB, < 128 VGPRs) four (its kernel 38.8 us,
// the same as three per CU with the 16 KB four-code table).
static int tiles_per_wg(int ntiles, int pairs, int per_cu = 2) {
  const int target = per_cu * device_cu_count();
  const int per_pair = std::max(1, target / std::max(pairs, 1));
  return std::max(1, (ntiles + per_pair - 1) / per_pair);
}

template <typename K>
static int launch_with_smem(K kfn, size_t smem, dim3 grid, hipStream_t st, const ContainerArgs& a,
                            const char* what) {
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, grid, dim3(kCThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return TTKV_OK;
}

template <int G, int BITS>
static int krt_ks(const ContainerArgs& a, int ks, dim3 grid, hipStream_t st) {
  switch (ks) {
    case 1: return launch_with_smem(container_krt_kernel<G, BITS, 1>, sizeof(KrtSmem<1>), grid, st, a, "container krt");
    case 2: return launch_with_smem(container_krt_kernel<G, BITS, 2>, sizeof(KrtSmem<2>), grid, st, a, "container krt");
    case 3: return launch_with_smem(container_krt_kernel<G, BITS, 3>, sizeof(KrtSmem<3>), grid, st, a, "container krt");
    case 4: return launch_with_smem(container_krt_kernel<G, BITS, 4>, sizeof(KrtSmem<4>), grid, st, a, "container krt");
    case 5: return launch_with_smem(container_krt_kernel<G, BITS, 5>, sizeof(KrtSmem<5>), grid, st, a, "container krt");
  }
  return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
}

template <int BITS>
static int krt_g(const ContainerArgs& a, int ks, dim3 grid, hipStream_t st) {
  switch (a.G) {
    case 1: return krt_ks<1, BITS>(a, ks, grid, st);
    case 2: return krt_ks<2, BITS>(a, ks, grid, st);
    case 3: return krt_ks<3, BITS>(a, ks, grid, st);
    case 4: return krt_ks<4, BITS>(a, ks, grid, st);
    case 8: return krt_ks<8, BITS>(a, ks, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "num_heads / H = " + std::to_string(a.G) +
                                           " query heads per KV head is not built (1,2,3,4,8)");
}

static int container_common(int H, int HQ, int d, int B, int n, int pb, int bits, bool need_rows,
                            int& G) {
  if (d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (H <= 0 || HQ <= 0 || HQ % H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  G = HQ / H;
  if (B < 0 || n < 0) return host_fail(TTKV_E_INVALID, "negative size");
  if (need_rows) {
    if (bits != 3 && bits != 4) return host_fail(TTKV_E_UNSUPPORTED, "row code width must be 3 or 4 bits");
    if (pb <= 0 || pb > 48)
      return host_fail(TTKV_E_UNSUPPORTED, "packed row bytes must be in 1..48 (<= 96 lanes at 4 bits)");
  }
  return TTKV_OK;
}

int container_krt(int H, int HQ, int d, int B, int n, int r1, const int8_t* cq, const float* cs,
                  const float* dec, int dec_per_seq, const uint8_t* bm, const uint8_t* pk,
                  const float* rs, int pb, int bits, const float* cosv, const float* sinv,
                  const float* q, float* s, hipStream_t st) {
  const bool has_res = bm != nullptr;
  int G = 0;
  if (int rc = container_common(H, HQ, d, B, n, pb, has_res ? bits : 3, has_res, G)) return rc;
  if (r1 <= 0) return host_fail(TTKV_E_INVALID, "r1 must be positive");
  const int ks = (r1 + 31) / 32;
  if (ks > 5) return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
  if (!cq || !cs || !dec || !cosv || !sinv || !q || !s)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (has_res && (!pk || !rs)) return host_fail(TTKV_E_INVALID, "residual arrays incomplete");
  if (((uintptr_t)cosv | (uintptr_t)sinv | (uintptr_t)bm | (uintptr_t)q) % 16)
    return host_fail(TTKV_E_INVALID, "cos / sin / bitmap / query must be 16-byte aligned");
  if (B == 0 || n == 0) return TTKV_OK;
  ContainerArgs a{};
  a.n = n;
  a.r1 = r1;
  a.H = H;
  a.G = G;
  a.B = B;
  a.PB = pb;
  a.dec_per_seq = dec_per_seq;
  a.has_res = has_res;
  a.cq = cq;
  a.cs = cs;
  a.dec = dec;
  a.bm = bm;
  a.pk = pk;
  a.rs = rs;
  a.cosv = cosv;
  a.sinv = sinv;
  a.q = q;
  a.s = s;
  a.tiles_per_wg = tiles_per_wg((n + kCTile - 1) / kCTile, H * B, ks <= 4 ? 3 : 2);
  const dim3 grid(((n + kCTile - 1) / kCTile + a.tiles_per_wg - 1) / a.tiles_per_wg, H, B);
  // without residual rows the staged bitmaps are zero and the 3-bit decode contributes 0
  return (has_res && bits == 4) ? krt_g<4>(a, ks, grid, st) : krt_g<3>(a, ks, grid, st);
}

template <int BITS>
static int vout_g(const ContainerArgs& a, dim3 grid, hipStream_t st) {
  switch (a.G) {
    case 1: return launch_with_smem(container_v_out_kernel<1, BITS>, sizeof(VoutSmem), grid, st, a, "container v_out");
    case 2: return launch_with_smem(container_v_out_kernel<2, BITS>, sizeof(VoutSmem), grid, st, a, "container v_out");
    case 3: return launch_with_smem(container_v_out_kernel<3, BITS>, sizeof(VoutSmem), grid, st, a, "container v_out");
    case 4: return launch_with_smem(container_v_out_kernel<4, BITS>, sizeof(VoutSmem), grid, st, a, "container v_out");
    case 8: return launch_with_smem(container_v_out_kernel<8, BITS>, sizeof(VoutSmem), grid, st, a, "container v_out");
  }
  return host_fail(TTKV_E_UNSUPPORTED, "num_heads / H = " + std::to_string(a.G) +
                                           " query heads per KV head is not built (1,2,3,4,8)");
}

int container_v_out(int H, int HQ, int d, int B, int n, const float* p, int64_t p_head_stride,
                    int64_t p_batch_stride, const uint8_t* bm, const uint8_t* pk, const float* rs,
                    int pb, int bits, float* o, hipStream_t st) {
  int G = 0;
  if (int rc = container_common(H, HQ, d, B, n, pb, bits, true, G)) return rc;
  if (!p || !bm || !pk || !rs || !o) return host_fail(TTKV_E_INVALID, "null pointer argument");
  if ((uintptr_t)bm % 16) return host_fail(TTKV_E_INVALID, "bitmap must be 16-byte aligned");
  if (p_head_stride < n || p_batch_stride < (int64_t)HQ * p_head_stride)
    return host_fail(TTKV_E_INVALID, "p strides are smaller than its [B, HQ, n] extent");
  if (B == 0 || n == 0) return TTKV_OK;
  ContainerArgs a{};
  a.n = n;
  a.H = H;
  a.G = G;
  a.B = B;
  a.PB = pb;
  a.bm = bm;
  a.pk = pk;
  a.rs = rs;
  a.p = p;
  a.p_head_stride = p_head_stride;
  a.p_batch_stride = p_batch_stride;
  a.o = o;
  a.tiles_per_wg = tiles_per_wg((n + kCVTile - 1) / kCVTile, H * B, 4);
  const dim3 grid(((n + kCVTile - 1) / kCVTile + a.tiles_per_wg - 1) / a.tiles_per_wg, H, B);
  return bits == 4 ? vout_g<4>(a, grid, st) : vout_g<3>(a, grid, st);
}

}  // namespace ttkv

// K2: multi-query read of the compressed store for chunked-prefill continuations. gfx950 / CDNA4.
//
// A continuation chunk of Q queries (positions p0 .. p0+Q-1, p0 = seq_len - Q) attends causally
// over all seq_len stored keys (the chunk's own keys were written by the store write first). The
// key tile is reconstructed ONCE per work item and reused by all of its 64 queries x G heads on
// MFMA, instead of once per query as a decode read would.
//
// Work item = (request, KV head h, block of 64 queries, key split). A 256-thread workgroup walks
// its key range in 64-key tiles:
//   commit    : the tile's slot bytes -> LDS (coefficients as exact fp16, this head's K and V rows)
//   decode    : bitmap + MSB-first code stream -> one code byte per (key, lane), as in K1 (3-bit
//               codes as fp8 signed bytes, 4-bit as offset-binary bytes)
//   transpose : V codes -> Vt[dim][key] = code - 2^(b-1) in fp16 (small integers, exact)
//   recon     : K_pre^T[dims x 16 keys] = Dec^T * coeff^T on MFMA 16x16x32 f16 (decoder fragments
//               resident in registers), + cs * acc + residual, RoPE in registers -> Kp[key][dim]
//   scores    : S^T[16 keys x 16 queries] = Kp * Q^T on MFMA; wave w owns queries 16w..16w+15
//               for all G heads of h; causal -inf where key > p0 + query
//   softmax   : online, base 2, per query column (reduced over the 4 lane groups)
//   P.V       : O^T[dims x queries] += Vt * (P * ruler_v)^T on MFMA. The probabilities stay in
//               registers: the MFMA k-slots of P^T and of Vt enumerate the same keys (lane group
//               g holds keys 4g..4g+3 of both 16-key halves of a 32-key step).
// Key splits of one item are combined in the same launch by the last workgroup to finish, with
// the write-through partial hand-off K1 uses.
//
// Precision. Both MFMA contractions that feed the scores carry fp32 accuracy: the decoder is split
// hi + lo in fp16 (decoder_f = int8 * fp16 ruler has <= 19 significant bits, so hi + lo is exact)
// and the rotated key is split hi + lo too, so each score is the fp32 dot of the fp16 query with
// the fp32 key up to fp32 rounding. Rounding either operand to a single fp16 instead moves the
// attention output by up to ~1.5e-3 (decoder) and ~3e-3 (rotated key) on the benchmark's keys,
// which have x8 outlier channels -- beyond the 2e-3 budget. P * ruler_v * 2^-ve is rounded to
// fp16 once for the P.V contraction (the V codes themselves are exact small integers); ve >= 0
// grows with the largest V ruler seen so that the product stays below 2^15 (P <= 2^8).
//
// Reference semantics: vllm_ttkv/impl.py:725-778 (_prefill_continuation: p0 = seq_len - q_len,
// scores over the whole store, softmax, V readout), vllm_ttkv/reference.py:112-146
// (raw_scores_multi: -inf where key > p0 + j), krt_triton.py:154-317 (multi-query scores),
// v_out_triton.py:158-293 (multi-query V readout).
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kPTile = 64;      // keys per tile
constexpr int kPQ = 64;         // queries per work item
constexpr int kPThreads = 256;
constexpr int kPRawDw = 17;     // dwords per staged head row (16 + slack): odd, so rows spread over banks
constexpr int kPCode = 144;     // bytes per code row
constexpr int kKpStride = 136;  // halves per reconstructed key row (128 + 8)
constexpr int kVtStride = 72;   // halves per transposed V row (64 keys + 8)
constexpr int kPSeg = 516;      // block ids of one key range staged in LDS

struct PrefillArgs {
  Geom g;
  int HQ, G;
  float scale, scale_log2;
  const void* q;
  int q_dtype;
  int64_t q_row_stride;
  const uint8_t* page;
  int64_t n_slots, slot_stride;
  int block_size;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* seq_lens;
  const int32_t* qsl;
  const int32_t* req_index;
  int num_reqs;
  const int32_t* dec_map;
  int64_t num_blocks;
  const int8_t* dec_q;  // decoder pool (see dec_ranks)
  const float* dec_scale;
  int64_t n_dec_slots;
  const float* cs_cache;
  void* out;
  int out_dtype;
  int64_t out_row_stride;
  float* s_out;
  int64_t s_head_stride, s_q_stride;
  float* ws_part;
  int* ws_cnt;
  int* err;
  int n_qb, kchunk, nsplit, nwork, max_seq, max_q;
  int ri0;  // first batch row of this launch (rows ri0 .. ri0 + num_reqs - 1)
};

template <int KSTEPS, bool EXACT>
struct PrefillSmem {
  static constexpr int kCoefStride = KSTEPS * 32 + 8;
  _Float16 coef[kPTile][kCoefStride];  // commit -> recon
  union {
    struct {
      uint32_t k[kPTile][kPRawDw];
      uint32_t gap[16];  // V rows 16 dwords off: a token's K and V rows on other banks
      uint32_t v[kPTile][kPRawDw];
    } raw;                                        // commit -> decode
    _Float16 kp[EXACT ? 2 : 1][kPTile][kKpStride];  // recon -> scores (hi, lo)
  } u;
  uint8_t kcode[kPTile][kPCode];  // decode -> recon
  uint8_t vcode[kPTile][kPCode];  // decode -> transpose
  _Float16 vt[kD][kVtStride];     // transpose -> P.V
  uint2 lut[256];
  int32_t seg[kPSeg];
  float cs[kPTile], krul[kPTile], vrul[kPTile];
  int is_last;
};

template <int G, int RB, int VB, int KSTEPS, bool SCORES, int CM>
__global__ __launch_bounds__(kPThreads, ((SCORES && G <= 3) || G <= 2) ? 2 : 1) void prefill_paged_kernel(PrefillArgs a) {
  constexpr bool EXACT = true;  // see the precision note at the top
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint16_t lut3s[kLut3Entries];  // static: its address folds into the loads
  PrefillSmem<KSTEPS, EXACT>& S = *reinterpret_cast<PrefillSmem<KSTEPS, EXACT>*>(smem_raw);
  static_assert(RB == VB, "K and V rows decode with one code path (3/3 and 4/4 are built)");
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // Work order: the query blocks and heads of one key range are consecutive and dealt to one
  // XCD (blocks go round-robin over the 8 XCDs), so they share that XCD's L2 for the slot bytes.
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= a.nwork) return;
  const int qb = w % a.n_qb;
  int t = w / a.n_qb;
  const int h = t % g.H;
  t /= g.H;
  const int sp = t % a.nsplit;
  const int ri = t / a.nsplit;
  if (ri >= a.num_reqs) return;
  const int r = a.req_index ? a.req_index[a.ri0 + ri] : a.ri0 + ri;
  const int q0 = a.qsl[r];
  int qlen = a.qsl[r + 1] - q0;
  int seq = a.seq_lens[r];
  const int blk0 = a.bt[(int64_t)r * a.bt_row_stride];
  const bool lead = (tid == 0 && sp == 0 && qb == 0 && h == 0);
  if (seq > a.max_seq || qlen > a.max_q) {  // the host sized grid and outputs from these bounds
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    seq = min(seq, a.max_seq);
    qlen = min(qlen, a.max_q);
  }
  const int p0 = seq - qlen;
  const int qa = qb * kPQ;
  if (qlen <= 0 || qa >= qlen) return;
  if (p0 < 0) {  // fewer stored keys than queries: not a continuation of this store
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    return;
  }
  const int qe = min(qlen, qa + kPQ);
  const int kmax = SCORES ? seq : min(seq, p0 + qe);  // keys any query of the block may see
  const int nparts = (kmax + a.kchunk - 1) / a.kchunk;
  if (sp >= nparts) return;
  const int k0 = sp * a.kchunk;
  const int k1 = min(kmax, k0 + a.kchunk);
  const int item = (ri * g.H + h) * a.n_qb + qb;

  int dslot = -1;
  if (blk0 >= 0 && blk0 < a.num_blocks) dslot = a.dec_map[blk0];
  if (dslot < 0 || dslot >= a.n_dec_slots) {
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    if constexpr (SCORES) {
      for (int i = tid; i < G * (qe - qa) * (k1 - k0); i += kPThreads) {
        const int kk = i % (k1 - k0);
        const int rest = i / (k1 - k0);
        const int qj = qa + rest % (qe - qa);
        const int gg = rest / (qe - qa);
        a.s_out[(int64_t)(h * G + gg) * a.s_head_stride + (int64_t)qj * a.s_q_stride + k0 + kk] = NAN;
      }
    } else if (sp == 0) {
      for (int i = tid; i < G * (qe - qa) * kD; i += kPThreads) {
        const int dim = i % kD;
        const int qj = qa + (i / kD) % (qe - qa);
        const int gg = i / kD / (qe - qa);
        store_act(a.out, a.out_dtype,
                  (int64_t)(q0 + qj) * a.out_row_stride + (int64_t)(h * G + gg) * kD + dim, NAN);
      }
    }
    return;
  }

  build_luts(S.lut, (RB == 3 || VB == 3) ? lut3s : nullptr, tid, kPThreads);

  // ---- query fragments (B operand of S^T = Kp Q^T): column = query 16*wv + n of the block
  const int qj = qa + 16 * wv + n;
  const bool qvalid = qj < qe;
  // (a column past the chunk loads the chunk's first query and discards it, so the loads carry
  // no branch and go out together)
  half8 qf[G][4];
  {
    const bool qvec = act_rows_aligned(a.q, a.q_dtype, a.q_row_stride);
    const int64_t qb = (int64_t)(q0 + (qvalid ? qj : qa)) * a.q_row_stride + (int64_t)h * G * kD +
                       8 * gq;
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float t[8];
        load_act_n<8>(a.q, a.q_dtype, qb + (int64_t)gg * kD + 32 * ks, qvec, t);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][ks][i] = qvalid ? (_Float16)t[i] : (_Float16)0.0f;
      }
  }

  // ---- decoder fragments (A operand of the reconstruction, M = dims), resident in registers
  // (int8 ranks 32s + 8gq .. +7 of the lane's two columns, 8 bytes per step, and their rulers;
  // 32 KSTEPS <= R, so every load is inside the decoder)
  const int HD = g.H * kD;
  const int R = dec_ranks(g.r1);
  const int8_t* decq = a.dec_q + ((int64_t)dslot * HD + h * kD) * R;
  const float* decs = a.dec_scale + (int64_t)dslot * R;
  half8 ahi[2][KSTEPS], alo[2][EXACT ? KSTEPS : 1];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int8_t* col = decq + (int64_t)(16 * (wv + 4 * mi) + n) * R;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      const u32x2v q8 = *gbl((const u32x2v*)(col + 32 * s + 8 * gq));
      const float4v s0 = *gbl((const float4v*)(decs + 32 * s + 8 * gq));
      const float4v s1 = *gbl((const float4v*)(decs + 32 * s + 8 * gq + 4));
      float v[8];
      dec_values4(q8[0], s0, v);
      dec_values4(q8[1], s1, v + 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = 32 * s + 8 * gq + j < g.r1 ? v[j] : 0.f;
        const _Float16 hi = (_Float16)f;
        ahi[mi][s][j] = hi;
        if constexpr (EXACT) alo[mi][s][j] = (_Float16)(f - (float)hi);
      }
    }
  }

  float4v o[SCORES ? 1 : 8][G];
  float m_run[G], l_run[G];
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    m_run[gg] = -INFINITY;
    l_run[gg] = 0.f;
#pragma unroll
    for (int dt = 0; dt < (SCORES ? 1 : 8); ++dt) o[dt][gg] = float4v{0.f, 0.f, 0.f, 0.f};
  }
  int ve = 0;  // V-ruler exponent of the P.V operand (see the softmax)
  float v_thr = 128.f, v_mul = 1.f;

  const int k_row_off = g.k_field + h * g.k_row;
  const int v_row_off = g.k_slot + h * g.v_row;
  const int ptok = tid >> 2;
  const int part = tid & 3;
  const int dl = 16 * wv + 4 * gq;
  const float voff = (float)(1 << (VB - 1));
  // staged rows: realigned, code streams byte-reversed per dword (slot bases are 16-aligned)
  const uint32_t ksel = stage_selector(k_row_off & 3, part != 0);
  const uint32_t vsel = stage_selector(v_row_off & 3, part != 0);
  // fp8 code unit of the hardware conversion (3-bit codes are decoded as fp8 signed bytes)
  const float inv_unit = 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
  // this key range's block ids, staged once (no global read on the per-tile address path)
  const int bfirst = k0 / a.block_size;
  const int nseg = (k1 - 1) / a.block_size - bfirst + 1;
  for (int i = tid; i < nseg; i += kPThreads) {
    int blk = a.bt[(int64_t)r * a.bt_row_stride + bfirst + i];
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, TTKV_ERR_BAD_BLOCK);
      blk = -1;
    }
    S.seg[i] = blk;
  }
  __syncthreads();
  auto slot_base = [&](int tt) -> const uint8_t* {
    if (ptok >= min(kPTile, k1 - tt)) return nullptr;
    const int pos = tt + ptok;
    const int bi = pos / a.block_size;
    const int blk = S.seg[bi - bfirst];
    if (blk < 0) return nullptr;
    const int64_t slot = (int64_t)blk * a.block_size + (pos - bi * a.block_size);
    return slot < a.n_slots ? a.page + slot * a.slot_stride : nullptr;
  };
  // the rows' 64-byte windows (16-aligned; each row lies inside its window, host-checked)
  const int k_win = k_row_off & ~15, v_win = v_row_off & ~15;
  RawSlotW<2 * KSTEPS, CM> P;
  fetch_raw_slot_w<2 * KSTEPS, CM>(P, slot_base(k0), part, g, k_win, v_win);

  // score-tensor rows 16-byte aligned: every 4-key group starts on a 16-byte boundary
  const bool s_vec = SCORES && ((uintptr_t)a.s_out % 16 == 0) && a.s_q_stride % 4 == 0 &&
                     a.s_head_stride % 4 == 0 && k0 % 4 == 0;
  for (int tt = k0; tt < k1; tt += kPTile) {
    const int ntile = min(kPTile, k1 - tt);
    // ------------------------------------------------------------ commit this tile's bytes
    {
      const float cs = commit_coef<2 * KSTEPS, CM>(P, (uint32_t*)&S.coef[ptok][0], part, g);
      if (part == 0) S.cs[ptok] = cs;
      stage_row_w(P.krow, (k_row_off & 15) >> 2, ksel, &S.u.raw.k[ptok][part * 4]);
      stage_row_w(P.vrow, (v_row_off & 15) >> 2, vsel, &S.u.raw.v[ptok][part * 4]);
    }
    if constexpr (SCORES)
      if (tt + kPTile < k1) fetch_raw_slot_w<2 * KSTEPS, CM>(P, slot_base(tt + kPTile), part, g, k_win, v_win);
    // No barrier: wave w commits and decodes the same 16 keys (16w .. 16w+15), and LDS accesses
    // of one wave complete in order (the fences only keep the compiler from moving them); the
    // previous tile's readers finished before its closing barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ------------------------------------------------------------ decode (thread = half row)
    // Decode, V transpose and reconstruction run at raised wave priority, so that where two
    // workgroups share a CU the other one's scores, softmax and P.V fill the slots they leave.
    __builtin_amdgcn_s_setprio(1);
    {
      // lanes 0..31: K rows, 32..63: V rows of this wave's 16 keys, two threads per row; one
      // decode call with per-lane row and destination (the two kinds share the code width)
      const bool is_v = lane >= 32;
      const int key = 16 * (tid >> 6) + ((lane >> 1) & 15);
      const int half = lane & 1;
      const uint32_t* row = is_v ? S.u.raw.v[key] : S.u.raw.k[key];
      decode_half_row_be<RB>(row, half, S.lut, lut3s,
                             is_v ? &S.vcode[key][64 * half] : &S.kcode[key][64 * half]);
      if (half == 0) {
        const float rul = f16_bits_to_float(staged_u16(row, kBitmapBytes + (is_v ? g.v_pb : g.k_pb)));
        if (is_v) {
          S.vrul[key] = key < ntile ? rul : 0.f;
        } else {
          // 3-bit codes come out as fp8 (c - 4) * unit: the ruler takes the 1 / unit
          S.krul[key] = RB == 3 ? rul * inv_unit : rul;
        }
      }
    }
    __syncthreads();
    // ------------------------------------------------------------ V transpose (4 keys x 4 dims)
    if constexpr (!SCORES) {
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int b = tid + kPThreads * it;
        const int kg = b & 15, dg = b >> 4;
        const uint32_t x0 = *(const uint32_t*)&S.vcode[4 * kg + 0][4 * dg];
        const uint32_t x1 = *(const uint32_t*)&S.vcode[4 * kg + 1][4 * dg];
        const uint32_t x2 = *(const uint32_t*)&S.vcode[4 * kg + 2][4 * dg];
        const uint32_t x3 = *(const uint32_t*)&S.vcode[4 * kg + 3][4 * dg];
        // 4x4 byte transpose: y_i = [x0.b_i, x1.b_i, x2.b_i, x3.b_i]
        const uint32_t a01l = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // x0b0 x1b0 x0b1 x1b1
        const uint32_t a01h = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // x0b2 x1b2 x0b3 x1b3
        const uint32_t a23l = __builtin_amdgcn_perm(x3, x2, 0x05010400u);
        const uint32_t a23h = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
        uint32_t y[4];
        y[0] = __builtin_amdgcn_perm(a23l, a01l, 0x05040100u);
        y[1] = __builtin_amdgcn_perm(a23l, a01l, 0x07060302u);
        y[2] = __builtin_amdgcn_perm(a23h, a01h, 0x05040100u);
        y[3] = __builtin_amdgcn_perm(a23h, a01h, 0x07060302u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t p01, p23;
          if constexpr (VB == 3) {  // fp8 signed codes -> exact fp16 integers c - 4
            p01 = __builtin_bit_cast(uint32_t,
                                     __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y[i], inv_unit, false));
            p23 = __builtin_bit_cast(uint32_t,
                                     __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y[i], inv_unit, true));
          } else {
            u8x4_to_f16_minus(y[i], voff, p01, p23);
          }
          *(uint2*)&S.vt[4 * dg + i][4 * kg] = make_uint2(p01, p23);
        }
      }
    }
    // ------------------------------------------------------------ recon + residual + RoPE -> Kp
    // RoPE angles of keys 16*nb + n, dims dl..dl+3 (cos) / 64+dl.. (sin), one block ahead
    auto angle_row = [&](int nb, float4v& cv, float4v& sv) {
      const int key = 16 * nb + n;
      const int pos = key < ntile ? tt + key : tt;
      cv = *(const float4v*)&a.cs_cache[(int64_t)pos * kD + dl];
      sv = *(const float4v*)&a.cs_cache[(int64_t)pos * kD + 64 + dl];
    };
    float4v cvn, svn;
    angle_row(0, cvn, svn);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int key = 16 * nb + n;
      const float4v cv = cvn, sv = svn;
      if (nb < 3) angle_row(nb + 1, cvn, svn);
      float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const half8 b = *(const half8*)&S.coef[key][32 * s + 8 * gq];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0][s], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1][s], b, acc1, 0, 0, 0);
        if constexpr (EXACT) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0][s], b, acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1][s], b, acc1, 0, 0, 0);
        }
      }
      const float cs = S.cs[key];
      const float kr = S.krul[key];
      // 3-bit: codes read as (c - 4) * unit (ruler carries 1 / unit); 4-bit: as c
      const float kb = RB == 3 ? 0.f : -8.f * kr;
      float vcl[4], vch[4];
      codes4<RB>(*(const uint32_t*)&S.kcode[key][dl], vcl);
      codes4<RB>(*(const uint32_t*)&S.kcode[key][64 + dl], vch);
      half2v yl[2], yh[2], zl[2], zh[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float kl = fmaf(cs, acc0[i], fmaf(vcl[i], kr, kb));
        const float kh = fmaf(cs, acc1[i], fmaf(vch[i], kr, kb));
        const float y1 = kl * cv[i] - kh * sv[i];
        const float y2 = kh * cv[i] + kl * sv[i];
        const _Float16 h1 = (_Float16)y1, h2 = (_Float16)y2;
        yl[i >> 1][i & 1] = h1;
        yh[i >> 1][i & 1] = h2;
        if constexpr (EXACT) {
          zl[i >> 1][i & 1] = (_Float16)(y1 - (float)h1);
          zh[i >> 1][i & 1] = (_Float16)(y2 - (float)h2);
        }
      }
      *(uint2*)&S.u.kp[0][key][dl] = make_uint2(__builtin_bit_cast(uint32_t, yl[0]),
                                                __builtin_bit_cast(uint32_t, yl[1]));
      *(uint2*)&S.u.kp[0][key][64 + dl] = make_uint2(__builtin_bit_cast(uint32_t, yh[0]),
                                                     __builtin_bit_cast(uint32_t, yh[1]));
      if constexpr (EXACT) {
        *(uint2*)&S.u.kp[EXACT ? 1 : 0][key][dl] = make_uint2(
            __builtin_bit_cast(uint32_t, zl[0]), __builtin_bit_cast(uint32_t, zl[1]));
        *(uint2*)&S.u.kp[EXACT ? 1 : 0][key][64 + dl] = make_uint2(
            __builtin_bit_cast(uint32_t, zh[0]), __builtin_bit_cast(uint32_t, zh[1]));
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // The next tile's bytes are in flight while this tile's scores, softmax and P.V run. Loads
    // complete in order (vmcnt), so they are requested only after the reconstruction's last
    // angle wait, which would otherwise also wait for them. The score-tensor mode requests them
    // at the commit instead: its score stores count on the same in-order counter (measured).
    if constexpr (!SCORES)
      if (tt + kPTile < k1) fetch_raw_slot_w<2 * KSTEPS, CM>(P, slot_base(tt + kPTile), part, g, k_win, v_win);
    __syncthreads();
    // ------------------------------------------------------------ scores S^T = Kp Q^T
    float4v sacc[4][G];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) sacc[kt][gg] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8 ka = *(const half8*)&S.u.kp[0][16 * kt + n][32 * ks + 8 * gq];
#pragma unroll
        for (int gg = 0; gg < G; ++gg)
          sacc[kt][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[gg][ks], sacc[kt][gg], 0, 0, 0);
        if constexpr (EXACT) {
          const half8 kl = *(const half8*)&S.u.kp[EXACT ? 1 : 0][16 * kt + n][32 * ks + 8 * gq];
#pragma unroll
          for (int gg = 0; gg < G; ++gg)
            sacc[kt][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qf[gg][ks], sacc[kt][gg], 0, 0, 0);
        }
      }
    }
    const int lim = p0 + qj;  // last key this lane's query may see
    if constexpr (SCORES) {
      // lane holds keys tt + 16kt + 4gq + jj of query qj: one 16-byte store per 4 keys where the
      // rows are 16-byte aligned and all 4 keys are in range, single stores otherwise
      if (qvalid) {
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
          float* srow = a.s_out + (int64_t)(h * G + gg) * a.s_head_stride + (int64_t)qj * a.s_q_stride;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
            const int key0 = tt + 16 * kt + 4 * gq;
            float4v v;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              v[jj] = key0 + jj <= lim ? sacc[kt][gg][jj] * a.scale : -INFINITY;
            if (s_vec && key0 + 3 < k1) {
              *(float4v*)&srow[key0] = v;
            } else {
#pragma unroll
              for (int jj = 0; jj < 4; ++jj)
                if (key0 + jj < k1) srow[key0 + jj] = v[jj];
            }
          }
        }
      }
    } else {
      // ---------------------------------------------------------- online softmax per column
      float4v vr[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) vr[kt] = *(const float4v*)&S.vrul[16 * kt + 4 * gq];
      {
        // P * ruler_v is carried at scale 2^-ve (ve grows, behind a ballot, with the largest
        // ruler seen) so that it stays an fp16 normal below 2^15; rulers are >= 0
        float vmx = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) vmx = fmaxf(vmx, max3_mfma(vr[kt][0], vr[kt][1], fmaxf(vr[kt][2], vr[kt][3])));
        if (__builtin_amdgcn_ballot_w64(vmx >= v_thr) != 0) {  // rare: a large V ruler
          const int ve_new = wave_max_i((int)(__float_as_uint(vmx) >> 23) - 127) - 6;
          const float f = ldexpf(1.f, ve - ve_new);
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int gg = 0; gg < G; ++gg) o[dt][gg] *= f;
          ve = ve_new;
          v_thr = ldexpf(1.f, 7 + ve);
          v_mul = ldexpf(1.f, -ve);
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) vr[kt] *= v_mul;
      }
      half8 pb[G][2];
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        float mt = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int key = tt + 16 * kt + 4 * gq + jj;
            const float tv = (key < k1 && key <= lim) ? sacc[kt][gg][jj] * a.scale_log2 : -INFINITY;
            sacc[kt][gg][jj] = tv;
            mt = fmaxf(mt, tv);
          }
        mt = cross_row_max(mt);
        // lazy rescaling: the reference point moves only when the column max grows by more
        // than 2^8 (p <= 256 otherwise); a fully masked tile leaves it at -inf
        if (mt > m_run[gg] + 8.f) {
          const float alpha = exp2f(m_run[gg] - mt);
          m_run[gg] = mt;
          l_run[gg] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) o[dt][gg] *= alpha;
        }
        const float mref = m_run[gg] == -INFINITY ? 0.f : m_run[gg];
        float ps = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float p = fast_exp2(sacc[kt][gg][jj] - mref);
            ps += p;
            pb[gg][kt >> 1][4 * (kt & 1) + jj] = (_Float16)(p * vr[kt][jj]);
          }
        l_run[gg] += cross_row_sum(ps);
      }
      // ---------------------------------------------------------- O^T += Vt (P ruler_v)^T
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const uint2 lo = *(const uint2*)&S.vt[16 * dt + n][32 * k2 + 4 * gq];
          const uint2 hi = *(const uint2*)&S.vt[16 * dt + n][32 * k2 + 16 + 4 * gq];
          const half8 va = __builtin_bit_cast(half8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
          for (int gg = 0; gg < G; ++gg)
            o[dt][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[gg][k2], o[dt][gg], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // Kp / Vt / coef are overwritten by the next tile
  }
  if constexpr (SCORES) {
    return;
  } else {
    if (ve != 0) {  // the V-ruler scale taken back (exact)
      const float vsc = ldexpf(1.f, ve);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int gg = 0; gg < G; ++gg) o[dt][gg] *= vsc;
    }
  }

  // ---------------------------------------------------------------- output / split-K hand-off
  if (nparts == 1) {
    if (qvalid) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const float inv = 1.f / l_run[gg];
        const int64_t ob = (int64_t)(q0 + qj) * a.out_row_stride + (int64_t)(h * G + gg) * kD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            store_act(a.out, a.out_dtype, ob + 16 * dt + 4 * gq + jj, o[dt][gg][jj] * inv);
      }
    }
    return;
  }
  constexpr int kRowF = kD + 2;
  const int64_t pstride = (int64_t)G * kPQ * kRowF;
  float* partp = a.ws_part + ((int64_t)item * a.nsplit + sp) * pstride;
  auto st_agent = [](float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (qvalid) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      float* pr = partp + (int64_t)(gg * kPQ + 16 * wv + n) * kRowF;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) st_agent(&pr[16 * dt + 4 * gq + jj], o[dt][gg][jj]);
      if (gq == 0) {
        st_agent(&pr[kD], m_run[gg]);
        st_agent(&pr[kD + 1], l_run[gg]);
      }
    }
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(&a.ws_cnt[item], 1, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
    S.is_last = (prev == nparts - 1);
  }
  __syncthreads();
  if (!S.is_last) return;
  // Every partial is complete in L2 (write-through stores, waited on before their counter
  // update). An agent-scope acquire drops this CU's L1 copies, after which plain loads see the
  // partials -- and, unlike atomic loads, the loads of all chunks can be in flight together.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  auto ld_agent = [](const float* p) { return *p; };
  const float* pbase = a.ws_part + (int64_t)item * a.nsplit * pstride;
  const int nq = qe - qa;
  for (int it = tid; it < G * nq * kD; it += kPThreads) {
    const int dim = it % kD;
    const int row = it / kD;  // gg * nq + query
    const int gg = row / nq;
    const int qq = row - gg * nq;
    const int64_t ro = (int64_t)(gg * kPQ + qq) * kRowF;
    float M = -INFINITY;
#pragma unroll 8
    for (int c = 0; c < nparts; ++c) M = fmaxf(M, ld_agent(&pbase[c * pstride + ro + kD]));
    float L = 0.f, O = 0.f;
#pragma unroll 8
    for (int c = 0; c < nparts; ++c) {
      const float* pc = pbase + c * pstride + ro;
      const float mc = ld_agent(&pc[kD]);
      const float f = mc == -INFINITY ? 0.f : exp2f(mc - M);
      L = fmaf(ld_agent(&pc[kD + 1]), f, L);
      O = fmaf(ld_agent(&pc[dim]), f, O);
    }
    store_act(a.out, a.out_dtype,
              (int64_t)(q0 + qa + qq) * a.out_row_stride + (int64_t)(h * G + gg) * kD + dim, O / L);
  }
  if (tid == 0)
    __hip_atomic_store(&a.ws_cnt[item], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ttkv

// ------------------------------------------------------------------------------------ host side
#include "ttkv_host.h"

namespace ttkv {

template <int G, int RB, int VB, int KSTEPS, bool SCORES, int CM = kCoefI8>
static int launch_prefill_t(const PrefillArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(PrefillSmem<KSTEPS, true>);
  auto kfn = prefill_paged_kernel<G, RB, VB, KSTEPS, SCORES, CM>;
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kPThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string("prefill launch: ") + hipGetErrorString(e));
  return TTKV_OK;
}

template <int RB, int VB, int KSTEPS, bool SCORES>
static int prefill_dispatch_g(const PrefillArgs& a, int grid, hipStream_t st) {
  switch (a.G) {
    case 1: return launch_prefill_t<1, RB, VB, KSTEPS, SCORES>(a, grid, st);
    case 2: return launch_prefill_t<2, RB, VB, KSTEPS, SCORES>(a, grid, st);
    case 3: return launch_prefill_t<3, RB, VB, KSTEPS, SCORES>(a, grid, st);
    case 4: return launch_prefill_t<4, RB, VB, KSTEPS, SCORES>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "num_heads / H = " + std::to_string(a.G) +
                                           " query heads per KV head is not built for the "
                                           "multi-query read (1, 2, 3, 4)");
}

template <int RB, int VB, bool SCORES>
static int prefill_dispatch_k(const PrefillArgs& a, int ksteps, int grid, hipStream_t st) {
  // the fp16 and 4-bit coefficient modes are built for G = 3 and 64 < r1 <= 128
  if (a.g.coef_mode != kCoefI8) {
    if (a.G != 3 || ksteps != 4)
      return host_fail(TTKV_E_UNSUPPORTED, "fp16 and 4-bit coefficients are built for num_heads "
                                           "/ H = 3 and 64 < r1 <= 128");
    return a.g.coef_mode == kCoefF16 ? launch_prefill_t<3, RB, VB, 4, SCORES, kCoefF16>(a, grid, st)
                                     : launch_prefill_t<3, RB, VB, 4, SCORES, kCoefI4G32>(a, grid, st);
  }
  switch (ksteps) {
    case 2: return prefill_dispatch_g<RB, VB, 2, SCORES>(a, grid, st);
    case 4: return prefill_dispatch_g<RB, VB, 4, SCORES>(a, grid, st);
    case 5: return prefill_dispatch_g<RB, VB, 5, SCORES>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
}

// Key range per split: enough splits that the grid fills the chip about once at two resident
// workgroups per CU, each split at least 256 keys.
// Workgroups resident per CU (the kernel's launch bound): the G <= 2 kernels and the score-mode
// kernels up to G = 3 fit two, the others one.
static int prefill_blocks_per_cu(int G, bool scores) {
  return ((scores && G <= 3) || G <= 2) ? 2 : 1;
}

// Key range per work item: the items fill about one round of resident workgroups (fewer key
// splits where only one workgroup fits a CU: each split's partials cost a write and a read).
static int prefill_kchunk(int items, int max_seq_len, int block_size, int per_cu) {
  const int64_t target = (int64_t)per_cu * device_cu_count();
  const int64_t want = std::max<int64_t>(1, (target + items - 1) / std::max(items, 1));
  int64_t kc = (std::max(max_seq_len, 1) + want - 1) / want;
  kc = (kc + kPTile - 1) / kPTile * kPTile;
  kc = std::max<int64_t>(kc, 4 * kPTile);
  // the block ids of one key range are staged in LDS: at most kPSeg of them
  const int64_t seg_cap = (int64_t)(kPSeg - 2) * std::max(block_size, 1) / kPTile * kPTile;
  return (int)std::max<int64_t>(std::min(kc, seg_cap), kPTile);
}

// Batch rows per launch: one arrival counter per (row, head, query block).
static int prefill_slice_reqs(const Geom& g, int num_reqs, int max_q_len) {
  const int n_qb = (max_q_len + kPQ - 1) / kPQ;
  return std::min(num_reqs, std::max(1, kMaxCounters / (g.H * n_qb)));
}

// Partials of a launch over nr rows (0 when its keys are not split).
static int64_t prefill_part_bytes(const Geom& g, int G, int nr, int max_q_len, int max_seq_len,
                                  int block_size) {
  const int n_qb = (max_q_len + kPQ - 1) / kPQ;
  const int items = nr * g.H * n_qb;
  const int kc = prefill_kchunk(items, max_seq_len, block_size, prefill_blocks_per_cu(G, false));
  const int nsplit = std::max(1, (max_seq_len + kc - 1) / kc);
  if (nsplit == 1) return 0;
  return (int64_t)items * nsplit * G * kPQ * (kD + 2) * 4;
}

int64_t prefill_workspace_bytes(const Geom& g, int G, int num_reqs, int max_q_len,
                                int max_seq_len, int block_size) {
  if (num_reqs <= 0 || max_q_len <= 0) return 0;
  if (continuation_applies(g, G, max_q_len))
    return continuation_workspace_bytes(g, G, num_reqs, max_q_len, max_seq_len);
  const int slice = prefill_slice_reqs(g, num_reqs, max_q_len);
  const int64_t part = std::max(
      prefill_part_bytes(g, G, slice, max_q_len, max_seq_len, block_size),
      prefill_part_bytes(g, G, (num_reqs - 1) % slice + 1, max_q_len, max_seq_len, block_size));
  return part ? kCounterBytes + part : 0;
}

int prefill_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                  int64_t q_row_stride, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                  int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                  const int32_t* seq_lens, const int32_t* qsl, const int32_t* req_index,
                  int num_reqs, int max_q_len, int max_seq_len, const int32_t* dec_map,
                  int64_t num_blocks, const int8_t* dec_q, const float* dec_scale,
                  int64_t n_dec_slots, const float* cs_cache, int64_t max_pos, void* out,
                  int out_dtype, int64_t out_row_stride, float* s_out, int64_t s_head_stride,
                  int64_t s_q_stride, void* ws, int64_t ws_bytes, int32_t* err, hipStream_t st) {
  const bool scores = s_out != nullptr;
  if (g.d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (!((g.res_bits == 3 && g.v_bits == 3) || (g.res_bits == 4 && g.v_bits == 4)))
    return host_fail(TTKV_E_UNSUPPORTED, "res_bits/v_bits must be 3/3 or 4/4");
  if (HQ <= 0 || HQ % g.H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  const int G = HQ / g.H;
  const int ksteps = g.r1 <= 64 ? 2 : g.r1 <= 128 ? 4 : g.r1 <= 160 ? 5 : 0;
  if (!ksteps) return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
  if (g.coef_mode != kCoefI8 && (G != 3 || ksteps != 4))
    return host_fail(TTKV_E_UNSUPPORTED, "fp16 and 4-bit coefficients are built for num_heads / "
                                         "H = 3 and 64 < r1 <= 128");
  // the coefficient window (32 * ksteps ranks) is read in 16-byte chunks from the slot's start
  const int win_bytes = g.coef_mode == kCoefI8 ? 32 * ksteps
                        : g.coef_mode == kCoefF16 ? 64 * ksteps : 16 * ksteps;
  if (win_bytes > g.k_slot)
    return host_fail(TTKV_E_UNSUPPORTED, "padded coefficient block exceeds the K slot");
  if (!rows_in_windows(g))
    return host_fail(TTKV_E_UNSUPPORTED, "a head row of " + std::to_string(g.k_row) + "/" +
                                             std::to_string(g.v_row) +
                                             " bytes straddles its 64-byte load window");
  if (!q || !page || !bt || !seq_lens || !qsl || !dec_map || !cs_cache || !err)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (int rc = check_dec_pool(dec_q, dec_scale)) return rc;
  if (!scores && !out) return host_fail(TTKV_E_INVALID, "out is null");
  if ((uintptr_t)page % 16 || slot_stride % 16 || slot_stride < g.blob)
    return host_fail(TTKV_E_INVALID,
                     "page must be 16-byte aligned with a slot stride that is a multiple of 16 "
                     "and >= the blob (" + std::to_string(g.blob) + " bytes)");
  if ((uintptr_t)cs_cache % 16) return host_fail(TTKV_E_INVALID, "cos_sin_cache not 16-aligned");
  if (q_dtype < 0 || q_dtype > 2 || (!scores && (out_dtype < 0 || out_dtype > 2)))
    return host_fail(TTKV_E_INVALID, "dtype code");
  if (block_size <= 0) return host_fail(TTKV_E_INVALID, "block_size");
  if (num_reqs < 0 || max_seq_len < 0 || max_q_len < 0)
    return host_fail(TTKV_E_INVALID, "negative batch size");
  if (scores && num_reqs > 1)
    return host_fail(TTKV_E_INVALID, "the scores tensor is per request: num_reqs must be 1");
  if (num_reqs == 0 || max_q_len == 0) return TTKV_OK;
  if (max_q_len > max_seq_len)
    return host_fail(TTKV_E_INVALID, "max_q_len exceeds max_seq_len");
  if ((int64_t)max_blocks * block_size < max_seq_len)
    return host_fail(TTKV_E_INVALID, "max_seq_len=" + std::to_string(max_seq_len) +
                                         " needs more blocks than the block table row holds");
  if (max_seq_len > max_pos)
    return host_fail(TTKV_E_INVALID, "position " + std::to_string(max_seq_len - 1) +
                                         " is past the model's cos_sin_cache (" +
                                         std::to_string(max_pos) + " entries)");
  PrefillArgs a{};
  a.g = g;
  a.HQ = HQ;
  a.G = G;
  a.scale = scale;
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
  a.seq_lens = seq_lens;
  a.qsl = qsl;
  a.req_index = req_index;
  a.num_reqs = num_reqs;
  a.dec_map = dec_map;
  a.num_blocks = num_blocks;
  a.dec_q = dec_q;
  a.dec_scale = dec_scale;
  a.n_dec_slots = n_dec_slots;
  a.cs_cache = cs_cache;
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_row_stride = out_row_stride;
  a.s_out = s_out;
  a.s_head_stride = s_head_stride;
  a.s_q_stride = s_q_stride;
  a.err = err;
  a.max_seq = max_seq_len;
  a.max_q = max_q_len;
  a.n_qb = (max_q_len + kPQ - 1) / kPQ;
  if ((int64_t)g.H * a.n_qb > kMaxCounters)
    return host_fail(TTKV_E_UNSUPPORTED, "max_q_len=" + std::to_string(max_q_len) +
                                             " is past the longest query chunk built");
  if (!scores) {
    const int64_t need = prefill_workspace_bytes(g, G, num_reqs, max_q_len, max_seq_len, block_size);
    if (need && (!ws || ws_bytes < need))
      return host_fail(TTKV_E_WORKSPACE, "prefill workspace needs " + std::to_string(need) +
                                             " bytes, got " + std::to_string(ws_bytes));
    if (need && (uintptr_t)ws % 256)
      return host_fail(TTKV_E_INVALID, "workspace not 256-byte aligned");
  }
  // chunks of more than one 64-query block: every key expanded once, then attended by all the
  // chunk's queries (ttkv_continuation.hip)
  // the score tensor of a long chunk from the expanded tiles, when the caller gave a workspace
  // for them (without one, the fused kernel below)
  if (scores && ws) {
    const int64_t need = continuation_scores_workspace_bytes(g, G, max_q_len, max_seq_len);
    if (need && ws_bytes >= need && (uintptr_t)ws % 256 == 0)
      return continuation_scores(g, HQ, scale, q, q_dtype, q_row_stride, page, n_slots,
                                 slot_stride, block_size, bt, bt_row_stride, seq_lens, qsl,
                                 max_q_len, max_seq_len, dec_map, num_blocks, dec_q, dec_scale,
                                 n_dec_slots, cs_cache, s_out, s_head_stride, s_q_stride, ws, err,
                                 st);
  }
  if (!scores && continuation_applies(g, G, max_q_len))
    return continuation_paged(g, HQ, scale, q, q_dtype, q_row_stride, page, n_slots, slot_stride,
                              block_size, bt, bt_row_stride, seq_lens, qsl, req_index, num_reqs,
                              max_q_len, max_seq_len, dec_map, num_blocks, dec_q, dec_scale,
                              n_dec_slots, cs_cache, out, out_dtype, out_row_stride, ws, err, st);
  const int slice = prefill_slice_reqs(g, num_reqs, max_q_len);
  for (int ri0 = 0; ri0 < num_reqs; ri0 += slice) {
    PrefillArgs b = a;
    b.ri0 = ri0;
    b.num_reqs = std::min(slice, num_reqs - ri0);
    const int items = b.num_reqs * g.H * a.n_qb;
    b.kchunk = prefill_kchunk(items, max_seq_len, block_size, prefill_blocks_per_cu(G, scores));
    b.nsplit = std::max(1, (max_seq_len + b.kchunk - 1) / b.kchunk);
    if (!scores && b.nsplit > 1) {  // counters [item]: items <= kMaxCounters
      b.ws_cnt = (int*)ws;
      b.ws_part = (float*)((char*)ws + kCounterBytes);
    }
    b.nwork = items * b.nsplit;
    const int grid = (b.nwork + 7) / 8 * 8;
    int rc;
    if (scores)
      rc = g.res_bits == 3 ? prefill_dispatch_k<3, 3, true>(b, ksteps, grid, st)
                           : prefill_dispatch_k<4, 4, true>(b, ksteps, grid, st);
    else
      rc = g.res_bits == 3 ? prefill_dispatch_k<3, 3, false>(b, ksteps, grid, st)
                           : prefill_dispatch_k<4, 4, false>(b, ksteps, grid, st);
    if (rc != TTKV_OK) return rc;
  }
  return TTKV_OK;
}

}  // namespace ttkv

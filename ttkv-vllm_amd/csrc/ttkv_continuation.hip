// K2 for continuation chunks of two or more queries, in two launches. gfx950 / CDNA4.
//
// The fused continuation kernel (ttkv_prefill.hip) reconstructs every key tile once per 64-query
// block and holds the decoder, query, score and output fragments of a whole work item at once
// (one wave per SIMD): Q / 64 reconstructions of every stored key for a chunk of Q queries, and
// one wave per SIMD to hide their latency. Here the work is split where the reuse is:
//
//   K2a expand : per (request, KV head, run of 64-key tiles): the commit / decode /
//                reconstruction of the fused kernel, once per key. Each tile is written to the
//                workspace as
//                  khi, klo [64 keys][16 chunks][8] fp16 -- the rotated key split hi + lo (its
//                                                       fp32 value to 22 significant bits); chunk c
//                                                       holds dims 4c..4c+3 and 64+4c..64+4c+3
//                                                       (tile_dims)
//                  vt       [128 dims][64 keys] fp16 -- the V codes c - 2^(b-1), exact small
//                                                       integers, keys in MFMA k-slot order
//                  vrul     [64] fp32               -- the V row rulers
//                Keys past the context are written as zeros (masked by the causal rule).
//   K2b attend : flash attention over those tiles. A 512-thread workgroup owns 128 queries x G
//                heads of one (request, KV head, key split); wave w owns queries 16w..16w+15.
//                Per 64-key tile: S^T = K Q^T on MFMA (hi and lo key halves against the fp16
//                query), causal -inf, online base-2 softmax per query column, O^T += Vt (P *
//                ruler_v)^T on MFMA with P * ruler_v * 2^-ve rounded to fp16 once (ve >= 0 grows
//                with the largest V ruler seen, keeping it below 2^15), in 32-key halves.
//                Waves 4..7 run half a tile behind waves 0..3 (three LDS tile buffers, one
//                barrier per tile), so each SIMD's two waves overlap MFMA with softmax. The
//                next tile is copied to LDS while the current ones are
//                computed, by direct global -> LDS DMA issued at the barrier. Key splits are
//                combined in the same launch by the last workgroup.
//
// The arithmetic is the fused kernel's, so results agree with it to fp32 rounding: the same
// exact fp16 coefficient / hi+lo decoder reconstruction, k = cs * acc + ruler * code, RoPE in
// fp32, the same hi+lo rotated key against the fp16 query, the same fp16 rounding of P * ruler_v.
//
// Reference semantics: vllm_ttkv/impl.py:725-778 (_prefill_continuation), reference.py:112-146
// (raw_scores_multi: -inf where key > p0 + j), krt_triton.py:154-317, v_out_triton.py:158-293.
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kXTile = 64;                 // keys per tile
constexpr int kXThreads = 256;             // expand workgroup
constexpr int kAThreads = 512;             // attend workgroup (8 waves)
constexpr int kAQ = 128;                   // queries per attend work item (16 per wave)
constexpr int kXSeg = 260;                 // block ids of one expand item staged in LDS
constexpr int kTileKhi = 0;                // byte offsets inside one workspace tile
constexpr int kTileKlo = kXTile * kD * 2;
constexpr int kTileVt = 2 * kXTile * kD * 2;
constexpr int kTileVrul = 3 * kXTile * kD * 2;
constexpr int kTileBytes = kTileVrul + kXTile * 4;  // 49,408
constexpr int kTileChunks = kTileBytes / 16;        // 3088 16-byte chunks
constexpr int kMaxParts = 48;             // key splits of one attend item (LDS weights)
constexpr int kXRawDw = 17;                // staged row dwords (16 + slack): odd, so rows spread over banks
constexpr int kXCode = 144;

// tile_dims: the 16-byte chunk c of a workspace key row holds dims 4c..4c+3 then 64+4c..64+4c+3
// -- exactly the 8 values one lane of the expand's reconstruction holds (dims dl..dl+3 and
// 64+dl..64+dl+3, dl = 4c), so each lane writes one 16-byte chunk per half. A dot product over
// all 128 dims does not depend on their order: the attend and scores kernels read the query's
// dims in the same order into the matching B fragments.
// Position of key k of a 64-key tile in the MFMA k-slot order of the P.V contraction: a 32-key
// step's lane group g holds keys 4g..4g+3 and 16+4g..16+4g+3, stored as 8 consecutive slots.
__host__ __device__ constexpr int vt_slot(int k) {
  return (k & 32) | (((k >> 2) & 3) << 3) | (((k >> 4) & 1) << 2) | (k & 3);
}

struct ExpandArgs {
  Geom g;
  const uint8_t* page;
  int64_t n_slots, slot_stride;
  int block_size;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* seq_lens;
  const int32_t* req_index;
  int ri0, num_reqs;
  const int32_t* dec_map;
  int64_t num_blocks;
  const int8_t* dec_q;  // decoder pool (see dec_ranks)
  const float* dec_scale;
  int64_t n_dec_slots;
  const float* cs_cache;
  uint8_t* tiles;     // [num_reqs][H][ntl] tiles of kTileBytes
  int ntl, tpi, nchunk, max_seq;
  int* err;
};

// The tile's outputs go from registers straight to the workspace: each store writes whole 32-byte
// (K) or 128-byte (V) row pieces, and the 4 waves complete every line in L2.
template <int KSTEPS>
struct ExpandSmem {
  static constexpr int kCoefStride = KSTEPS * 32 + 8;
  _Float16 coef[kXTile][kCoefStride];  // commit -> recon
  uint32_t rawk[kXTile][kXRawDw];      // commit -> decode
  uint32_t rawgap[16];                 // V rows 16 dwords off: a token's K and V rows on other banks
  uint32_t rawv[kXTile][kXRawDw];
  uint8_t kcode[kXTile][kXCode];       // decode -> recon
  uint8_t vcode[kXTile][kXCode];       // decode -> transpose
  uint2 lut[256];
  int32_t seg[kXSeg];
  float cs[kXTile], krul[kXTile], vrul[kXTile];
};

template <int RB, int VB, int KSTEPS, int CM>
__global__ __launch_bounds__(kXThreads, 2) void expand_kernel(ExpandArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint16_t lut3s[kLut3Entries];  // static: its address folds into the loads
  ExpandSmem<KSTEPS>& S = *reinterpret_cast<ExpandSmem<KSTEPS>*>(smem_raw);
  static_assert(RB == VB, "K and V rows decode with one code path (3/3 and 4/4 are built)");
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // items ((row, chunk), head), the H heads of one chunk consecutive and on one XCD (blocks go
  // round-robin over the 8 XCDs) so they share its L2 for the chunk's coefficient bytes
  const int nwork = a.num_reqs * a.nchunk * g.H;
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= nwork) return;
  const int h = w % g.H;
  const int c = (w / g.H) % a.nchunk;
  const int ri = w / g.H / a.nchunk;
  const int r = a.req_index ? a.req_index[a.ri0 + ri] : a.ri0 + ri;
  const int seq = min(max(a.seq_lens[r], 0), a.max_seq);  // the launcher checked the bounds
  const int ntiles = (seq + kXTile - 1) / kXTile;
  const int t_lo = c * a.tpi;
  const int t_hi = min(ntiles, t_lo + a.tpi);
  if (t_lo >= t_hi) return;
  const int k0 = t_lo * kXTile;
  const int k1 = min(seq, t_hi * kXTile);

  const int blk0 = a.bt[(int64_t)r * a.bt_row_stride];
  int dslot = -1;
  if (blk0 >= 0 && blk0 < a.num_blocks) dslot = a.dec_map[blk0];
  if (dslot < 0 || dslot >= a.n_dec_slots) {  // the attend launch writes this request's NaN rows
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    return;
  }

  build_luts(S.lut, (RB == 3 || VB == 3) ? lut3s : nullptr, tid, kXThreads);

  // decoder fragments (A operand, M = dims), hi + lo fp16, resident in registers
  // (int8 ranks 32s + 8gq .. +7 of the lane's two columns, 8 bytes per step, and their rulers;
  // 32 KSTEPS <= R, so every load is inside the decoder)
  const int HD = g.H * kD;
  const int R = dec_ranks(g.r1);
  const int8_t* decq = a.dec_q + ((int64_t)dslot * HD + h * kD) * R;
  const float* decs = a.dec_scale + (int64_t)dslot * R;
  u32x2v dq[2][KSTEPS];
  float4v dsc[2 * KSTEPS];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int8_t* col = decq + (int64_t)(16 * (wv + 4 * mi) + n) * R;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) dq[mi][s] = *gbl((const u32x2v*)(col + 32 * s + 8 * gq));
  }
#pragma unroll
  for (int s = 0; s < 2 * KSTEPS; ++s)
    dsc[s] = *gbl((const float4v*)(decs + 32 * (s >> 1) + 8 * gq + 4 * (s & 1)));
  half8 ahi[2][KSTEPS], alo[2][KSTEPS];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      float v[8];
      dec_values4(dq[mi][s][0], dsc[2 * s], v);
      dec_values4(dq[mi][s][1], dsc[2 * s + 1], v + 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = 32 * s + 8 * gq + j < g.r1 ? v[j] : 0.f;
        const _Float16 hi = (_Float16)f;
        ahi[mi][s][j] = hi;
        alo[mi][s][j] = (_Float16)(f - (float)hi);
      }
    }
  }

  const int k_row_off = g.k_field + h * g.k_row;
  const int v_row_off = g.k_slot + h * g.v_row;
  const int ptok = tid >> 2;
  const int part = tid & 3;
  const int dl = 16 * wv + 4 * gq;
  const float voff = (float)(1 << (VB - 1));
  const uint32_t ksel = stage_selector(k_row_off & 3, part != 0);
  const uint32_t vsel = stage_selector(v_row_off & 3, part != 0);
  const float inv_unit = 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
  const int bfirst = k0 / a.block_size;
  const int nseg = (k1 - 1) / a.block_size - bfirst + 1;  // <= kXSeg (host-bounded)
  for (int i = tid; i < nseg; i += kXThreads) {
    int blk = a.bt[(int64_t)r * a.bt_row_stride + bfirst + i];
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, TTKV_ERR_BAD_BLOCK);
      blk = -1;
    }
    S.seg[i] = blk;
  }
  __syncthreads();
  auto slot_base = [&](int tt) -> const uint8_t* {
    if (ptok >= min(kXTile, k1 - tt)) return nullptr;
    const int pos = tt + ptok;
    const int bi = pos / a.block_size;
    const int blk = S.seg[bi - bfirst];
    if (blk < 0) return nullptr;
    const int64_t slot = (int64_t)blk * a.block_size + (pos - bi * a.block_size);
    return slot < a.n_slots ? a.page + slot * a.slot_stride : nullptr;
  };
  const int k_win = k_row_off & ~15, v_win = v_row_off & ~15;
  RawSlotW<2 * KSTEPS, CM> P;
  fetch_raw_slot_w<2 * KSTEPS, CM>(P, slot_base(k0), part, g, k_win, v_win);
  uint8_t* tile_out = a.tiles + (((int64_t)ri * g.H + h) * a.ntl + t_lo) * kTileBytes;

  for (int tt = k0; tt < k1; tt += kXTile, tile_out += kTileBytes) {
    const int ntile = min(kXTile, k1 - tt);
    // ------------------------------------------------------------ commit this tile's bytes
    {
      const float cs = commit_coef<2 * KSTEPS, CM>(P, (uint32_t*)&S.coef[ptok][0], part, g);
      if (part == 0) S.cs[ptok] = cs;
      stage_row_w(P.krow, (k_row_off & 15) >> 2, ksel, &S.rawk[ptok][part * 4]);
      stage_row_w(P.vrow, (v_row_off & 15) >> 2, vsel, &S.rawv[ptok][part * 4]);
    }
    // This tile's angle rows, then the next tile's slot bytes, are requested before any of the
    // tile's stores: loads and stores complete in order (vmcnt), so a load issued after the
    // stores could only be waited on together with them.
    float4v cvA[4], svA[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int key = 16 * nb + n;
      const int pos = key < ntile ? tt + key : tt;
      cvA[nb] = *gbl((const float4v*)&a.cs_cache[(int64_t)pos * kD + dl]);
      svA[nb] = *gbl((const float4v*)&a.cs_cache[(int64_t)pos * kD + 64 + dl]);
    }
    if (tt + kXTile < k1)
      fetch_raw_slot_w<2 * KSTEPS, CM>(P, slot_base(tt + kXTile), part, g, k_win, v_win);
    // No barrier: wave w commits and decodes the same 16 keys (16w .. 16w+15), and LDS accesses
    // of one wave complete in order (the fences only keep the compiler from moving them); the
    // previous tile's readers finished before its closing barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_s_setprio(1);
    // ------------------------------------------------------------ decode (thread = half row)
    {
      // lanes 0..31: K rows, 32..63: V rows of this wave's 16 keys, two threads per row; one
      // decode call with per-lane row and destination (the two kinds share the code width)
      const bool is_v = lane >= 32;
      const int key = 16 * wv + ((lane >> 1) & 15);
      const int half = lane & 1;
      const uint32_t* row = is_v ? S.rawv[key] : S.rawk[key];
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
    // vt[dim][slot] = code - 2^(b-1) in fp16 (exact), key 4kg + j at slot vt_slot(4kg) + j; the
    // 16 threads of one dim group write that dim row's 128 bytes
    auto* vt_out = gblw((u32x2v*)(tile_out + kTileVt));
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int b = tid + kXThreads * it;
      const int kg = b & 15, dg = b >> 4;
      const uint32_t x0 = *(const uint32_t*)&S.vcode[4 * kg + 0][4 * dg];
      const uint32_t x1 = *(const uint32_t*)&S.vcode[4 * kg + 1][4 * dg];
      const uint32_t x2 = *(const uint32_t*)&S.vcode[4 * kg + 2][4 * dg];
      const uint32_t x3 = *(const uint32_t*)&S.vcode[4 * kg + 3][4 * dg];
      const uint32_t a01l = __builtin_amdgcn_perm(x1, x0, 0x05010400u);
      const uint32_t a01h = __builtin_amdgcn_perm(x1, x0, 0x07030602u);
      const uint32_t a23l = __builtin_amdgcn_perm(x3, x2, 0x05010400u);
      const uint32_t a23h = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
      uint32_t y[4];
      y[0] = __builtin_amdgcn_perm(a23l, a01l, 0x05040100u);
      y[1] = __builtin_amdgcn_perm(a23l, a01l, 0x07060302u);
      y[2] = __builtin_amdgcn_perm(a23h, a01h, 0x05040100u);
      y[3] = __builtin_amdgcn_perm(a23h, a01h, 0x07060302u);
      // the 4 keys 4kg..4kg+3 are consecutive slots
      const int slot0 = vt_slot(4 * kg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t p01, p23;
        if constexpr (VB == 3) {
          p01 = __builtin_bit_cast(uint32_t,
                                   __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y[i], inv_unit, false));
          p23 = __builtin_bit_cast(uint32_t,
                                   __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(y[i], inv_unit, true));
        } else {
          u8x4_to_f16_minus(y[i], voff, p01, p23);
        }
        vt_out[((4 * dg + i) * kXTile + slot0) >> 2] = u32x2v{p01, p23};
      }
    }
    if (tid < kXTile / 4)
      gblw((u32x4*)(tile_out + kTileVrul))[tid] = *(const u32x4*)&S.vrul[4 * tid];
    // ------------------------------------------------------------ recon + residual + RoPE -> K
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int key = 16 * nb + n;
      const float4v cv = cvA[nb], sv = svA[nb];
      float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const half8 b = *(const half8*)&S.coef[key][32 * s + 8 * gq];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0][s], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1][s], b, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0][s], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1][s], b, acc1, 0, 0, 0);
      }
      const float cs = S.cs[key];
      const float kr = S.krul[key];
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
        zl[i >> 1][i & 1] = (_Float16)(y1 - (float)h1);
        zh[i >> 1][i & 1] = (_Float16)(y2 - (float)h2);
      }
      // khi / klo [key][chunk]: this lane's dims dl..dl+3 and 64+dl..64+dl+3 are chunk dl / 4
      // (tile_dims), one 16-byte store each
      auto* kh_out = gblw((u32x4*)(tile_out + kTileKhi + key * kD * 2));
      auto* kl_out = gblw((u32x4*)(tile_out + kTileKlo + key * kD * 2));
      kh_out[dl >> 2] = u32x4{__builtin_bit_cast(uint32_t, yl[0]), __builtin_bit_cast(uint32_t, yl[1]),
                              __builtin_bit_cast(uint32_t, yh[0]), __builtin_bit_cast(uint32_t, yh[1])};
      kl_out[dl >> 2] = u32x4{__builtin_bit_cast(uint32_t, zl[0]), __builtin_bit_cast(uint32_t, zl[1]),
                              __builtin_bit_cast(uint32_t, zh[0]), __builtin_bit_cast(uint32_t, zh[1])};
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();  // coef / kcode / vcode / rulers are overwritten by the next tile
  }
}

// ------------------------------------------------------------------------------------ attend
struct AttendArgs {
  Geom g;
  int HQ, G;
  float scale_log2;
  const void* q;
  int q_dtype;
  int64_t q_row_stride;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* seq_lens;
  const int32_t* qsl;
  const int32_t* req_index;
  int ri0, num_reqs;
  const int32_t* dec_map;
  int64_t num_blocks, n_dec_slots;
  const uint8_t* tiles;
  int ntl;
  void* out;
  int out_dtype;
  int64_t out_row_stride;
  float* ws_part;
  int* ws_cnt;
  int* err;
  int n_qb, kchunk, nsplit, max_seq, max_q;
};

// one 64-key tile in LDS (three are resident: see the loop): khi, klo rows of 16 chunks and vt
// rows of 8 chunks, chunk c of row k at
// c ^ (k & 7) (rows read by lanes 0..7 of a wave land in 8 different bank groups); then vrul
struct AttendTile {
  u32x4 khi[kXTile][16];
  u32x4 klo[kXTile][16];
  u32x4 vt[kD][8];
  float vrul[kXTile];
};
struct AttendSmem {
  AttendTile t[3];
  int is_last;
};

template <int G>
__global__ __launch_bounds__(kAThreads, 2) void attend_kernel(AttendArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  AttendSmem& S = *reinterpret_cast<AttendSmem*>(smem_raw);
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // items (row, head, split, query block): the query blocks of one key range consecutive, on one
  // XCD, so they read the same workspace tiles through its L2
  const int nwork = a.num_reqs * g.H * a.nsplit * a.n_qb;
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= nwork) return;
  const int qb = w % a.n_qb;
  int t = w / a.n_qb;
  const int sp = t % a.nsplit;
  t /= a.nsplit;
  const int h = t % g.H;
  const int ri = t / g.H;
  const int r = a.req_index ? a.req_index[a.ri0 + ri] : a.ri0 + ri;
  const int q0 = a.qsl[r];
  int qlen = a.qsl[r + 1] - q0;
  int seq = a.seq_lens[r];
  const bool lead = (tid == 0 && sp == 0 && qb == 0 && h == 0);
  if (seq > a.max_seq || qlen > a.max_q) {
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    seq = min(seq, a.max_seq);
    qlen = min(qlen, a.max_q);
  }
  const int p0 = seq - qlen;
  const int qa = qb * kAQ;
  if (qlen <= 0 || qa >= qlen) return;
  if (p0 < 0) {
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    return;
  }
  const int qe = min(qlen, qa + kAQ);
  const int kmax = min(seq, p0 + qe);  // keys any query of the block may see
  const int nparts = (kmax + a.kchunk - 1) / a.kchunk;
  if (sp >= nparts) return;
  const int k0 = sp * a.kchunk;
  const int k1 = min(kmax, k0 + a.kchunk);
  const int item = (ri * g.H + h) * a.n_qb + qb;

  const int blk0 = a.bt[(int64_t)r * a.bt_row_stride];
  int dslot = -1;
  if (blk0 >= 0 && blk0 < a.num_blocks) dslot = a.dec_map[blk0];
  if (dslot < 0 || dslot >= a.n_dec_slots) {  // expand skipped this request: NaN rows
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    if (sp == 0)
      for (int i = tid; i < G * (qe - qa) * kD; i += kAThreads) {
        const int dim = i % kD;
        const int qq = qa + (i / kD) % (qe - qa);
        const int gg = i / kD / (qe - qa);
        store_act(a.out, a.out_dtype,
                  (int64_t)(q0 + qq) * a.out_row_stride + (int64_t)(h * G + gg) * kD + dim, NAN);
      }
    return;
  }

  const uint8_t* tbase = a.tiles + ((int64_t)ri * g.H + h) * a.ntl * kTileBytes;
  // Tile copies global -> LDS by DMA (global_load_lds_dwordx4): one wave instruction fills 64
  // consecutive 16-byte chunks of a buffer's image, each lane gathering the workspace chunk that
  // belongs in its slot (chunk c of row k sits at c ^ (k & 7)). Wave w moves image chunks
  // 64 (w + 8 i): 4 instructions for the K half, 2 for the V half, and wave 0 the 16 vrul
  // chunks. Each wave waits for its own (vmcnt(0)) before the next barrier.
  // source chunk of this lane's slot in each of its 6 full instructions (the same every tile)
  int dsrc[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int P = (i < 4 ? 64 * (wv + 8 * i) : 2048 + 64 * (wv + 8 * (i - 4))) + lane;
    if (P < 2048) {
      const int row = (P >> 4) & 63, pc = P & 15;
      dsrc[i] = (P & ~1023) + row * 16 + (pc ^ (row & 7));
    } else {
      const int row = (P - 2048) >> 3, pc = P & 7;
      dsrc[i] = 2048 + row * 8 + (pc ^ (row & 7));
    }
  }
  auto dma_tile = [&](AttendTile& T, int tile) {
    const u32x4* src = (const u32x4*)(tbase + (int64_t)tile * kTileBytes);
    typedef __attribute__((address_space(3))) void* lds_ptr;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int c0 = i < 4 ? 64 * (wv + 8 * i) : 2048 + 64 * (wv + 8 * (i - 4));
      __builtin_amdgcn_global_load_lds(gbl(src + dsrc[i]), (lds_ptr)((u32x4*)&T + c0), 16, 0, 0);
    }
    if (wv == 0 && lane < kTileChunks - 3072)  // the 16 vrul chunks, unswizzled
      __builtin_amdgcn_global_load_lds(gbl(src + 3072 + lane), (lds_ptr)((u32x4*)&T + 3072), 16, 0, 0);
  };

  // query fragments (B operand of S^T = K Q^T): column n = query qa + 16 wv + n of head h*G+gg
  const int qj = qa + 16 * wv + n;
  const bool qvalid = qj < qe;
  half8 qf[G][4];
  {
    const bool qvec = act_rows_aligned(a.q, a.q_dtype, a.q_row_stride);
    // k-step ks, lane group gq: the dims of key chunk 4 ks + gq (tile_dims)
    const int64_t qrow = (int64_t)(q0 + (qvalid ? qj : qa)) * a.q_row_stride + (int64_t)h * G * kD +
                         4 * gq;
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float tq[8];
        load_act_n<4>(a.q, a.q_dtype, qrow + (int64_t)gg * kD + 16 * ks, qvec, tq);
        load_act_n<4>(a.q, a.q_dtype, qrow + (int64_t)gg * kD + 64 + 16 * ks, qvec, tq + 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][ks][i] = qvalid ? (_Float16)tq[i] : (_Float16)0.0f;
      }
  }
  float4v o[8][G];
  float m_run[G], l_run[G];
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    m_run[gg] = -INFINITY;
    l_run[gg] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt][gg] = float4v{0.f, 0.f, 0.f, 0.f};
  }

  const int tl0 = k0 / kXTile, ntl_item = (k1 + kXTile - 1) / kXTile - tl0;
  const int lim = p0 + qj;  // last key this lane's query may see
  const float sl2 = a.scale_log2;

  // One half step: keys 32 hf .. 32 hf + 31 of tile tl (buffer T): scores, softmax, P.V.
  // LDS byte offsets of this lane's fragments inside a tile image: the swizzle only involves
  // row & 7 = n & 7, so they are fixed per lane (rows add multiples of 16 rows)
  uint32_t koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = n * 256 + (((4 * ks + gq) ^ (n & 7)) << 4);
  uint32_t voff[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) voff[hf] = 32768 + n * 128 + (((4 * hf + gq) ^ (n & 7)) << 4);
  float l_lane[G];  // per-lane partial normalisers, summed over the column at the end
#pragma unroll
  for (int gg = 0; gg < G; ++gg) l_lane[gg] = 0.f;
  // P * ruler_v is carried at scale 2^-ve so that it stays an fp16 normal below 2^15 (P <= 2^8):
  // ve grows, behind a ballot, when a half step brings a ruler of 2^(7 + ve) or more, and the
  // wave's accumulators are rescaled by an exact power of two (ve is per wave: its own rows)
  int ve = 0;
  float v_thr = 128.f, v_mul = 1.f;

  auto half_step = [&](const AttendTile& T, int tl, int hf) {
    const int tt = tl * kXTile;
    const char* tb = (const char*)&T;
    // -------------------------------------------------------- scores S^T = K Q^T
    float4v sacc[2][G];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const char* rb = tb + (32 * hf + 16 * k2) * 256;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8 ka = *(const half8*)(rb + koff[ks]);
        const half8 kl = *(const half8*)(rb + 16384 + koff[ks]);
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
          sacc[k2][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              ka, qf[gg][ks], ks ? sacc[k2][gg] : float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          sacc[k2][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qf[gg][ks], sacc[k2][gg], 0, 0, 0);
        }
      }
    }
    // -------------------------------------------------------- causal mask (boundary tiles only)
    // key t is visible to this lane's query iff t <= min(k1 - 1, p0 + qj); a tile whose every
    // key is visible to the block's first query needs no mask (a uniform branch)
    if (!(tt + kXTile <= k1 && tt + kXTile - 1 <= p0 + qa)) {
      const int last = min(k1 - 1, lim) - (tt + 32 * hf + 4 * gq);
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int gg = 0; gg < G; ++gg)
            sacc[k2][gg][jj] = 16 * k2 + jj <= last ? sacc[k2][gg][jj] : -INFINITY;
    }
    // -------------------------------------------------------- online softmax per column
    // (raw scores; the scale enters the exponent's fma, and m_run is in scaled units)
    float4v vr0 = *(const float4v*)(tb + 49152 + (32 * hf + 4 * gq) * 4);
    float4v vr1 = *(const float4v*)(tb + 49152 + (32 * hf + 16 + 4 * gq) * 4);
    {
      // rulers are >= 0 (rows past the context carry 0)
      const float vmx = fmaxf(max3_mfma(vr0[0], vr0[1], vr0[2]),
                              max3_mfma(vr0[3], vr1[0], fmaxf(vr1[1], fmaxf(vr1[2], vr1[3]))));
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
      vr0 *= v_mul;
      vr1 *= v_mul;
    }
    half8 pb[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const float m01 = max3_mfma(sacc[0][gg][0], sacc[0][gg][1], sacc[0][gg][2]);
      const float m23 = max3_mfma(sacc[0][gg][3], sacc[1][gg][0], sacc[1][gg][1]);
      float mt = max3_mfma(m01, m23, max3_mfma(sacc[1][gg][2], sacc[1][gg][3], sacc[1][gg][3]));
      mt *= sl2;
      // Lazy rescaling: the reference point moves only when a column max grows by more than 2^8
      // (p <= 256 otherwise), which is rare after a column's first tile, so the column max and
      // the rescale sit behind a wave-uniform ballot. A fully masked column stays at -inf.
      if (__builtin_amdgcn_ballot_w64(mt > m_run[gg] + 8.f) != 0) {
        const float cm = cross_row_max(mt);
        const bool up = cm > m_run[gg] + 8.f;  // the same in the column's 4 lanes
        const float alpha = up ? exp2f(m_run[gg] - cm) : 1.f;
        m_run[gg] = up ? cm : m_run[gg];
        l_lane[gg] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt][gg] *= alpha;
      }
      const float nref = m_run[gg] == -INFINITY ? 0.f : -m_run[gg];
      float ps = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float pr = fast_exp2(fmaf(sacc[k2][gg][jj], sl2, nref));
          ps += pr;
          pb[gg][4 * k2 + jj] = (_Float16)(pr * (k2 ? vr1[jj] : vr0[jj]));
        }
      l_lane[gg] += ps;
    }
    // -------------------------------------------------------- O^T += Vt (P ruler_v)^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const half8 va = *(const half8*)(tb + dt * 2048 + voff[hf]);
#pragma unroll
      for (int gg = 0; gg < G; ++gg)
        o[dt][gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[gg], o[dt][gg], 0, 0, 0);
    }
  };

  // Waves 4..7 run half a tile behind waves 0..3, so that the two waves sharing a SIMD are in
  // different phases (one's MFMAs beside the other's softmax). Barrier k: waves 0..3 have
  // finished tiles < k, waves 4..7 tiles < k - 1 and half 0 of tile k - 1. Between barriers k
  // and k + 1 tiles k - 1 and k are read and tile k + 1 is written, into buffer (k + 1) % 3,
  // whose last reader (tile k - 2) finished before barrier k.
  dma_tile(S.t[0], tl0);
  const bool late = wv >= 4;
  for (int k = 0; k <= ntl_item; ++k) {
    // this wave's DMA writes have landed (the barrier's workgroup-scope fence does not wait for
    // them), then every wave's have
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (k + 1 < ntl_item) dma_tile(S.t[(k + 1) % 3], tl0 + k + 1);
    if (!late) {
      if (k < ntl_item) {
        half_step(S.t[k % 3], tl0 + k, 0);
        half_step(S.t[k % 3], tl0 + k, 1);
      }
    } else {
      if (k >= 1) half_step(S.t[(k - 1) % 3], tl0 + k - 1, 1);
      if (k < ntl_item) half_step(S.t[k % 3], tl0 + k, 0);
    }
  }

#pragma unroll
  for (int gg = 0; gg < G; ++gg) l_run[gg] = cross_row_sum(l_lane[gg]);
  if (ve != 0) {  // the V-ruler scale taken back (exact)
    const float vsc = ldexpf(1.f, ve);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int gg = 0; gg < G; ++gg) o[dt][gg] *= vsc;
  }

  // ---------------------------------------------------------------- output / split-K hand-off
  // out rows aligned for 4-element stores (16 bytes fp32, 8 bytes fp16 / bf16)
  const bool ovec = (uintptr_t)a.out % 16 == 0 && a.out_row_stride % 4 == 0;
  if (nparts == 1) {
    if (qvalid) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const float inv = 1.f / l_run[gg];
        const int64_t ob = (int64_t)(q0 + qj) * a.out_row_stride + (int64_t)(h * G + gg) * kD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
          store_act4(a.out, a.out_dtype, ob + 16 * dt + 4 * gq, o[dt][gg] * inv, ovec);
      }
    }
    return;
  }
  // Partials of split sp: O rows [G * kAQ][kD] (16-byte stores), then (m, l) per row.
  constexpr int kRows = G * kAQ;
  const int64_t pstride = (int64_t)kRows * (kD + 2);
  float* po = a.ws_part + ((int64_t)item * a.nsplit + sp) * pstride;
  float* pml = po + (int64_t)kRows * kD;
  if (qvalid) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const int row = gg * kAQ + 16 * wv + n;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) store_agent16(&po[(int64_t)row * kD + 16 * dt + 4 * gq], o[dt][gg]);
      if (gq == 0) store_agent8(&pml[2 * row], float2v{m_run[gg], l_run[gg]});
    }
  }
  // the write-through partial stores are complete at the device-coherent level before the
  // counter update (no L2 writeback needed on this side)
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(&a.ws_cnt[item], 1, __ATOMIC_ACQ_REL,
                                            __HIP_MEMORY_SCOPE_AGENT);
    S.is_last = (prev == nparts - 1);
  }
  __syncthreads();
  if (!S.is_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // combine: per row the weights exp2(m_c - M) / L of every split (in the tile buffers' LDS,
  // free now), then each output float4 as one weighted sum of the splits' float4s, four outputs'
  // loads in flight at a time
  const float* pbase = a.ws_part + (int64_t)item * a.nsplit * pstride;
  const int nq = qe - qa;
  float* wsm = (float*)&S.t[0];  // [nparts][kRows], nparts <= kMaxParts (host-bounded)
  for (int row = tid; row < kRows; row += kAThreads) {
    if (row % kAQ >= nq) continue;
    float M = -INFINITY;
    for (int c = 0; c < nparts; ++c) M = fmaxf(M, pbase[c * pstride + (int64_t)kRows * kD + 2 * row]);
    float L = 0.f;
    for (int c = 0; c < nparts; ++c) {
      const float* ml = pbase + c * pstride + (int64_t)kRows * kD + 2 * row;
      const float e = ml[0] == -INFINITY ? 0.f : exp2f(ml[0] - M);
      L = fmaf(ml[1], e, L);
      wsm[c * kRows + row] = e;
    }
    const float inv = 1.f / L;
    for (int c = 0; c < nparts; ++c) wsm[c * kRows + row] *= inv;
  }
  __syncthreads();
  const int nout = G * nq * (kD / 4);
  for (int i0 = tid; i0 < nout; i0 += 4 * kAThreads) {
    float4v acc[4];
    int rowv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = float4v{0.f, 0.f, 0.f, 0.f};
      const int it = min(i0 + u * kAThreads, nout - 1);
      const int rr = it >> 5;  // gg * nq + qq
      rowv[u] = (rr / nq) * kAQ + rr % nq;
    }
    for (int c = 0; c < nparts; ++c) {
      float4v x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int it = min(i0 + u * kAThreads, nout - 1);
        x[u] = *gbl((const float4v*)&pbase[c * pstride + (int64_t)rowv[u] * kD + 4 * (it & 31)]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += wsm[c * kRows + rowv[u]] * x[u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int it = i0 + u * kAThreads;
      if (it >= nout) continue;
      const int gg = rowv[u] / kAQ, qq = rowv[u] % kAQ;
      const int64_t ob = (int64_t)(q0 + qa + qq) * a.out_row_stride + (int64_t)(h * G + gg) * kD +
                         4 * (it & 31);
      store_act4(a.out, a.out_dtype, ob, acc[u], ovec);
    }
  }
  if (tid == 0)
    __hip_atomic_store(&a.ws_cnt[item], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------ scores
// The score tensor of one request (krt_multi_from_slots) from the expanded tiles:
//   s[p, j, t] = scale * q[j, p] . k_t,   -inf where t > p0 + j
// for a 512-thread workgroup per (KV head, 128 queries, key range); wave w owns queries
// 16w..16w+15 for all G heads. Per 64-key tile: the tile's K halves by DMA (double-buffered, one
// barrier per tile), S^T = K Q^T on MFMA (hi and lo key halves against the fp16 query), then 16-byte
// stores of 4 keys per lane. Nothing is reduced, so key ranges need no combine.
struct ScoresArgs {
  Geom g;
  int G;
  float scale;
  const void* q;
  int q_dtype;
  int64_t q_row_stride;
  const int32_t* bt;
  const int32_t* seq_lens;
  const int32_t* qsl;
  const int32_t* dec_map;
  int64_t num_blocks, n_dec_slots;
  const uint8_t* tiles;
  int ntl;
  float* s_out;
  int64_t s_head_stride, s_q_stride;
  int* err;
  int n_qb, kchunk, nsplit, max_seq, max_q;
};

struct ScoresTile {
  u32x4 khi[kXTile][16];
  u32x4 klo[kXTile][16];
};
struct ScoresSmem {
  ScoresTile t[2];
};

template <int G>
__global__ __launch_bounds__(kAThreads, 2) void scores_kernel(ScoresArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  ScoresSmem& S = *reinterpret_cast<ScoresSmem*>(smem_raw);
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // items (head, key range, query block), the query blocks of one key range consecutive on one
  // XCD so they read the same tiles through its L2
  const int nwork = g.H * a.nsplit * a.n_qb;
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= nwork) return;
  const int qb = w % a.n_qb;
  const int sp = (w / a.n_qb) % a.nsplit;
  const int h = w / a.n_qb / a.nsplit;
  const int q0 = a.qsl[0];
  int qlen = a.qsl[1] - q0;
  int seq = a.seq_lens[0];
  const bool lead = tid == 0 && sp == 0 && qb == 0 && h == 0;
  if (seq > a.max_seq || qlen > a.max_q) {
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    seq = min(seq, a.max_seq);
    qlen = min(qlen, a.max_q);
  }
  const int p0 = seq - qlen;
  const int qa = qb * kAQ;
  if (qlen <= 0 || qa >= qlen) return;
  if (p0 < 0) {
    if (lead) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
    return;
  }
  const int qe = min(qlen, qa + kAQ);
  const int k0 = sp * a.kchunk;
  const int k1 = min(seq, k0 + a.kchunk);
  if (k0 >= k1) return;

  const int blk0 = a.bt[0];
  int dslot = -1;
  if (blk0 >= 0 && blk0 < a.num_blocks) dslot = a.dec_map[blk0];
  if (dslot < 0 || dslot >= a.n_dec_slots) {  // expand skipped the request: NaN scores
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    for (int i = tid; i < G * (qe - qa) * (k1 - k0); i += kAThreads) {
      const int kk = i % (k1 - k0);
      const int rest = i / (k1 - k0);
      const int qj = qa + rest % (qe - qa);
      const int gg = rest / (qe - qa);
      a.s_out[(int64_t)(h * G + gg) * a.s_head_stride + (int64_t)qj * a.s_q_stride + k0 + kk] = NAN;
    }
    return;
  }

  const uint8_t* tbase = a.tiles + (int64_t)h * a.ntl * kTileBytes;
  // K-half DMA: wave w moves image chunks 64 (w + 8 i), i < 4 (see attend_kernel's dma_tile)
  int dsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int P = 64 * (wv + 8 * i) + lane;
    const int row = (P >> 4) & 63, pc = P & 15;
    dsrc[i] = (P & ~1023) + row * 16 + (pc ^ (row & 7));
  }
  auto dma_k = [&](ScoresTile& T, int tile) {
    const u32x4* src = (const u32x4*)(tbase + (int64_t)tile * kTileBytes);
    typedef __attribute__((address_space(3))) void* lds_ptr;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(gbl(src + dsrc[i]), (lds_ptr)((u32x4*)&T + 64 * (wv + 8 * i)),
                                       16, 0, 0);
  };

  const int qj = qa + 16 * wv + n;
  const bool qvalid = qj < qe;
  half8 qf[G][4];
  {
    const bool qvec = act_rows_aligned(a.q, a.q_dtype, a.q_row_stride);
    // k-step ks, lane group gq: the dims of key chunk 4 ks + gq (tile_dims)
    const int64_t qrow = (int64_t)(q0 + (qvalid ? qj : qa)) * a.q_row_stride + (int64_t)h * G * kD +
                         4 * gq;
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float tq[8];
        load_act_n<4>(a.q, a.q_dtype, qrow + (int64_t)gg * kD + 16 * ks, qvec, tq);
        load_act_n<4>(a.q, a.q_dtype, qrow + (int64_t)gg * kD + 64 + 16 * ks, qvec, tq + 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][ks][i] = qvalid ? (_Float16)tq[i] : (_Float16)0.0f;
      }
  }
  uint32_t koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = n * 256 + (((4 * ks + gq) ^ (n & 7)) << 4);
  // score rows 16-byte aligned: a lane's 4 consecutive keys are one store
  const bool s_vec = ((uintptr_t)a.s_out % 16 == 0) && a.s_q_stride % 4 == 0 &&
                     a.s_head_stride % 4 == 0;
  const int lim = p0 + qj;  // last key this lane's query may see

  const int tl0 = k0 / kXTile, ntl_item = (k1 + kXTile - 1) / kXTile - tl0;
  dma_k(S.t[0], tl0);
  for (int k = 0; k < ntl_item; ++k) {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA has landed
    __syncthreads();  // every wave's has; every wave is done with the other buffer
    if (k + 1 < ntl_item) dma_k(S.t[(k + 1) & 1], tl0 + k + 1);
    const char* tb = (const char*)&S.t[k & 1];
    const int tt = (tl0 + k) * kXTile;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float4v sacc[G];
      const char* rb = tb + 16 * kt * 256;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8 ka = *(const half8*)(rb + koff[ks]);
        const half8 kl = *(const half8*)(rb + 16384 + koff[ks]);
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
          sacc[gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              ka, qf[gg][ks], ks ? sacc[gg] : float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          sacc[gg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qf[gg][ks], sacc[gg], 0, 0, 0);
        }
      }
      // lane holds keys key0 .. key0 + 3 of query qj, head h*G + gg
      const int key0 = tt + 16 * kt + 4 * gq;
      if (qvalid) {
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
          float* srow = a.s_out + (int64_t)(h * G + gg) * a.s_head_stride + (int64_t)qj * a.s_q_stride;
          float4v v;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            v[jj] = key0 + jj <= lim ? sacc[gg][jj] * a.scale : -INFINITY;
          if (s_vec && key0 + 3 < k1) {
            *gblw((float4v*)&srow[key0]) = v;
          } else {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              if (key0 + jj < k1) srow[key0 + jj] = v[jj];
          }
        }
      }
    }
  }
}

}  // namespace ttkv

// ------------------------------------------------------------------------------------ host side
#include "ttkv_host.h"

namespace ttkv {

namespace {

// Where the two-launch path applies: chunks of more than one 64-query block, G <= 3 (the attend
// kernel's fragments for 16 queries x G heads fit 256 registers per lane), r1 <= 128.
bool continuation_eligible(const Geom& g, int G, int max_q_len) {
  // every chunk of two or more queries: at 4 x 7,656 keys two launches beat the fused kernel
  // from Q = 2 (137 against 147 us) to Q = 64 (169 against 327 us)
  return max_q_len > 1 && G >= 1 && G <= 3 && g.r1 <= 128;
}

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Rows per launch: one arrival counter per (row, head, query block), and at most 1 GiB of
// expanded tiles.
int cont_slice_reqs(const Geom& g, int num_reqs, int max_q_len, int max_seq_len) {
  const int n_qb = ceil_div(max_q_len, kAQ);
  const int64_t per_row = (int64_t)g.H * ceil_div(max_seq_len, kXTile) * kTileBytes;
  const int by_tiles = (int)std::max<int64_t>(1, ((int64_t)1 << 30) / std::max<int64_t>(per_row, 1));
  return std::max(1, std::min({num_reqs, kMaxCounters / (g.H * n_qb), by_tiles}));
}

// Keys per attend split: the items fill about one round of the chip (one 8-wave workgroup per
// CU), each split a whole number of tiles, at least 4.
int cont_kchunk(int items, int max_seq_len) {
  const int64_t target = device_cu_count();
  const int64_t want = std::min<int64_t>(
      kMaxParts, std::max<int64_t>(1, (target + items - 1) / std::max(items, 1)));
  int64_t kc = (std::max(max_seq_len, 1) + want - 1) / want;
  kc = (kc + kXTile - 1) / kXTile * kXTile;
  return (int)std::max<int64_t>(kc, 4 * kXTile);
}

struct ContShape {
  int ntl, n_qb, kchunk, nsplit;
  int64_t part_bytes, tile_bytes;
};

ContShape cont_shape(const Geom& g, int G, int nr, int max_q_len, int max_seq_len) {
  ContShape s{};
  s.ntl = ceil_div(max_seq_len, kXTile);
  s.n_qb = ceil_div(max_q_len, kAQ);
  const int items = nr * g.H * s.n_qb;
  s.kchunk = cont_kchunk(items, max_seq_len);
  s.nsplit = std::max(1, ceil_div(max_seq_len, s.kchunk));
  s.part_bytes = s.nsplit > 1 ? (int64_t)items * s.nsplit * G * kAQ * (kD + 2) * 4 : 0;
  s.tile_bytes = (int64_t)nr * g.H * s.ntl * kTileBytes;
  return s;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

template <int RB, int VB, int KSTEPS, int CM = kCoefI8>
int launch_expand_t(const ExpandArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(ExpandSmem<KSTEPS>);
  auto kfn = expand_kernel<RB, VB, KSTEPS, CM>;
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kXThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string("expand launch: ") + hipGetErrorString(e));
  return TTKV_OK;
}

int launch_expand(const ExpandArgs& a, int ksteps, int grid, hipStream_t st) {
  const bool b3 = a.g.res_bits == 3;
  // the fp16 and 4-bit coefficient modes are built for 64 < r1 <= 128
  if (a.g.coef_mode != kCoefI8 && ksteps != 4)
    return host_fail(TTKV_E_UNSUPPORTED, "fp16 and 4-bit coefficients are built for 64 < r1 <= 128");
  if (a.g.coef_mode == kCoefF16)
    return b3 ? launch_expand_t<3, 3, 4, kCoefF16>(a, grid, st)
              : launch_expand_t<4, 4, 4, kCoefF16>(a, grid, st);
  if (a.g.coef_mode == kCoefI4G32)
    return b3 ? launch_expand_t<3, 3, 4, kCoefI4G32>(a, grid, st)
              : launch_expand_t<4, 4, 4, kCoefI4G32>(a, grid, st);
  switch (ksteps) {
    case 2: return b3 ? launch_expand_t<3, 3, 2>(a, grid, st) : launch_expand_t<4, 4, 2>(a, grid, st);
    case 4: return b3 ? launch_expand_t<3, 3, 4>(a, grid, st) : launch_expand_t<4, 4, 4>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "r1 > 128 is not built for the expand launch");
}

template <int G>
int launch_attend_t(const AttendArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(AttendSmem);
  auto kfn = attend_kernel<G>;
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kAThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string("attend launch: ") + hipGetErrorString(e));
  return TTKV_OK;
}

template <int G>
int launch_scores_t(const ScoresArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(ScoresSmem);
  auto kfn = scores_kernel<G>;
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kAThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string("scores launch: ") + hipGetErrorString(e));
  return TTKV_OK;
}

// shared by the attention and score paths: the expand launch over rows ri0 .. ri0 + nr - 1
int expand_rows(const Geom& g, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                int block_size, const int32_t* bt, int64_t bt_row_stride, const int32_t* seq_lens,
                const int32_t* req_index, int ri0, int nr, int ntl, int max_seq_len,
                const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                const float* dec_scale, int64_t n_dec_slots, const float* cs_cache, uint8_t* tiles,
                int32_t* err, hipStream_t st) {
  ExpandArgs e{};
  e.g = g;
  e.page = page;
  e.n_slots = n_slots;
  e.slot_stride = slot_stride;
  e.block_size = block_size;
  e.bt = bt;
  e.bt_row_stride = bt_row_stride;
  e.seq_lens = seq_lens;
  e.req_index = req_index;
  e.ri0 = ri0;
  e.num_reqs = nr;
  e.dec_map = dec_map;
  e.num_blocks = num_blocks;
  e.dec_q = dec_q;
  e.dec_scale = dec_scale;
  e.n_dec_slots = n_dec_slots;
  e.cs_cache = cs_cache;
  e.tiles = tiles;
  e.ntl = ntl;
  e.max_seq = max_seq_len;
  e.err = err;
  // tiles per item: about one round of two workgroups per CU, and the item's block ids fit the
  // LDS stage
  const int64_t total = (int64_t)nr * g.H * ntl;
  int tpi = ceil_div(total, 2 * (int64_t)device_cu_count());
  tpi = std::min(tpi, std::max(1, (kXSeg - 2) * block_size / kXTile));
  tpi = std::max(1, std::min(tpi, ntl));
  e.tpi = tpi;
  e.nchunk = ceil_div(ntl, tpi);
  const int ework = nr * e.nchunk * g.H;
  return launch_expand(e, g.r1 <= 64 ? 2 : 4, (ework + 7) / 8 * 8, st);
}
}  // namespace

int64_t continuation_scores_workspace_bytes(const Geom& g, int G, int max_q_len,
                                            int max_seq_len) {
  if (!continuation_eligible(g, G, max_q_len)) return 0;
  return (int64_t)g.H * ceil_div(max_seq_len, kXTile) * kTileBytes;
}

// The score tensor of one request through the expand launch and the scores kernel (caller:
// prefill_paged in scores mode, which has checked the arguments and the workspace size).
int continuation_scores(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                        int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                        int64_t slot_stride, int block_size, const int32_t* bt,
                        int64_t bt_row_stride, const int32_t* seq_lens, const int32_t* qsl,
                        int max_q_len, int max_seq_len, const int32_t* dec_map, int64_t num_blocks,
                        const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                        const float* cs_cache, float* s_out, int64_t s_head_stride,
                        int64_t s_q_stride, void* ws, int32_t* err, hipStream_t st) {
  const int G = HQ / g.H;
  const int ntl = ceil_div(max_seq_len, kXTile);
  uint8_t* tiles = (uint8_t*)ws;
  if (int rc = expand_rows(g, page, n_slots, slot_stride, block_size, bt, bt_row_stride, seq_lens,
                           nullptr, 0, 1, ntl, max_seq_len, dec_map, num_blocks, dec_q, dec_scale,
                           n_dec_slots, cs_cache, tiles, err, st))
    return rc;
  ScoresArgs b{};
  b.g = g;
  b.G = G;
  b.scale = scale;
  b.q = q;
  b.q_dtype = q_dtype;
  b.q_row_stride = q_row_stride;
  b.bt = bt;
  b.seq_lens = seq_lens;
  b.qsl = qsl;
  b.dec_map = dec_map;
  b.num_blocks = num_blocks;
  b.n_dec_slots = n_dec_slots;
  b.tiles = tiles;
  b.ntl = ntl;
  b.s_out = s_out;
  b.s_head_stride = s_head_stride;
  b.s_q_stride = s_q_stride;
  b.err = err;
  b.n_qb = ceil_div(max_q_len, kAQ);
  b.max_seq = max_seq_len;
  b.max_q = max_q_len;
  // key ranges: about one round of two workgroups per CU, each at least 4 tiles
  const int items = g.H * b.n_qb;
  const int64_t want = std::max<int64_t>(1, (2 * (int64_t)device_cu_count() + items - 1) / items);
  int64_t kc = (std::max(max_seq_len, 1) + want - 1) / want;
  kc = std::max<int64_t>((kc + kXTile - 1) / kXTile * kXTile, 4 * kXTile);
  b.kchunk = (int)kc;
  b.nsplit = std::max(1, ceil_div(max_seq_len, kc));
  const int work = g.H * b.nsplit * b.n_qb;
  const int grid = (work + 7) / 8 * 8;
  switch (G) {
    case 1: return launch_scores_t<1>(b, grid, st);
    case 2: return launch_scores_t<2>(b, grid, st);
    case 3: return launch_scores_t<3>(b, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "scores: G > 3");
}

bool continuation_applies(const Geom& g, int G, int max_q_len) {
  return continuation_eligible(g, G, max_q_len);
}

int64_t continuation_workspace_bytes(const Geom& g, int G, int num_reqs, int max_q_len,
                                     int max_seq_len) {
  if (num_reqs <= 0 || max_q_len <= 0) return 0;
  const int slice = cont_slice_reqs(g, num_reqs, max_q_len, max_seq_len);
  int64_t need = 0;
  for (int nr : {slice, (num_reqs - 1) % slice + 1}) {
    const ContShape s = cont_shape(g, G, nr, max_q_len, max_seq_len);
    need = std::max(need, kCounterBytes + align256(s.part_bytes) + s.tile_bytes);
  }
  return need;
}

// The two-launch continuation read (caller: prefill_paged, which has checked the arguments and
// the workspace size).
int continuation_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                       int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                       int64_t slot_stride, int block_size, const int32_t* bt,
                       int64_t bt_row_stride, const int32_t* seq_lens, const int32_t* qsl,
                       const int32_t* req_index, int num_reqs, int max_q_len, int max_seq_len,
                       const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                       const float* dec_scale, int64_t n_dec_slots, const float* cs_cache,
                       void* out, int out_dtype, int64_t out_row_stride, void* ws, int32_t* err,
                       hipStream_t st) {
  const int G = HQ / g.H;
  const int slice = cont_slice_reqs(g, num_reqs, max_q_len, max_seq_len);
  for (int ri0 = 0; ri0 < num_reqs; ri0 += slice) {
    const int nr = std::min(slice, num_reqs - ri0);
    const ContShape s = cont_shape(g, G, nr, max_q_len, max_seq_len);
    uint8_t* tiles = (uint8_t*)ws + kCounterBytes + align256(s.part_bytes);

    if (int rc = expand_rows(g, page, n_slots, slot_stride, block_size, bt, bt_row_stride,
                             seq_lens, req_index, ri0, nr, s.ntl, max_seq_len, dec_map,
                             num_blocks, dec_q, dec_scale, n_dec_slots, cs_cache, tiles, err, st))
      return rc;

    AttendArgs b{};
    b.g = g;
    b.HQ = HQ;
    b.G = G;
    b.scale_log2 = scale * 1.4426950408889634f;
    b.q = q;
    b.q_dtype = q_dtype;
    b.q_row_stride = q_row_stride;
    b.bt = bt;
    b.bt_row_stride = bt_row_stride;
    b.seq_lens = seq_lens;
    b.qsl = qsl;
    b.req_index = req_index;
    b.ri0 = ri0;
    b.num_reqs = nr;
    b.dec_map = dec_map;
    b.num_blocks = num_blocks;
    b.n_dec_slots = n_dec_slots;
    b.tiles = tiles;
    b.ntl = s.ntl;
    b.out = out;
    b.out_dtype = out_dtype;
    b.out_row_stride = out_row_stride;
    b.ws_cnt = (int*)ws;
    b.ws_part = (float*)((char*)ws + kCounterBytes);
    b.err = err;
    b.n_qb = s.n_qb;
    b.kchunk = s.kchunk;
    b.nsplit = s.nsplit;
    b.max_seq = max_seq_len;
    b.max_q = max_q_len;
    const int awork = nr * g.H * s.nsplit * s.n_qb;
    const int grid = (awork + 7) / 8 * 8;
    int rc = TTKV_OK;
    switch (G) {
      case 1: rc = launch_attend_t<1>(b, grid, st); break;
      case 2: rc = launch_attend_t<2>(b, grid, st); break;
      case 3: rc = launch_attend_t<3>(b, grid, st); break;
      default: rc = host_fail(TTKV_E_UNSUPPORTED, "attend: G > 3");
    }
    if (rc != TTKV_OK) return rc;
  }
  return TTKV_OK;
}

}  // namespace ttkv

// K1: fused paged decode read over compressed (pre-RoPE, tensor-train) KV slots, one launch per
// layer for the whole decode batch. gfx950 / CDNA4.
//
// Work item = (request r, KV head h, token chunk c). The chunk length comes from the batch's own
// lengths, computed on the device by every workgroup (the work plan below), so a ragged batch
// spreads its total tokens over one round of resident workgroups. A 256-thread workgroup (4
// waves) walks its chunk in 64-token tiles with the next tile's raw bytes prefetched into
// registers while the current one is computed:
//   commit  : prefetched bytes -> LDS: coefficients as fp16 MFMA B-fragments (int8 is exact in
//             fp16; the fp16 mode's values are copied; the 4-bit mode's q * group scale is exact
//             in fp16, commit_coef); this head's K and V rows realigned, the code streams
//             byte-reversed per dword (one v_perm each) so that a code window is one v_alignbit.
//   decode  : one thread per half row. Per bitmap byte, the next 8 codes are spread one per byte
//             through a 64-entry two-code table (3-bit) or nibble perms (4-bit) and scattered onto their
//             lanes with one v_perm driven by a 256-entry selector table (both tables built in
//             LDS by the workgroup at start). 3-bit codes come out as
//             fp8 bytes of the signed value c - 4 (0 outside the bitmap), which the arithmetic
//             reads two at a time with v_cvt_pk_f32_fp8.
//   recon   : K_pre^T[128 x 16 tokens] = Dec^T[128 x r1] * coeff^T[r1 x 16] on MFMA 16x16x32 f16
//             (only that shape). The decoder is split hi + lo in fp16 and both halves are applied; decoder_f values
//             are int8 * fp16 row rulers (<= 19 significant bits), so hi + lo is exact and the
//             products are exact in the fp32 accumulator. Wave w owns dims {16w..16w+15} and
//             {64+16w..64+16w+15}, so each RoPE pair (j, j+64) sits in one lane and the decoder
//             fragments stay in registers for the whole chunk.
//   rope    : k / cs = acc + (ruler / cs) * (code - 2^(b-1)), rotated by the row's absolute
//             position. The coefficient ruler cs is a per-token factor of the key, so it is
//             applied to the score instead (with scale * log2 e).
//   q.k     : on MFMA: S[p, token] = Q[p, dims] * Y[dims, token] over the wave's 32 dims, with the
//             rotated keys split hi + lo in fp16 (22 significant bits) and the query split the
//             same way; partial scores of the 4 waves are summed through LDS.
//   softmax : online, base 2, evaluated redundantly by every wave (lane = token, no barrier). The
//             reference point moves only when some score exceeds it by more than 2^8 (a ballot),
//             so the wave-wide max is rarely computed; sums stay per lane until the end.
//   P.V     : on MFMA, O^T[dims, heads] += V^T[dims, tokens] * P'^T[tokens, heads] with
//             P' = P * ruler_v * 2^-ve rounded to fp16 once (ve >= 0 grows with the largest V
//             ruler seen, so P' stays below 2^15) and the codes as exact fp16 integers
//             (c - 2^(b-1)). The V^T operand is read straight from the decoded code rows with
//             the gfx950 LDS transpose read (ds_read_tr8_b64); P'^T from a per-wave LDS row.
// Chunks of one (r, h) are combined in the same launch by the last workgroup to finish
// (write-through partials + a relaxed arrival counter, agent-scope loads), which also resets the
// counter to zero. The counters sit at the
// workspace's fixed 64 KiB head, the partials after it, indexed by (chunk item) so their count
// follows the plan.
//
// Reference semantics: vllm_ttkv/reference.py:63-163 (dense K, per-row RoPE, scores, softmax,
// V readout), vllm_ttkv/impl.py:511-540 (scale then softmax), decode.py:54-122 (vLLM cos/sin
// half layout), decode.py:307-339 (slot = block_table[r, t/bs]*bs + t%bs); bit format
// codec/ttkv_packed_cache.py:50-100, 138-167, 247-271.
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kTile = 64;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRawDw = 17;      // dwords per staged head row (49-50 B rows + window slack); odd so
                                // threads reading the same offset of different rows hit distinct banks
constexpr int kCodeStride = 144;  // bytes per code row (128 + bank stagger)
constexpr int kSegMax = 260;    // block ids staged per chunk
constexpr int kPlanLanes = 4;   // requests per lane in the work plan
constexpr int kPlanReqs = 64 * kPlanLanes;  // requests per launch (larger batches: several)

struct DecodeArgs {
  Geom g;
  int HQ, G;
  float scale_log2;
  const void* q;
  int q_dtype;
  int64_t q_row_stride;
  const uint8_t* page;
  int64_t n_slots, slot_stride;
  int block_size, bs_shift;
  const int32_t* bt;
  int64_t bt_row_stride;
  int max_blocks;
  const int32_t* seq_lens;
  const int32_t* qsl;
  int num_reqs;
  const int32_t* dec_map;
  int64_t num_blocks;
  const int8_t* dec_q;  // decoder pool (see dec_ranks)
  const float* dec_scale;
  int64_t n_dec_slots;
  const float* cs_cache;
  int64_t max_pos;
  void* out;
  int out_dtype;
  int64_t out_row_stride;
  float* ws_part;
  int* ws_cnt;
  int* err;
  int chunk_cap, target, max_seq;  // chunk length cap, work items aimed at, longest context
};

// KU = coefficient window in 16-wide k units: r1 is padded to 16 * KU; the reconstruction runs
// KU / 2 MFMA steps of k = 32 and, for odd KU, one of k = 16.
template <int KU, int G>
struct DecodeSmem {
  static constexpr int kCoefStride = KU * 16 + 8;  // fp16 per token row
  static constexpr int kSP = G <= 4 ? 4 : 8;           // score slots per token
  _Float16 coef[kTile][kCoefStride];
  uint32_t rawk[kTile][kRawDw];
  uint32_t rawgap[16];  // V rows 16 dwords off: a wave's K and V rows of one token on other banks
  uint32_t rawv[kTile][kRawDw];
  uint8_t kcode[kTile][kCodeStride];
  uint8_t vcode[2][kTile][kCodeStride];  // by tile parity: the next tile's decode runs beside P.V
  float spart[kWaves][kTile][kSP];  // per wave partial q.k [wave][token][head]
  _Float16 pw[kWaves][G][kTile];    // per wave P' = P * ruler_v (fp16), the P.V B operand
  uint2 lut[256];
  int32_t seg[kSegMax];
  float cs[kTile];  // coefficient ruler
  float kr[kTile];  // K residual ruler / (cs * unit)
  float vr[2][kTile];  // V ruler, by tile parity
  float f[2][kTile];   // cs * scale * log2(e), by tile parity
  float m[G], l[G];
  int is_last;
};

// One-round split-K combine for up to NC chunks: each thread requests every chunk's (max, sum,
// output) value for its outputs (it = tid + u * kThreads) in one round, then combines them in
// registers. Chunks past n_chunks re-read the last one and are not used. The partials were
// written through to the device-coherent level and are read with agent-scope loads.
template <int G, int NC>
__device__ __forceinline__ void combine_regs(const float* pbase, int64_t cstride, int n_chunks,
                                             int tid, void* out, int out_dtype, int64_t orow,
                                             int h) {
  constexpr int kOut = (G * kD + kThreads - 1) / kThreads;  // outputs per thread
  float mv[kOut][NC], lv[kOut][NC], ov[kOut][NC];
#pragma unroll
  for (int u = 0; u < kOut; ++u) {
    const int it = min(tid + u * kThreads, G * kD - 1);
    const int p = it / kD;
    const int dim = it - p * kD;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const float* pc = pbase + min(cc, n_chunks - 1) * cstride + p * (kD + 2);
      mv[u][cc] = ld_agent(&pc[kD]);
      lv[u][cc] = ld_agent(&pc[kD + 1]);
      ov[u][cc] = ld_agent(&pc[dim]);
    }
  }
#pragma unroll
  for (int u = 0; u < kOut; ++u) {
    const int it = tid + u * kThreads;
    if (it < G * kD) {
      const int p = it / kD;
      const int dim = it - p * kD;
      float M = -INFINITY;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) M = cc < n_chunks ? fmaxf(M, mv[u][cc]) : M;
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const float f = cc < n_chunks ? exp2f(mv[u][cc] - M) : 0.f;
        L = fmaf(lv[u][cc], f, L);
        O = fmaf(ov[u][cc], f, O);
      }
      store_act(out, out_dtype, orow + (int64_t)(h * G + p) * kD + dim, O / L);
    }
  }
}

// QLO: the query's low fp16 part can be non-zero (fp32 / bf16 queries), so the scores take the
// third product qlo * yhi; an fp16 query is its own hi part and skips it.
template <int G, int RB, int VB, int KU, bool QLO, int CM>
__global__ __launch_bounds__(kThreads, 2) void decode_paged_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  __shared__ uint16_t lut3s[kLut3Entries];  // static: its address folds into the loads
  using Smem = DecodeSmem<KU, G>;
  Smem& S = *reinterpret_cast<Smem*>(smem_raw);
  static_assert(RB == VB, "K and V rows decode with one code path (3/3 and 4/4 are built)");
  constexpr int KSTEPS = KU / 2;  // k = 32 steps
  constexpr bool KTAIL = KU & 1;  // one more k = 16 step
  constexpr int kSP = Smem::kSP;
  const Geom& g = a.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // ---- work plan, from the batch's own lengths (no host round trip). Every wave computes it
  // alike: the lengths of requests lane + 64 i; the shortest chunk (a multiple of the tile) whose
  // (request, chunk, head) items fit `rounds` full rounds of resident blocks, each request
  // having at least one chunk; and then this block's item. Items are enumerated chunk-major --
  // (chunk c, request r, head h) over the requests that have a chunk c -- so the H heads of one
  // (request, chunk) read the same coefficient bytes and every request's chunk c the same rows
  // of the angle table (positions are absolute). Blocks are dealt round-robin to the 8 XCDs, so
  // each XCD takes a contiguous range of items and both are fetched from HBM about once per XCD.
  // Each request's query row and first block id are loaded with its length (one round trip), then
  // its decoder slot.
  const int nper = (a.num_reqs + 63) >> 6;  // groups of 64 requests in use (uniform)
  int seql[kPlanLanes], nchl[kPlanLanes], qsll[kPlanLanes], blk0l[kPlanLanes], decl[kPlanLanes];
  int tot = 0, over = 0;
#pragma unroll
  for (int i = 0; i < kPlanLanes; ++i) {
    const int rr = lane + 64 * i;
    seql[i] = 0;
    qsll[i] = 0;
    blk0l[i] = -1;
    if (i < nper && rr < a.num_reqs) {
      const int sr = a.seq_lens[rr];
      qsll[i] = a.qsl[rr];
      blk0l[i] = a.max_blocks > 0 ? a.bt[(int64_t)rr * a.bt_row_stride] : -1;
      over |= sr > a.max_seq;
      seql[i] = min(max(sr, 0), a.max_seq);  // the host sized the launch from max_seq
      tot += seql[i];                         // host: num_reqs * max_seq < 2^31
    }
  }
  // each request's decoder slot, requested now: its round trip overlaps the chunk search below
#pragma unroll
  for (int i = 0; i < kPlanLanes; ++i)
    decl[i] = blk0l[i] >= 0 && blk0l[i] < a.num_blocks ? a.dec_map[blk0l[i]] : -1;
  tot = wave_sum_i(tot);
  const bool any_over = __builtin_amdgcn_ballot_w64(over) != 0;
  if (blockIdx.x == 0 && tid == 0 && any_over) atomicOr(a.err, TTKV_ERR_SEQ_LEN);
  int chunk;
  {
    int tl[kPlanLanes];  // tiles per request
#pragma unroll
    for (int i = 0; i < kPlanLanes; ++i) tl[i] = (seql[i] + kTile - 1) / kTile;
    // items at chunk = m tiles: ceil(ceil(n / 64) / m) = ceil(n / (64 m)) chunks per request
    auto items_at = [&](int m) {
      int sum = 0;
#pragma unroll
      for (int i = 0; i < kPlanLanes; ++i)
        if (i < nper && lane + 64 * i < a.num_reqs) sum += max(1, (tl[i] + m - 1) / m);
      return wave_sum_i(sum) * g.H;
    };
    const int rounds = max(1, (a.num_reqs * g.H + a.target - 1) / a.target);
    const int64_t budget = (int64_t)rounds * a.target;
    const int m_cap = a.chunk_cap / kTile;
    // no chunk below tot * H / budget tiles can fit (items fall as the chunk grows): start there,
    // gallop up to a chunk that fits, then bisect; the cap is taken when nothing fits
    int m = (int)min<int64_t>(m_cap, max<int64_t>(1, ((int64_t)tot * g.H + budget * kTile - 1) /
                                                         (budget * kTile)));
    if (items_at(m) > budget) {
      int bad = m, good = -1, step = 1;
      while (good < 0 && bad < m_cap) {
        const int t = min(m_cap, bad + step);
        if (items_at(t) <= budget) good = t;
        else bad = t;
        step <<= 1;
      }
      if (good < 0) {
        m = m_cap;
      } else {
        while (good - bad > 1) {
          const int mid = (bad + good) >> 1;
          if (items_at(mid) <= budget) good = mid;
          else bad = mid;
        }
        m = good;
      }
    }
    chunk = m * kTile;
  }
  int nreq_items = 0, maxc = 0;
#pragma unroll
  for (int i = 0; i < kPlanLanes; ++i) {
    nchl[i] = 0;
    if (i < nper && lane + 64 * i < a.num_reqs) nchl[i] = max(1, (seql[i] + chunk - 1) / chunk);
    nreq_items += nchl[i];
    maxc = max(maxc, nchl[i]);
  }
  // items: <= rounds * target < target + num_reqs * H, or, when nothing fits, the host's count
  // with every request at max_seq and the capped chunk -- the grid is sized for the larger
  const int n_pairs = wave_sum_i(nreq_items);
  const int n_items = n_pairs * g.H;
  maxc = wave_max_i(maxc);
  const int per_xcd = (n_items + 7) >> 3;
  if ((int)(blockIdx.x >> 3) >= per_xcd) return;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= n_items) return;
  const int h = w % g.H;
  const int j = w / g.H;
  // (chunk c, request r) of pair j: c is the largest with P(c) <= j, P(c) = sum_r min(nch_r, c);
  // r is the (j - P(c))-th request with more than c chunks; base = chunks of the requests before
  // r (its partials follow theirs). When every request has the same count this is a division.
  int c = 0, r = 0, base = 0;
  if (n_pairs == maxc * a.num_reqs) {
    c = j / a.num_reqs;
    r = j - c * a.num_reqs;
    base = r * maxc;
  } else {
    int pc = 0, hi = maxc;
    while (hi - c > 1) {
      const int mid = (c + hi) >> 1;
      int pm = 0;
#pragma unroll
      for (int i = 0; i < kPlanLanes; ++i)
        if (i < nper) pm += min(nchl[i], mid);
      pm = wave_sum_i(pm);
      if (pm <= j) {
        c = mid;
        pc = pm;
      } else {
        hi = mid;
      }
    }
    int k = j - pc;
    bool found = false;
#pragma unroll
    for (int i = 0; i < kPlanLanes; ++i) {
      if (i < nper && !found) {
        const uint64_t msk = __builtin_amdgcn_ballot_w64(nchl[i] > c);
        const int cnt = __builtin_popcountll(msk);
        if (k < cnt) {
          const uint64_t below = lane ? msk & (~0ull >> (64 - lane)) : 0ull;
          const bool hit = ((msk >> lane) & 1ull) && __builtin_popcountll(below) == k;
          r = 64 * i + __builtin_ctzll(__builtin_amdgcn_ballot_w64(hit));
          found = true;
        } else {
          k -= cnt;
        }
      }
    }
    int bl = 0;
#pragma unroll
    for (int i = 0; i < kPlanLanes; ++i)
      if (i < nper) bl += lane + 64 * i < r ? nchl[i] : 0;
    base = wave_sum_i(bl);
  }
  int n_chunks = 0, seq = 0, qrow_r = 0, dslot = -1;
#pragma unroll
  for (int i = 0; i < kPlanLanes; ++i) {
    if ((r >> 6) == i) {
      n_chunks = __builtin_amdgcn_readlane(nchl[i], r & 63);
      seq = __builtin_amdgcn_readlane(seql[i], r & 63);
      qrow_r = __builtin_amdgcn_readlane(qsll[i], r & 63);
      dslot = __builtin_amdgcn_readlane(decl[i], r & 63);
    }
  }

  const int t0 = c * chunk;
  const int ptok = tid >> 2;  // token / part handled by this thread in prefetch + commit
  const int part = tid & 3;
  // block id of this thread's token in the first tile (position clamped into the context)
  const int64_t bt_row = (int64_t)r * a.bt_row_stride;
  const int pos0 = min(t0 + ptok, seq - 1);
  const int bi0 = a.bs_shift >= 0 ? pos0 >> a.bs_shift : pos0 / a.block_size;
  const int64_t qrow = qrow_r;
  const int blk_t0 = seq > 0 ? a.bt[bt_row + bi0] : -1;
  if (seq <= 0) {  // empty context: the reference's einsum over zero rows is 0
    for (int i = tid; i < G * kD; i += kThreads)
      store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G) * kD + i, 0.f);
    return;
  }
  const int t1 = min(seq, t0 + chunk);

  // This chunk's block ids (at most kSegMax, host-bounded), requested in the same round trip as
  // the first tile's block id and the decoder slot: they depend on the plan only, and are staged
  // into LDS after the code tables are built.
  const int bfirst = t0 / a.block_size;
  const int nseg = (t1 - 1) / a.block_size - bfirst + 1;
  constexpr int kSegPer = (kSegMax + kThreads - 1) / kThreads;
  int segv[kSegPer];
#pragma unroll
  for (int k = 0; k < kSegPer; ++k) {
    const int i = tid + kThreads * k;
    segv[k] = i < nseg ? a.bt[bt_row + bfirst + i] : -1;
  }

  // The first tile's bytes (bad block ids are flagged when the chunk's ids are staged); the
  // decoder slot (the device registry keyed by the request's first block) came with the plan
  const int k_row_off = g.k_field + h * g.k_row;
  const int v_row_off = g.k_slot + h * g.v_row;
  // the rows' 64-byte windows (16-aligned; each row lies inside its window, host-checked)
  const int k_win = k_row_off & ~15, v_win = v_row_off & ~15;
  RawSlotW<KU, CM> P;
  {
    const uint8_t* base = nullptr;
    if (ptok < min(kTile, t1 - t0) && blk_t0 >= 0 && blk_t0 < a.num_blocks) {
      const int64_t slot = (int64_t)blk_t0 * a.block_size + (pos0 - bi0 * a.block_size);
      if (slot < a.n_slots) base = a.page + slot * a.slot_stride;
    }
    fetch_raw_slot_w<KU, CM>(P, base, part, g, k_win, v_win);
  }
  if (dslot < 0 || dslot >= a.n_dec_slots) {
    if (tid == 0) atomicOr(a.err, TTKV_ERR_NO_DECODER);
    if (c == 0)
      for (int i = tid; i < G * kD; i += kThreads)
        store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G) * kD + i, NAN);
    return;
  }

  // ---- decoder and query values for the MFMA fragments: loaded now, so that their latency
  // overlaps the table and block-id staging
  const int dl = 16 * wv + 4 * gq;
  const int HD = g.H * kD;
  // int8 ranks 32s + 8gq .. +7 of each of the lane's two columns (one 8-byte load per step; the
  // k = 16 tail step: ranks 32 KSTEPS + 4gq .. +3, 4 bytes) and their rulers (one float4 per 4
  // ranks, the same for both columns). 16 KU <= R, so every load is inside the decoder.
  const int R = dec_ranks(g.r1);
  const int8_t* decq = a.dec_q + ((int64_t)dslot * HD + h * kD) * R;
  const float* decs = a.dec_scale + (int64_t)dslot * R;
  u32x2v dq[2][KSTEPS];
  uint32_t dqt[2] = {0u, 0u};
  float4v dsc[2 * KSTEPS + 1];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int8_t* col = decq + (int64_t)(16 * (wv + 4 * mi) + n) * R;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) dq[mi][s] = *gbl((const u32x2v*)(col + 32 * s + 8 * gq));
    if constexpr (KTAIL) dqt[mi] = *gbl((const uint32_t*)(col + 32 * KSTEPS + 4 * gq));
  }
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    dsc[2 * s] = *gbl((const float4v*)(decs + 32 * s + 8 * gq));
    dsc[2 * s + 1] = *gbl((const float4v*)(decs + 32 * s + 8 * gq + 4));
  }
  dsc[2 * KSTEPS] = KTAIL ? *gbl((const float4v*)(decs + 32 * KSTEPS + 4 * gq))
                          : float4v{0.f, 0.f, 0.f, 0.f};
  // (rows n >= G of the fragment are zero: they load head G - 1 and discard it, so the loads
  // carry no branch and go out together)
  float qraw[8];
  {
    const bool qvec = act_rows_aligned(a.q, a.q_dtype, a.q_row_stride);
    const int64_t qb = qrow * a.q_row_stride + (int64_t)(h * G + min(n, G - 1)) * kD;
    load_act_n<4>(a.q, a.q_dtype, qb + dl, qvec, qraw);
    load_act_n<4>(a.q, a.q_dtype, qb + 64 + dl, qvec, qraw + 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) qraw[j] = n < G ? qraw[j] : 0.f;
  }

  // ---- code tables, and this chunk's block ids
  build_luts(S.lut, (RB == 3 || VB == 3) ? lut3s : nullptr, tid, kThreads);
#pragma unroll
  for (int k = 0; k < kSegPer; ++k) {
    const int i = tid + kThreads * k;
    if (i < nseg) {
      int blk = segv[k];
      if (blk < 0 || blk >= a.num_blocks) {
        atomicOr(a.err, TTKV_ERR_BAD_BLOCK);
        blk = -1;
      }
      S.seg[i] = blk;
    }
  }

  // slot bases are 16-aligned, so a row's byte misalignment is fixed per head
  const uint32_t ksel = stage_selector(k_row_off & 3, part != 0);
  const uint32_t vsel = stage_selector(v_row_off & 3, part != 0);
  // fp8 code unit of the hardware conversion (2^-9 for OCP e4m3, 2^-10 for FNUZ); codes of 4
  // bits are converted as plain bytes
  const float inv_unit = 1.0f / __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
  const float inv_unit_k = RB == 3 ? inv_unit : 1.0f;

  __syncthreads();  // seg

  auto slot_base = [&](int tt) -> const uint8_t* {
    if (ptok >= min(kTile, t1 - tt)) return nullptr;
    const int pos = tt + ptok;
    const int bi = a.bs_shift >= 0 ? pos >> a.bs_shift : pos / a.block_size;
    const int blk = S.seg[bi - bfirst];
    if (blk < 0) return nullptr;
    const int64_t slot = (int64_t)blk * a.block_size + (pos - bi * a.block_size);
    if (slot >= a.n_slots) return nullptr;
    return a.page + slot * a.slot_stride;
  };

  // ---- decoder fragments (A operand, M = dims, K = r1), hi/lo fp16, resident in registers.
  half8 ahi[2][KSTEPS], alo[2][KSTEPS];
  half8 thi[2], tlo[2];  // k = 16 tail step (odd KU), upper halves zero
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
    float vt[4];
    dec_values4(dqt[mi], dsc[2 * KSTEPS], vt);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = KTAIL && j < 4 && 32 * KSTEPS + 4 * gq + j < g.r1 ? vt[j & 3] : 0.f;
      const _Float16 hi = (_Float16)f;
      thi[mi][j] = hi;
      tlo[mi][j] = (_Float16)(f - (float)hi);
    }
  }

  // ---- query fragments (A operand of q.k, M = heads, K = this wave's 32 dims in the order of
  // the rotated-key fragments: 8*gq + i <-> dim dl + i, 8*gq + 4 + i <-> dim 64 + dl + i),
  // split hi + lo in fp16; rows >= G are zero.
  half8 qhi, qlo;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const _Float16 hi = (_Float16)qraw[j];
    qhi[j] = hi;
    qlo[j] = (_Float16)(qraw[j] - (float)hi);
  }

  // P.V accumulators on MFMA: O^T[dims, heads] for the wave's two dim tiles; lane (n, gq) holds
  // dims 4gq..4gq+3 of the tile for query head n (n < G; the other columns stay zero)
  float4v oacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  float m_run[G], l_lane[G];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    m_run[p] = -INFINITY;
    l_lane[p] = 0.f;
  }
  // P' = P * ruler_v is carried at scale 2^-ve so that it stays an fp16 normal below 2^15: P <=
  // 2^8 (lazy rescale), so every ruler of a tile must stay below 2^(7 + ve). ve starts at 0 (no
  // scaling: rulers below 128, i.e. V rows up to |v| ~ 384 at 3 bits) and grows, behind a ballot,
  // when a tile brings a larger ruler; the accumulators are then rescaled by an exact power of
  // two, and the output takes 2^ve back at the end. Every wave sees the same rulers, so ve is
  // the same in all of them.
  int ve = 0;
  float v_thr = 128.f, v_mul = 1.f;
  // V^T A-fragments come from the decoded code rows through the LDS transpose read: in each
  // 16-lane group, lanes 2j and 2j+1 address the two 8-byte halves of row j (token 8gq + j) of
  // the tile's 16 dims, and lane n receives column n (dim n) of those 8 rows, i.e. exactly
  // A[dim n][tokens 8gq .. 8gq+7].
  const int tr_tok = 8 * gq + (n >> 1);
  const int tr_col = 8 * (n & 1);

  // RoPE angle rows (shared by every request and head, L2-resident): this lane's 4 dims of the
  // token it reconstructs in block nb, requested one block ahead inside the reconstruction. Block
  // 0's row of the NEXT tile is requested after the reconstruction, where the registers allow.
  constexpr bool kAngle0Ahead = G <= 4;
  float4v cv0, sv0;
  auto angle_row = [&](int ts, int nb, float4v& cv, float4v& sv) {
    const int tok = 16 * nb + n;
    const int64_t pos = tok < min(kTile, t1 - ts) ? ts + tok : ts;
    cv = *gbl((const float4v*)&a.cs_cache[pos * kD + dl]);
    sv = *gbl((const float4v*)&a.cs_cache[pos * kD + 64 + dl]);
  };
  if constexpr (kAngle0Ahead) angle_row(t0, 0, cv0, sv0);

  for (int tt = t0, tp = 0; tt < t1; tt += kTile, tp ^= 1) {
    const int ntile = min(kTile, t1 - tt);
    // the next tile's slot address first: its block-id read overlaps the commit
    const uint8_t* next_base = tt + kTile < t1 ? slot_base(tt + kTile) : nullptr;
    // ---------------------------------------------------------------- commit prefetched bytes
    {
      const float cs = commit_coef<KU, CM>(P, (uint32_t*)&S.coef[ptok][0], part, g);
      if (part == 0) S.cs[ptok] = cs;
      stage_row_w(P.krow, (k_row_off & 15) >> 2, ksel, &S.rawk[ptok][part * 4]);
      stage_row_w(P.vrow, (v_row_off & 15) >> 2, vsel, &S.rawv[ptok][part * 4]);
    }
    // No barrier: wave w commits and decodes the same 16 tokens (16w .. 16w+15), and LDS
    // accesses of one wave complete in order (the fences only keep the compiler from moving
    // them). The buffers this tile writes are free: the previous tile's reconstruction read
    // coef / kcode / kr before the last barrier, and its softmax and P.V read the other parity of
    // vcode / vr / f.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // The next tile's slot bytes, requested as soon as the commit has freed P: they arrive during
    // the decode and reconstruction instead of stalling the next commit (measured: the bytes took
    // ~2k cycles, longer than the softmax and P.V they used to overlap). The reconstruction's
    // angle loads queue behind them (loads complete in order) but are issued a decode later.
    if (tt + kTile < t1) fetch_raw_slot_w<KU, CM>(P, next_base, part, g, k_win, v_win);
    // ---------------------------------------------------------------- decode (thread = half row)
    // The decode and reconstruction are each workgroup's critical chain; the co-resident
    // workgroup's softmax, P.V and commit fill the issue slots they leave. Raising this wave's
    // priority for these two phases lets them run ahead (headline 172 -> 159 us, measured).
    __builtin_amdgcn_s_setprio(1);
    {
      // lanes 0..31: K rows, 32..63: V rows of this wave's 16 tokens, two threads per row; one
      // decode call with per-lane row and destination (the two kinds share the code width)
      const bool is_v = lane >= 32;
      const int tok = 16 * wv + ((lane >> 1) & 15);
      const int half = lane & 1;
      const uint32_t* row = is_v ? S.rawv[tok] : S.rawk[tok];
      uint8_t* dst = is_v ? &S.vcode[tp][tok][64 * half] : &S.kcode[tok][64 * half];
      decode_half_row_be<RB>(row, half, S.lut, lut3s, dst);
      if (half == 0) {
        const float rul = f16_bits_to_float(staged_u16(row, kBitmapBytes + (is_v ? g.v_pb : g.k_pb)));
        if (is_v) {
          S.vr[tp][tok] = rul;
        } else {
          const float cs = S.cs[tok];
          // the hardware reciprocal (1 ulp) instead of an IEEE divide, which would lengthen the
          // K lanes' branch
          S.kr[tok] = cs != 0.f ? rul * inv_unit_k * __builtin_amdgcn_rcpf(cs) : 0.f;
          S.f[tp][tok] = cs * a.scale_log2;
        }
      }
    }
    __syncthreads();
    // ---------------------------------------------------------------- recon + rope + q.k
    float4v cvn, svn;
    if constexpr (kAngle0Ahead) {
      cvn = cv0;
      svn = sv0;
    } else {
      angle_row(tt, 0, cvn, svn);
    }
    // Software-pipelined over the 4 token blocks: block nb + 1's MFMAs are issued before block nb's
    // epilogue (residual, RoPE, hi/lo split, scores), which has no dependence on them, so the two
    // overlap within the wave (reconstruction phase 3.65k -> 3.17k cycles per tile, measured).
    auto recon_mfma = [&](int nb, float krp, float4v& acc0, float4v& acc1) {
      const int tok = 16 * nb + n;
      // 4-bit codes arrive as c: the -8 * ruler offset enters as the accumulator's start
      const float kb = RB == 4 ? -8.f * krp : 0.f;
      acc0 = float4v{kb, kb, kb, kb};
      acc1 = float4v{kb, kb, kb, kb};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const half8 b = *(const half8*)&S.coef[tok][32 * s + 8 * gq];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[0][s], b, acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[0][s], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[1][s], b, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[1][s], b, acc1, 0, 0, 0);
      }
      if constexpr (KTAIL) {
        // The k = 16 tail runs as a 16x16x32 step whose upper k half is zero in A and B (lane
        // (n, gq) holds k 8gq..8gq+7 of a 32-wide step; the tail's k 4gq..4gq+3 sit in its first
        // four). One MFMA shape per accumulator chain: on gfx950 a 16x16x16 step reading a
        // 16x16x32 step's result as its accumulator gave wrong sums when the compiler placed the
        // two a few instructions apart (measured; extra wait states between them also fixed it).
        const half4 b4 = *(const half4*)&S.coef[tok][32 * KSTEPS + 4 * gq];
        const half8 b = {b4[0], b4[1], b4[2], b4[3], 0, 0, 0, 0};
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(thi[0], b, acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(tlo[0], b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(thi[1], b, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(tlo[1], b, acc1, 0, 0, 0);
      }
    };
    float krA = S.kr[n];
    float4v accA0, accA1;
    recon_mfma(0, krA, accA0, accA1);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int tok = 16 * nb + n;
      const float4v cv = cvn, sv = svn;
      if (nb < 3) angle_row(tt, nb + 1, cvn, svn);
      float4v accB0 = accA0, accB1 = accA1;
      float krB = krA;
      if (nb < 3) {
        krB = S.kr[tok + 16];
        recon_mfma(nb + 1, krB, accB0, accB1);
      }
      float vl[4], vh[4];
      codes4<RB>(*(const uint32_t*)&S.kcode[tok][dl], vl);
      codes4<RB>(*(const uint32_t*)&S.kcode[tok][64 + dl], vh);
      float y[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float kl = fmaf(krA, vl[i], accA0[i]);
        const float kh = fmaf(krA, vh[i], accA1[i]);
        y[i] = kl * cv[i] - kh * sv[i];
        y[4 + i] = kh * cv[i] + kl * sv[i];
      }
      half8 yhi, ylo;
      split8(y, yhi, ylo);
      float4v sacc = {0.f, 0.f, 0.f, 0.f};
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi, yhi, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi, ylo, sacc, 0, 0, 0);
      if constexpr (QLO) sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo, yhi, sacc, 0, 0, 0);
      // lane (n, gq) holds heads 4*gq .. 4*gq+3 of token n
      if (4 * gq < G) *(float4v*)&S.spart[wv][tok][4 * gq] = sacc;
      accA0 = accB0;
      accA1 = accB1;
      krA = krB;
    }
    __builtin_amdgcn_s_setprio(0);
    // ---------------------------------------------------------------- next tile's first angle row
    if constexpr (kAngle0Ahead)
      if (tt + kTile < t1) angle_row(tt + kTile, 0, cv0, sv0);
    __syncthreads();
    // ---------------------------------------------------------------- online softmax (every wave)
    {
      const bool valid = lane < ntile;
      const float ft = S.f[tp][lane];
      const float vrt = S.vr[tp][lane];
      float sum[kSP];
#pragma unroll
      for (int i = 0; i < kSP; ++i) sum[i] = 0.f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
#pragma unroll
        for (int i = 0; i < kSP; i += 4) {
          const float4v x = *(const float4v*)&S.spart[ww][lane][i];
          sum[i] += x[0];
          sum[i + 1] += x[1];
          sum[i + 2] += x[2];
          sum[i + 3] += x[3];
        }
      }
      float amul = 1.f;  // this lane's factor for its head column n of the P.V accumulators
      if (__builtin_amdgcn_ballot_w64(vrt >= v_thr) != 0) {  // rare: a large V ruler
        // rulers are >= 0: the biased exponent field orders them; vrt < 2^(ex + 1)
        const int ex = wave_max_i((int)(__float_as_uint(vrt) >> 23) - 127);
        const int ve_new = ex - 6;
        amul = ldexpf(1.f, ve - ve_new);
        ve = ve_new;
        v_thr = ldexpf(1.f, 7 + ve);
        v_mul = ldexpf(1.f, -ve);
      }
      const float vrs = vrt * v_mul;
#pragma unroll
      for (int p = 0; p < G; ++p) {
        const float s = valid ? sum[p] * ft : -INFINITY;
        // Lazy rescaling: the reference point m_run only moves when some score exceeds it by
        // more than 2^8, so most tiles skip the wave-wide max (p stays <= 256; fp32 has the
        // range). m_run is the same in every lane and wave (same inputs), so the branch is
        // uniform.
        if (__builtin_amdgcn_ballot_w64(s > m_run[p] + 8.f) != 0) {
          const float mt = wave_max(s);
          const float alpha = exp2f(m_run[p] - mt);
          m_run[p] = mt;
          l_lane[p] *= alpha;
          amul = n == p ? alpha * amul : amul;
        }
        const float pr = fast_exp2(s - m_run[p]);
        l_lane[p] += pr;
        // P' = P * ruler_v * 2^-ve, rounded to fp16 once (the V codes are exact integers);
        // tokens past the tile's end have P = 0 and all-zero decoded rows
        S.pw[wv][p][lane] = (_Float16)(pr * vrs);
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) oacc[mi] *= amul;
    }
    // ---------------------------------------------------------------- P.V on MFMA
    // O^T[dims, heads] += V^T[dims, tokens] * P'^T[tokens, heads], 32 tokens per k-step. The B
    // operand (lane (n, gq): P' of head n, tokens 8gq..8gq+7) is this wave's own LDS row, written
    // just above by other lanes of the wave: LDS accesses of one wave complete in order, and the
    // wavefront fence keeps the compiler from reordering them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      half8 bp = {};
      if (n < G) bp = *(const half8*)&S.pw[wv][n][32 * kk + 8 * gq];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const uint8_t* src = &S.vcode[tp][32 * kk + tr_tok][16 * (wv + 4 * mi) + tr_col];
        typedef int v2i __attribute__((ext_vector_type(2)));
        const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) v2i*)(src));
        half8 av;
        if constexpr (VB == 3) {
          // fp8 bytes of (c - 4) scaled by the fp8 unit's inverse: exact small integers
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
            const half2v a = __builtin_bit_cast(half2v, lo) - bias;
            const half2v b = __builtin_bit_cast(half2v, hi) - bias;
            av[4 * w] = a[0];
            av[4 * w + 1] = a[1];
            av[4 * w + 2] = b[0];
            av[4 * w + 3] = b[1];
          }
        }
        oacc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bp, oacc[mi], 0, 0, 0);
      }
    }
  }

  // the V-ruler scale 2^-ve taken back (exact)
  if (ve != 0) {
    const float vsc = ldexpf(1.f, ve);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) oacc[mi] *= vsc;
  }
  // ---- normalisers: the per-lane partial sums over the wave (every wave holds the same)
#pragma unroll
  for (int p = 0; p < G; ++p) l_lane[p] = wave_sum(l_lane[p]);
  if (tid == 0) {
#pragma unroll
    for (int p = 0; p < G; ++p) {
      S.m[p] = m_run[p];
      S.l[p] = l_lane[p];
    }
  }
  __syncthreads();

  if (n_chunks == 1) {
    if (n < G) {
      const float inv = 1.f / S.l[n];
      const int64_t ob = qrow * a.out_row_stride + (int64_t)(h * G + n) * kD;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        store_act(a.out, a.out_dtype, ob + dl + i, oacc[0][i] * inv);
        store_act(a.out, a.out_dtype, ob + 64 + dl + i, oacc[1][i] * inv);
      }
    }
    return;
  }

  // ---- split-K partial: [G][kD + 2] per (r, h, c): unnormalised o, running max, running sum
  const int64_t pstride = (int64_t)G * (kD + 2);
  float* partp = a.ws_part + ((int64_t)(base + c) * g.H + h) * pstride;
  // The partial is written with agent-scope (write-through) atomic stores and waited on before
  // the counter update, so no cache-wide release fence is needed.
  auto st_agent = [](float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (n < G) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st_agent(&partp[n * (kD + 2) + dl + i], oacc[0][i]);
      st_agent(&partp[n * (kD + 2) + 64 + dl + i], oacc[1][i]);
    }
  }
  if (tid < G) {
    st_agent(&partp[tid * (kD + 2) + kD], S.m[tid]);
    st_agent(&partp[tid * (kD + 2) + kD + 1], S.l[tid]);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = arrive(&a.ws_cnt[r * g.H + h]);
    S.is_last = (prev == n_chunks - 1);
  }
  __syncthreads();
  if (!S.is_last) return;
  // Every partial was stored write-through and completed before its counter update, so the
  // agent-scope loads below (ld_agent: coherent across the XCDs' L2s, with no L2 invalidate) see
  // them; the loads of all chunks are in flight together.

  const float* pbase = a.ws_part + ((int64_t)base * g.H + h) * pstride;
  const int64_t cstride = (int64_t)g.H * pstride;  // between chunks of one request and head
  // Many chunks: weights in LDS (the tile buffers are free now) -- every chunk's (max, sum) in
  // one round of loads, the per-head max and normaliser by one wave per head, then each output's
  // chunk loads issued together: a few memory round trips whatever the chunk count. Up to 8
  // chunks (24 for G <= 4), every value a thread's outputs need is requested in one round and
  // combined in registers (combine_regs): one round trip. (Partials live past this XCD's L2; a round trip took ~2.8 us at
  // the headline, and the former two rounds per output, four per thread, made this combine
  // ~11.5 us of the launch's tail.)
  float* wsh = reinterpret_cast<float*>(&S.coef[0][0]);
  constexpr int kWCap = (int)(sizeof(S.coef) / sizeof(float));
  const int ncp = n_chunks * G;
  const int64_t orow = qrow * a.out_row_stride;
  if (n_chunks <= 8) {
    combine_regs<G, 8>(pbase, cstride, n_chunks, tid, a.out, a.out_dtype, orow, h);
  } else if (G <= 4 && n_chunks <= 24) {
    // (batch 1 at ~1k tokens: 17 chunks per head)
    if constexpr (G <= 4) combine_regs<G, 24>(pbase, cstride, n_chunks, tid, a.out, a.out_dtype, orow, h);
  } else if (2 * ncp <= kWCap) {
    for (int i = tid; i < ncp; i += kThreads) {
      const int cc = i / G, p = i - cc * G;
      const float* pc = pbase + cc * cstride + p * (kD + 2);
      wsh[i] = ld_agent(&pc[kD]);
      wsh[ncp + i] = ld_agent(&pc[kD + 1]);
    }
    __syncthreads();
    for (int p = wv; p < G; p += kWaves) {  // wave-uniform: whole waves take a head each
      float mx = -INFINITY;
      for (int cc = lane; cc < n_chunks; cc += 64) mx = fmaxf(mx, wsh[cc * G + p]);
      mx = wave_max(mx);
      float L = 0.f;
      for (int cc = lane; cc < n_chunks; cc += 64)
        L = fmaf(wsh[ncp + cc * G + p], exp2f(wsh[cc * G + p] - mx), L);
      const float invL = 1.f / wave_sum(L);
      for (int cc = lane; cc < n_chunks; cc += 64)
        wsh[cc * G + p] = exp2f(wsh[cc * G + p] - mx) * invL;
    }
    __syncthreads();
    for (int it = tid; it < G * kD; it += kThreads) {
      const int p = it / kD;
      const int dim = it - p * kD;
      const float* po = pbase + p * (kD + 2) + dim;
      float O = 0.f;
      for (int c0 = 0; c0 < n_chunks; c0 += 32) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = c0 + j < n_chunks ? ld_agent(&po[(c0 + j) * cstride]) : 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j)
          if (c0 + j < n_chunks) O = fmaf(v[j], wsh[(c0 + j) * G + p], O);
      }
      store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G + p) * kD + dim, O);
    }
  } else {  // more chunks than the LDS weights hold: two passes per output
    for (int it = tid; it < G * kD; it += kThreads) {
      const int p = it / kD;
      const int dim = it - p * kD;
      float M = -INFINITY;
#pragma unroll 8
      for (int cc = 0; cc < n_chunks; ++cc) M = fmaxf(M, ld_agent(&pbase[cc * cstride + p * (kD + 2) + kD]));
      float L = 0.f, O = 0.f;
#pragma unroll 8
      for (int cc = 0; cc < n_chunks; ++cc) {
        const float* pc = pbase + cc * cstride + p * (kD + 2);
        const float f = exp2f(ld_agent(&pc[kD]) - M);
        L = fmaf(ld_agent(&pc[kD + 1]), f, L);
        O = fmaf(ld_agent(&pc[dim]), f, O);
      }
      store_act(a.out, a.out_dtype, qrow * a.out_row_stride + (int64_t)(h * G + p) * kD + dim,
                O / L);
    }
  }
  if (tid == 0) __hip_atomic_store(&a.ws_cnt[r * g.H + h], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ttkv


// ------------------------------------------------------------------------------------ host side
#include "ttkv_host.h"

namespace ttkv {

template <int G, int RB, int VB, int KU, int CM = kCoefI8>
static int launch_decode_t(const DecodeArgs& a, int grid, hipStream_t st) {
  const size_t smem = sizeof(DecodeSmem<KU, G>);
  auto kfn = a.q_dtype == TTKV_DTYPE_F16 ? decode_paged_kernel<G, RB, VB, KU, false, CM>
                                         : decode_paged_kernel<G, RB, VB, KU, true, CM>;
  if (int rc = raise_smem_limit((const void*)kfn, smem)) return rc;
  hipLaunchKernelGGL(kfn, dim3(grid), dim3(kThreads), smem, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host_fail(TTKV_E_LAUNCH, std::string("decode launch: ") +
                                                           hipGetErrorString(e));
  return TTKV_OK;
}

template <int RB, int VB, int KU>
static int dispatch_g(const DecodeArgs& a, int grid, hipStream_t st) {
  switch (a.G) {
    case 1: return launch_decode_t<1, RB, VB, KU>(a, grid, st);
    case 2: return launch_decode_t<2, RB, VB, KU>(a, grid, st);
    case 3: return launch_decode_t<3, RB, VB, KU>(a, grid, st);
    case 4: return launch_decode_t<4, RB, VB, KU>(a, grid, st);
    case 8: return launch_decode_t<8, RB, VB, KU>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "num_heads / H = " + std::to_string(a.G) +
                                           " query heads per KV head is not built (1,2,3,4,8)");
}

// The fp16 and 4-bit coefficient modes are built for G = 3 and r1 in 65..128 (the shapes their
// tests and benchmark use).
template <int RB, int VB, int CM>
static int dispatch_mode(const DecodeArgs& a, int ku, int grid, hipStream_t st) {
  if (a.G == 3 && ku == 7) return launch_decode_t<3, RB, VB, 7, CM>(a, grid, st);
  if (a.G == 3 && ku == 8) return launch_decode_t<3, RB, VB, 8, CM>(a, grid, st);
  return host_fail(TTKV_E_UNSUPPORTED, "fp16 and 4-bit coefficients are built for num_heads / H "
                                       "= 3 and 64 < r1 <= 128");
}

template <int RB, int VB>
static int dispatch_k(const DecodeArgs& a, int ku, int grid, hipStream_t st) {
  if (a.g.coef_mode == kCoefF16) return dispatch_mode<RB, VB, kCoefF16>(a, ku, grid, st);
  if (a.g.coef_mode == kCoefI4G32) return dispatch_mode<RB, VB, kCoefI4G32>(a, ku, grid, st);
  switch (ku) {
    case 4: return dispatch_g<RB, VB, 4>(a, grid, st);
    case 7: return dispatch_g<RB, VB, 7>(a, grid, st);
    case 8: return dispatch_g<RB, VB, 8>(a, grid, st);
    case 10: return dispatch_g<RB, VB, 10>(a, grid, st);
  }
  return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
}

// Requests per launch: the work plan holds kPlanReqs of them, and a launch's token total must fit
// an int. Larger batches run as several launches over consecutive request ranges.
static int decode_slice_reqs(int num_reqs, int max_seq_len) {
  const int64_t by_total = std::max<int64_t>(1, (int64_t)INT32_MAX / std::max(max_seq_len, 1));
  return (int)std::min<int64_t>(std::min<int64_t>(num_reqs, kPlanReqs), by_total);
}

struct DecodeShape {
  int chunk_cap, target;
  int64_t items_cap;  // (request, chunk, head) items any batch of this shape can need
};

// The kernel picks its chunk length from the batch's token total T: 64 * ceil(T * H / target / 64),
// clamped to [64, chunk_cap]. The batch with every request at max_seq_len gives the longest
// chunk and bounds the item count when the cap binds; otherwise the items are at most
// sum_r (seq_r / chunk + 1) * H <= target + num_reqs * H.
static DecodeShape decode_shape(int num_reqs, int H, int max_seq_len, int block_size) {
  DecodeShape s;
  s.target = 2 * device_cu_count();  // one round at 2 resident blocks per CU
  // the block ids of one chunk are staged in LDS: at most kSegMax of them
  const int64_t seg_cap = (int64_t)(kSegMax - 2) * std::max(block_size, 1) / kTile * kTile;
  s.chunk_cap = (int)std::max<int64_t>(std::min<int64_t>(seg_cap, 4096), kTile);
  const int64_t work = (int64_t)num_reqs * H * std::max(max_seq_len, 1);
  int64_t chunk = (work + s.target - 1) / s.target;
  chunk = std::min<int64_t>(std::max<int64_t>((chunk + kTile - 1) / kTile * kTile, kTile),
                            s.chunk_cap);
  const int64_t uniform = (int64_t)num_reqs * H * std::max<int64_t>(1, (max_seq_len + chunk - 1) / chunk);
  s.items_cap = std::max<int64_t>((int64_t)s.target + (int64_t)num_reqs * H, uniform);
  return s;
}

int64_t decode_workspace_bytes(const Geom& g, int G, int num_reqs, int max_seq_len,
                               int block_size) {
  const int nr = decode_slice_reqs(num_reqs, max_seq_len);
  const DecodeShape s = decode_shape(nr, g.H, max_seq_len, block_size);
  return kCounterBytes + s.items_cap * G * (kD + 2) * 4;
}

int decode_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                 int64_t q_row_stride, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                 int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                 const int32_t* seq_lens, const int32_t* qsl, int num_reqs, int max_seq_len,
                 const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                 const float* dec_scale, int64_t n_dec_slots, const float* cs_cache,
                 int64_t max_pos, void* out, int out_dtype, int64_t out_row_stride, void* ws,
                 int64_t ws_bytes, int32_t* err, hipStream_t st) {
  if (g.d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (!((g.res_bits == 3 && g.v_bits == 3) || (g.res_bits == 4 && g.v_bits == 4)))
    return host_fail(TTKV_E_UNSUPPORTED, "res_bits/v_bits must be 3/3 or 4/4");
  if (HQ <= 0 || HQ % g.H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  if (g.H * kPlanReqs > kMaxCounters) return host_fail(TTKV_E_UNSUPPORTED, "H > 64 KV heads");
  const int G = HQ / g.H;
  // coefficient window in 16-wide k units (r1 padded to 16 * ku)
  const int ku = g.r1 <= 64 ? 4 : g.r1 <= 112 ? 7 : g.r1 <= 128 ? 8 : g.r1 <= 160 ? 10 : 0;
  if (!ku) return host_fail(TTKV_E_UNSUPPORTED, "r1 > 160 is not built");
  if (g.coef_mode != kCoefI8 && (G != 3 || (ku != 7 && ku != 8)))
    return host_fail(TTKV_E_UNSUPPORTED, "fp16 and 4-bit coefficients are built for num_heads / "
                                         "H = 3 and 64 < r1 <= 128");
  // the coefficient window (16 * ku ranks) is read in 16-byte chunks from the slot's start
  const int win_bytes = g.coef_mode == kCoefI8 ? 16 * ku : g.coef_mode == kCoefF16 ? 32 * ku
                                                                                 : 16 * ((ku + 1) / 2);
  if (win_bytes > g.k_slot)
    return host_fail(TTKV_E_UNSUPPORTED, "padded coefficient block exceeds the K slot");
  if (!rows_in_windows(g))
    return host_fail(TTKV_E_UNSUPPORTED, "a head row of " + std::to_string(g.k_row) + "/" +
                                             std::to_string(g.v_row) +
                                             " bytes straddles its 64-byte load window");
  if (!q || !page || !bt || !seq_lens || !qsl || !dec_map || !cs_cache || !out || !err)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (int rc = check_dec_pool(dec_q, dec_scale)) return rc;
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
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.bt = bt;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.qsl = qsl;
  a.num_reqs = num_reqs;
  a.dec_map = dec_map;
  a.num_blocks = num_blocks;
  a.dec_q = dec_q;
  a.dec_scale = dec_scale;
  a.n_dec_slots = n_dec_slots;
  a.cs_cache = cs_cache;
  a.max_pos = max_pos;
  a.out = out;
  a.out_dtype = out_dtype;
  a.out_row_stride = out_row_stride;
  a.err = err;
  a.max_seq = max_seq_len;
  if (max_seq_len > kTile) {  // a request may be split into chunks: partials + counters
    const int64_t need = decode_workspace_bytes(g, G, num_reqs, max_seq_len, block_size);
    if (!ws || ws_bytes < need)
      return host_fail(TTKV_E_WORKSPACE, "decode workspace needs " + std::to_string(need) +
                                             " bytes, got " + std::to_string(ws_bytes));
    if ((uintptr_t)ws % 256) return host_fail(TTKV_E_INVALID, "workspace not 256-byte aligned");
  }
  const int slice = decode_slice_reqs(num_reqs, max_seq_len);
  for (int r0 = 0; r0 < num_reqs; r0 += slice) {
    // (slices run in stream order on one workspace: each leaves the counters zero for the next)
    DecodeArgs b = a;
    b.num_reqs = std::min(slice, num_reqs - r0);
    b.seq_lens = seq_lens + r0;
    b.qsl = qsl + r0;
    b.bt = bt + (int64_t)r0 * bt_row_stride;
    const DecodeShape sh = decode_shape(b.num_reqs, g.H, max_seq_len, block_size);
    b.chunk_cap = sh.chunk_cap;
    b.target = sh.target;
    if (max_seq_len > kTile) {  // counters [r * H + h]: kPlanReqs * H <= kMaxCounters
      b.ws_cnt = (int*)ws;
      b.ws_part = (float*)((char*)ws + kCounterBytes);
    }
    const int grid = (int)((sh.items_cap + 7) / 8 * 8);
    const int rc = g.res_bits == 3 ? dispatch_k<3, 3>(b, ku, grid, st)
                                   : dispatch_k<4, 4>(b, ku, grid, st);
    if (rc != TTKV_OK) return rc;
  }
  return TTKV_OK;
}

}  // namespace ttkv

// ---------------------------------------------------------------- no-allocation variant
// For callers that cannot allocate (code under graph capture, serving loops that forbid it): the
// split-K counters and partials live in a file-scope device array instead of a caller workspace.
// Each device holds its own copy for the life of the process. Host code never passes `scratch`
// itself (its host-side name is not a device address): the device address is looked up once per
// device with hipGetSymbolAddress and kept. Calls on one device share the array, so calls that
// overlap in time on one device race; the counters are left zero by every call.
#include <mutex>

namespace ttkv {

constexpr int64_t kScratchBytes = 8ll << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;

__global__ void clear_counters_kernel(int* cnt, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    cnt[i] = 0;
}

// Device address of `scratch` on the current device, looked up (and its counter region cleared
// by a kernel on `st`) on the first call there; null on failure, with the error recorded.
static void* scratch_address(hipStream_t st) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    host_fail(TTKV_E_LAUNCH, "hipGetDevice failed");
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    host_fail(TTKV_E_UNSUPPORTED, "device ordinal " + std::to_string(dev) + " >= 64");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      host_fail(TTKV_E_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") +
                                   hipGetErrorString(e));
      return nullptr;
    }
    hipLaunchKernelGGL(clear_counters_kernel, dim3(16), dim3(256), 0, st, (int*)p, kMaxCounters);
    const hipError_t le = hipGetLastError();
    if (le != hipSuccess) {
      host_fail(TTKV_E_LAUNCH, std::string("scratch clear launch: ") + hipGetErrorString(le));
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

int64_t decode_noalloc_scratch_bytes() { return kScratchBytes; }

int decode_paged_noalloc(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                         int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                         int64_t slot_stride, int block_size, const int32_t* bt,
                         int64_t bt_row_stride, int max_blocks, const int32_t* seq_lens,
                         const int32_t* qsl, int num_reqs, int max_seq_len, const int32_t* dec_map,
                         int64_t num_blocks, const int8_t* dec_q, const float* dec_scale,
                         int64_t n_dec_slots, const float* cs_cache, int64_t max_pos, void* out,
                         int out_dtype, int64_t out_row_stride, int32_t* err, hipStream_t st) {
  if (g.H <= 0 || HQ <= 0 || HQ % g.H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  if (block_size <= 0 || num_reqs < 0 || max_seq_len < 0)
    return host_fail(TTKV_E_INVALID, "block_size / batch size");
  const int64_t need = decode_workspace_bytes(g, HQ / g.H, num_reqs, max_seq_len, block_size);
  if (need > kScratchBytes)
    return host_fail(TTKV_E_WORKSPACE,
                     "this batch needs " + std::to_string(need) + " bytes of split-K scratch; "
                     "the no-allocation entry point holds " + std::to_string(kScratchBytes) +
                     " (use ttkv_decode_paged with a workspace)");
  void* ws = scratch_address(st);
  if (!ws) return TTKV_E_LAUNCH;
  return decode_paged(g, HQ, scale, q, q_dtype, q_row_stride, page, n_slots, slot_stride,
                      block_size, bt, bt_row_stride, max_blocks, seq_lens, qsl, num_reqs,
                      max_seq_len, dec_map, num_blocks, dec_q, dec_scale, n_dec_slots, cs_cache,
                      max_pos, out, out_dtype, out_row_stride, ws, kScratchBytes, err, st);
}

}  // namespace ttkv

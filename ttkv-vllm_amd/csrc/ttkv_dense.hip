// Benchmark comparator: dense fp16/bf16 paged decode attention over an uncompressed KV cache of
// the same shapes as K1's workload. It has no counterpart in the compressed path; it measures what
// a plain paged KV cache costs per cached token on this GPU (the reference's bench compares its
// read with dense attention too, bench_decode_read.py:132-151). It is built as a byte-streaming
// kernel, the way a dense decode read is best built on this GPU, so that the comparison is
// against a read near the HBM bound rather than a weak one.
//
// Cache layout (vLLM's paged KV): k_cache / v_cache [num_blocks * block_size, H, d] in the model
// dtype; slot of position t of request r = block_table[r, t / bs] * bs + t % bs. A token's K row
// of all H heads (H * 256 bytes at d = 128) is one contiguous run, and so is its V row.
//
// Two launches (split-K over token chunks, then a reduction; vLLM's own paged attention v2 has
// the same structure):
//   dense_decode_kernel : work item = (request, token chunk), ALL KV heads, so every slot row is
//       read whole and once. The chunk comes from a work plan computed on the device from the
//       batch's own lengths: the shortest multiple of 16 tokens that spreads the batch's total
//       tokens over `target` items (each request at least one chunk), so a ragged batch fills
//       the chip by its total work, not by its longest request. Wave w takes head group w % 2
//       (4 heads: lane group g = head 4 * hg + g, 16 lanes of 8 dims each, one 16-byte K and V
//       load per lane and token) and token stream w / 2; per step it loads 4 tokens with the
//       next step's loads in flight, dots the G query heads of each head (packed fp16 dot
//       products for fp16 caches), keeps one online softmax per (head, query head) and
//       accumulates P.V in fp32. The two streams of a head group are merged through LDS. A
//       request with one chunk is written out directly; otherwise the item's unnormalised
//       partials (o, max, sum per head and query head) go to the workspace.
//   dense_reduce_kernel : one wave per (request, query head) with two or more chunks: the
//       chunks' maxima and sums one per lane, their weights through LDS, two output dims per
//       lane with a batch of up to 64 chunks' loads in flight together. The decode launch
//       leaves each request's (first item, chunk count) at the head of the workspace.
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kDThreads = 256;
constexpr int kDSeg = 1026;     // block ids of one chunk staged in LDS
constexpr int kDPlanLanes = 4;  // requests per lane in the work plan (256 per launch)
constexpr int kDHeads = 8;      // KV heads the kernel is built for (2 head groups of 4)
constexpr int kDGran = 16;      // chunk granularity in tokens
constexpr int kDMetaBytes = 4096;  // workspace head: (first item, chunk count) per request

struct DenseArgs {
  int H, HQ, G;
  float scale_log2;
  const void* q;
  int64_t q_row_stride;
  const uint16_t* kc;
  const uint16_t* vc;
  int dtype;  // TTKV_DTYPE_F16 or BF16 for q, cache and out
  int64_t n_slots;
  int block_size, bs_shift;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* seq_lens;
  const int32_t* qsl;
  int num_reqs;
  void* out;
  int64_t out_row_stride;
  int2* ws_meta;   // [requests] (first item, chunk count), written by the decode launch
  float* ws_part;  // [items][H][G][kD + 2]
  int target;      // work items aimed at (resident workgroups of the launch)
  int chunk_cap;   // longest chunk in tokens (a multiple of 64 whose block ids fit the LDS stage)
  int max_seq;     // longest context the launch was sized for
};

__device__ __forceinline__ void unpack8(uint4 x, int dt, float f[8]) {
  const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (dt == TTKV_DTYPE_F16) {
      f[2 * i] = f16_bits_to_float(w[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_float(w[i] >> 16);
    } else {
      f[2 * i] = bf16_bits_to_float(w[i] & 0xffffu);
      f[2 * i + 1] = bf16_bits_to_float(w[i] >> 16);
    }
  }
}

// Inclusive prefix sum over the wave's lanes (all lanes active).
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o);
    v += lane >= o ? t : 0;
  }
  return v;
}

// The device work plan, computed alike by every wave of both kernels: the chunk length and each
// request's chunk count and first item. Block `blk` of the decode launch (rq < 0), or request
// `rq` of the reduction, resolves to its item, request, chunk, context length and the request's
// first item and chunk count. Blocks are dealt to the 8 XCDs round-robin, so each XCD takes a
// contiguous range of ceil(items / 8) items: sized by the items, not by the grid (which is sized
// for the most items any batch of the launch's shape can plan), so that no XCD receives more
// items than it has resident slots while another idles.
struct DensePlan {
  int chunk, n_items;
  int it, r, c, seq, first, n_chunks;
};

__device__ __forceinline__ DensePlan dense_plan(const DenseArgs& a, int blk, int rq) {
  const int lane = threadIdx.x & 63;
  const int nper = (a.num_reqs + 63) >> 6;
  int sl[kDPlanLanes], nch[kDPlanLanes], ex[kDPlanLanes];
  int tiles = 0;
#pragma unroll
  for (int i = 0; i < kDPlanLanes; ++i) {
    const int rr = lane + 64 * i;
    sl[i] = (i < nper && rr < a.num_reqs) ? min(max(a.seq_lens[rr], 0), a.max_seq) : 0;
    tiles += (sl[i] + kDGran - 1) / kDGran;
  }
  tiles = wave_sum_i(tiles);
  DensePlan P{};
  const int m_tiles = min(max(1, (tiles + a.target - 1) / a.target), a.chunk_cap / kDGran);
  P.chunk = m_tiles * kDGran;
  int carry = 0;
#pragma unroll
  for (int i = 0; i < kDPlanLanes; ++i) {
    const int rr = lane + 64 * i;
    nch[i] = (i < nper && rr < a.num_reqs) ? max(1, (sl[i] + P.chunk - 1) / P.chunk) : 0;
    const int incl = wave_incl_scan(nch[i]);
    ex[i] = carry + incl - nch[i];
    carry += __shfl(incl, 63);
  }
  P.n_items = carry;
  P.n_chunks = 0;
  int it = 0;
  if (rq < 0) {
    const int per_xcd = (P.n_items + 7) >> 3;
    it = (blk >> 3) < per_xcd ? (blk & 7) * per_xcd + (blk >> 3) : P.n_items;
  }
  P.it = it;
#pragma unroll
  for (int i = 0; i < kDPlanLanes; ++i) {
    const int rr = lane + 64 * i;
    const bool mine = rq >= 0 ? rr == rq : (nch[i] > 0 && ex[i] <= it && it < ex[i] + nch[i]);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(mine && rr < a.num_reqs);
    if (hit) {
      const int ln = __builtin_ctzll(hit);
      P.r = 64 * i + ln;
      P.first = __shfl(ex[i], ln);
      P.c = it - P.first;
      P.seq = __shfl(sl[i], ln);
      P.n_chunks = __shfl(nch[i], ln);
    }
  }
  return P;
}

template <int G, int DT>
__global__ __launch_bounds__(kDThreads, 2) void dense_decode_kernel(DenseArgs a) {
  constexpr int NST = 2;  // token streams per head group
  __shared__ float red_o[4][4][G][kD];  // [wave][head in group][query head][dim]
  __shared__ float red_m[4][4][G], red_l[4][4][G];
  __shared__ int seg[kDSeg];
  const int tid = threadIdx.x;
  // the wave index and the item's bounds in scalar registers: the streaming loop's trip count is
  // uniform (scalar branches, no exec-mask bookkeeping around the loads)
  const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 4;   // head within the group
  const int sub = lane & 15;  // dims 8*sub .. 8*sub+7
  const int hg = wv & 1, stream = wv >> 1;
  const int head = 4 * hg + hl;

  const DensePlan P = dense_plan(a, blockIdx.x, -1);
  const int it = P.it;
  if (it >= P.n_items) return;
  if (P.c == 0 && tid == 0) a.ws_meta[P.r] = make_int2(P.first, P.n_chunks);
  const int64_t qrow = a.qsl[P.r];
  const int t0 = __builtin_amdgcn_readfirstlane(P.c * P.chunk);
  const int t1 = __builtin_amdgcn_readfirstlane(min(P.seq, t0 + P.chunk));
  if (t1 <= t0) {  // empty context: the attention over zero rows is 0
    for (int i = tid; i < a.HQ * kD; i += kDThreads)
      store_act(a.out, DT, qrow * a.out_row_stride + i, 0.f);
    return;
  }
  const int bfirst = t0 >> a.bs_shift;
  const int nseg = ((t1 - 1) >> a.bs_shift) - bfirst + 1;
  for (int i = tid; i < nseg; i += kDThreads)
    seg[i] = a.bt[(int64_t)P.r * a.bt_row_stride + bfirst + i];

  // query: fp16 caches take packed fp16 pairs (dot products on v_dot2), bf16 fp32 values
  uint32_t qp[G][4];
  float qf[G][8];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const uint4 x = ld_global16((const uint16_t*)a.q + qrow * a.q_row_stride +
                                (int64_t)(head * G + p) * kD + 8 * sub);
    qp[p][0] = x.x;
    qp[p][1] = x.y;
    qp[p][2] = x.z;
    qp[p][3] = x.w;
    if constexpr (DT != TTKV_DTYPE_F16) unpack8(x, DT, qf[p]);
  }
  float o[G][8], m[G], l[G];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    m[p] = -INFINITY;
    l[p] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[p][i] = 0.f;
  }
  __syncthreads();  // seg
  const int bmask = a.block_size - 1;
  const int lane_off = head * kD + 8 * sub;  // elements within a slot's row
  constexpr int64_t kRow = (int64_t)kDHeads * kD;
  constexpr int kStep = 4;  // tokens per wave step
  // Loads are unconditional (positions past the chunk re-read its last row, whose scores are
  // masked to -inf), issued in the same order in every copy of the step, from a wave-uniform row
  // address plus the lane's 32-bit offset: with a branch per token the compiler could not count
  // the loads in flight across the join and waited for all of them, the next step's included,
  // before any use (headline 100 -> 83 us per launch with the two register sets below).
  const uint32_t lane_byte = (uint32_t)lane_off * 2u;
  auto load_step = [&](int tb, uint4* kx, uint4* vx) {
#pragma unroll
    for (int u = 0; u < kStep; ++u) {
      const int t = min(tb + u, t1 - 1);
      const int blk = __builtin_amdgcn_readfirstlane(seg[(t >> a.bs_shift) - bfirst]);
      const int64_t slot = (int64_t)blk * a.block_size + (t & bmask);
      const char* kr = (const char*)a.kc + slot * (kRow * 2);
      const char* vr = (const char*)a.vc + slot * (kRow * 2);
      kx[u] = ld_stream16(kr + lane_byte);
      vx[u] = ld_stream16(vr + lane_byte);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto step = [&](int tb, const uint4* kx, const uint4* vx) {
    float s[G][kStep];
#pragma unroll
    for (int u = 0; u < kStep; ++u) {
      const bool ok = tb + u < t1;
      float kf[8];
      if constexpr (DT != TTKV_DTYPE_F16) unpack8(kx[u], DT, kf);
      const uint32_t kw[4] = {kx[u].x, kx[u].y, kx[u].z, kx[u].w};
#pragma unroll
      for (int p = 0; p < G; ++p) {
        float acc = 0.f;
        if constexpr (DT == TTKV_DTYPE_F16) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, qp[p][i]),
                                         __builtin_bit_cast(half2v, kw[i]), acc, false);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) acc = fmaf(qf[p][i], kf[i], acc);
        }
        s[p][u] = ok ? row_sum(acc) * a.scale_log2 : -INFINITY;
      }
    }
    // online softmax per (head, query head): the 16 lanes of a head hold the same scores; the
    // reference point moves only when a score exceeds it by more than 2^8 (p <= 256 otherwise)
#pragma unroll
    for (int p = 0; p < G; ++p) {
      float mt = s[p][0];
#pragma unroll
      for (int u = 1; u < kStep; ++u) mt = fmaxf(mt, s[p][u]);
      if (__builtin_amdgcn_ballot_w64(mt > m[p] + 8.f) != 0) {
        const float mn = fmaxf(m[p], mt);
        const float alpha = m[p] == -INFINITY ? 0.f : exp2f(m[p] - mn);
        m[p] = mn;
        l[p] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[p][i] *= alpha;
      }
#pragma unroll
      for (int u = 0; u < kStep; ++u) {
        s[p][u] = fast_exp2(s[p][u] - m[p]);
        l[p] += s[p][u];
      }
    }
#pragma unroll
    for (int u = 0; u < kStep; ++u) {
      float vf[8];
      unpack8(vx[u], DT, vf);
#pragma unroll
      for (int p = 0; p < G; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[p][i] = fmaf(s[p][u], vf[i], o[p][i]);
    }
  };
  // Two register sets in turn, so the next step's loads are in flight during a step; the
  // scheduling barriers keep the compiler from hoisting a step's arithmetic above them.
  constexpr int kAdv = kStep * NST;  // tokens between a stream's consecutive steps
  uint4 ka[kStep], va[kStep], kb[kStep], vb[kStep];
  int tb = t0 + kStep * stream;
  load_step(tb, ka, va);
  while (tb < t1) {
    load_step(tb + kAdv, kb, vb);
    __builtin_amdgcn_sched_barrier(0);
    step(tb, ka, va);
    tb += kAdv;
    if (tb >= t1) break;
    load_step(tb + kAdv, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    step(tb, kb, vb);
    tb += kAdv;
  }
  // ---- merge the two streams of each head group through LDS
  if (sub == 0) {
#pragma unroll
    for (int p = 0; p < G; ++p) {
      red_m[wv][hl][p] = m[p];
      red_l[wv][hl][p] = l[p];
    }
  }
  __syncthreads();
  if (stream != 0) {
#pragma unroll
    for (int p = 0; p < G; ++p) {
      const float M = fmaxf(red_m[hg][hl][p], m[p]);
      const float f = m[p] == -INFINITY ? 0.f : exp2f(m[p] - M);
#pragma unroll
      for (int i = 0; i < 8; ++i) red_o[wv][hl][p][8 * sub + i] = o[p][i] * f;
    }
  }
  __syncthreads();
  if (stream != 0) return;
  // stream 0 of each head group: merged o, max, sum of its 4 heads
  const int wo = wv + 2;  // the other stream's wave
  float* partp = nullptr;
  if (P.n_chunks > 1)
    partp = a.ws_part + ((int64_t)it * kDHeads + head) * G * (kD + 2);
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const float mo = red_m[wo][hl][p];
    const float M = fmaxf(m[p], mo);
    const float f = m[p] == -INFINITY ? 0.f : exp2f(m[p] - M);
    const float L = l[p] * f + (mo == -INFINITY ? 0.f : red_l[wo][hl][p] * exp2f(mo - M));
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = fmaf(o[p][i], f, red_o[wo][hl][p][8 * sub + i]);
    if (P.n_chunks == 1) {
      const float inv = 1.f / L;
      const int64_t ob = qrow * a.out_row_stride + (int64_t)(head * G + p) * kD + 8 * sub;
#pragma unroll
      for (int i = 0; i < 8; ++i) store_act(a.out, DT, ob + i, v[i] * inv);
    } else {
      float* pp = partp + p * (kD + 2);
#pragma unroll
      for (int i = 0; i < 8; ++i) pp[8 * sub + i] = v[i];
      if (sub == 0) {
        pp[kD] = M;
        pp[kD + 1] = L;
      }
    }
  }
}

// One wave per (request, query head) whose request has two or more chunks: the chunks' partials
// combined into the output, in batches of up to 64 chunks. Lane c holds chunk c's max and sum;
// the chunk weights go through LDS to every lane, and each lane combines two output dims, with
// all of the batch's output loads in flight together. The request's item range comes from the
// decode launch (no plan here).
template <int G, int DT>
__global__ __launch_bounds__(64) void dense_reduce_kernel(DenseArgs a) {
  __shared__ float wgt[64];
  const int lane = threadIdx.x;
  const int rq = blockIdx.x / a.HQ, hq = blockIdx.x % a.HQ;
  if (rq >= a.num_reqs) return;
  const int2 meta = a.ws_meta[rq];
  const int first = meta.x, nch = meta.y;
  if (nch <= 1) return;
  const int h = hq / G, p = hq % G;
  const int64_t cstride = (int64_t)kDHeads * G * (kD + 2);  // between consecutive items
  const float* ph = a.ws_part + ((int64_t)first * kDHeads + h) * G * (kD + 2) + p * (kD + 2);
  float M = -INFINITY, L = 0.f, O0 = 0.f, O1 = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 64) {
    const int nb = min(64, nch - c0);
    // chunks past the batch re-read its last chunk (valid, finite) and get weight 0
    const float* pl = ph + (int64_t)(c0 + min(lane, nb - 1)) * cstride;
    const float mc = lane < nb ? pl[kD] : -INFINITY;
    const float lc = pl[kD + 1];
    float2v ov[64];
#pragma unroll
    for (int j = 0; j < 64; ++j)
      ov[j] = *(const float2v*)(ph + (int64_t)(c0 + min(j, nb - 1)) * cstride + 2 * lane);
    const float mb = fmaxf(M, wave_max(mc));
    // a non-empty chunk's max is finite, so mb is; the running terms start at zero
    const float f = M == -INFINITY ? 0.f : exp2f(M - mb);
    const float wc = mc == -INFINITY ? 0.f : exp2f(mc - mb);
    L = fmaf(L, f, wave_sum(lc * wc));
    wgt[lane] = wc;
    __syncthreads();
    O0 *= f;
    O1 *= f;
#pragma unroll
    for (int j = 0; j < 64; j += 4) {
      const float4v w = *(const float4v*)&wgt[j];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        O0 = fmaf(ov[j + k][0], w[k], O0);
        O1 = fmaf(ov[j + k][1], w[k], O1);
      }
    }
    __syncthreads();  // wgt is rewritten by the next batch
    M = mb;
  }
  const float inv = 1.f / L;
  const int64_t ob = (int64_t)a.qsl[rq] * a.out_row_stride + (int64_t)hq * kD + 2 * lane;
  store_act(a.out, DT, ob, O0 * inv);
  store_act(a.out, DT, ob + 1, O1 * inv);
}

}  // namespace ttkv

#include "ttkv_host.h"

namespace ttkv {

// Resident workgroups of the G/DT build on this device (the plan's item target), at most two per
// CU: longer chunks stream longer runs per workgroup.
template <int G, int DT>
static int dense_slots() {
  static int slots = 0;
  if (!slots) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, dense_decode_kernel<G, DT>,
                                                     kDThreads, 0) != hipSuccess || per_cu < 1)
      per_cu = 2;
    slots = std::min(per_cu, 2) * device_cu_count();
  }
  return slots;
}

static int dense_target(int G, int dtype) {
  const bool f16 = dtype == TTKV_DTYPE_F16;
  switch (G) {
    case 1: return f16 ? dense_slots<1, TTKV_DTYPE_F16>() : dense_slots<1, TTKV_DTYPE_BF16>();
    case 2: return f16 ? dense_slots<2, TTKV_DTYPE_F16>() : dense_slots<2, TTKV_DTYPE_BF16>();
    case 3: return f16 ? dense_slots<3, TTKV_DTYPE_F16>() : dense_slots<3, TTKV_DTYPE_BF16>();
    default: return f16 ? dense_slots<4, TTKV_DTYPE_F16>() : dense_slots<4, TTKV_DTYPE_BF16>();
  }
}

static int dense_chunk_cap(int block_size) {
  return (int)std::max<int64_t>(kDGran, (int64_t)(kDSeg - 2) * std::max(block_size, 1) / kDGran *
                                            kDGran);
}

// Requests per launch: the plan's 256.
static int dense_slice_reqs(int num_reqs) { return std::min(num_reqs, kDPlanLanes * 64); }

// (request, chunk) items a launch can plan: at most target + one per request from rounding,
// more when the chunk cap binds
static int64_t dense_max_items(int nr, int max_seq_len, int block_size, int target) {
  const int64_t cap = dense_chunk_cap(block_size);
  return (int64_t)target + 1 + (int64_t)nr * (2 + (std::max(max_seq_len, 1) + cap - 1) / cap);
}

int64_t dense_workspace_bytes(int H, int G, int num_reqs, int max_seq_len, int block_size) {
  if (num_reqs <= 0 || G < 1 || G > 4 || H != kDHeads) return 256;
  const int slice = std::max(1, dense_slice_reqs(num_reqs));
  const int target = std::max(dense_target(G, TTKV_DTYPE_F16), dense_target(G, TTKV_DTYPE_BF16));
  return kDMetaBytes + dense_max_items(slice, max_seq_len, block_size, target) * kDHeads * G *
                            (kD + 2) * 4;
}

template <int G, int DT>
static int launch_dense_t(const DenseArgs& a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((dense_decode_kernel<G, DT>), dim3(grid), dim3(kDThreads), 0, st, a);
  hipLaunchKernelGGL((dense_reduce_kernel<G, DT>), dim3(a.num_reqs * a.HQ), dim3(64), 0,
                     st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return host_fail(TTKV_E_LAUNCH, std::string("dense launch: ") + hipGetErrorString(e));
  return TTKV_OK;
}

int dense_decode_paged(int H, int HQ, int d, float scale, const void* q, int64_t q_row_stride,
                       const void* k_cache, const void* v_cache, int dtype, int64_t n_slots,
                       int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                       const int32_t* seq_lens, const int32_t* qsl, int num_reqs, int max_seq_len,
                       void* out, int64_t out_row_stride, void* ws, int64_t ws_bytes,
                       hipStream_t st) {
  if (d != kD) return host_fail(TTKV_E_UNSUPPORTED, "head dim must be 128");
  if (H <= 0 || HQ % H) return host_fail(TTKV_E_INVALID, "num_heads is not a multiple of H");
  if (H != kDHeads) return host_fail(TTKV_E_UNSUPPORTED, "the dense comparator is built for H = 8");
  if (dtype != TTKV_DTYPE_F16 && dtype != TTKV_DTYPE_BF16)
    return host_fail(TTKV_E_INVALID, "dense cache dtype must be fp16 or bf16");
  if (!q || !k_cache || !v_cache || !bt || !seq_lens || !qsl || !out)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || q_row_stride % 8)
    return host_fail(TTKV_E_INVALID, "q / caches must be 16-byte aligned");
  if (num_reqs == 0) return TTKV_OK;
  if (block_size <= 0 || (block_size & (block_size - 1)))
    return host_fail(TTKV_E_UNSUPPORTED, "the dense comparator takes a power-of-two block size");
  if ((int64_t)max_blocks * block_size < max_seq_len)
    return host_fail(TTKV_E_INVALID, "max_seq_len needs more blocks than the block table holds");
  const int G = HQ / H;
  if (G < 1 || G > 4) return host_fail(TTKV_E_UNSUPPORTED, "G must be 1..4 for the dense comparator");
  const int64_t need = dense_workspace_bytes(H, G, num_reqs, max_seq_len, block_size);
  if (!ws || ws_bytes < need || (uintptr_t)ws % 256)
    return host_fail(TTKV_E_WORKSPACE, "dense workspace needs " + std::to_string(need) +
                                           " bytes, 256-aligned");
  DenseArgs a{};
  a.H = H;
  a.HQ = HQ;
  a.G = G;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.q = q;
  a.q_row_stride = q_row_stride;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.dtype = dtype;
  a.n_slots = n_slots;
  a.block_size = block_size;
  a.bs_shift = __builtin_ctz((unsigned)block_size);
  a.bt = bt;
  a.bt_row_stride = bt_row_stride;
  a.out = out;
  a.out_row_stride = out_row_stride;
  a.max_seq = max_seq_len;
  a.target = dense_target(G, dtype);
  a.chunk_cap = dense_chunk_cap(block_size);
  a.ws_meta = (int2*)ws;
  a.ws_part = (float*)((char*)ws + kDMetaBytes);
  const int slice = dense_slice_reqs(num_reqs);
  for (int r0 = 0; r0 < num_reqs; r0 += slice) {
    DenseArgs b = a;
    b.num_reqs = std::min(slice, num_reqs - r0);
    b.seq_lens = seq_lens + r0;
    b.qsl = qsl + r0;
    b.bt = bt + (int64_t)r0 * bt_row_stride;
    const int64_t items = dense_max_items(b.num_reqs, max_seq_len, block_size, a.target);
    const int grid = (int)((items + 7) / 8 * 8);
    const bool f16 = dtype == TTKV_DTYPE_F16;
    int rc = TTKV_OK;
    switch (G) {
      case 1: rc = f16 ? launch_dense_t<1, TTKV_DTYPE_F16>(b, grid, st) : launch_dense_t<1, TTKV_DTYPE_BF16>(b, grid, st); break;
      case 2: rc = f16 ? launch_dense_t<2, TTKV_DTYPE_F16>(b, grid, st) : launch_dense_t<2, TTKV_DTYPE_BF16>(b, grid, st); break;
      case 3: rc = f16 ? launch_dense_t<3, TTKV_DTYPE_F16>(b, grid, st) : launch_dense_t<3, TTKV_DTYPE_BF16>(b, grid, st); break;
      case 4: rc = f16 ? launch_dense_t<4, TTKV_DTYPE_F16>(b, grid, st) : launch_dense_t<4, TTKV_DTYPE_BF16>(b, grid, st); break;
    }
    if (rc != TTKV_OK) return rc;
  }
  return TTKV_OK;
}

}  // namespace ttkv

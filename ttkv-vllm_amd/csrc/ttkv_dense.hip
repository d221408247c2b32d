// Benchmark comparator: dense fp16/bf16 paged decode attention of the same shapes and launch
// structure as K1 (one launch per layer over the batch, split-K over token chunks combined in the
// same launch). It has no counterpart in the compressed path; it measures what a plain paged KV
// cache costs per cached token on this GPU (the reference's bench compares its read with dense
// attention too, bench_decode_read.py:132-151).
//
// Cache layout (vLLM's paged KV): k_cache / v_cache [num_blocks * block_size, H, d] in the model
// dtype; slot of position t of request r = block_table[r, t / bs] * bs + t % bs.
//
// Work item = (request, KV head, token chunk). 16 lanes own one token (8 dims each, one 16-byte
// load per lane for K and for V); a wave walks 16 tokens per step with the next step's loads in
// flight, dots the G query heads of the KV head, rescales its online softmax once per step and
// accumulates P.V. Lane groups and waves are merged at the end, then chunks as in K1.
#include <math.h>

#include "ttkv_device.h"

namespace ttkv {

constexpr int kDThreads = 256;
constexpr int kDSeg = 1026;  // block ids of one chunk staged in LDS
constexpr int kDUnroll = 4;  // 4-token steps per wave iteration (loads of the next iteration in flight)

struct DenseArgs {
  int H, HQ, G;
  float scale_log2;
  const void* q;
  int64_t q_row_stride;
  const uint16_t* kc;
  const uint16_t* vc;
  int dtype;  // TTKV_DTYPE_F16 or BF16 for q, cache and out
  int64_t n_slots;
  int block_size;
  const int32_t* bt;
  int64_t bt_row_stride;
  const int32_t* seq_lens;
  const int32_t* qsl;
  int num_reqs;
  void* out;
  int64_t out_row_stride;
  float* ws_part;
  int* ws_cnt;
  int chunk, max_chunks, nwork, max_seq;
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

template <int G, int DT>
__global__ __launch_bounds__(kDThreads) void dense_decode_kernel(DenseArgs a) {
  __shared__ float red_o[4][G][kD];
  __shared__ float red_m[4][4][G], red_l[4][4][G];
  __shared__ int is_last;
  __shared__ int seg[kDSeg];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int grp = lane >> 4;  // token slot within the wave step
  const int sub = lane & 15;  // dims 8*sub .. 8*sub+7
  const int per_xcd = gridDim.x >> 3;
  const int w = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (w >= a.nwork) return;
  const int h = w % a.H;
  const int rc = w / a.H;
  const int r = rc % a.num_reqs;
  const int c = rc / a.num_reqs;
  if (c >= a.max_chunks) return;
  const int seq = min(a.seq_lens[r], a.max_seq);
  const int n_chunks = (seq + a.chunk - 1) / a.chunk;
  if (c >= n_chunks) return;
  const int t0 = c * a.chunk, t1 = min(seq, t0 + a.chunk);
  const int64_t qrow = a.qsl[r];
  const int bfirst = t0 / a.block_size;
  const int nseg = (t1 - 1) / a.block_size - bfirst + 1;
  for (int i = tid; i < nseg; i += kDThreads)
    seg[i] = a.bt[(int64_t)r * a.bt_row_stride + bfirst + i];
  __syncthreads();

  float q[G][8];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const uint4 x = ld_global16((const uint16_t*)a.q + qrow * a.q_row_stride +
                                (int64_t)(h * G + p) * kD + 8 * sub);
    unpack8(x, DT, q[p]);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[p][i] *= a.scale_log2;
  }
  float o[G][8], m[G], l[G];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    m[p] = -INFINITY;
    l[p] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[p][i] = 0.f;
  }
  const int64_t row_elems = (int64_t)a.H * kD;
  auto slot_off = [&](int t) -> int64_t {
    const int bi = t / a.block_size;
    const int blk = seg[bi - bfirst];
    return ((int64_t)blk * a.block_size + (t - bi * a.block_size)) * row_elems + (int64_t)h * kD +
           8 * sub;
  };
  // Each wave owns steps of 4 * kDUnroll tokens (4 lane groups x kDUnroll); the next step's K/V loads are
  // issued before the current step is computed. One softmax rescale per step.
  constexpr int kStep = 4 * kDUnroll;
  uint4 kx[kDUnroll], vx[kDUnroll];
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  int tb = t0 + kStep * wv;
#pragma unroll
  for (int u = 0; u < kDUnroll; ++u) {
    const int t = tb + 4 * u + grp;
    const int64_t off = t < t1 ? slot_off(t) : -1;
    kx[u] = off >= 0 ? ld_global16(a.kc + off) : zero4;
    vx[u] = off >= 0 ? ld_global16(a.vc + off) : zero4;
  }
  for (; tb < t1; tb += 4 * kStep) {
    uint4 kn[kDUnroll], vn[kDUnroll];
#pragma unroll
    for (int u = 0; u < kDUnroll; ++u) {
      const int t = tb + 4 * kStep + 4 * u + grp;
      const int64_t off = t < t1 ? slot_off(t) : -1;
      kn[u] = off >= 0 ? ld_global16(a.kc + off) : zero4;
      vn[u] = off >= 0 ? ld_global16(a.vc + off) : zero4;
    }
    float s[G][kDUnroll];
#pragma unroll
    for (int u = 0; u < kDUnroll; ++u) {
      float kf[8];
      unpack8(kx[u], DT, kf);
      const bool ok = tb + 4 * u + grp < t1;
#pragma unroll
      for (int p = 0; p < G; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(q[p][i], kf[i], acc);
        s[p][u] = ok ? row_sum(acc) : -INFINITY;
      }
    }
#pragma unroll
    for (int p = 0; p < G; ++p) {
      float mt = s[p][0];
#pragma unroll
      for (int u = 1; u < kDUnroll; ++u) mt = fmaxf(mt, s[p][u]);
      mt = cross_row_max(mt);
      const float mn = fmaxf(m[p], mt);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = exp2f(m[p] - mref);
      m[p] = mn;
      float ls = 0.f;
#pragma unroll
      for (int u = 0; u < kDUnroll; ++u) {
        s[p][u] = fast_exp2(s[p][u] - mref);
        ls += s[p][u];
      }
      l[p] = l[p] * alpha + cross_row_sum(ls);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[p][i] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < kDUnroll; ++u) {
      float vf[8];
      unpack8(vx[u], DT, vf);
#pragma unroll
      for (int p = 0; p < G; ++p)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[p][i] = fmaf(s[p][u], vf[i], o[p][i]);
    }
#pragma unroll
    for (int u = 0; u < kDUnroll; ++u) {
      kx[u] = kn[u];
      vx[u] = vn[u];
    }
  }
  // merge the 4 lane groups of each wave, then the 4 waves, through LDS
  if (sub == 0) {  // m, l are wave-uniform: the 4 lane groups share one running softmax
#pragma unroll
    for (int p = 0; p < G; ++p) {
      red_m[wv][grp][p] = grp == 0 ? m[p] : -INFINITY;
      red_l[wv][grp][p] = grp == 0 ? l[p] : 0.f;
    }
  }
  __syncthreads();
  float M[G];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    M[p] = -INFINITY;
    for (int i = 0; i < 16; ++i) M[p] = fmaxf(M[p], red_m[i >> 2][i & 3][p]);
  }
  for (int i = tid; i < 4 * G * kD; i += kDThreads) (&red_o[0][0][0])[i] = 0.f;
  __syncthreads();
#pragma unroll
  for (int p = 0; p < G; ++p) {
    const float f = m[p] == -INFINITY ? 0.f : exp2f(m[p] - M[p]);
#pragma unroll
    for (int i = 0; i < 8; ++i) atomicAdd(&red_o[wv][p][8 * sub + i], o[p][i] * f);
  }
  __syncthreads();
  float L[G];
#pragma unroll
  for (int p = 0; p < G; ++p) {
    L[p] = 0.f;
    for (int i = 0; i < 16; ++i) {
      const float mi = red_m[i >> 2][i & 3][p];
      L[p] += mi == -INFINITY ? 0.f : red_l[i >> 2][i & 3][p] * exp2f(mi - M[p]);
    }
  }
  if (n_chunks == 1) {
    for (int i = tid; i < G * kD; i += kDThreads) {
      const int p = i / kD, d = i % kD;
      const float v = red_o[0][p][d] + red_o[1][p][d] + red_o[2][p][d] + red_o[3][p][d];
      store_act(a.out, DT, qrow * a.out_row_stride + (int64_t)(h * G + p) * kD + d, v / L[p]);
    }
    return;
  }
  const int64_t pstride = (int64_t)G * (kD + 2);
  float* partp = a.ws_part + ((int64_t)(r * a.H + h) * a.max_chunks + c) * pstride;
  for (int i = tid; i < G * kD; i += kDThreads) {
    const int p = i / kD, d = i % kD;
    const float v = red_o[0][p][d] + red_o[1][p][d] + red_o[2][p][d] + red_o[3][p][d];
    __hip_atomic_store(&partp[p * (kD + 2) + d], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid < G) {
    __hip_atomic_store(&partp[tid * (kD + 2) + kD], M[tid], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&partp[tid * (kD + 2) + kD + 1], L[tid], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(&a.ws_cnt[r * a.H + h], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == n_chunks - 1);
  }
  __syncthreads();
  if (!is_last) return;
  const float* pbase = a.ws_part + (int64_t)(r * a.H + h) * a.max_chunks * pstride;
  for (int i = tid; i < G * kD; i += kDThreads) {
    const int p = i / kD, d = i % kD;
    float Mx = -INFINITY;
    for (int cc = 0; cc < n_chunks; ++cc)
      Mx = fmaxf(Mx, __hip_atomic_load(&pbase[cc * pstride + p * (kD + 2) + kD], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT));
    float Lx = 0.f, Ox = 0.f;
    for (int cc = 0; cc < n_chunks; ++cc) {
      const float* pc = pbase + cc * pstride + p * (kD + 2);
      const float f = exp2f(__hip_atomic_load(&pc[kD], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - Mx);
      Lx = fmaf(__hip_atomic_load(&pc[kD + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), f, Lx);
      Ox = fmaf(__hip_atomic_load(&pc[d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), f, Ox);
    }
    store_act(a.out, DT, qrow * a.out_row_stride + (int64_t)(h * G + p) * kD + d, Ox / Lx);
  }
  if (tid == 0)
    __hip_atomic_store(&a.ws_cnt[r * a.H + h], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace ttkv

#include "ttkv_host.h"

namespace ttkv {

int dense_chunk_for(int num_reqs, int H, int max_seq_len, int block_size) {
  const int64_t work = (int64_t)num_reqs * H * std::max(max_seq_len, 1);
  const int64_t target = 2LL * device_cu_count();  // 2 resident workgroups per CU
  int64_t chunk = (work + target - 1) / target;
  chunk = (chunk + 255) / 256 * 256;
  chunk = std::min<int64_t>(std::max<int64_t>(chunk, 256), 8192);
  const int64_t seg_cap = (int64_t)(kDSeg - 2) * std::max(block_size, 1) / 256 * 256;
  return (int)std::max<int64_t>(std::min(chunk, seg_cap), 256);
}

// Requests per launch: one arrival counter per (request, head).
static int dense_slice_reqs(int H, int num_reqs) {
  return std::min(num_reqs, std::max(1, kMaxCounters / std::max(H, 1)));
}

static int64_t dense_part_bytes(int H, int G, int nr, int max_seq_len, int block_size) {
  const int chunk = dense_chunk_for(nr, H, max_seq_len, block_size);
  const int max_chunks = std::max(1, (max_seq_len + chunk - 1) / chunk);
  return (int64_t)nr * H * max_chunks * G * (kD + 2) * 4;
}

int64_t dense_workspace_bytes(int H, int G, int num_reqs, int max_seq_len, int block_size) {
  if (num_reqs <= 0) return kCounterBytes;
  const int slice = dense_slice_reqs(H, num_reqs);
  return kCounterBytes +
         std::max(dense_part_bytes(H, G, slice, max_seq_len, block_size),
                  dense_part_bytes(H, G, (num_reqs - 1) % slice + 1, max_seq_len, block_size));
}

template <int G, int DT>
static int launch_dense_t(const DenseArgs& a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((dense_decode_kernel<G, DT>), dim3(grid), dim3(kDThreads), 0, st, a);
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
  if (dtype != TTKV_DTYPE_F16 && dtype != TTKV_DTYPE_BF16)
    return host_fail(TTKV_E_INVALID, "dense cache dtype must be fp16 or bf16");
  if (!q || !k_cache || !v_cache || !bt || !seq_lens || !qsl || !out)
    return host_fail(TTKV_E_INVALID, "null pointer argument");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || q_row_stride % 8)
    return host_fail(TTKV_E_INVALID, "q / caches must be 16-byte aligned");
  if (num_reqs == 0) return TTKV_OK;
  if ((int64_t)max_blocks * block_size < max_seq_len)
    return host_fail(TTKV_E_INVALID, "max_seq_len needs more blocks than the block table holds");
  DenseArgs a{};
  a.H = H;
  a.HQ = HQ;
  a.G = HQ / H;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.q = q;
  a.q_row_stride = q_row_stride;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.dtype = dtype;
  a.n_slots = n_slots;
  a.block_size = block_size;
  a.bt = bt;
  a.bt_row_stride = bt_row_stride;
  a.seq_lens = seq_lens;
  a.qsl = qsl;
  a.num_reqs = num_reqs;
  a.out = out;
  a.out_row_stride = out_row_stride;
  a.max_seq = max_seq_len;
  if (a.G < 1 || a.G > 4) return host_fail(TTKV_E_UNSUPPORTED, "G must be 1..4 for the dense comparator");
  if (H > kMaxCounters) return host_fail(TTKV_E_UNSUPPORTED, "H");
  const bool multi = dense_chunk_for(dense_slice_reqs(H, num_reqs), H, max_seq_len, block_size) <
                     max_seq_len;
  if (multi) {
    const int64_t need = dense_workspace_bytes(H, a.G, num_reqs, max_seq_len, block_size);
    if (!ws || ws_bytes < need || (uintptr_t)ws % 256)
      return host_fail(TTKV_E_WORKSPACE, "dense workspace needs " + std::to_string(need) +
                                             " bytes, 256-aligned");
  }
  const int slice = dense_slice_reqs(H, num_reqs);
  for (int r0 = 0; r0 < num_reqs; r0 += slice) {
    DenseArgs b = a;
    b.num_reqs = std::min(slice, num_reqs - r0);
    b.seq_lens = seq_lens + r0;
    b.qsl = qsl + r0;
    b.bt = bt + (int64_t)r0 * bt_row_stride;
    b.chunk = dense_chunk_for(b.num_reqs, H, max_seq_len, block_size);
    b.max_chunks = std::max(1, (max_seq_len + b.chunk - 1) / b.chunk);
    if (b.max_chunks > 1) {  // counters [r * H + h] <= kMaxCounters
      b.ws_cnt = (int*)ws;
      b.ws_part = (float*)((char*)ws + kCounterBytes);
    }
    b.nwork = b.num_reqs * b.max_chunks * H;
    const int grid = (b.nwork + 7) / 8 * 8;
    const bool f16 = dtype == TTKV_DTYPE_F16;
    int rc = TTKV_OK;
    switch (a.G) {
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

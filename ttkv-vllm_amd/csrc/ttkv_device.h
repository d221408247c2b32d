// Device helpers shared by the read kernels (K1 decode, K2 multi-query): exact int8 -> fp16
// conversion, the LUT-driven bitmap/code-stream decode of one packed head row, and cross-lane
// reductions on DPP and the gfx950 permlane swaps. Bit format: codec/ttkv_packed_cache.py:50-100,
// 138-167 (bitmap MSB-first per byte, lane order; codes MSB-first in lane order).
#pragma once

#include "ttkv_common.h"

namespace ttkv {

// int8 x4 (little-endian in a dword) -> two packed fp16 pairs, exact.
__device__ __forceinline__ void i8x4_to_f16(uint32_t x, uint32_t& p01, uint32_t& p23) {
  const uint32_t u = x ^ 0x80808080u;  // b + 128 as unsigned bytes
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  p01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, lo) - bias);
  p23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, hi) - bias);
}

// 4 code bytes (little-endian) -> two fp16 pairs holding code - off, exact.
__device__ __forceinline__ void u8x4_to_f16_minus(uint32_t x, float off, uint32_t& p01,
                                                  uint32_t& p23) {
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);  // 1024 + b0, 1024 + b1
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
  const _Float16 bias = (_Float16)(1024.0f + off);
  const half2v b2 = {bias, bias};
  p01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, lo) - b2);
  p23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, hi) - b2);
}

// Spread the 8 codes at the top of a 32-bit MSB-first window (code k at bits 31-B*k-B+1 ..
// 31-B*k) into bytes: e0 = codes 0..3, e1 = codes 4..7 (byte i of e0 = code i).
template <int BITS>
__device__ __forceinline__ void spread8(uint32_t w, uint32_t& e0, uint32_t& e1) {
  if constexpr (BITS == 4) {
    // nibbles: code k at bits 28-4k. bytes of (w >> 4) & 0x0f0f0f0f hold codes 6,4,2,0 at bytes
    // 0..3; bytes of w & 0x0f0f0f0f hold codes 7,5,3,1. Interleave with v_perm.
    const uint32_t ev = (w >> 4) & 0x0f0f0f0fu;  // byte0 = c6, byte1 = c4, byte2 = c2, byte3 = c0
    const uint32_t od = w & 0x0f0f0f0fu;         // byte0 = c7, byte1 = c5, byte2 = c3, byte3 = c1
    // e0 = [c0, c1, c2, c3]: c0 = ev.b3, c1 = od.b3, c2 = ev.b2, c3 = od.b2  (S0 = ev: 4-7, S1 = od)
    e0 = __builtin_amdgcn_perm(ev, od, 0x02060307u);
    // e1 = [c4, c5, c6, c7]: c4 = ev.b1, c5 = od.b1, c6 = ev.b0, c7 = od.b0
    e1 = __builtin_amdgcn_perm(ev, od, 0x00040105u);
  } else {
    e0 = __builtin_amdgcn_ubfe(w, 32 - BITS, BITS) |
         (__builtin_amdgcn_ubfe(w, 32 - 2 * BITS, BITS) << 8) |
         (__builtin_amdgcn_ubfe(w, 32 - 3 * BITS, BITS) << 16) |
         (__builtin_amdgcn_ubfe(w, 32 - 4 * BITS, BITS) << 24);
    e1 = __builtin_amdgcn_ubfe(w, 32 - 5 * BITS, BITS) |
         (__builtin_amdgcn_ubfe(w, 32 - 6 * BITS, BITS) << 8) |
         (__builtin_amdgcn_ubfe(w, 32 - 7 * BITS, BITS) << 16) |
         (__builtin_amdgcn_ubfe(w, 32 - 8 * BITS, BITS) << 24);
  }
}

// Wide fetch of the slot bytes one of a token's 4 loader threads needs for one KV head: 16-byte
// loads only (5 per thread instead of one per dword). Part p loads coefficient chunks p, p+4,
// p+8 (bytes 16c .. 16c+15 of the coefficient window: 16 ranks of int8, 8 of fp16 or 32 of 4-bit
// values per chunk; a chunk past the window is clamped to the window's last one and never
// committed), chunk p of the 64-byte-aligned windows holding this head's K row and V row (each
// row lies inside its window: misalignment + row length <= 64, checked by the host; a chunk past
// the blob is clamped inside it and covers no row byte), and the dword holding the coefficient
// ruler (int8 mode) or the scale of group p (4-bit mode; the fp16 mode has neither).
template <int KU, int CM = kCoefI8>
struct RawSlotW {
  // coefficient chunks of the 16*KU-rank window
  static constexpr int kCoefChunks = CM == kCoefI8 ? KU : CM == kCoefF16 ? 2 * KU : (KU + 1) / 2;
  static constexpr int kChunks = (kCoefChunks + 3) / 4;  // coefficient chunks per part
  u32x4 coef[kChunks];
  u32x4 krow, vrow;
  uint32_t rul;
};

template <int KU, int CM = kCoefI8>
__device__ __forceinline__ void fetch_raw_slot_w(RawSlotW<KU, CM>& P, const uint8_t* base,
                                                 int part, const Geom& g, int k_win, int v_win) {
  using R = RawSlotW<KU, CM>;
  if (!base) {
#pragma unroll
    for (int i = 0; i < R::kChunks; ++i) P.coef[i] = u32x4{0u, 0u, 0u, 0u};
    P.krow = P.vrow = u32x4{0u, 0u, 0u, 0u};
    P.rul = 0u;
    return;
  }
#pragma unroll
  for (int i = 0; i < R::kChunks; ++i)
    P.coef[i] = *gbl((const u32x4*)(base + 16 * min(part + 4 * i, R::kCoefChunks - 1)));
  P.krow = *gbl((const u32x4*)(base + min(k_win + 16 * part, g.blob - 16)));
  P.vrow = *gbl((const u32x4*)(base + min(v_win + 16 * part, g.blob - 16)));
  if constexpr (CM == kCoefI4G32)
    P.rul = *gbl((const uint32_t*)(base + ((g.coeff_bytes + 2 * min(part, g.coef_groups - 1)) & ~3)));
  else if constexpr (CM == kCoefI8)
    P.rul = *gbl((const uint32_t*)(base + (g.coeff_bytes & ~3)));
  else
    P.rul = 0u;
}

// Commit of one token's coefficients: this part's chunks become fp16 MFMA B values in the token's
// LDS row `crow` (one dword = two consecutive ranks, ranks 0 .. 16*KU-1), exactly. Returns the
// coefficient ruler the key is scaled by afterwards: the int8 mode's fp16 ruler, 1 for the fp16
// and 4-bit modes (their values are the coefficients themselves).
//  - int8: 16 ranks per chunk; bytes past r1 (the ruler, head 0's row) are finite int8 values
//    that meet zero decoder ranks, so they contribute exactly 0.
//  - fp16: 8 ranks per chunk, copied; ranks >= r1 (other fields' bytes, maybe not finite) are
//    zeroed.
//  - 4-bit: 32 ranks (one group) per chunk. Per word, each pair of ranks (2m, 2m+1) becomes
//    fp16 1024 + (q + 8) by one shift-and-or into the exponent of 1024, then (x - 1032) * scale,
//    both exact (|q| <= 8 and the scale's 8 significant bits need 11). Words past the values
//    (the scales, head 0's row) are taken as zero and groups past the last have scale 0.
template <int KU, int CM>
__device__ __forceinline__ float commit_coef(const RawSlotW<KU, CM>& P, uint32_t* crow, int part,
                                             const Geom& g) {
  using R = RawSlotW<KU, CM>;
  static_assert(CM != kCoefI4G32 || R::kChunks == 1, "4-bit mode: one group per loader part");
#pragma unroll
  for (int i = 0; i < R::kChunks; ++i) {
    const int cch = part + 4 * i;
    if (cch >= R::kCoefChunks) continue;
    if constexpr (CM == kCoefI8) {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) i8x4_to_f16(P.coef[i][j], h[2 * j], h[2 * j + 1]);
      *(u32x4*)&crow[8 * cch] = u32x4{h[0], h[1], h[2], h[3]};
      *(u32x4*)&crow[8 * cch + 4] = u32x4{h[4], h[5], h[6], h[7]};
    } else if constexpr (CM == kCoefF16) {
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 8 * cch + 2 * j;
        h[j] = P.coef[i][j] & ((r < g.r1 ? 0x0000ffffu : 0u) | (r + 1 < g.r1 ? 0xffff0000u : 0u));
      }
      *(u32x4*)&crow[4 * cch] = u32x4{h[0], h[1], h[2], h[3]};
    } else {
      const uint32_t sb = (g.coeff_bytes + 2 * part) & 2 ? P.rul >> 16 : P.rul & 0xffffu;
      const _Float16 sc = part < g.coef_groups ? __builtin_bit_cast(_Float16, (uint16_t)sb)
                                               : (_Float16)0.0f;
      const half2v s2 = {sc, sc};
      const half2v bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if (32 * cch + 8 * w >= 16 * KU) continue;  // past the window (KU odd)
        const uint32_t x = (16 * cch + 4 * w < g.coeff_bytes ? P.coef[i][w] : 0u) ^ 0x88888888u;
        uint32_t o[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const half2v v = __builtin_bit_cast(half2v, ((x >> (4 * m)) & 0x000f000fu) | 0x64006400u);
          o[m] = __builtin_bit_cast(uint32_t, (v - bias) * s2);
        }
        *(u32x4*)&crow[16 * cch + 4 * w] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
  if constexpr (CM == kCoefI8)
    return f16_bits_to_float((g.coeff_bytes & 2) ? P.rul >> 16 : P.rul & 0xffffu);
  else
    return 1.f;
}

// Stage dwords 4*part .. 4*part+3 of a head row for the decode (the big-endian staged layout
// below): this thread holds chunk `part` of the row's 64-byte window, the quad neighbour (lane
// + 1) chunk part + 1, fetched with one DPP move per dword. `m4`/`sel`: the row's misalignment in
// the window in dwords (wave-uniform) and the v_perm selector for its byte part and this part's
// byte reversal (stage_selector). Part 3's neighbour is itself: those staged bytes lie past the
// row and are never decoded.
__device__ __forceinline__ void stage_row_w(const u32x4& mine, int m4, uint32_t sel, uint32_t* dst) {
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[i] = mine[i];
    // quad_perm [1, 2, 3, 3]: each lane reads lane + 1 of its quad
    w[4 + i] = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine[i], 0xF9, 0xF, 0xF, false);
  }
  switch (m4) {  // wave-uniform
#define TTKV_STAGE_CASE(M)                                                          \
  case M:                                                                           \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) dst[i] =                          \
        __builtin_amdgcn_perm(w[(M) + i + 1], w[(M) + i], sel);                     \
    break;
    TTKV_STAGE_CASE(0)
    TTKV_STAGE_CASE(1)
    TTKV_STAGE_CASE(2)
    default:
      TTKV_STAGE_CASE(3)
#undef TTKV_STAGE_CASE
  }
}

// 2^x on the hardware exp unit (one v_exp_f32). Softmax weights below 2^-126 flush to zero,
// which is far below fp32 resolution of the sums they join; -inf gives 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) in one v_max3_f32. fmaxf chains compile to v_max with every operand first
// quieted (v_max_f32 x, x, x) because the compiler cannot rule out signalling NaNs; MFMA results
// are never signalling NaNs, so the callers skip that.
__device__ __forceinline__ float max3_mfma(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Cross-lane helpers on DPP and the gfx950 permlane swaps (VALU ops, no LDS round trip).
__device__ __forceinline__ int dpp_i(int iv, int ctrl_sel) {
  switch (ctrl_sel) {  // dpp control must be a constant
    case 0: return __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false);   // xor 1
    case 1: return __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false);   // xor 2
    case 2: return __builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, false);  // row_ror 4
    default: return __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false); // row_ror 8
  }
}
__device__ __forceinline__ float dpp_f(float v, int ctrl_sel) {
  return __builtin_bit_cast(float, dpp_i(__builtin_bit_cast(int, v), ctrl_sel));
}
// Integer sum / max over the whole wave, returned as a wave-uniform (scalar) value; all lanes
// must be active.
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i(v, 0);
  v += dpp_i(v, 1);
  v += dpp_i(v, 2);
  v += dpp_i(v, 3);
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = (int)r[0] + (int)r[1];
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_amdgcn_readfirstlane((int)r[0] + (int)r[1]);
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i(v, 0));
  v = max(v, dpp_i(v, 1));
  v = max(v, dpp_i(v, 2));
  v = max(v, dpp_i(v, 3));
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((int)r[0], (int)r[1]);
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_amdgcn_readfirstlane(max((int)r[0], (int)r[1]));
}
// Sum / max over the 16 lanes of each row (every lane gets its row's result).
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f(v, 0);
  v += dpp_f(v, 1);
  v += dpp_f(v, 2);
  v += dpp_f(v, 3);
  return v;
}
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, dpp_f(v, 0));
  v = fmaxf(v, dpp_f(v, 1));
  v = fmaxf(v, dpp_f(v, 2));
  v = fmaxf(v, dpp_f(v, 3));
  return v;
}
// Lanes l and l^16 / l^32 exchanged: returns (value of rows {0,2}, value of rows {1,3}) etc.
__device__ __forceinline__ void swap16(float v, float& a, float& b) {
  const int iv = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
  a = __builtin_bit_cast(float, (int)r[0]);  // rows [0,0,2,2]
  b = __builtin_bit_cast(float, (int)r[1]);  // rows [1,1,3,3]
}
__device__ __forceinline__ void swap32(float v, float& a, float& b) {
  const int iv = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
  a = __builtin_bit_cast(float, (int)r[0]);  // halves [lo, lo]
  b = __builtin_bit_cast(float, (int)r[1]);  // halves [hi, hi]
}
// Sum over lanes {l, l^16, l^32, l^48} (the four rows at the same row position).
__device__ __forceinline__ float cross_row_sum(float v) {
  float a, b;
  swap16(v, a, b);
  v = a + b;
  swap32(v, a, b);
  return a + b;
}
__device__ __forceinline__ float cross_row_max(float v) {
  float a, b;
  swap16(v, a, b);
  v = fmaxf(a, b);
  swap32(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float wave_max(float v) { return cross_row_max(row_max(v)); }
__device__ __forceinline__ float wave_sum(float v) { return cross_row_sum(row_sum(v)); }
// Broadcast row `nb` (lanes 16nb..16nb+15) of v to all four rows: out[nb].
__device__ __forceinline__ void bcast_rows(float v, float out[4]) {
  float r02, r13, a, b;
  swap16(v, r02, r13);      // r02 = rows [0,0,2,2], r13 = rows [1,1,3,3]
  swap32(r02, a, b);        // a = [r0 x4], b = [r2 x4]
  out[0] = a;
  out[2] = b;
  swap32(r13, a, b);        // a = [r1 x4], b = [r3 x4]
  out[1] = a;
  out[3] = b;
}


// y - h for h the low / high fp16 half of a packed pair, in one v_fma_mix_f32 (the fp16 operand is
// widened exactly; the difference of a value and its fp16 truncation is exact in fp32).
__device__ __forceinline__ float minus_lo16(float y, half2v h) {
  float r;
  __asm__("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(y));
  return r;
}
__device__ __forceinline__ float minus_hi16(float y, half2v h) {
  float r;
  __asm__("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
          : "=v"(r)
          : "v"(h), "v"(y));
  return r;
}

// hi + lo fp16 split of 8 fp32 values (22 significant bits): hi truncated, lo the exact
// remainder rounded toward zero.
__device__ __forceinline__ void split8(const float y[8], half8& hi, half8& lo) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(y[i], y[i + 1]);
    const half2v hh = {(_Float16)h[0], (_Float16)h[1]};
    const auto l = __builtin_amdgcn_cvt_pkrtz(minus_lo16(y[i], hh), minus_hi16(y[i + 1], hh));
    hi[i] = hh[0];
    hi[i + 1] = hh[1];
    lo[i] = (_Float16)l[0];
    lo[i + 1] = (_Float16)l[1];
  }
}

// ------------------------------------------------------------------ big-endian staged rows
// The read kernels stage a head row in LDS as dwords 0..3 = bitmap (as stored) and dwords 4.. =
// code stream with each dword byte-reversed, so that the MSB-first stream reads as big-endian
// words: stream bit b is bit 31 - (b & 31) of word b >> 5. One v_perm per dword does the
// realignment (the row starts at any byte) and the reversal together.
//
// v_perm_b32(S0, S1, sel): byte k of the result is byte sel.k of the 8 bytes {S1 (0..3), S0
// (4..7)}; selector 0x0c gives 0x00.
__device__ __forceinline__ uint32_t stage_selector(int sh, bool reverse) {
  const uint32_t s = (uint32_t)sh;
  return reverse ? ((s + 3u) | ((s + 2u) << 8) | ((s + 1u) << 16) | (s << 24))
                 : (s | ((s + 1u) << 8) | ((s + 2u) << 16) | ((s + 3u) << 24));
}

// The 16-bit ruler at row byte `rb` (little-endian), read back from a staged row whose bytes
// from 16 on are reversed within their dwords.
__device__ __forceinline__ uint32_t staged_u16(const uint32_t* row, int rb) {
  const uint32_t lo = (row[rb >> 2] >> (8 * (3 - (rb & 3)))) & 0xffu;
  const int rb1 = rb + 1;
  const uint32_t hi = (row[rb1 >> 2] >> (8 * (3 - (rb1 & 3)))) & 0xffu;
  return lo | (hi << 8);
}

// Codes are handed to the arithmetic as fp8 (e4m3) bytes holding the signed value c - 2^(b-1)
// in sign-magnitude: magnitude k <= 15 is byte k in both e4m3 variants (k * 2^-9 in OCP e4m3,
// k * 2^-10 in the FNUZ one; the kernels read the unit back from the hardware conversion).
// Lanes outside the bitmap get byte 0 (+0), i.e. residual 0, with no fix-up pass.

// The decode tables, built in LDS by the workgroup itself (a few hundred VALU operations per
// thread, no memory traffic at kernel start):
//   lut3[x]  (3-bit codes): x = 6 bits holding 2 codes, the first in the top 3 bits -> the 2
//            codes as fp8 signed bytes (c - 4), first code in the low byte. The byte map
//            c -> fp8(c - 4) is one v_perm over the 8-byte table {84 83 82 81 00 01 02 03}. The
//            64 entries fill 32 dwords, one per bank, so any gather by a wave is conflict-free
//            (a 4096-entry table of 4-code entries takes half the lookups but ~4x the bank
//            passes per lookup, and 16 KB of LDS).
//   lut[B]   selectors that move the byte-spread codes of bitmap byte B (MSB = first lane) onto its
//            set lanes: lane k gets the rank of its bit among B's set bits, 0x0c (zero) if unset.
constexpr int kLut3Entries = 64;
__device__ __forceinline__ uint16_t lut3_entry(uint32_t x) {
  const uint32_t c = (x >> 3) | ((x & 7u) << 8);
  return (uint16_t)__builtin_amdgcn_perm(0x03020100u, 0x81828384u, c);
}
__device__ __forceinline__ uint2 scatter_entry(uint32_t B) {
  uint32_t s0 = 0, s1 = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t present = (B >> (7 - k)) & 1u;
    const uint32_t idx = __builtin_popcount(B >> (8 - k));  // set bits before lane k
    const uint32_t sel = present ? idx : 0x0cu;
    if (k < 4) s0 |= sel << (8 * k);
    else s1 |= sel << (8 * (k - 4));
  }
  return make_uint2(s0, s1);
}
__device__ __forceinline__ void build_luts(uint2* lut, uint16_t* lut3, int tid, int nthreads) {
  for (int i = tid; i < 256; i += nthreads) lut[i] = scatter_entry((uint32_t)i);
  if (lut3)
    for (int i = tid; i < kLut3Entries; i += nthreads) lut3[i] = lut3_entry((uint32_t)i);
}

// Decode the 32 lanes of bitmap dword `bm` of one big-endian staged head row (code stream at
// `st`, this dword's first code at rank `rank`, advanced past it) into one byte per lane at
// dst[0..31].
//   BITS == 3: fp8 signed bytes (c - 4), 0 outside the bitmap; needs lut3 (build_luts).
//   BITS == 4: offset-binary code bytes c, 8 outside the bitmap.
// Per bitmap byte: the code window at bit offset bp is one v_alignbit of the words holding bits
// bp-1 and bp+31 (shift (-bp) mod 32; word -1 is the last bitmap dword, read but unused).
template <int BITS>
__device__ __forceinline__ void decode_dword_be(const uint32_t* st, uint32_t bm, int& rank,
                                                const uint2* lut, const uint16_t* lut3,
                                                uint8_t* dst) {
  uint32_t B[4];
  int bp[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    B[m] = __builtin_amdgcn_ubfe(bm, 8 * m, 8);
    bp[m] = rank * BITS;
    rank += __builtin_popcount(B[m]);
  }
  uint2 sel[4];
  uint32_t w[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    sel[m] = lut[B[m]];
    const uint32_t* wp = st + ((bp[m] - 1) >> 5);
    w[m] = __builtin_amdgcn_alignbit(wp[0], wp[1], (uint32_t)(-bp[m]));
  }
  uint32_t e0[4], e1[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if constexpr (BITS == 3) {
      e0[m] = (uint32_t)lut3[w[m] >> 26] | ((uint32_t)lut3[(w[m] >> 20) & 63u] << 16);
      e1[m] = (uint32_t)lut3[(w[m] >> 14) & 63u] | ((uint32_t)lut3[(w[m] >> 8) & 63u] << 16);
    } else {
      spread8<4>(w[m] ^ 0x88888888u, e0[m], e1[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint2 out;
    out.x = __builtin_amdgcn_perm(e1[m], e0[m], sel[m].x);
    out.y = __builtin_amdgcn_perm(e1[m], e0[m], sel[m].y);
    if constexpr (BITS == 4) {
      out.x ^= 0x08080808u;
      out.y ^= 0x08080808u;
    }
    *(uint2*)(dst + 8 * m) = out;
  }
}

// Decode dims [64*half, 64*half+64) of one big-endian staged head row (dwords 0..3 the bitmap,
// dwords 4.. the code stream) into one byte per lane at dst[0..63].
template <int BITS>
__device__ __forceinline__ void decode_half_row_be(const uint32_t* row, int half, const uint2* lut,
                                                   const uint16_t* lut3, uint8_t* dst) {
  const uint32_t bm0 = row[2 * half], bm1 = row[2 * half + 1];
  int rank = half ? __builtin_popcount(row[0]) + __builtin_popcount(row[1]) : 0;
  decode_dword_be<BITS>(row + 4, bm0, rank, lut, lut3, dst);
  decode_dword_be<BITS>(row + 4, bm1, rank, lut, lut3, dst + 32);
}

// Decode dims [32*qr, 32*qr+32) of one staged head row into dst[0..31] (four threads per row).
template <int BITS>
__device__ __forceinline__ void decode_quarter_row_be(const uint32_t* row, int qr,
                                                      const uint2* lut, const uint16_t* lut3,
                                                      uint8_t* dst) {
  int rank = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) rank += i < qr ? __builtin_popcount(row[i]) : 0;
  decode_dword_be<BITS>(row + 4, row[qr], rank, lut, lut3, dst);
}

// Four decoded code bytes -> floats. BITS == 3: fp8 signed bytes -> (c - 4) * unit, two per
// v_cvt_pk_f32_fp8. BITS == 4: offset-binary bytes -> c (the caller removes the offset).
template <int BITS>
__device__ __forceinline__ void codes4(uint32_t x, float v[4]) {
  if constexpr (BITS == 3) {
    const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)x, false);
    const auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)x, true);
    v[0] = a[0];
    v[1] = a[1];
    v[2] = b[0];
    v[3] = b[1];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((x >> (8 * i)) & 0xffu);
  }
}

}  // namespace ttkv

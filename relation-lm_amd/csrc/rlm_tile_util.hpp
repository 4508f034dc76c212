// Helpers of the matrix-core-filtered selection kernels (rlm_select_tile.hip,
// rlm_multi_tile.hip): bf16 MFMA candidate scores, the fp32 -> bf16 hi/lo
// split of a query, statistics loads, wave maxima and member numbering.
#pragma once

#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef double f64x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Bound of |s~ - s| for the bf16 MFMA scores: eps = kErrScale * ||q||_1 * max|k|
// (+ kErrAbs for products that underflow fp32).
constexpr float kErrScale = 1.220703125e-4f;          // 2^-13
constexpr float kErrAbs = 7.888609052210118e-31f;     // 2^-100

__device__ __forceinline__ int clamp_pos(int64_t v) {
  constexpr int64_t kLim = int64_t(1) << 30;
  return static_cast<int>(v < -kLim ? -kLim : (v > kLim ? kLim : v));
}

// Max |x| bits of eight bf16 values (two per 32-bit word), packed 16-bit max.
__device__ __forceinline__ u16x2_t absmax8(const uint4& v, u16x2_t m) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, w[i] & 0x7fff7fffu));
  return m;
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Wave-wide maxima (every lane gets the result).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = umax32(v, dpp_u32<kDppXor1>(v));
  v = umax32(v, dpp_u32<kDppXor2>(v));
  v = umax32(v, dpp_u32<kDppHalfMirror>(v));
  v = umax32(v, dpp_u32<kDppMirror>(v));
  uint32_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    best = umax32(best, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16 * r)));
  return best;
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, static_cast<int>(dpp_u32<kDppXor1>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u32<kDppXor2>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u32<kDppHalfMirror>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int>(dpp_u32<kDppMirror>(static_cast<uint32_t>(v))));
  int best = __builtin_amdgcn_readlane(v, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) best = max(best, __builtin_amdgcn_readlane(v, 16 * r));
  return best;
}
__device__ __forceinline__ double group_max_f64(double v, int G) {
  if (G >= 2) v = fmax(v, dpp_f64<kDppXor1>(v));
  if (G >= 4) v = fmax(v, dpp_f64<kDppXor2>(v));
  if (G >= 8) v = fmax(v, dpp_f64<kDppHalfMirror>(v));
  if (G >= 16) v = fmax(v, dpp_f64<kDppMirror>(v));
  return v;
}

__device__ __forceinline__ f32x4_t mfma_bf16(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Eight fp32 -> bf16 hi (round to nearest even) and bf16 lo = bf16(x - hi).
__device__ __forceinline__ void split_hi_lo(const float (&x)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    const float h0 = __uint_as_float(h[i] << 16);
    const float h1 = __uint_as_float(h[i] & 0xffff0000u);
    l[i] = pack_bf16x2(x[2 * i] - h0, x[2 * i + 1] - h1);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

template <typename TS>
__device__ __forceinline__ void load_stat8(const TS* src, float (&out)[8]);
template <>
__device__ __forceinline__ void load_stat8<float>(const float* src, float (&out)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(src);
  const float4 c = *reinterpret_cast<const float4*>(src + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
}
template <>
__device__ __forceinline__ void load_stat8<bf16>(const bf16* src, float (&out)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(src);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// Member indices of the candidates flagged in `mask` (bit i: candidate
// lane + 64 i), numbered candidate slot by slot; returns the member count.
template <int NCL>
__device__ __forceinline__ int number_members(uint32_t mask, int (&mi)[NCL]) {
  int base = 0;
#pragma unroll
  for (int i = 0; i < NCL; ++i) {
    const uint64_t bal = __builtin_amdgcn_ballot_w64((mask >> i) & 1u);
    mi[i] = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                       static_cast<uint32_t>(bal >> 32),
                       __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
    base += __builtin_popcountll(bal);
  }
  return base;
}

}  // namespace
}  // namespace rlm

// Shared device helpers and host-side argument validation for the gfx950
// routed relation path.  Everything here is CDNA4-specific: wave64, LDS
// ordering within a wave, bf16 as raw 16-bit storage.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "relation_lm_hip.h"

namespace rlm {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element types
// ---------------------------------------------------------------------------

struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16 v) { return static_cast<float>(v); }

// Two floats -> two bf16 (lo in bits 0..15), round-to-nearest-even, in one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Round-to-nearest-even float -> bf16.
__device__ __forceinline__ bf16 f32_to_bf16(float f) {
  bf16 out;
  out.bits = static_cast<uint16_t>(pack_bf16x2(f, 0.0f));
  return out;
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return f32_to_bf16(v); }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) { return static_cast<f16>(v); }

// The two bf16 halves of a 32-bit word as floats.
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Four consecutive outputs of one row, converted to TO and written with one
// store (16 bytes for fp32, 8 bytes for 16-bit types).
template <typename TO>
__device__ __forceinline__ void put4(TO* dst, float v0, float v1, float v2, float v3) {
  if constexpr (sizeof(TO) == 4) {
    *reinterpret_cast<float4*>(dst) = make_float4(v0, v1, v2, v3);
  } else if constexpr (__is_same(TO, bf16)) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
  } else {
    const f16 h[4] = {static_cast<f16>(v0), static_cast<f16>(v1), static_cast<f16>(v2),
                      static_cast<f16>(v3)};
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h[0])) |
                       (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h[1])) << 16),
                   static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h[2])) |
                       (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h[3])) << 16));
  }
}

// Four consecutive elements starting at p (p aligned to 4 elements).
__device__ __forceinline__ float4 load4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ float4 load4(const bf16* p) {
  uint2 raw = *reinterpret_cast<const uint2*>(p);
  return make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                     __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
}
__device__ __forceinline__ float4 load4(const f16* p) {
  const f16* q = p;
  return make_float4(static_cast<float>(q[0]), static_cast<float>(q[1]),
                     static_cast<float>(q[2]), static_cast<float>(q[3]));
}

// Scalar element of a runtime-typed tensor (small parameter tensors only).
__device__ __forceinline__ float load_any_f(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case RLM_BF16:
      return to_f32(static_cast<const bf16*>(p)[i]);
    case RLM_F16:
      return to_f32(static_cast<const f16*>(p)[i]);
    default:
      return static_cast<const float*>(p)[i];
  }
}
__device__ __forceinline__ int64_t load_any_i(const void* p, int dtype, int64_t i) {
  return dtype == RLM_I64 ? static_cast<const int64_t*>(p)[i]
                          : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

// ---------------------------------------------------------------------------
// Range-checked buffer access
// ---------------------------------------------------------------------------
//
// Raw buffer loads/stores through a resource descriptor whose size is the
// tensor's byte size: an access past the end reads zero / is dropped by the
// hardware, so a gather with an invalid index needs no branch -- its offset is
// set to kNoOffset.  Every buffer addressed this way is smaller than 2 GiB
// (checked on the host), so kNoOffset plus any in-row offset stays past it.

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kNoOffset = 0x80000000u;
constexpr int kRawBufferWord3 = 0x00020000;  // gfx9 family: raw (untyped) buffer

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           kRawBufferWord3);
}
__device__ __forceinline__ uint4 buf_load_b128(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint2 buf_load_b64(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load_b32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint16_t buf_load_b16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ void buf_store_f32(float v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
}
// 16 bytes per lane from global memory straight into LDS: lane i's bytes land
// at lds_addr + 16*i (lds_addr wave-uniform, an LDS byte address).  Issued as
// inline assembly so that the compiler does not follow it with a full
// vmcnt(0) before the next LDS access; the caller waits (s_waitcnt vmcnt +
// barrier) before the data is read.  The LDS base travels in M0, passed as an
// operand bound to that register ("{m0}"), so the compiler writes M0 itself
// and knows it holds this value.
__device__ __forceinline__ void lds_dma16(rsrc_t r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(r), "{m0}"(lds_addr)
               : "memory");
}
// The same with a wave-uniform byte offset added to every lane's (soff, an SGPR).
__device__ __forceinline__ void lds_dma16(rsrc_t r, uint32_t lds_addr, uint32_t voff,
                                          uint32_t soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "{m0}"(lds_addr)
               : "memory");
}
// s_waitcnt immediate that waits until at most n vector-memory operations of
// this wave are outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14),
// leaving the export and LDS counters untouched.
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// A wave-uniform condition that the compiler must treat as lane-varying.
// Selects on a uniform condition may be turned into a branch with the loads
// that feed one side sunk into it (each branch join then waits for its
// load); on a lane-varying condition they stay v_cndmask.  Costs one v_mov.
__device__ __forceinline__ bool varying(bool c) {
  uint32_t z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return c != (z != 0u);
}

// Branch-free loads of one int32 / int64 index (low word always, high word only
// for int64: the other load gets an out-of-range offset and reads 0) and of one
// fp32 / bf16 / fp16 element (a 4-byte and a 2-byte load, the one that does not
// match the dtype out of range).  Issued early and decoded after the round
// trip, so no load waits at a dtype branch.
struct IndexWords {
  uint32_t lo, hi;
};
__device__ __forceinline__ IndexWords issue_index(const void* base, int dtype, uint32_t count,
                                                  uint32_t i, bool valid) {
  const bool is64 = dtype == RLM_I64;
  const rsrc_t r = make_rsrc(base, count * (is64 ? 8u : 4u));
  return {buf_load_b32(r, valid ? i * (is64 ? 8u : 4u) : kNoOffset),
          buf_load_b32(r, valid && is64 ? 8u * i + 4u : kNoOffset)};
}
__device__ __forceinline__ int64_t decode_index(IndexWords w, int dtype) {
  return dtype == RLM_I64
             ? static_cast<int64_t>((static_cast<uint64_t>(w.hi) << 32) | w.lo)
             : static_cast<int64_t>(static_cast<int32_t>(w.lo));
}
struct FloatWords {
  uint32_t w32;  // fp32 element (0 for 16-bit dtypes)
  uint32_t w16;  // 16-bit element (0 for fp32)
};
__device__ __forceinline__ FloatWords issue_float(const void* base, int dtype, uint32_t count,
                                                  uint32_t i, bool valid) {
  const bool is32 = dtype == RLM_F32;
  const rsrc_t r = make_rsrc(base, count * (is32 ? 4u : 2u));
  return {buf_load_b32(r, valid && is32 ? 4u * i : kNoOffset),
          static_cast<uint32_t>(buf_load_b16(r, valid && !is32 ? 2u * i : kNoOffset))};
}
__device__ __forceinline__ float decode_float(FloatWords w, int dtype) {
  const float fh = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w.w16)));
  return dtype == RLM_F32 ? __uint_as_float(w.w32)
                          : (dtype == RLM_BF16 ? __uint_as_float(w.w16 << 16) : fh);
}

// Unconditional (branch-free) loads of one int32/int64 index and of four
// consecutive fp32/bf16/fp16 elements: both dtype interpretations are read
// from in-bounds addresses (the unused one from element 0) and the result is
// selected, so no load waits at a dtype branch.  `f4_issue` needs >= 4 elements.
__device__ __forceinline__ int64_t index_at(const void* base, int dtype, int64_t i) {
  const uint32_t* w = static_cast<const uint32_t*>(base);
  const bool is64 = varying(dtype == RLM_I64);
  const uint32_t lo = w[is64 ? 2 * i : i];
  const uint32_t hi = w[is64 ? 2 * i + 1 : i];
  // int32: the high word is lo's sign; one expression for both dtypes.
  const uint32_t top = is64 ? hi : static_cast<uint32_t>(static_cast<int32_t>(lo) >> 31);
  return static_cast<int64_t>((static_cast<uint64_t>(top) << 32) | lo);
}
struct F4Words {
  uint2 a, b;  // fp32 reading (16 bytes)
  uint2 h;     // 16-bit reading (8 bytes)
};
__device__ __forceinline__ F4Words f4_issue(const void* base, int dtype, int64_t i4) {
  const bool is32 = varying(dtype == RLM_F32);
  const uint2* w = static_cast<const uint2*>(base);
  return {w[is32 ? 2 * i4 : 0], w[is32 ? 2 * i4 + 1 : 0], w[is32 ? 0 : i4]};
}
__device__ __forceinline__ float4 f4_decode(const F4Words& v, int dtype) {
  // Both interpretations computed, one selected per element (selects, not
  // branches, so the loads stay where they are issued).
  const bool is32 = varying(dtype == RLM_F32);
  const bool isbf = varying(dtype == RLM_BF16);
  const uint32_t w32[4] = {v.a.x, v.a.y, v.b.x, v.b.y};
  const uint32_t e[4] = {v.h.x & 0xffffu, v.h.x >> 16, v.h.y & 0xffffu, v.h.y >> 16};
  float f[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float fb = __uint_as_float(e[k] << 16);
    const float fh = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(e[k])));
    f[k] = is32 ? __uint_as_float(w32[k]) : (isbf ? fb : fh);
  }
  return make_float4(f[0], f[1], f[2], f[3]);
}

// One element of type T at byte offset `off`, as float.
template <typename T>
__device__ __forceinline__ float buf_load_elem(rsrc_t r, uint32_t off);
template <>
__device__ __forceinline__ float buf_load_elem<float>(rsrc_t r, uint32_t off) {
  return __uint_as_float(buf_load_b32(r, off));
}
template <>
__device__ __forceinline__ float buf_load_elem<bf16>(rsrc_t r, uint32_t off) {
  return __uint_as_float(static_cast<uint32_t>(buf_load_b16(r, off)) << 16);
}
template <>
__device__ __forceinline__ float buf_load_elem<f16>(rsrc_t r, uint32_t off) {
  return static_cast<float>(__builtin_bit_cast(f16, buf_load_b16(r, off)));
}

// ---------------------------------------------------------------------------
// Elementwise math
// ---------------------------------------------------------------------------

// Exact (erf) GELU, x * Phi(x) (relation_reduce.py:139), with erf by
// Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26
// (1 - erf(z) = t (a1 + a2 t + ... + a5 t^4) exp(-z^2), t = 1/(1 + p z), z >= 0,
// |error| <= 1.5e-7), constants folded: for a = |x|,
//   h = Phi(-a) = 0.5 * (1 - erf(a/sqrt2)) = t * poly(t) * exp(-x^2/2),
//   t = 1/(1 + p a/sqrt2), poly with the A&S coefficients halved,
// and GELU(x) = x h for x < 0, x - x h for x >= 0, i.e. max(x, 0) - a h: one
// fused multiply-add.  Forming a h directly keeps the relative accuracy of the
// negative tail (no 1 + erf cancellation).  10 VALU operations plus one v_rcp
// and one v_exp.
__device__ __forceinline__ float gelu_erf(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752440f, a, 1.0f));
  float y = fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
  y = fmaf(y, t, 0.5f * 1.421413741f);
  y = fmaf(y, t, 0.5f * -0.284496736f);
  y = fmaf(y, t, 0.5f * 0.254829592f);
  y *= t;
  const float e = __builtin_amdgcn_exp2f(x * (x * (-0.5f * 1.44269504088896340736f)));
  // max(x, 0) on the bit pattern: one integer max, where fmaxf would first
  // quiet a possible signalling NaN (x is usually a matrix-core result).
  return fmaf(-a, y * e, __int_as_float(max(__float_as_int(x), 0)));
}

// Renumbers workgroup `i` of `count` so that each XCD (the hardware deals
// workgroups round-robin over 8 XCDs) receives a contiguous range of logical
// tile ids, so that workgroups with neighbouring logical ids share one L2.
__device__ __forceinline__ int64_t xcd_tile(int64_t i, int64_t count) {
  constexpr int kXcd = 8;
  const int64_t per = count / kXcd, rem = count % kXcd;
  const int64_t x = i % kXcd;
  return x * per + (x < rem ? x : rem) + i / kXcd;
}

// ---------------------------------------------------------------------------
// Wave-level primitives (wave64)
// ---------------------------------------------------------------------------

// Orders LDS traffic between lanes of one wave: a wave's LDS operations are
// executed in issue order, so only compiler reordering has to be fenced.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP lane exchanges within a row of 16 lanes (no LDS traffic):
//   quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2),
//   row_half_mirror (lane i <-> 7 - i within 8), row_mirror (i <-> 15 - i).
// After the two quad steps every lane of a quad holds the same value, so the
// mirrors pair each quad (or half row) with its neighbour, which is all a
// commutative reduction needs.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(u));
  const uint64_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(u >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t u) {
  const uint64_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(u));
  const uint64_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(u >> 32));
  return lo | (hi << 32);
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64);
// every lane of a group ends with the same bits.
__device__ __forceinline__ double group_sum_f64(double v, int G) {
  if (G >= 2) v += dpp_f64<kDppXor1>(v);
  if (G >= 4) v += dpp_f64<kDppXor2>(v);
  if (G >= 8) v += dpp_f64<kDppHalfMirror>(v);
  if (G >= 16) v += dpp_f64<kDppMirror>(v);
  if (G >= 32) v += __shfl_xor(v, 16, kWave);
  if (G >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// Maximum over the wave, returned in every lane (rows reduced with DPP, the
// four row maxima combined through readlane).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint64_t o = dpp_u64<kDppXor1>(v);
  v = v > o ? v : o;
  o = dpp_u64<kDppXor2>(v);
  v = v > o ? v : o;
  o = dpp_u64<kDppHalfMirror>(v);
  v = v > o ? v : o;
  o = dpp_u64<kDppMirror>(v);
  v = v > o ? v : o;
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v), 16 * r);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), 16 * r);
    const uint64_t x = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
    best = x > best ? x : best;
  }
  return best;
}

// Maximum over the wave held in every lane, all in VALU: DPP steps within the
// 16-lane rows, then v_permlane16/32_swap between rows (no SGPR round trips).
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t wave_max_u64_v(uint64_t v) {
  v = umax64(v, dpp_u64<kDppXor1>(v));
  v = umax64(v, dpp_u64<kDppXor2>(v));
  v = umax64(v, dpp_u64<kDppHalfMirror>(v));
  v = umax64(v, dpp_u64<kDppMirror>(v));
  auto lo = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v),
                                             false, false);
  auto hi = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v >> 32),
                                             static_cast<uint32_t>(v >> 32), false, false);
  v = umax64(static_cast<uint64_t>(lo[0]) | (static_cast<uint64_t>(hi[0]) << 32),
             static_cast<uint64_t>(lo[1]) | (static_cast<uint64_t>(hi[1]) << 32));
  lo = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false,
                                        false);
  hi = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v >> 32),
                                        static_cast<uint32_t>(v >> 32), false, false);
  return umax64(static_cast<uint64_t>(lo[0]) | (static_cast<uint64_t>(hi[0]) << 32),
                static_cast<uint64_t>(lo[1]) | (static_cast<uint64_t>(hi[1]) << 32));
}

__device__ __forceinline__ uint32_t wave_max_u32_v(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppMirror>(v));
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r[0], r[1]);
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(r[0], r[1]);
}

// Maximum 64-bit selection key over the wave, returned in every lane: the
// score half first (32-bit steps), then -- only when several lanes share the
// top score -- the tie half among those lanes.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
  const uint32_t hi = static_cast<uint32_t>(v >> 32);
  const uint32_t lo = static_cast<uint32_t>(v);
  const uint32_t mhi = wave_max_u32_v(hi);
  const uint64_t tied = __builtin_amdgcn_ballot_w64(hi == mhi);
  uint32_t mlo;
  if (__builtin_popcountll(tied) == 1)
    mlo = static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(lo), static_cast<int>(__builtin_ctzll(tied))));
  else
    mlo = wave_max_u32_v(hi == mhi ? lo : 0u);
  return (static_cast<uint64_t>(mhi) << 32) | mlo;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the same bits
// (each step adds a pair in both orders, and float addition commutes).
__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v)));
  return v;
}

// Sum of the neighbouring 16-lane rows (0,1) and (2,3), then of the two
// 32-lane halves: v_permlane16/32_swap exchange whole rows in VALU.
__device__ __forceinline__ float swap16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Wave64 sum / max with DPP row steps and two row swaps (no LDS round trips);
// every lane gets the same bits.
__device__ __forceinline__ float wave_sum_f32(float v) {
  return swap32_sum(swap16_sum(row16_sum(v)));
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v))));
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Order-preserving map float -> uint32 (+0.0 and -0.0 map to the same key,
// so they tie as they do under float comparison).
__device__ __forceinline__ uint32_t ordered_key(float f) {
  const uint32_t u = (f == 0.0f) ? 0u : __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
// 64-bit selection key: larger score first, then the smaller tie index.
__device__ __forceinline__ uint64_t select_key(float score, uint32_t tie_index) {
  return (static_cast<uint64_t>(ordered_key(score)) << 32) |
         static_cast<uint64_t>(0xffffffffu - tie_index);
}
__device__ __forceinline__ uint32_t key_index(uint64_t key) {
  return 0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu);
}
__device__ __forceinline__ float key_score(uint64_t key) {
  return key_to_float(static_cast<uint32_t>(key >> 32));
}

// ---------------------------------------------------------------------------
// Host-side validation
// ---------------------------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

inline bool is_float_dtype(int d) { return d == RLM_F32 || d == RLM_BF16 || d == RLM_F16; }
inline bool is_index_dtype(int d) { return d == RLM_I32 || d == RLM_I64; }
const char* dtype_name(int d);
// Bytes per element of an rlm dtype.
inline int64_t dtype_size(int d) { return (d == RLM_F32 || d == RLM_I32) ? 4 : (d == RLM_I64 ? 8 : 2); }

// Checks that `t` is a non-null, contiguous tensor of the given rank.
bool check_tensor(const rlm_tensor* t, const char* name, int ndim);
// Checks that `t` is a non-null 2-d tensor of unit column stride whose row
// stride is at least its width (row-strided views such as cache[:, t]).
bool check_rows(const rlm_tensor* t, const char* name);
// Checks t->shape[dim] == value.
bool check_dim(const rlm_tensor* t, const char* name, int dim, int64_t value);
bool check_dtype_float(const rlm_tensor* t, const char* name);
bool check_dtype_is(const rlm_tensor* t, const char* name, int dtype);
bool check_same_dtype(const rlm_tensor* a, const char* an, const rlm_tensor* b, const char* bn);

#define RLM_REQUIRE(cond, ...)      \
  do {                              \
    if (!(cond)) {                  \
      ::rlm::set_error(__VA_ARGS__); \
      return hipErrorInvalidValue;  \
    }                               \
  } while (0)

#define RLM_TRY(expr)                              \
  do {                                             \
    if (!(expr)) return hipErrorInvalidValue;      \
  } while (0)

// Launch status of the last kernel, with the error message recorded.
hipError_t launch_status(const char* what);

// Split-K partial products of the decode GEMM (rlm_gemm.hip): part[z] [M,N] fp32.
hipError_t linear_partials_impl(const rlm_tensor* input, const rlm_tensor* weight,
                                const rlm_tensor* part, hipStream_t stream);

}  // namespace rlm

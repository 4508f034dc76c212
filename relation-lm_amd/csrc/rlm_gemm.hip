// Dense projections for gfx950: out[M,N] = A[M,K] @ W[N,K]^T (+ bias[N]).
//
// Serves the packed 576->512 sparse-cache projection
// (src/relation_lm/inference/packed_cache.py:52-57), the expanded-cache
// projection and the relation MLP's second linear of the reference's callers.
//
// 16-bit weights (bf16/f16): v_mfma_f32_16x16x32_{bf16,f16} with fp32
//   accumulation.  A 64x64 workgroup tile is four waves of 32x32 (2x2 MFMA
//   tiles); A and W k-slices of 32 are staged in LDS.  A may be fp32 (the
//   relation hidden); it is rounded to the weight type while staging.
// fp32 weights: fp32 FMA on the same tiling (4x4 outputs per thread), so the
//   fp32 mode never passes through reduced precision.
#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 64;
constexpr int kBN = 64;
constexpr int kBK = 32;
constexpr int kPad = 8;  // 16-bit elements of padding per LDS row

struct GemmParams {
  int64_t M, N, K;
  int64_t lda;  // input row stride in elements (>= K)
  const void* a;
  const void* w;
  const void* bias;
  int bias_dtype;
  void* out;
};

// 16-bit bit pattern of v in the MFMA input type W (bf16 or f16).
template <typename W>
__device__ __forceinline__ uint16_t to_bits(float v);
template <>
__device__ __forceinline__ uint16_t to_bits<bf16>(float v) { return f32_to_bf16(v).bits; }
template <>
__device__ __forceinline__ uint16_t to_bits<f16>(float v) {
  const f16 h = static_cast<f16>(v);
  return __builtin_bit_cast(uint16_t, h);
}

// Eight consecutive A elements as W bit patterns (zero past K).
template <typename TA, typename W>
__device__ __forceinline__ uint4 load_a8(const TA* row, int64_t k, int64_t K) {
  uint16_t v[8];
  if constexpr (sizeof(TA) == 2 && sizeof(W) == 2 && __is_same(TA, W)) {
    if (k + 8 <= K) return *reinterpret_cast<const uint4*>(row + k);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = k + i < K ? reinterpret_cast<const uint16_t*>(row)[k + i] : 0;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = k + i < K ? to_bits<W>(to_f32(row[k + i])) : 0;
  }
  uint4 r;
  r.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
  r.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
  r.z = v[4] | (static_cast<uint32_t>(v[5]) << 16);
  r.w = v[6] | (static_cast<uint32_t>(v[7]) << 16);
  return r;
}

template <typename W>
__device__ __forceinline__ f32x4 mfma16(const u16x8& a, const u16x8& b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16<bf16>(const u16x8& a, const u16x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<f16>(const u16x8& a, const u16x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <typename TA, typename W, typename TO>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(const GemmParams p) {
  __shared__ __align__(16) uint16_t As[kBM][kBK + kPad];
  __shared__ __align__(16) uint16_t Bs[kBN][kBK + kPad];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kBN;
  const int wm = (wave >> 1) * 32;
  const int wn = (wave & 1) * 32;
  const TA* A = static_cast<const TA*>(p.a);
  const W* Wt = static_cast<const W*>(p.w);

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int lrow = tid >> 2;        // 0..63
  const int lk = (tid & 3) * 8;     // 0,8,16,24
  for (int64_t k0 = 0; k0 < p.K; k0 += kBK) {
    {
      const int64_t m = m0 + lrow;
      uint4 va = make_uint4(0, 0, 0, 0);
      if (m < p.M) va = load_a8<TA, W>(A + m * p.lda, k0 + lk, p.K);
      *reinterpret_cast<uint4*>(&As[lrow][lk]) = va;
      const int64_t n = n0 + lrow;
      uint4 vb = make_uint4(0, 0, 0, 0);
      if (n < p.N) vb = load_a8<W, W>(Wt + n * p.K, k0 + lk, p.K);
      *reinterpret_cast<uint4*>(&Bs[lrow][lk]) = vb;
    }
    __syncthreads();
    const int r16 = lane & 15;
    const int kq = (lane >> 4) * 8;
    u16x8 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      a[i] = *reinterpret_cast<const u16x8*>(&As[wm + i * 16 + r16][kq]);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      b[j] = *reinterpret_cast<const u16x8*>(&Bs[wn + j * 16 + r16][kq]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma16<W>(a[i], b[j], acc[i][j]);
    __syncthreads();
  }

  TO* out = static_cast<TO*>(p.out);
  const int col16 = lane & 15;
  const int row4 = (lane >> 4) * 4;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn + j * 16 + col16;
    if (n >= p.N) continue;
    const float bv = p.bias ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm + i * 16 + row4 + e;
        if (m < p.M) out[m * p.N + n] = from_f32<TO>(acc[i][j][e] + bv);
      }
    }
  }
}

template <typename TO>
__global__ void __launch_bounds__(256) gemm_f32_kernel(const GemmParams p) {
  __shared__ float As[kBK][kBM + 4];
  __shared__ float Bs[kBK][kBN + 4];
  const int tid = threadIdx.x;
  const int tx = tid & 15;
  const int ty = tid >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kBN;
  const float* A = static_cast<const float*>(p.a);
  const float* Wt = static_cast<const float*>(p.w);
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int64_t k0 = 0; k0 < p.K; k0 += kBK) {
    for (int idx = tid; idx < kBM * kBK; idx += 256) {
      const int r = idx / kBK;
      const int k = idx % kBK;
      const int64_t m = m0 + r, n = n0 + r, kk = k0 + k;
      As[k][r] = (m < p.M && kk < p.K) ? A[m * p.lda + kk] : 0.0f;
      Bs[k][r] = (n < p.N && kk < p.K) ? Wt[n * p.K + kk] : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int k = 0; k < kBK; ++k) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[k][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[k][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
    }
    __syncthreads();
  }
  TO* out = static_cast<TO*>(p.out);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + tx + 16 * j;
    if (n >= p.N) continue;
    const float bv = p.bias ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + ty + 16 * i;
      if (m < p.M) out[m * p.N + n] = from_f32<TO>(acc[i][j] + bv);
    }
  }
}

template <typename TA, typename W>
hipError_t launch_mfma_out(const GemmParams& p, int out_dtype, dim3 grid, hipStream_t s) {
  if (out_dtype == RLM_F32) {
    hipLaunchKernelGGL((gemm_mfma_kernel<TA, W, float>), grid, dim3(256), 0, s, p);
  } else if (out_dtype == RLM_BF16) {
    hipLaunchKernelGGL((gemm_mfma_kernel<TA, W, bf16>), grid, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((gemm_mfma_kernel<TA, W, f16>), grid, dim3(256), 0, s, p);
  }
  return launch_status("linear");
}

hipError_t linear_impl(const rlm_tensor* input, const rlm_tensor* weight, const rlm_tensor* bias,
                       const rlm_tensor* out, hipStream_t stream, const char* what) {
  RLM_TRY(check_rows(input, "input"));
  RLM_TRY(check_tensor(weight, "weight", 2));
  RLM_TRY(check_tensor(out, "out", 2));
  RLM_TRY(check_dtype_float(input, "input"));
  RLM_TRY(check_dtype_float(weight, "weight"));
  RLM_TRY(check_dtype_float(out, "out"));
  const int64_t M = input->shape[0], K = input->shape[1], N = weight->shape[0];
  RLM_TRY(check_dim(weight, "weight", 1, K));
  RLM_TRY(check_dim(out, "out", 0, M));
  RLM_TRY(check_dim(out, "out", 1, N));
  if (bias != nullptr) {
    RLM_TRY(check_tensor(bias, "bias", 1));
    RLM_TRY(check_dtype_float(bias, "bias"));
    RLM_TRY(check_dim(bias, "bias", 0, N));
  }
  GemmParams p{};
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = M > 1 ? input->stride[0] : K;
  p.a = input->data;
  p.w = weight->data;
  p.bias = bias ? bias->data : nullptr;
  p.bias_dtype = bias ? bias->dtype : RLM_F32;
  p.out = out->data;
  if (M == 0 || N == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((N + kBN - 1) / kBN),
                  static_cast<unsigned>((M + kBM - 1) / kBM));
  RLM_REQUIRE(grid.y <= 0x7fffffffu && grid.x <= 0x7fffffffu, "%s: problem too large", what);
  if (weight->dtype == RLM_F32) {
    RLM_REQUIRE(input->dtype == RLM_F32, "%s: fp32 weights need fp32 input (got %s)", what,
                dtype_name(input->dtype));
    if (out->dtype == RLM_F32)
      hipLaunchKernelGGL((gemm_f32_kernel<float>), grid, dim3(256), 0, stream, p);
    else if (out->dtype == RLM_BF16)
      hipLaunchKernelGGL((gemm_f32_kernel<bf16>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<f16>), grid, dim3(256), 0, stream, p);
    return launch_status(what);
  }
  RLM_REQUIRE(K % 8 == 0 && p.lda % 8 == 0,
              "%s: reduction dim and input row stride must be multiples of 8 for 16-bit weights",
              what);
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(input->data) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(weight->data) & 15u) == 0,
              "%s: input and weight must be 16-byte aligned", what);
  RLM_REQUIRE(input->dtype == weight->dtype || input->dtype == RLM_F32,
              "%s: input must be fp32 or share the weight dtype", what);
  if (weight->dtype == RLM_BF16) {
    if (input->dtype == RLM_F32) return launch_mfma_out<float, bf16>(p, out->dtype, grid, stream);
    return launch_mfma_out<bf16, bf16>(p, out->dtype, grid, stream);
  }
  if (input->dtype == RLM_F32) return launch_mfma_out<float, f16>(p, out->dtype, grid, stream);
  return launch_mfma_out<f16, f16>(p, out->dtype, grid, stream);
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_linear(const rlm_tensor* input, const rlm_tensor* weight,
                                 const rlm_tensor* bias, const rlm_tensor* out,
                                 hipStream_t stream) {
  clear_error();
  return linear_impl(input, weight, bias, out, stream, "linear");
}

extern "C" hipError_t rlm_packed_sparse_cache_projection(const rlm_tensor* memory,
                                                         const rlm_tensor* weight,
                                                         const rlm_tensor* out,
                                                         hipStream_t stream) {
  clear_error();
  RLM_REQUIRE(memory != nullptr && out != nullptr && memory->dtype == out->dtype,
              "packed_sparse_cache_projection: output dtype must equal the memory dtype");
  return linear_impl(memory, weight, nullptr, out, stream, "packed_sparse_cache_projection");
}

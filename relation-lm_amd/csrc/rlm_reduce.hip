// Relation reduce for gfx950: factorized relation hidden (gather + product
// GEMM + GELU), the fused current-row cache update, and the fused LayerNorm /
// active-K softmax / partner sum.
//
// Reference semantics: src/relation_lm/kernels/relation_reduce.py:72-450.
//
// hidden_kernel: a workgroup owns 64 consecutive (query, partner) rows of the
//   flattened [Q*K] row space and 64 hidden columns.  The gathered product
//   rows a*p (fp32, rounded as the reference does) and the W_m tile are staged
//   in LDS r-major, 64 r at a time; each thread accumulates a 4x4 fp32 block.
//   Out-of-range indices read zero rows instead of faulting.
// norm_reduce_kernel: one wavefront per query; each lane owns D/64 columns,
//   LayerNorm moments are wave64 reductions, the K softmax weights live in
//   lanes 0..K-1 and are broadcast by shuffles.
#include "rlm_common.hpp"

namespace rlm {
namespace {

constexpr int kRows = 64;   // (query, partner) rows per workgroup
constexpr int kCols = 64;   // hidden columns per workgroup
constexpr int kRC = 64;     // relation-dim chunk staged in LDS

struct HiddenParams {
  int64_t B, Tq, T;   // batch, queries per row, cache rows
  int R, H, K;
  int64_t rows;       // B*Tq*K
  const void* expanded;   // [B,T,2H]
  const void* operand;    // [B,T,R]
  const void* anchor;     // [B*Tq]
  const void* partner;    // [B*Tq*K]
  int index_dtype_a, index_dtype_p;
  const void* wm;         // [H,R]
  // cache update (decode only): wa/wp [H,R], b1 [H], position
  const void* wa;
  const void* wp;
  const void* b1;
  const void* pos;
  int pos_dtype;
  void* expanded_out;     // same buffer as expanded (mutated)
  float* out;             // [rows, H]
};

__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

// Fresh expanded value of row `t` (relation_reduce.py:215-236): half 0 is the
// anchor half W_a op[t] + b1, half 1 the partner half W_p op[t].  The cache
// write and every use of row t evaluate this same function, so the stored row
// is the rounding of exactly the fp32 value the hidden uses.
template <typename T>
__device__ __forceinline__ float fresh_value(const HiddenParams& p, int half, int64_t b,
                                             int64_t t, int n) {
  const T* w = static_cast<const T*>(half == 0 ? p.wa : p.wp) + static_cast<int64_t>(n) * p.R;
  const T* op = static_cast<const T*>(p.operand) + (b * p.T + t) * p.R;
  float acc = 0.0f;
  for (int r = 0; r < p.R; ++r) acc += to_f32(w[r]) * to_f32(op[r]);
  if (half == 0) acc += to_f32(static_cast<const T*>(p.b1)[n]);
  return acc;
}

template <typename T, bool UPDATE>
__global__ void __launch_bounds__(256) hidden_kernel(const HiddenParams p) {
  __shared__ float prodT[kRC][kRows];     // prodT[r][row]
  __shared__ float wT[kRC][kCols + 4];    // wT[r][col]
  __shared__ int64_t row_b[kRows], row_a[kRows], row_p[kRows];

  const int tid = threadIdx.x;
  const int tx = tid & 15;   // column group
  const int ty = tid >> 4;   // row group
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kRows;
  const int n0 = blockIdx.x * kCols;
  const int64_t QK = p.Tq * p.K;

  if (tid < kRows) {
    const int64_t row = r0 + tid;
    int64_t b = 0, a = -1, pp = -1;
    if (row < p.rows) {
      const int64_t q = row / p.K;
      b = q / p.Tq;
      a = load_any_i(p.anchor, p.index_dtype_a, q);
      pp = load_any_i(p.partner, p.index_dtype_p, row);
    }
    row_b[tid] = b;
    row_a[tid] = a;
    row_p[tid] = pp;
  }

  int64_t t = -1;
  if (UPDATE) {
    t = load_any_i(p.pos, p.pos_dtype, 0);
    if (t < 0 || t >= p.T) t = -1;  // out-of-range position: nothing to write or reuse
    // The tile holding row (b, k=0) writes batch b's fresh row for its columns.
    if (t >= 0) {
      const int64_t b_lo = (r0 + QK - 1) / QK;
      int64_t b_hi = (r0 + kRows - 1) / QK;
      if (b_hi > p.B - 1) b_hi = p.B - 1;
      const int64_t items = (b_hi - b_lo + 1) * 2 * kCols;
      for (int64_t idx = tid; idx < items; idx += 256) {
        const int c = static_cast<int>(idx % kCols);
        const int half = static_cast<int>((idx / kCols) % 2);
        const int64_t b = b_lo + idx / (2 * kCols);
        const int n = n0 + c;
        if (n >= p.H) continue;
        T* dst = static_cast<T*>(p.expanded_out) + (b * p.T + t) * (2 * static_cast<int64_t>(p.H)) +
                 static_cast<int64_t>(half) * p.H + n;
        *dst = from_f32<T>(fresh_value<T>(p, half, b, t, n));
      }
    }
  }
  __syncthreads();

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

  const T* operand = static_cast<const T*>(p.operand);
  const T* wm = static_cast<const T*>(p.wm);
  for (int rc = 0; rc < p.R; rc += kRC) {
    __syncthreads();
    // product rows: prodT[r][row] = fp32(op[a][r] * op[p][r])
    for (int idx = tid; idx < kRows * kRC; idx += 256) {
      const int row = idx / kRC;
      const int r = idx % kRC;
      float v = 0.0f;
      const int64_t a = row_a[row], pp = row_p[row], b = row_b[row];
      if (rc + r < p.R && a >= 0 && a < p.T && pp >= 0 && pp < p.T) {
        const float oa = to_f32(operand[(b * p.T + a) * p.R + rc + r]);
        const float op = to_f32(operand[(b * p.T + pp) * p.R + rc + r]);
        v = op * oa;
      }
      prodT[r][row] = v;
    }
    // W_m tile: wT[r][col] = W_m[n0+col][rc+r]
    for (int idx = tid; idx < kCols * kRC; idx += 256) {
      const int col = idx / kRC;
      const int r = idx % kRC;
      const int n = n0 + col;
      wT[r][col] = (n < p.H && rc + r < p.R) ? to_f32(wm[static_cast<int64_t>(n) * p.R + rc + r])
                                             : 0.0f;
    }
    __syncthreads();
    const int rlen = p.R - rc < kRC ? p.R - rc : kRC;
    for (int r = 0; r < rlen; ++r) {
      float av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = prodT[r][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = wT[r][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * wv[j];
    }
  }
  const T* expanded = static_cast<const T*>(p.expanded);
  const int64_t xrow = 2 * static_cast<int64_t>(p.H);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = ty + 16 * i;
    const int64_t grow = r0 + row;
    if (grow >= p.rows) continue;
    const int64_t b = row_b[row], a = row_a[row], pp = row_p[row];
    const bool a_ok = a >= 0 && a < p.T;
    const bool p_ok = pp >= 0 && pp < p.T;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = tx + 16 * j;
      const int n = n0 + col;
      if (n >= p.H) continue;
      // Row t is being rewritten by this launch: never read it, recompute it.
      float xa, xp;
      if (UPDATE && t >= 0 && a == t)
        xa = fresh_value<T>(p, 0, b, t, n);
      else
        xa = a_ok ? to_f32(expanded[(b * p.T + a) * xrow + n]) : 0.0f;
      if (UPDATE && t >= 0 && pp == t)
        xp = fresh_value<T>(p, 1, b, t, n);
      else
        xp = p_ok ? to_f32(expanded[(b * p.T + pp) * xrow + p.H + n]) : 0.0f;
      const float h = acc[i][j] + (xa + xp);
      p.out[grow * p.H + n] = gelu_erf(h);
    }
  }
}

struct NormParams {
  int64_t Q, Tq;
  int K, D;
  const void* raw;      // [Q,K,D]
  const float* scores;  // [Q,K]
  const void* w;
  const void* bias;
  int w_dtype, b_dtype;
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  float eps;
  float* out;           // [Q,D]
};

template <typename TR, int VPL>
__global__ void __launch_bounds__(256) norm_reduce_kernel(const NormParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (q >= p.Q) return;
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  // k_limit = clamp(ceil(log2(t + 2)), 1, K) == clamp(bit_length(t + 1), 1, K)
  const int64_t n = t + 1;
  int k_limit = n > 0 ? 64 - __clzll(static_cast<unsigned long long>(n)) : 0;
  k_limit = k_limit < 1 ? 1 : (k_limit > p.K ? p.K : k_limit);

  // Softmax weights: lane k holds partner k (K <= 64).
  const float s = lane < p.K ? p.scores[q * p.K + lane] : -INFINITY;
  const bool active = lane < p.K && lane < k_limit && s > -1.0e30f;
  const float safe = active ? s : -1.0e4f;
  const float m = wave_max_f32(lane < p.K ? safe : -INFINITY);
  float prob = active ? expf(safe - m) : 0.0f;
  const float total = wave_sum_f32(prob);
  prob = prob / fmaxf(total, 1.0e-9f);

  float gam[VPL], bet[VPL], ctx[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int d = lane + kWave * i;
    gam[i] = d < p.D ? load_any_f(p.w, p.w_dtype, d) : 0.0f;
    bet[i] = d < p.D ? load_any_f(p.bias, p.b_dtype, d) : 0.0f;
    ctx[i] = 0.0f;
  }
  const float inv_d = 1.0f / static_cast<float>(p.D);
  const TR* raw = static_cast<const TR*>(p.raw) + q * p.K * static_cast<int64_t>(p.D);
  for (int k = 0; k < p.K; ++k) {
    const float pk = __shfl(prob, k, kWave);
    if (pk == 0.0f) continue;  // wave-uniform: inactive rows contribute exactly 0
    const TR* row = raw + static_cast<int64_t>(k) * p.D;
    float x[VPL];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int d = lane + kWave * i;
      x[i] = d < p.D ? to_f32(row[d]) : 0.0f;
      sum += x[i];
    }
    const float mean = wave_sum_f32(sum) * inv_d;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int d = lane + kWave * i;
      x[i] = d < p.D ? x[i] - mean : 0.0f;
      sq += x[i] * x[i];
    }
    const float var = wave_sum_f32(sq) * inv_d;
    const float inv_std = rsqrtf(var + p.eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) ctx[i] += (x[i] * inv_std * gam[i] + bet[i]) * pk;
  }
  float* out = p.out + q * static_cast<int64_t>(p.D);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int d = lane + kWave * i;
    if (d < p.D) out[d] = ctx[i];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

hipError_t launch_hidden(HiddenParams& p, int dtype, bool update, hipStream_t stream) {
  if (p.rows == 0 || p.H == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((p.H + kCols - 1) / kCols),
                  static_cast<unsigned>((p.rows + kRows - 1) / kRows));
  RLM_REQUIRE(grid.y <= 65535u * 1024u, "too many relation rows");
#define RLM_HIDDEN_CASE(ID, T)                                                           \
  if (dtype == ID) {                                                                     \
    if (update)                                                                          \
      hipLaunchKernelGGL((hidden_kernel<T, true>), grid, dim3(256), 0, stream, p);       \
    else                                                                                 \
      hipLaunchKernelGGL((hidden_kernel<T, false>), grid, dim3(256), 0, stream, p);      \
    return launch_status("relation_hidden");                                             \
  }
  RLM_HIDDEN_CASE(RLM_F32, float)
  RLM_HIDDEN_CASE(RLM_BF16, bf16)
  RLM_HIDDEN_CASE(RLM_F16, f16)
#undef RLM_HIDDEN_CASE
  set_error("relation_hidden: unsupported dtype %s", dtype_name(dtype));
  return hipErrorInvalidValue;
}

hipError_t hidden_impl(bool seq, const rlm_tensor* expanded_cache,
                       const rlm_tensor* operand_cache, const rlm_tensor* anchor_index,
                       const rlm_tensor* partner_index, const rlm_tensor* product_weight,
                       const rlm_tensor* out, HiddenParams& p) {
  RLM_TRY(check_tensor(operand_cache, "operand_cache", 3));
  RLM_TRY(check_dtype_float(operand_cache, "operand_cache"));
  RLM_TRY(check_tensor(product_weight, "product_weight", 2));
  RLM_TRY(check_tensor(expanded_cache, "expanded_cache", 3));
  const int64_t B = operand_cache->shape[0];
  const int64_t T = operand_cache->shape[1];
  const int64_t R = operand_cache->shape[2];
  const int64_t H = product_weight->shape[0];
  RLM_TRY(check_dim(product_weight, "product_weight", 1, R));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 0, B));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 1, T));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 2, 2 * H));
  RLM_TRY(check_same_dtype(expanded_cache, "expanded_cache", operand_cache, "operand_cache"));
  RLM_TRY(check_same_dtype(product_weight, "product_weight", operand_cache, "operand_cache"));
  const int qd = seq ? 2 : 1;
  RLM_TRY(check_tensor(anchor_index, "anchor_index", qd));
  RLM_TRY(check_tensor(partner_index, "partner_index", qd + 1));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype) && is_index_dtype(partner_index->dtype),
              "anchor_index/partner_index must be int32 or int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, B));
  RLM_TRY(check_dim(partner_index, "partner_index", 0, B));
  const int64_t Tq = seq ? anchor_index->shape[1] : 1;
  if (seq) RLM_TRY(check_dim(partner_index, "partner_index", 1, Tq));
  const int64_t K = partner_index->shape[qd];
  RLM_REQUIRE(R >= 1 && R <= 4096 && H <= (1 << 20) && K <= 4096,
              "relation dim, hidden dim or partner count out of range");
  RLM_TRY(check_tensor(out, "out", qd + 2));
  RLM_TRY(check_dtype_is(out, "out", RLM_F32));
  RLM_TRY(check_dim(out, "out", 0, B));
  if (seq) RLM_TRY(check_dim(out, "out", 1, Tq));
  RLM_TRY(check_dim(out, "out", qd, K));
  RLM_TRY(check_dim(out, "out", qd + 1, H));
  p.B = B;
  p.Tq = Tq;
  p.T = T;
  p.R = static_cast<int>(R);
  p.H = static_cast<int>(H);
  p.K = static_cast<int>(K);
  p.rows = B * Tq * K;
  p.expanded = expanded_cache->data;
  p.expanded_out = expanded_cache->data;
  p.operand = operand_cache->data;
  p.anchor = anchor_index->data;
  p.partner = partner_index->data;
  p.index_dtype_a = anchor_index->dtype;
  p.index_dtype_p = partner_index->dtype;
  p.wm = product_weight->data;
  p.out = static_cast<float*>(out->data);
  return hipSuccess;
}

template <int VPL>
hipError_t launch_norm_vpl(const NormParams& p, int dtype, hipStream_t stream) {
  const int waves = 4;
  const dim3 grid(static_cast<unsigned>((p.Q + waves - 1) / waves));
#define RLM_NORM_CASE(ID, T)                                                                  \
  if (dtype == ID) {                                                                          \
    hipLaunchKernelGGL((norm_reduce_kernel<T, VPL>), grid, dim3(waves * kWave), 0, stream, p); \
    return launch_status("relation_norm_reduce");                                            \
  }
  RLM_NORM_CASE(RLM_F32, float)
  RLM_NORM_CASE(RLM_BF16, bf16)
  RLM_NORM_CASE(RLM_F16, f16)
#undef RLM_NORM_CASE
  set_error("relation_norm_reduce: unsupported raw dtype %s", dtype_name(dtype));
  return hipErrorInvalidValue;
}

hipError_t norm_impl(bool seq, const rlm_tensor* raw, const rlm_tensor* partner_scores,
                     const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
                     const rlm_tensor* position, double norm_eps, const rlm_tensor* out,
                     hipStream_t stream) {
  clear_error();
  const int qd = seq ? 2 : 1;
  RLM_TRY(check_tensor(raw, "raw", qd + 2));
  RLM_TRY(check_dtype_float(raw, "raw"));
  const int64_t B = raw->shape[0];
  const int64_t Tq = seq ? raw->shape[1] : 1;
  const int64_t K = raw->shape[qd];
  const int64_t D = raw->shape[qd + 1];
  RLM_REQUIRE(K >= 1 && K <= 64, "relation_norm_reduce supports 1 <= K <= 64, got %lld",
              (long long)K);
  RLM_REQUIRE(D >= 1 && D <= 2048, "relation_norm_reduce supports 1 <= D <= 2048, got %lld",
              (long long)D);
  RLM_TRY(check_tensor(partner_scores, "partner_scores", qd + 1));
  RLM_TRY(check_dtype_is(partner_scores, "partner_scores", RLM_F32));
  RLM_TRY(check_dim(partner_scores, "partner_scores", 0, B));
  if (seq) RLM_TRY(check_dim(partner_scores, "partner_scores", 1, Tq));
  RLM_TRY(check_dim(partner_scores, "partner_scores", qd, K));
  RLM_TRY(check_tensor(norm_weight, "norm_weight", 1));
  RLM_TRY(check_dtype_float(norm_weight, "norm_weight"));
  RLM_TRY(check_dim(norm_weight, "norm_weight", 0, D));
  RLM_TRY(check_tensor(norm_bias, "norm_bias", 1));
  RLM_TRY(check_dtype_float(norm_bias, "norm_bias"));
  RLM_TRY(check_dim(norm_bias, "norm_bias", 0, D));
  RLM_TRY(check_tensor(out, "out", qd + 1));
  RLM_TRY(check_dtype_is(out, "out", RLM_F32));
  RLM_TRY(check_dim(out, "out", 0, B));
  if (seq) RLM_TRY(check_dim(out, "out", 1, Tq));
  RLM_TRY(check_dim(out, "out", qd, D));
  NormParams p{};
  RLM_REQUIRE(position != nullptr && is_index_dtype(position->dtype),
              "position: expected an int32/int64 tensor");
  if (!seq) {
    RLM_TRY(check_tensor(position, "position", 0));
    p.pos_sb = 0;
    p.pos_sq = 0;
  } else if (position->ndim == 1) {
    RLM_TRY(check_tensor(position, "positions", 1));
    RLM_TRY(check_dim(position, "positions", 0, Tq));
    p.pos_sb = 0;
    p.pos_sq = 1;
  } else {
    RLM_TRY(check_tensor(position, "positions", 2));
    RLM_TRY(check_dim(position, "positions", 0, B));
    RLM_TRY(check_dim(position, "positions", 1, Tq));
    p.pos_sb = Tq;
    p.pos_sq = 1;
  }
  p.Q = B * Tq;
  p.Tq = Tq;
  p.K = static_cast<int>(K);
  p.D = static_cast<int>(D);
  p.raw = raw->data;
  p.scores = static_cast<const float*>(partner_scores->data);
  p.w = norm_weight->data;
  p.bias = norm_bias->data;
  p.w_dtype = norm_weight->dtype;
  p.b_dtype = norm_bias->dtype;
  p.pos = position->data;
  p.pos_dtype = position->dtype;
  p.eps = static_cast<float>(norm_eps);
  p.out = static_cast<float*>(out->data);
  if (p.Q == 0) return hipSuccess;
  const int vpl = static_cast<int>((D + kWave - 1) / kWave);
  if (vpl <= 2) return launch_norm_vpl<2>(p, raw->dtype, stream);
  if (vpl <= 4) return launch_norm_vpl<4>(p, raw->dtype, stream);
  if (vpl <= 8) return launch_norm_vpl<8>(p, raw->dtype, stream);
  if (vpl <= 12) return launch_norm_vpl<12>(p, raw->dtype, stream);
  if (vpl <= 16) return launch_norm_vpl<16>(p, raw->dtype, stream);
  if (vpl <= 24) return launch_norm_vpl<24>(p, raw->dtype, stream);
  return launch_norm_vpl<32>(p, raw->dtype, stream);
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_relation_hidden_cached(const rlm_tensor* expanded_cache,
                                                 const rlm_tensor* operand_cache,
                                                 const rlm_tensor* anchor_index,
                                                 const rlm_tensor* partner_index,
                                                 const rlm_tensor* product_weight,
                                                 const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  HiddenParams p{};
  hipError_t err = hidden_impl(false, expanded_cache, operand_cache, anchor_index, partner_index,
                               product_weight, out, p);
  if (err != hipSuccess) return err;
  return launch_hidden(p, operand_cache->dtype, false, stream);
}

extern "C" hipError_t rlm_relation_hidden_cached_seq(const rlm_tensor* expanded_cache,
                                                     const rlm_tensor* operand_cache,
                                                     const rlm_tensor* anchor_index,
                                                     const rlm_tensor* partner_index,
                                                     const rlm_tensor* product_weight,
                                                     const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  HiddenParams p{};
  hipError_t err = hidden_impl(true, expanded_cache, operand_cache, anchor_index, partner_index,
                               product_weight, out, p);
  if (err != hipSuccess) return err;
  return launch_hidden(p, operand_cache->dtype, false, stream);
}

extern "C" hipError_t rlm_relation_hidden_cache_update(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias, const rlm_tensor* position,
    const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  HiddenParams p{};
  hipError_t err = hidden_impl(false, expanded_cache, operand_cache, anchor_index, partner_index,
                               product_weight, out, p);
  if (err != hipSuccess) return err;
  RLM_TRY(check_tensor(anchor_weight, "anchor_weight", 2));
  RLM_TRY(check_tensor(partner_weight, "partner_weight", 2));
  RLM_TRY(check_tensor(first_bias, "first_bias", 1));
  RLM_TRY(check_dim(anchor_weight, "anchor_weight", 0, p.H));
  RLM_TRY(check_dim(anchor_weight, "anchor_weight", 1, p.R));
  RLM_TRY(check_dim(partner_weight, "partner_weight", 0, p.H));
  RLM_TRY(check_dim(partner_weight, "partner_weight", 1, p.R));
  RLM_TRY(check_dim(first_bias, "first_bias", 0, p.H));
  RLM_TRY(check_same_dtype(anchor_weight, "anchor_weight", operand_cache, "operand_cache"));
  RLM_TRY(check_same_dtype(partner_weight, "partner_weight", operand_cache, "operand_cache"));
  RLM_TRY(check_same_dtype(first_bias, "first_bias", operand_cache, "operand_cache"));
  RLM_REQUIRE(position != nullptr && is_index_dtype(position->dtype),
              "position: expected an int32/int64 0-d tensor");
  RLM_TRY(check_tensor(position, "position", 0));
  p.wa = anchor_weight->data;
  p.wp = partner_weight->data;
  p.b1 = first_bias->data;
  p.pos = position->data;
  p.pos_dtype = position->dtype;
  return launch_hidden(p, operand_cache->dtype, true, stream);
}

extern "C" hipError_t rlm_relation_norm_reduce(const rlm_tensor* raw,
                                               const rlm_tensor* partner_scores,
                                               const rlm_tensor* norm_weight,
                                               const rlm_tensor* norm_bias,
                                               const rlm_tensor* position, double norm_eps,
                                               const rlm_tensor* out, hipStream_t stream) {
  return norm_impl(false, raw, partner_scores, norm_weight, norm_bias, position, norm_eps, out,
                   stream);
}

extern "C" hipError_t rlm_relation_norm_reduce_seq(const rlm_tensor* raw,
                                                   const rlm_tensor* partner_scores,
                                                   const rlm_tensor* norm_weight,
                                                   const rlm_tensor* norm_bias,
                                                   const rlm_tensor* positions, double norm_eps,
                                                   const rlm_tensor* out, hipStream_t stream) {
  return norm_impl(true, raw, partner_scores, norm_weight, norm_bias, positions, norm_eps, out,
                   stream);
}

// Multi-anchor relation block for gfx950: the work of one layer after the
// routed multi-anchor selection, and the row LayerNorm / block statistics the
// layer needs around it.
//
// Reference semantics (dense eager torch, src/relation_lm/models/
// multi_relation_blocks.py):
//   * per (query, slot, partner) row: relation_mlp = Linear -> GELU -> Linear ->
//     LayerNorm (:47-52, :150-163).  The two Linears run on the library's
//     factorized hidden op and MFMA linear; this file applies the LayerNorm;
//   * per-slot partner weights: softmax over the K partners with inactive ones
//     at -1e4, times the active mask, renormalised by max(sum, 1e-9) -- no
//     k_limit (:164-168);
//   * slot context = sum_k w_k LN(row_k), times the slot's activity (:169-170);
//   * slot weights softmax(slot_mix_logits) times activity, renormalised by
//     max(sum, 1e-9) (:172-176); context = sum_s w_s slot_context_s (:177);
//   * output = hidden + sigmoid(residual_gate) * context (:178);
//   * LayerNorm of input_norm / final_norm (:39, :111, :198, :207);
//   * block statistics: mean and biased std of router keys per block and
//     channel (DistilledBlockRouter.block_statistics, routing/block_router.py).
// Slot s of the query at position t is active iff s <= t (:82-84).
//
// Mapping: one wave per query (reduce) or per row (LayerNorm); lane owns column
// groups g = lane + 64 i (4 columns each), so every row is read with coalesced
// 16-byte (fp32) or 8-byte (16-bit) loads and reduced with wave sums.  All of a
// query's row loads of one batch are issued before any is reduced.
#include "rlm_common.hpp"

namespace rlm {
namespace {

__device__ __forceinline__ void store4f(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void store4f(bf16* p, float4 v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
}
__device__ __forceinline__ void store4f(f16* p, float4 v) {
  f16 h[4] = {static_cast<f16>(v.x), static_cast<f16>(v.y), static_cast<f16>(v.z),
              static_cast<f16>(v.w)};
  *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(h);
}

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// Value of lane `src` (any lane, dynamic index).
__device__ __forceinline__ float lane_value(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}

struct MultiReduceParams {
  int64_t Q, Tq;
  int S, K, D;
  const void* raw;          // [Q, S*K, D]
  const float* scores;      // [Q, S, K]
  const void* w;            // [D] LayerNorm weight
  const void* b;            // [D] LayerNorm bias
  int w_dtype, b_dtype;
  const void* slot_logits;  // [S]
  int slot_dtype;
  const void* gate;         // [] residual gate logit
  int gate_dtype;
  const void* hidden;       // [Q, D] residual input
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  float eps;
  void* out;                // [Q, D], hidden's dtype
  float* context;           // [Q, D] fp32 or null
  const void* rb;           // [D] bias added to every raw row as it is loaded, or null
  int rb_dtype;
};

// Row weight of lane l = (slot l / K, partner l % K), 0 for l >= S*K:
// slot weight * partner weight, with the reference's masks and renormalisations.
__device__ float row_weight(const MultiReduceParams& p, float score, int64_t t, int lane) {
  const int SK = p.S * p.K;
  const bool live = lane < SK;
  const int s = live ? lane / p.K : 0;
  const int k0 = s * p.K;
  const bool slot_active = live && s <= t;
  const bool partner_active = live && score > -INFINITY && score < INFINITY;
  const float safe = partner_active ? score : -1.0e4f;
  // Softmax over the slot's K partners (all of them, inactive ones at -1e4).
  float m = -INFINITY;
  for (int k = 0; k < p.K; ++k) m = fmaxf(m, lane_value(safe, k0 + k));
  const float e = expf(safe - m);
  float total = 0.0f;
  for (int k = 0; k < p.K; ++k) total += lane_value(e, k0 + k);
  const float prob = (e / total) * (partner_active ? 1.0f : 0.0f);
  float active_total = 0.0f;
  for (int k = 0; k < p.K; ++k) active_total += lane_value(prob, k0 + k);
  const float pw = prob / fmaxf(active_total, 1.0e-9f);
  // Slot weights: softmax of the mix logits, times activity, renormalised.
  float lm = -INFINITY;
  for (int j = 0; j < p.S; ++j) lm = fmaxf(lm, load_any_f(p.slot_logits, p.slot_dtype, j));
  float lsum = 0.0f, asum = 0.0f, mine = 0.0f;
  for (int j = 0; j < p.S; ++j) {
    const float v = expf(load_any_f(p.slot_logits, p.slot_dtype, j) - lm);
    lsum += v;
    if (j <= t) asum += v;
    if (j == s) mine = v;
  }
  // (v / lsum) * active / max(sum_active (v / lsum), 1e-9), as the reference.
  const float sw = slot_active ? (mine / lsum) / fmaxf(asum / lsum, 1.0e-9f) : 0.0f;
  return live ? sw * pw : 0.0f;
}

template <typename TR, typename TH, int G, int RB>
__global__ void __launch_bounds__(256) multi_reduce_kernel(const MultiReduceParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (q >= p.Q) return;
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  const int SK = p.S * p.K;
  const int groups = p.D >> 2;
  const int64_t t = index_at(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  const float score = p.scores[q * SK + (lane < SK ? lane : 0)];
  const TR* raw = static_cast<const TR*>(p.raw) + q * SK * static_cast<int64_t>(p.D);
  const TH* hid = static_cast<const TH*>(p.hidden) + q * static_cast<int64_t>(p.D);
  F4Words gw[G], bw[G], rbw[G];
  float4 h4[G];
  const bool has_rb = p.rb != nullptr;  // uniform
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    const int gs = g < groups ? g : 0;
    gw[i] = f4_issue(p.w, p.w_dtype, gs);
    bw[i] = f4_issue(p.b, p.b_dtype, gs);
    rbw[i] = f4_issue(has_rb ? p.rb : p.b, has_rb ? p.rb_dtype : p.b_dtype, gs);
    h4[i] = load4(hid + 4 * gs);
  }
  float4 x[RB][G];
  auto load_batch = [&](int r0) {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr)
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int g = lane + kWave * i;
        const bool in = r0 + rr < SK && g < groups;
        const float4 v = load4(raw + static_cast<int64_t>(in ? r0 + rr : 0) * p.D + 4 * (in ? g : 0));
        x[rr][i] = in ? v : f4_zero();
      }
  };
  load_batch(0);
  // The second Linear's bias, decoded once and added to each raw row before its
  // statistics (fp32 adds, as the GEMM epilogue would).  Zero without a bias and
  // on lanes past the row, whose row values must stay zero for the row sums.
  float4 rb4[G];
#pragma unroll
  for (int i = 0; i < G; ++i)
    rb4[i] = has_rb && lane + kWave * i < groups ? f4_decode(rbw[i], p.rb_dtype) : f4_zero();
  auto add_bias = [&]() {
#pragma unroll
    for (int rr = 0; rr < RB; ++rr)
#pragma unroll
      for (int i = 0; i < G; ++i) {
        x[rr][i].x += rb4[i].x;
        x[rr][i].y += rb4[i].y;
        x[rr][i].z += rb4[i].z;
        x[rr][i].w += rb4[i].w;
      }
  };
  const float weight = row_weight(p, score, t, lane);
  const float inv_d = 1.0f / static_cast<float>(p.D);
  float4 acc[G];
#pragma unroll
  for (int i = 0; i < G; ++i) acc[i] = f4_zero();
  float wsum = 0.0f;
  for (int r0 = 0; r0 < SK; r0 += RB) {
    if (r0 > 0) load_batch(r0);
    if (has_rb) add_bias();  // uniform
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      if (r0 + rr >= SK) break;
      const float wr = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(weight), r0 + rr));
      if (wr == 0.0f) continue;  // wave-uniform: rows of inactive partners / slots add exactly 0
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < G; ++i) sum += (x[rr][i].x + x[rr][i].y) + (x[rr][i].z + x[rr][i].w);
      const float mean = wave_sum_f32(sum) * inv_d;
      float sq = 0.0f;
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int g = lane + kWave * i;
        if (g < groups) {
          const float dx = x[rr][i].x - mean, dy = x[rr][i].y - mean;
          const float dz = x[rr][i].z - mean, dw = x[rr][i].w - mean;
          sq += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
      }
      const float rstd = rsqrtf(wave_sum_f32(sq) * inv_d + p.eps);
      const float a = wr * rstd;
      const float c = -a * mean;
#pragma unroll
      for (int i = 0; i < G; ++i) {
        acc[i].x = fmaf(a, x[rr][i].x, acc[i].x + c);
        acc[i].y = fmaf(a, x[rr][i].y, acc[i].y + c);
        acc[i].z = fmaf(a, x[rr][i].z, acc[i].z + c);
        acc[i].w = fmaf(a, x[rr][i].w, acc[i].w + c);
      }
      wsum += wr;
    }
  }
  // context = gamma * sum_r w_r rstd_r (x_r - mean_r) + beta * sum_r w_r.
  const float gate = 1.0f / (1.0f + expf(-load_any_f(p.gate, p.gate_dtype, 0)));
  TH* out = static_cast<TH*>(p.out) + q * static_cast<int64_t>(p.D);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    if (g >= groups) continue;
    const float4 gm = f4_decode(gw[i], p.w_dtype);
    const float4 bt = f4_decode(bw[i], p.b_dtype);
    const float4 ctx = make_float4(fmaf(gm.x, acc[i].x, bt.x * wsum), fmaf(gm.y, acc[i].y, bt.y * wsum),
                                   fmaf(gm.z, acc[i].z, bt.z * wsum), fmaf(gm.w, acc[i].w, bt.w * wsum));
    if (p.context) store4f(p.context + q * static_cast<int64_t>(p.D) + 4 * g, ctx);
    store4f(out + 4 * g, make_float4(fmaf(gate, ctx.x, h4[i].x), fmaf(gate, ctx.y, h4[i].y),
                                     fmaf(gate, ctx.z, h4[i].z), fmaf(gate, ctx.w, h4[i].w)));
  }
}

struct LayerNormParams {
  int64_t rows;
  int D;
  const void* x;   // [rows, D]
  const void* w;
  const void* b;
  int w_dtype, b_dtype;
  float eps;
  void* out;       // [rows, D], x's dtype
};

template <typename T, int G>
__global__ void __launch_bounds__(256) layer_norm_kernel(const LayerNormParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= p.rows) return;
  const int groups = p.D >> 2;
  const T* x = static_cast<const T*>(p.x) + row * p.D;
  float4 v[G];
  F4Words gw[G], bw[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    const int gs = g < groups ? g : 0;
    v[i] = g < groups ? load4(x + 4 * gs) : f4_zero();
    gw[i] = f4_issue(p.w, p.w_dtype, gs);
    bw[i] = f4_issue(p.b, p.b_dtype, gs);
  }
  const float inv_d = 1.0f / static_cast<float>(p.D);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mean = wave_sum_f32(sum) * inv_d;
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    if (g < groups) {
      const float dx = v[i].x - mean, dy = v[i].y - mean, dz = v[i].z - mean, dw = v[i].w - mean;
      sq += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
  }
  const float rstd = rsqrtf(wave_sum_f32(sq) * inv_d + p.eps);
  T* out = static_cast<T*>(p.out) + row * p.D;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    if (g >= groups) continue;
    const float4 gm = f4_decode(gw[i], p.w_dtype);
    const float4 bt = f4_decode(bw[i], p.b_dtype);
    store4f(out + 4 * g, make_float4(fmaf((v[i].x - mean) * rstd, gm.x, bt.x),
                                     fmaf((v[i].y - mean) * rstd, gm.y, bt.y),
                                     fmaf((v[i].z - mean) * rstd, gm.z, bt.z),
                                     fmaf((v[i].w - mean) * rstd, gm.w, bt.w)));
  }
}

struct BlockStatsParams {
  int64_t B, T;
  int C, NB, BS;
  const void* keys;  // [B, T, C]
  float* mean;       // [B, NB, C]
  float* std;        // [B, NB, C]
};

// One thread per (batch row, block, channel); consecutive threads take
// consecutive channels, so every key row is read coalesced.  Two passes over
// the block's rows (mean, then the mean squared deviation), fp32.
template <typename T>
__global__ void __launch_bounds__(256) block_stats_kernel(const BlockStatsParams p) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = p.B * p.NB * p.C;
  if (i >= total) return;
  const int c = static_cast<int>(i % p.C);
  const int64_t bj = i / p.C;
  const int j = static_cast<int>(bj % p.NB);
  const int64_t b = bj / p.NB;
  const T* k = static_cast<const T*>(p.keys) + (b * p.T + static_cast<int64_t>(j) * p.BS) * p.C + c;
  float sum = 0.0f;
  for (int r = 0; r < p.BS; ++r) sum += to_f32(k[static_cast<int64_t>(r) * p.C]);
  const float mean = sum / static_cast<float>(p.BS);
  float sq = 0.0f;
  for (int r = 0; r < p.BS; ++r) {
    const float d = to_f32(k[static_cast<int64_t>(r) * p.C]) - mean;
    sq = fmaf(d, d, sq);
  }
  p.mean[i] = mean;
  p.std[i] = sqrtf(sq / static_cast<float>(p.BS));
}

template <int G>
hipError_t launch_multi_reduce(const MultiReduceParams& p, int raw_dtype, int hid_dtype,
                               hipStream_t stream) {
  constexpr int kWaves = 4;
  constexpr int RB = G <= 2 ? 8 : 4;
  const dim3 grid(static_cast<unsigned>((p.Q + kWaves - 1) / kWaves));
#define RLM_MR_CASE(RID, TR, HID, TH)                                                            \
  if (raw_dtype == RID && hid_dtype == HID) {                                                    \
    hipLaunchKernelGGL((multi_reduce_kernel<TR, TH, G, RB>), grid, dim3(kWaves * kWave), 0,     \
                       stream, p);                                                               \
    return launch_status("multi_relation_reduce");                                              \
  }
  RLM_MR_CASE(RLM_F32, float, RLM_F32, float)
  RLM_MR_CASE(RLM_F32, float, RLM_BF16, bf16)
  RLM_MR_CASE(RLM_F32, float, RLM_F16, f16)
  RLM_MR_CASE(RLM_BF16, bf16, RLM_F32, float)
  RLM_MR_CASE(RLM_BF16, bf16, RLM_BF16, bf16)
  RLM_MR_CASE(RLM_BF16, bf16, RLM_F16, f16)
  RLM_MR_CASE(RLM_F16, f16, RLM_F32, float)
  RLM_MR_CASE(RLM_F16, f16, RLM_BF16, bf16)
  RLM_MR_CASE(RLM_F16, f16, RLM_F16, f16)
#undef RLM_MR_CASE
  set_error("multi_relation_reduce: unsupported dtypes raw %s / hidden %s", dtype_name(raw_dtype),
            dtype_name(hid_dtype));
  return hipErrorInvalidValue;
}

template <int G>
hipError_t launch_layer_norm(const LayerNormParams& p, int dtype, hipStream_t stream) {
  constexpr int kWaves = 4;
  const dim3 grid(static_cast<unsigned>((p.rows + kWaves - 1) / kWaves));
#define RLM_LN_CASE(ID, T)                                                                       \
  if (dtype == ID) {                                                                             \
    hipLaunchKernelGGL((layer_norm_kernel<T, G>), grid, dim3(kWaves * kWave), 0, stream, p);     \
    return launch_status("layer_norm");                                                         \
  }
  RLM_LN_CASE(RLM_F32, float)
  RLM_LN_CASE(RLM_BF16, bf16)
  RLM_LN_CASE(RLM_F16, f16)
#undef RLM_LN_CASE
  set_error("layer_norm: unsupported dtype %s", dtype_name(dtype));
  return hipErrorInvalidValue;
}

bool check_vector(const rlm_tensor* t, const char* name, int64_t n) {
  return check_tensor(t, name, 1) && check_dtype_float(t, name) && check_dim(t, name, 0, n);
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_multi_relation_reduce_seq(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* slot_mix_logits,
    const rlm_tensor* residual_gate, const rlm_tensor* hidden, const rlm_tensor* positions,
    double norm_eps, const rlm_tensor* out, const rlm_tensor* context, const rlm_tensor* raw_bias,
    hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(partner_scores, "partner_scores", 4));
  RLM_TRY(check_dtype_is(partner_scores, "partner_scores", RLM_F32));
  const int64_t B = partner_scores->shape[0], Tq = partner_scores->shape[1];
  const int64_t S = partner_scores->shape[2], K = partner_scores->shape[3];
  RLM_REQUIRE(S >= 1 && K >= 1 && S * K <= 64,
              "multi_relation_reduce supports 1 <= slots * partners <= 64, got %lld x %lld",
              (long long)S, (long long)K);
  RLM_TRY(check_tensor(raw, "raw", 4));
  RLM_TRY(check_dtype_float(raw, "raw"));
  RLM_TRY(check_dim(raw, "raw", 0, B));
  RLM_TRY(check_dim(raw, "raw", 1, Tq));
  RLM_TRY(check_dim(raw, "raw", 2, S * K));
  const int64_t D = raw->shape[3];
  RLM_REQUIRE(D >= 4 && D % 4 == 0 && D <= 2048,
              "multi_relation_reduce needs d_model a multiple of 4 in [4, 2048], got %lld",
              (long long)D);
  RLM_TRY(check_vector(norm_weight, "norm_weight", D));
  RLM_TRY(check_vector(norm_bias, "norm_bias", D));
  RLM_TRY(check_vector(slot_mix_logits, "slot_mix_logits", S));
  RLM_TRY(check_tensor(residual_gate, "residual_gate", 0));
  RLM_TRY(check_dtype_float(residual_gate, "residual_gate"));
  RLM_TRY(check_tensor(hidden, "hidden", 3));
  RLM_TRY(check_dtype_float(hidden, "hidden"));
  RLM_TRY(check_dim(hidden, "hidden", 0, B));
  RLM_TRY(check_dim(hidden, "hidden", 1, Tq));
  RLM_TRY(check_dim(hidden, "hidden", 2, D));
  RLM_TRY(check_tensor(out, "out", 3));
  RLM_TRY(check_same_dtype(out, "out", hidden, "hidden"));
  RLM_TRY(check_dim(out, "out", 0, B));
  RLM_TRY(check_dim(out, "out", 1, Tq));
  RLM_TRY(check_dim(out, "out", 2, D));
  MultiReduceParams p{};
  if (context != nullptr) {
    RLM_TRY(check_tensor(context, "context", 3));
    RLM_TRY(check_dtype_is(context, "context", RLM_F32));
    RLM_TRY(check_dim(context, "context", 0, B));
    RLM_TRY(check_dim(context, "context", 1, Tq));
    RLM_TRY(check_dim(context, "context", 2, D));
    p.context = static_cast<float*>(context->data);
  }
  RLM_REQUIRE(positions != nullptr && is_index_dtype(positions->dtype),
              "positions: expected an int32/int64 tensor");
  if (positions->ndim == 1) {
    RLM_TRY(check_tensor(positions, "positions", 1));
    RLM_TRY(check_dim(positions, "positions", 0, Tq));
    p.pos_sb = 0;
    p.pos_sq = 1;
  } else {
    RLM_TRY(check_tensor(positions, "positions", 2));
    RLM_TRY(check_dim(positions, "positions", 0, B));
    RLM_TRY(check_dim(positions, "positions", 1, Tq));
    p.pos_sb = Tq;
    p.pos_sq = 1;
  }
  for (const rlm_tensor* t : {raw, hidden, out})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "raw, hidden and out must be 16-byte aligned");
  p.Q = B * Tq;
  p.Tq = Tq;
  p.S = static_cast<int>(S);
  p.K = static_cast<int>(K);
  p.D = static_cast<int>(D);
  p.raw = raw->data;
  p.scores = static_cast<const float*>(partner_scores->data);
  p.w = norm_weight->data;
  p.b = norm_bias->data;
  p.w_dtype = norm_weight->dtype;
  p.b_dtype = norm_bias->dtype;
  p.slot_logits = slot_mix_logits->data;
  p.slot_dtype = slot_mix_logits->dtype;
  p.gate = residual_gate->data;
  p.gate_dtype = residual_gate->dtype;
  p.hidden = hidden->data;
  p.pos = positions->data;
  p.pos_dtype = positions->dtype;
  p.eps = static_cast<float>(norm_eps);
  p.out = out->data;
  if (raw_bias != nullptr) {
    RLM_TRY(check_vector(raw_bias, "raw_bias", D));
    p.rb = raw_bias->data;
    p.rb_dtype = raw_bias->dtype;
  }
  if (p.Q == 0) return hipSuccess;
  const int groups = static_cast<int>((D / 4 + kWave - 1) / kWave);
  if (groups <= 1) return launch_multi_reduce<1>(p, raw->dtype, hidden->dtype, stream);
  if (groups <= 2) return launch_multi_reduce<2>(p, raw->dtype, hidden->dtype, stream);
  if (groups <= 3) return launch_multi_reduce<3>(p, raw->dtype, hidden->dtype, stream);
  if (groups <= 4) return launch_multi_reduce<4>(p, raw->dtype, hidden->dtype, stream);
  return launch_multi_reduce<8>(p, raw->dtype, hidden->dtype, stream);
}

extern "C" hipError_t rlm_layer_norm(const rlm_tensor* input, const rlm_tensor* weight,
                                     const rlm_tensor* bias, double eps, const rlm_tensor* out,
                                     hipStream_t stream) {
  clear_error();
  RLM_REQUIRE(input != nullptr && input->ndim >= 1 && input->ndim <= RLM_MAX_DIMS,
              "input: expected a 1-d to %d-d tensor", RLM_MAX_DIMS);
  RLM_TRY(check_tensor(input, "input", input->ndim));
  RLM_TRY(check_dtype_float(input, "input"));
  const int64_t D = input->shape[input->ndim - 1];
  RLM_REQUIRE(D >= 4 && D % 4 == 0 && D <= 2048,
              "layer_norm needs a last dimension that is a multiple of 4 in [4, 2048], got %lld",
              (long long)D);
  RLM_TRY(check_vector(weight, "weight", D));
  RLM_TRY(check_vector(bias, "bias", D));
  RLM_TRY(check_tensor(out, "out", input->ndim));
  RLM_TRY(check_same_dtype(out, "out", input, "input"));
  int64_t rows = 1;
  for (int i = 0; i < input->ndim; ++i) {
    RLM_TRY(check_dim(out, "out", i, input->shape[i]));
    if (i + 1 < input->ndim) rows *= input->shape[i];
  }
  for (const rlm_tensor* t : {input, out})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "input and out must be 16-byte aligned");
  LayerNormParams p{};
  p.rows = rows;
  p.D = static_cast<int>(D);
  p.x = input->data;
  p.w = weight->data;
  p.b = bias->data;
  p.w_dtype = weight->dtype;
  p.b_dtype = bias->dtype;
  p.eps = static_cast<float>(eps);
  p.out = out->data;
  if (rows == 0) return hipSuccess;
  const int groups = static_cast<int>((D / 4 + kWave - 1) / kWave);
  if (groups <= 1) return launch_layer_norm<1>(p, input->dtype, stream);
  if (groups <= 2) return launch_layer_norm<2>(p, input->dtype, stream);
  if (groups <= 3) return launch_layer_norm<3>(p, input->dtype, stream);
  if (groups <= 4) return launch_layer_norm<4>(p, input->dtype, stream);
  return launch_layer_norm<8>(p, input->dtype, stream);
}

extern "C" hipError_t rlm_block_statistics(const rlm_tensor* keys, int64_t block_size,
                                           const rlm_tensor* out_mean, const rlm_tensor* out_std,
                                           hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(keys, "keys", 3));
  RLM_TRY(check_dtype_float(keys, "keys"));
  const int64_t B = keys->shape[0], T = keys->shape[1], C = keys->shape[2];
  RLM_REQUIRE(block_size >= 1 && T % block_size == 0,
              "block_statistics: the key length %lld must be a multiple of block_size %lld",
              (long long)T, (long long)block_size);
  const int64_t NB = T / block_size;
  for (const rlm_tensor* t : {out_mean, out_std}) {
    const char* name = t == out_mean ? "out_mean" : "out_std";
    RLM_TRY(check_tensor(t, name, 3));
    RLM_TRY(check_dtype_is(t, name, RLM_F32));
    RLM_TRY(check_dim(t, name, 0, B));
    RLM_TRY(check_dim(t, name, 1, NB));
    RLM_TRY(check_dim(t, name, 2, C));
  }
  RLM_REQUIRE(B * T * C < (int64_t(1) << 40), "block_statistics: keys too large");
  BlockStatsParams p{};
  p.B = B;
  p.T = T;
  p.C = static_cast<int>(C);
  p.NB = static_cast<int>(NB);
  p.BS = static_cast<int>(block_size);
  p.keys = keys->data;
  p.mean = static_cast<float*>(out_mean->data);
  p.std = static_cast<float*>(out_std->data);
  const int64_t total = B * NB * C;
  if (total == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  switch (keys->dtype) {
    case RLM_F32:
      hipLaunchKernelGGL((block_stats_kernel<float>), grid, dim3(256), 0, stream, p);
      break;
    case RLM_BF16:
      hipLaunchKernelGGL((block_stats_kernel<bf16>), grid, dim3(256), 0, stream, p);
      break;
    default:
      hipLaunchKernelGGL((block_stats_kernel<f16>), grid, dim3(256), 0, stream, p);
      break;
  }
  return launch_status("block_statistics");
}

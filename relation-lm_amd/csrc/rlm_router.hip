// Router cache update for gfx950: one decode token of both router streams --
// the depthwise causal conv (kernel 3) from the two previous raw rows, the
// raw/conv cache writes at the token's position, and the mean / biased std of
// the block that holds the token.
//
// Reference semantics: src/relation_lm/kernels/router_cache.py:9-197 (the
// decode-time form of DistilledBlockRouter._causal_conv / block_statistics,
// block_router.py:50-68).
//
// Mapping: one wavefront per (batch row, stream); a lane owns one router
// column (columns beyond 64 loop).  The update is latency-bound, so the fast
// form (one state dtype, block size 8/16/32/64) issues every load of a lane in
// one batch and keeps the block's conv rows in registers for both moments; a
// general form covers mixed dtypes and other block sizes.  The current row's
// value is taken from registers rather than re-read after its own store (the
// reference substitutes it the same way, :113-117).
//
// Numerics follow the reference's fp32 evaluation order: conv = raw*w2, then
// + (prev1*w1), then + (prev2*w0), each product rounded before its add; the
// block mean is the fp32 sum of the BS rows divided by BS and the variance the
// mean squared deviation from it.
//
// A position outside [0, T) writes zeros to `out` and touches no cache (the
// reference reads and writes out of bounds there); a block index past the
// statistics' block count updates no statistics; block rows past the cache
// end count as zero.
//
// Ring-buffer form (contexts beyond the cache length T, a power of two): any
// position t >= 0 is accepted; position p lives in cache row p mod T and block
// j's statistics in slot j mod NB (NB * BS == T).  Rows of the token's block
// past t still hold positions from T earlier, so they count as zero -- the
// value a fresh cache gives them in the linear form.
#include "rlm_common.hpp"

namespace rlm {
namespace {

struct RouterParams {
  int B, T, D, NB, BS;
  const void* raw[2];        // [B, D] rows, stride raw_stride
  int64_t raw_stride[2];
  int raw_dtype[2];
  void* raw_cache[2];        // [B, T, D]
  void* conv_cache[2];       // [B, T, D]
  int raw_cache_dtype[2], conv_cache_dtype[2];
  void* mean[2];             // [B, NB, D]
  void* stdev[2];
  int mean_dtype[2], std_dtype[2];
  const void* weight[2];     // [D, 3]
  int weight_dtype[2];
  const void* pos;
  int pos_dtype;
  int ring;                  // ring-buffer caches
  float* out;                // [B, 2, D]
};

__device__ __forceinline__ void store_any_f(void* p, int dtype, int64_t i, float v) {
  switch (dtype) {
    case RLM_BF16: static_cast<bf16*>(p)[i] = f32_to_bf16(v); break;
    case RLM_F16: static_cast<f16*>(p)[i] = static_cast<f16>(v); break;
    default: static_cast<float*>(p)[i] = v; break;
  }
}

template <typename T>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  static_cast<T*>(p)[i] = from_f32<T>(v);
}

// Fast form: raw rows of type TR; raw/conv caches, statistics and conv weights
// all of type TC; block size BS known at compile time.  Every load of a lane
// -- this token's raw value, the two previous raw rows, the weights and the
// block's BS conv rows -- is issued before any is used.
template <int BS, typename TR, typename TC>
__global__ void __launch_bounds__(kWave) router_cache_fast_kernel(const RouterParams p) {
  const int b = blockIdx.x;
  const int side = blockIdx.y;  // 0 anchor stream, 1 partner stream
  const int lane = threadIdx.x;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, 0);
  float* out = p.out + (static_cast<int64_t>(b) * 2 + side) * p.D;
  if (t < 0 || (!p.ring && t >= p.T)) {
    for (int c = lane; c < p.D; c += kWave) out[c] = 0.0f;
    return;
  }
  const int64_t mask = p.T - 1;  // ring row mask
  const int64_t row_t = static_cast<int64_t>(b) * p.T + (p.ring ? (t & mask) : t);
  const int64_t j = t / BS;
  const int64_t slot = p.ring ? (j & (p.NB - 1)) : j;
  const int64_t first = p.ring ? ((j * BS) & mask) : j * BS;  // the block's first cache row
  const bool stats = slot < p.NB;
  const TR* raw = static_cast<const TR*>(p.raw[side]) + b * p.raw_stride[side];
  const TC* raw_cache = static_cast<const TC*>(p.raw_cache[side]);
  const TC* weight = static_cast<const TC*>(p.weight[side]);
  // This batch row's conv cache: rows past its end are out of range (read 0).
  const uint32_t row_bytes = static_cast<uint32_t>(p.D) * sizeof(TC);
  const rsrc_t conv_rsrc = make_rsrc(
      static_cast<const unsigned char*>(p.conv_cache[side]) + static_cast<int64_t>(b) * p.T * row_bytes,
      static_cast<uint32_t>(p.T) * row_bytes);
  // Previous rows, clamped where unused (t < 1, t < 2).
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t prev1 = t >= 1 ? (p.ring ? row0 + ((t - 1) & mask) : row_t - 1) : row_t;
  const int64_t prev2 = t >= 2 ? (p.ring ? row0 + ((t - 2) & mask) : row_t - 2) : row_t;
  for (int c = lane; c < p.D; c += kWave) {
    const float x = to_f32(raw[c]);
    const float p1 = to_f32(raw_cache[prev1 * p.D + c]);
    const float p2 = to_f32(raw_cache[prev2 * p.D + c]);
    const float w0 = to_f32(weight[3 * c]);
    const float w1 = to_f32(weight[3 * c + 1]);
    const float w2 = to_f32(weight[3 * c + 2]);
    const uint32_t base = static_cast<uint32_t>(first) * row_bytes + c * sizeof(TC);
    float rows[BS];
#pragma unroll
    for (int r = 0; r < BS; ++r) rows[r] = buf_load_elem<TC>(conv_rsrc, base + r * row_bytes);
    float conv;
    {
#pragma clang fp contract(off)
      conv = x * w2;
      if (t >= 1) conv = conv + p1 * w1;
      if (t >= 2) conv = conv + p2 * w0;
    }
    store_elem<TC>(p.raw_cache[side], row_t * p.D + c, x);
    store_elem<TC>(p.conv_cache[side], row_t * p.D + c, conv);
    out[c] = conv;
    if (!stats) continue;
    // Block statistics over all BS rows; the token's own row from registers
    // (ring form: rows past it count as zero).
    const int own = static_cast<int>(t - j * BS);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      rows[r] = r == own ? conv : ((p.ring && r > own) ? 0.0f : rows[r]);
      sum += rows[r];
    }
    const float mean = sum / static_cast<float>(BS);
    float sq = 0.0f;
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      const float d = rows[r] - mean;
      sq += d * d;
    }
    const int64_t s = (static_cast<int64_t>(b) * p.NB + slot) * p.D + c;
    store_elem<TC>(p.mean[side], s, mean);
    store_elem<TC>(p.stdev[side], s, sqrtf(sq / static_cast<float>(BS)));
  }
}

// General form: any float dtype per tensor, any block size.
__global__ void __launch_bounds__(kWave) router_cache_kernel(const RouterParams p) {
  const int b = blockIdx.x;
  const int side = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, 0);
  float* out = p.out + (static_cast<int64_t>(b) * 2 + side) * p.D;
  if (t < 0 || (!p.ring && t >= p.T)) {
    for (int c = lane; c < p.D; c += kWave) out[c] = 0.0f;
    return;
  }
  const int BS = p.BS;
  const int64_t mask = p.T - 1;
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  auto row_of = [&](int64_t pos) { return row0 + (p.ring ? (pos & mask) : pos); };
  const int64_t row_t = row_of(t);
  const int64_t j = t / BS;
  const int64_t slot = p.ring ? (j & (p.NB - 1)) : j;
  const int64_t first = j * BS;
  for (int c = lane; c < p.D; c += kWave) {
    const float x = load_any_f(p.raw[side], p.raw_dtype[side], b * p.raw_stride[side] + c);
    const float p1 = t >= 1 ? load_any_f(p.raw_cache[side], p.raw_cache_dtype[side],
                                         row_of(t - 1) * p.D + c)
                            : 0.0f;
    const float p2 = t >= 2 ? load_any_f(p.raw_cache[side], p.raw_cache_dtype[side],
                                         row_of(t - 2) * p.D + c)
                            : 0.0f;
    const float w0 = load_any_f(p.weight[side], p.weight_dtype[side], 3 * c);
    const float w1 = load_any_f(p.weight[side], p.weight_dtype[side], 3 * c + 1);
    const float w2 = load_any_f(p.weight[side], p.weight_dtype[side], 3 * c + 2);
    float conv;
    {
#pragma clang fp contract(off)
      conv = x * w2;
      if (t >= 1) conv = conv + p1 * w1;
      if (t >= 2) conv = conv + p2 * w0;
    }
    store_any_f(p.raw_cache[side], p.raw_cache_dtype[side], row_t * p.D + c, x);
    store_any_f(p.conv_cache[side], p.conv_cache_dtype[side], row_t * p.D + c, conv);
    out[c] = conv;
    if (slot >= p.NB) continue;
    auto block_row = [&](int r) {
      const int64_t idx = first + r;
      if (idx == t) return conv;
      if (p.ring) return idx < t ? load_any_f(p.conv_cache[side], p.conv_cache_dtype[side],
                                              row_of(idx) * p.D + c)
                                 : 0.0f;
      return idx < p.T ? load_any_f(p.conv_cache[side], p.conv_cache_dtype[side],
                                    (static_cast<int64_t>(b) * p.T + idx) * p.D + c)
                       : 0.0f;
    };
    float sum = 0.0f;
    for (int r = 0; r < BS; ++r) sum += block_row(r);
    const float mean = sum / static_cast<float>(BS);
    float sq = 0.0f;
    for (int r = 0; r < BS; ++r) {
      const float d = block_row(r) - mean;
      sq += d * d;
    }
    const int64_t s = (static_cast<int64_t>(b) * p.NB + slot) * p.D + c;
    store_any_f(p.mean[side], p.mean_dtype[side], s, mean);
    store_any_f(p.stdev[side], p.std_dtype[side], s, sqrtf(sq / static_cast<float>(BS)));
  }
}

// Statistics tensors are [B, NB, ...] with D values per block, contiguous.
bool check_stats(const rlm_tensor* t, const char* name, int64_t B, int64_t D, int64_t* nb) {
  if (t == nullptr || t->ndim < 2) {
    set_error("%s: expected a [B, blocks, ...] tensor", name);
    return false;
  }
  if (!check_tensor(t, name, t->ndim) || !check_dtype_float(t, name)) return false;
  int64_t per_block = 1;
  for (int i = 2; i < t->ndim; ++i) per_block *= t->shape[i];
  if (t->shape[0] != B || per_block != D) {
    set_error("%s: expected [B=%lld, blocks, ...] with %lld values per block", name,
              (long long)B, (long long)D);
    return false;
  }
  *nb = t->shape[1];
  return true;
}

template <typename TR, typename TC>
hipError_t launch_fast(const RouterParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.B), 2);
  switch (p.BS) {
    case 8: hipLaunchKernelGGL((router_cache_fast_kernel<8, TR, TC>), grid, dim3(kWave), 0, stream, p); break;
    case 16: hipLaunchKernelGGL((router_cache_fast_kernel<16, TR, TC>), grid, dim3(kWave), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((router_cache_fast_kernel<32, TR, TC>), grid, dim3(kWave), 0, stream, p); break;
    default: hipLaunchKernelGGL((router_cache_fast_kernel<64, TR, TC>), grid, dim3(kWave), 0, stream, p); break;
  }
  return launch_status("router_cache_update");
}

template <typename TC>
hipError_t launch_fast_tc(const RouterParams& p, hipStream_t stream) {
  switch (p.raw_dtype[0]) {
    case RLM_BF16: return launch_fast<bf16, TC>(p, stream);
    case RLM_F16: return launch_fast<f16, TC>(p, stream);
    default: return launch_fast<float, TC>(p, stream);
  }
}

hipError_t router_update_impl(
    bool ring, const rlm_tensor* anchor_raw, const rlm_tensor* partner_raw,
    const rlm_tensor* anchor_raw_cache, const rlm_tensor* partner_raw_cache,
    const rlm_tensor* anchor_conv_cache, const rlm_tensor* partner_conv_cache,
    const rlm_tensor* anchor_mean, const rlm_tensor* anchor_std,
    const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    const rlm_tensor* position, int64_t block_size, const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  RLM_TRY(check_rows(anchor_raw, "anchor_raw"));
  RLM_TRY(check_rows(partner_raw, "partner_raw"));
  RLM_TRY(check_dtype_float(anchor_raw, "anchor_raw"));
  RLM_TRY(check_dtype_float(partner_raw, "partner_raw"));
  const int64_t B = anchor_raw->shape[0], D = anchor_raw->shape[1];
  RLM_TRY(check_dim(partner_raw, "partner_raw", 0, B));
  RLM_TRY(check_dim(partner_raw, "partner_raw", 1, D));
  const rlm_tensor* caches[4] = {anchor_raw_cache, partner_raw_cache, anchor_conv_cache,
                                 partner_conv_cache};
  const char* cache_names[4] = {"anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache",
                                "partner_conv_cache"};
  for (int i = 0; i < 4; ++i) {
    RLM_TRY(check_tensor(caches[i], cache_names[i], 3));
    RLM_TRY(check_dtype_float(caches[i], cache_names[i]));
    RLM_TRY(check_dim(caches[i], cache_names[i], 0, B));
    RLM_TRY(check_dim(caches[i], cache_names[i], 1, anchor_raw_cache->shape[1]));
    RLM_TRY(check_dim(caches[i], cache_names[i], 2, D));
  }
  const int64_t T = anchor_raw_cache->shape[1];
  int64_t nb[4];
  RLM_TRY(check_stats(anchor_mean, "anchor_mean", B, D, &nb[0]));
  RLM_TRY(check_stats(anchor_std, "anchor_std", B, D, &nb[1]));
  RLM_TRY(check_stats(partner_mean, "partner_mean", B, D, &nb[2]));
  RLM_TRY(check_stats(partner_std, "partner_std", B, D, &nb[3]));
  RLM_REQUIRE(nb[1] == nb[0] && nb[2] == nb[0] && nb[3] == nb[0],
              "router statistics must all have the same number of blocks");
  for (const rlm_tensor* w : {anchor_conv_weight, partner_conv_weight}) {
    const char* name = w == anchor_conv_weight ? "anchor_conv_weight" : "partner_conv_weight";
    RLM_TRY(check_tensor(w, name, 2));
    RLM_TRY(check_dtype_float(w, name));
    RLM_TRY(check_dim(w, name, 0, D));
    RLM_TRY(check_dim(w, name, 1, 3));
  }
  RLM_REQUIRE(position != nullptr && position->ndim == 0 && is_index_dtype(position->dtype) &&
                  position->data != nullptr,
              "position: expected a 0-d int32/int64 device tensor");
  RLM_REQUIRE(block_size > 0 && block_size <= (int64_t(1) << 20),
              "block_size must be positive, got %lld", (long long)block_size);
  RLM_TRY(check_tensor(out, "out", 3));
  RLM_TRY(check_dtype_is(out, "out", RLM_F32));
  RLM_TRY(check_dim(out, "out", 0, B));
  RLM_TRY(check_dim(out, "out", 1, 2));
  RLM_TRY(check_dim(out, "out", 2, D));
  RLM_REQUIRE(B < (int64_t(1) << 31) && T < (int64_t(1) << 31) && D < (int64_t(1) << 31) &&
                  nb[0] < (int64_t(1) << 31),
              "router cache dimensions must be below 2^31");
  if (ring)
    RLM_REQUIRE(T > 0 && (T & (T - 1)) == 0 && nb[0] * block_size == T,
                "ring-buffer caches need a power-of-two cache length equal to blocks * "
                "block_size (cache length %lld, %lld blocks of %lld)",
                (long long)T, (long long)nb[0], (long long)block_size);
  if (B == 0 || D == 0) return hipSuccess;
  RouterParams p{};
  p.ring = ring ? 1 : 0;
  p.B = static_cast<int>(B);
  p.T = static_cast<int>(T);
  p.D = static_cast<int>(D);
  p.NB = static_cast<int>(nb[0]);
  p.BS = static_cast<int>(block_size);
  const rlm_tensor* raws[2] = {anchor_raw, partner_raw};
  const rlm_tensor* means[2] = {anchor_mean, partner_mean};
  const rlm_tensor* stds[2] = {anchor_std, partner_std};
  const rlm_tensor* weights[2] = {anchor_conv_weight, partner_conv_weight};
  for (int s = 0; s < 2; ++s) {
    p.raw[s] = raws[s]->data;
    p.raw_stride[s] = B > 1 ? raws[s]->stride[0] : D;
    p.raw_dtype[s] = raws[s]->dtype;
    p.raw_cache[s] = caches[s]->data;
    p.raw_cache_dtype[s] = caches[s]->dtype;
    p.conv_cache[s] = caches[2 + s]->data;
    p.conv_cache_dtype[s] = caches[2 + s]->dtype;
    p.mean[s] = means[s]->data;
    p.mean_dtype[s] = means[s]->dtype;
    p.stdev[s] = stds[s]->data;
    p.std_dtype[s] = stds[s]->dtype;
    p.weight[s] = weights[s]->data;
    p.weight_dtype[s] = weights[s]->dtype;
  }
  p.pos = position->data;
  p.pos_dtype = position->dtype;
  p.out = static_cast<float*>(out->data);
  const int64_t conv_row_block = T * D * (anchor_conv_cache->dtype == RLM_F32 ? 4 : 2);
  RLM_REQUIRE(conv_row_block + block_size * D * 4 < (int64_t(1) << 31),
              "a batch row of the conv caches must be smaller than 2 GiB");
  // One state dtype (fp32 or bf16) for caches, statistics and weights, one raw
  // dtype, and a block size of 8/16/32/64 take the fast kernel.
  const int tc = anchor_conv_cache->dtype;
  bool uniform = tc == RLM_F32 || tc == RLM_BF16;
  for (const rlm_tensor* x : {partner_raw_cache, anchor_raw_cache, partner_conv_cache,
                              anchor_mean, anchor_std, partner_mean, partner_std,
                              anchor_conv_weight, partner_conv_weight})
    uniform = uniform && x->dtype == tc;
  uniform = uniform && partner_raw->dtype == anchor_raw->dtype;
  const bool fast_bs = block_size == 8 || block_size == 16 || block_size == 32 || block_size == 64;
  if (uniform && fast_bs)
    return tc == RLM_BF16 ? launch_fast_tc<bf16>(p, stream) : launch_fast_tc<float>(p, stream);
  hipLaunchKernelGGL(router_cache_kernel, dim3(static_cast<unsigned>(B), 2), dim3(kWave), 0,
                     stream, p);
  return launch_status("router_cache_update");
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_router_cache_update(
    const rlm_tensor* anchor_raw, const rlm_tensor* partner_raw,
    const rlm_tensor* anchor_raw_cache, const rlm_tensor* partner_raw_cache,
    const rlm_tensor* anchor_conv_cache, const rlm_tensor* partner_conv_cache,
    const rlm_tensor* anchor_mean, const rlm_tensor* anchor_std,
    const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    const rlm_tensor* position, int64_t block_size, const rlm_tensor* out, hipStream_t stream) {
  return router_update_impl(false, anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache,
                            anchor_conv_cache, partner_conv_cache, anchor_mean, anchor_std,
                            partner_mean, partner_std, anchor_conv_weight, partner_conv_weight,
                            position, block_size, out, stream);
}

extern "C" hipError_t rlm_router_cache_update_ring(
    const rlm_tensor* anchor_raw, const rlm_tensor* partner_raw,
    const rlm_tensor* anchor_raw_cache, const rlm_tensor* partner_raw_cache,
    const rlm_tensor* anchor_conv_cache, const rlm_tensor* partner_conv_cache,
    const rlm_tensor* anchor_mean, const rlm_tensor* anchor_std,
    const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    const rlm_tensor* position, int64_t block_size, const rlm_tensor* out, hipStream_t stream) {
  return router_update_impl(true, anchor_raw, partner_raw, anchor_raw_cache, partner_raw_cache,
                            anchor_conv_cache, partner_conv_cache, anchor_mean, anchor_std,
                            partner_mean, partner_std, anchor_conv_weight, partner_conv_weight,
                            position, block_size, out, stream);
}

// Decode step: packed sparse-cache projection with the router cache update as
// its epilogue (the reference's roadmap item "fold the router cache update
// into the packed projection", README.md:148-149), in one launch.
//
// Same results, bit for bit, as packed_projection_to_caches followed by
// router_cache_update (rlm_gemm.hip, rlm_router.hip): every output column is
// the same sum in the same order -- eight waves split the reduction into
// 32-wide slices w, w+8, w+16, each wave accumulates its slices in order and
// the eight partial tiles are added in wave order -- and the router update is
// the fp32 evaluation of router_cache_fast_kernel on the bf16/f16-rounded
// router rows of the projection.
//
// Grid: one workgroup per 16 output columns of the cache segments (anchor key,
// partner key, operand, partner-anchor; their rows also go to row `position`
// of the four caches), plus one workgroup per router stream.  A router
// workgroup computes its stream's D (<= 64) router columns itself -- every
// wave takes its slices for all D/16 column tiles -- so the update needs no
// other workgroup: it rounds the columns to the output dtype, writes them,
// and then runs the update of batch row b on wave b (and b + 8).  The update's
// own loads (the two previous raw rows, the conv weights and the block's conv
// rows) depend only on the position and are issued before the projection's.
#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kPRWaves = 8;
constexpr int kPRSlices = 3;       // slices per wave: K <= 8 * 3 * 32
constexpr int kPRMaxK = kPRWaves * kPRSlices * 32;
constexpr int kPRMaxM = 16;
constexpr int kPRMaxD = 64;

struct ProjRouterParams {
  int M, N, K, Nmain, D;   // rows; packed width; input width; first router column; router dim
  int64_t lda;
  const void* a;           // memory [M, K]
  const void* w;           // weight [N, K]
  void* out;               // packed [M, N]
  uint32_t a_bytes, w_bytes;
  int64_t seg_lo[4], seg_hi[4], seg_rows[4];
  void* seg_dst[4];        // the four token caches [M, rows, width]
  const void* pos;
  int pos_dtype;
  int T, NB;               // router caches: rows, statistics blocks
  void* raw_cache[2];      // [M, T, D]
  void* conv_cache[2];
  void* mean[2];           // [M, NB, D]
  void* stdev[2];
  const void* cweight[2];  // [D, 3]
  float* rout;             // [M, 2, D]
};

template <typename W>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16<bf16>(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<f16>(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <typename TIO, int BS, typename TC, bool RING>
__global__ void __launch_bounds__(kPRWaves * kWave) proj_router_kernel(const ProjRouterParams p) {
  __shared__ f32x4 part[kPRWaves][kPRMaxD / 16][kWave];
  __shared__ float rawl[kPRMaxM][kPRMaxD];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int ntm = p.Nmain / 16;
  const bool router = static_cast<int>(blockIdx.x) >= ntm;  // uniform
  const int side = router ? static_cast<int>(blockIdx.x) - ntm : 0;
  const int n0 = router ? p.Nmain + side * p.D : 16 * static_cast<int>(blockIdx.x);
  const int tiles = router ? p.D / 16 : 1;
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, 0);

  // ---- Router update inputs of batch rows wave, wave + 8 and column lane.
  const bool t_ok = t >= 0 && (RING || t < p.T);
  const int64_t mask = p.T - 1;
  const int64_t j = t_ok ? t / BS : 0;
  const int64_t slot = RING ? (j & (p.NB - 1)) : j;
  const int64_t first = RING ? ((j * BS) & mask) : j * BS;
  const uint32_t row_bytes = static_cast<uint32_t>(p.D) * sizeof(TC);
  float p1[2], p2[2], w0 = 0.f, w1 = 0.f, w2 = 0.f, rows[2][BS];
  if (router) {
    const TC* rc = static_cast<const TC*>(p.raw_cache[side]);
    const TC* cw = static_cast<const TC*>(p.cweight[side]);
    const int c = lane < p.D ? lane : 0;
    w0 = to_f32(cw[3 * c]);
    w1 = to_f32(cw[3 * c + 1]);
    w2 = to_f32(cw[3 * c + 2]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int b = wave + kPRWaves * h;
      const int bc = b < p.M ? b : 0;
      const int64_t row0 = static_cast<int64_t>(bc) * p.T;
      const int64_t row_t = row0 + (RING ? (t & mask) : (t_ok ? t : 0));
      const int64_t prev1 = t >= 1 && t_ok ? (RING ? row0 + ((t - 1) & mask) : row_t - 1) : row_t;
      const int64_t prev2 = t >= 2 && t_ok ? (RING ? row0 + ((t - 2) & mask) : row_t - 2) : row_t;
      p1[h] = to_f32(rc[prev1 * p.D + c]);
      p2[h] = to_f32(rc[prev2 * p.D + c]);
      // The block's conv rows of batch row b (rows past the cache end read 0).
      const rsrc_t cr = make_rsrc(static_cast<const unsigned char*>(p.conv_cache[side]) +
                                      static_cast<int64_t>(bc) * p.T * row_bytes,
                                  static_cast<uint32_t>(p.T) * row_bytes);
      const uint32_t base = static_cast<uint32_t>(first) * row_bytes + c * sizeof(TC);
#pragma unroll
      for (int r = 0; r < BS; ++r) rows[h][r] = buf_load_elem<TC>(cr, base + r * row_bytes);
    }
  }

  // ---- Projection: wave w takes slices w, w + 8, w + 16 for each column tile.
  const rsrc_t ar = make_rsrc(p.a, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  const bool m_ok = r16 < p.M;
  const uint32_t arow = static_cast<uint32_t>(r16 * p.lda * static_cast<int64_t>(sizeof(TIO)));
  uint4 araw[kPRSlices], braw[kPRSlices][kPRMaxD / 16];
#pragma unroll
  for (int u = 0; u < kPRSlices; ++u) {
    const int k = (wave + kPRWaves * u) * 32 + kq;
    const bool in = k < p.K;
    const uint32_t kb = static_cast<uint32_t>(in ? k : 0) * static_cast<uint32_t>(sizeof(TIO));
    araw[u] = buf_load_b128(ar, m_ok && in ? arow + kb : kNoOffset);
#pragma unroll
    for (int tt = 0; tt < kPRMaxD / 16; ++tt) {
      const int n = n0 + 16 * tt + r16;
      const uint32_t wrow = static_cast<uint32_t>(n) * static_cast<uint32_t>(p.K * sizeof(TIO));
      braw[u][tt] = buf_load_b128(wr, tt < tiles && in ? wrow + kb : kNoOffset);
    }
  }
  f32x4 acc[kPRMaxD / 16];
#pragma unroll
  for (int tt = 0; tt < kPRMaxD / 16; ++tt) {
    acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < kPRSlices; ++u) acc[tt] = mfma16<TIO>(araw[u], braw[u][tt], acc[tt]);
    if (tt < tiles) part[wave][tt][lane] = acc[tt];
  }
  __syncthreads();
  if (wave < tiles) {  // wave tt adds the partial tiles of column tile tt in wave order
    f32x4 sum = part[0][wave][lane];
#pragma unroll
    for (int w = 1; w < kPRWaves; ++w) sum += part[w][wave][lane];
    const int n = n0 + 16 * wave + r16;
    TIO* out = static_cast<TIO*>(p.out);
    const int seg = router ? -1 : (n < p.seg_hi[0] ? 0 : n < p.seg_hi[1] ? 1 : n < p.seg_hi[2] ? 2 : 3);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = (lane >> 4) * 4 + e;
      if (m >= p.M) continue;
      const TIO v = from_f32<TIO>(sum[e] + 0.0f);  // as the unfused store (bias 0)
      out[static_cast<int64_t>(m) * p.N + n] = v;
      if (router) {
        rawl[m][16 * wave + r16] = to_f32(v);
      } else if (n < p.seg_hi[3]) {
        // Cache-row scatter; a position outside the cache writes nothing.
        const int64_t rows_s = p.seg_rows[seg];
        if (t >= 0 && (RING || t < rows_s)) {
          const int64_t row = RING ? (t & (rows_s - 1)) : t;
          const int64_t width = p.seg_hi[seg] - p.seg_lo[seg];
          static_cast<TIO*>(p.seg_dst[seg])[(m * rows_s + row) * width + (n - p.seg_lo[seg])] = v;
        }
      }
    }
  }
  if (!router) return;  // uniform
  __syncthreads();

  // ---- Router update (router_cache_fast_kernel's evaluation order).
  if (lane >= p.D) return;
  const int c = lane;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int b = wave + kPRWaves * h;
    if (b >= p.M) continue;
    float* rout = p.rout + (static_cast<int64_t>(b) * 2 + side) * p.D;
    if (!t_ok) {
      rout[c] = 0.0f;
      continue;
    }
    const int64_t row_t = static_cast<int64_t>(b) * p.T + (RING ? (t & mask) : t);
    const float x = rawl[b][c];
    float conv;
    {
#pragma clang fp contract(off)
      conv = x * w2;
      if (t >= 1) conv = conv + p1[h] * w1;
      if (t >= 2) conv = conv + p2[h] * w0;
    }
    static_cast<TC*>(p.raw_cache[side])[row_t * p.D + c] = from_f32<TC>(x);
    static_cast<TC*>(p.conv_cache[side])[row_t * p.D + c] = from_f32<TC>(conv);
    rout[c] = conv;
    if (slot >= p.NB) continue;
    const int own = static_cast<int>(t - j * BS);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      rows[h][r] = r == own ? conv : ((RING && r > own) ? 0.0f : rows[h][r]);
      sum += rows[h][r];
    }
    const float mean = sum / static_cast<float>(BS);
    float sq = 0.0f;
#pragma unroll
    for (int r = 0; r < BS; ++r) {
      const float d = rows[h][r] - mean;
      sq += d * d;
    }
    const int64_t s = (static_cast<int64_t>(b) * p.NB + slot) * p.D + c;
    static_cast<TC*>(p.mean[side])[s] = from_f32<TC>(mean);
    static_cast<TC*>(p.stdev[side])[s] = from_f32<TC>(sqrtf(sq / static_cast<float>(BS)));
  }
}

template <typename TIO, typename TC, bool RING>
hipError_t launch_pr_bs(const ProjRouterParams& p, int bs, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.Nmain / 16 + 2));
  const dim3 block(kPRWaves * kWave);
  switch (bs) {
    case 8: hipLaunchKernelGGL((proj_router_kernel<TIO, 8, TC, RING>), grid, block, 0, stream, p); break;
    case 16: hipLaunchKernelGGL((proj_router_kernel<TIO, 16, TC, RING>), grid, block, 0, stream, p); break;
    case 32: hipLaunchKernelGGL((proj_router_kernel<TIO, 32, TC, RING>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((proj_router_kernel<TIO, 64, TC, RING>), grid, block, 0, stream, p); break;
  }
  return launch_status("packed_projection_router_update");
}

template <typename TIO, typename TC>
hipError_t launch_pr(const ProjRouterParams& p, int bs, bool ring, hipStream_t stream) {
  return ring ? launch_pr_bs<TIO, TC, true>(p, bs, stream) : launch_pr_bs<TIO, TC, false>(p, bs, stream);
}

// Whether the one-launch form applies; otherwise the two ops run in turn.
bool fused_applies(const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
                   const rlm_tensor* const (&caches)[4], const rlm_tensor* const (&router)[10],
                   int64_t block_size) {
  if (memory->ndim != 2 || weight->ndim != 2 || out->ndim != 2) return false;
  const int io = memory->dtype;
  if ((io != RLM_BF16 && io != RLM_F16) || weight->dtype != io || out->dtype != io) return false;
  const int64_t M = memory->shape[0], K = memory->shape[1], N = weight->shape[0];
  if (M < 1 || M > kPRMaxM || K > kPRMaxK || K % 8 != 0 || weight->shape[1] != K) return false;
  if (out->shape[0] != M || out->shape[1] != N || out->stride[0] != N) return false;
  if (memory->stride[1] != 1 || (M > 1 && memory->stride[0] % 8 != 0)) return false;
  if ((reinterpret_cast<uintptr_t>(memory->data) & 15u) || (reinterpret_cast<uintptr_t>(weight->data) & 15u))
    return false;
  int64_t lo = 0;
  for (const rlm_tensor* c : caches) lo += c->shape[2];
  const int64_t D = router[0]->shape[2];  // raw caches [M, T, D]
  if (lo % 16 != 0 || D % 16 != 0 || D > kPRMaxD || lo + 2 * D != N) return false;
  if (block_size != 8 && block_size != 16 && block_size != 32 && block_size != 64) return false;
  const int tc = router[0]->dtype;
  if (tc != RLM_F32 && tc != RLM_BF16) return false;
  for (const rlm_tensor* r : router)
    if (r->dtype != tc) return false;
  return true;
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_packed_projection_router_update(
    const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
    const rlm_tensor* anchor_keys, const rlm_tensor* partner_keys,
    const rlm_tensor* operand_cache, const rlm_tensor* partner_anchor_cache,
    const rlm_tensor* position, int32_t ring, const rlm_tensor* anchor_raw_cache,
    const rlm_tensor* partner_raw_cache, const rlm_tensor* anchor_conv_cache,
    const rlm_tensor* partner_conv_cache, const rlm_tensor* anchor_mean,
    const rlm_tensor* anchor_std, const rlm_tensor* partner_mean, const rlm_tensor* partner_std,
    const rlm_tensor* anchor_conv_weight, const rlm_tensor* partner_conv_weight,
    int64_t block_size, const rlm_tensor* router_out, hipStream_t stream) {
  clear_error();
  RLM_REQUIRE(memory != nullptr && weight != nullptr && out != nullptr && router_out != nullptr,
              "packed_projection_router_update: missing tensor");
  // The projection with its cache writes, validated by its own entry point's rules.
  const rlm_tensor* caches[4] = {anchor_keys, partner_keys, operand_cache, partner_anchor_cache};
  const rlm_tensor* router[10] = {anchor_raw_cache,  partner_raw_cache, anchor_conv_cache,
                                  partner_conv_cache, anchor_mean,      anchor_std,
                                  partner_mean,       partner_std,      anchor_conv_weight,
                                  partner_conv_weight};
  for (const rlm_tensor* t : caches)
    RLM_REQUIRE(t != nullptr && t->ndim == 3, "packed_projection_router_update: token caches must be [B, T, width]");
  for (const rlm_tensor* t : router)
    RLM_REQUIRE(t != nullptr && t->ndim >= 2, "packed_projection_router_update: missing router tensor");
  const bool fused = fused_applies(memory, weight, out, caches, router, block_size);
  if (!fused) {
    // Two launches: the projection with its cache writes, then the router
    // update on the router segments of the packed output.
    hipError_t err = rlm_packed_projection_to_caches(memory, weight, out, anchor_keys, partner_keys,
                                                     operand_cache, partner_anchor_cache, position,
                                                     ring, stream);
    if (err != hipSuccess) return err;
    RLM_REQUIRE(out->ndim == 2 && anchor_raw_cache->ndim == 3, "packed_projection_router_update: bad shapes");
    const int64_t D = anchor_raw_cache->shape[2];
    const int64_t N = out->shape[1];
    RLM_REQUIRE(N >= 2 * D, "packed_projection_router_update: packed width %lld < 2 * router dim %lld",
                (long long)N, (long long)D);
    rlm_tensor ra = *out, rp = *out;
    ra.ndim = rp.ndim = 2;
    ra.shape[1] = rp.shape[1] = D;
    const int64_t es = dtype_size(out->dtype);
    ra.data = static_cast<unsigned char*>(out->data) + (N - 2 * D) * es;
    rp.data = static_cast<unsigned char*>(out->data) + (N - D) * es;
    return ring ? rlm_router_cache_update_ring(&ra, &rp, anchor_raw_cache, partner_raw_cache,
                                               anchor_conv_cache, partner_conv_cache, anchor_mean,
                                               anchor_std, partner_mean, partner_std,
                                               anchor_conv_weight, partner_conv_weight, position,
                                               block_size, router_out, stream)
                : rlm_router_cache_update(&ra, &rp, anchor_raw_cache, partner_raw_cache,
                                          anchor_conv_cache, partner_conv_cache, anchor_mean,
                                          anchor_std, partner_mean, partner_std, anchor_conv_weight,
                                          partner_conv_weight, position, block_size, router_out,
                                          stream);
  }
  // Full validation of both halves (shapes, dtypes, positions, ring rules),
  // then one launch.
  const int64_t M = memory->shape[0], K = memory->shape[1], N = weight->shape[0];
  const char* names[4] = {"anchor_keys", "partner_keys", "operand_cache", "partner_anchor_cache"};
  ProjRouterParams p{};
  int64_t lo = 0;
  for (int s = 0; s < 4; ++s) {
    RLM_TRY(check_tensor(caches[s], names[s], 3));
    RLM_TRY(check_dtype_is(caches[s], names[s], out->dtype));
    RLM_TRY(check_dim(caches[s], names[s], 0, M));
    const int64_t rows = caches[s]->shape[1];
    RLM_REQUIRE(rows >= 1, "%s: empty cache", names[s]);
    if (ring)
      RLM_REQUIRE((rows & (rows - 1)) == 0,
                  "%s: ring-buffer caches need a power-of-two length, got %lld", names[s],
                  (long long)rows);
    p.seg_lo[s] = lo;
    p.seg_hi[s] = lo + caches[s]->shape[2];
    p.seg_rows[s] = rows;
    p.seg_dst[s] = caches[s]->data;
    lo = p.seg_hi[s];
  }
  RLM_REQUIRE(position != nullptr && position->ndim == 0 && is_index_dtype(position->dtype) &&
                  position->data != nullptr,
              "position: expected a 0-d int32/int64 device tensor");
  const int64_t D = anchor_raw_cache->shape[2];
  const int64_t T = anchor_raw_cache->shape[1];
  const char* rnames[4] = {"anchor_raw_cache", "partner_raw_cache", "anchor_conv_cache",
                           "partner_conv_cache"};
  for (int i = 0; i < 4; ++i) {
    RLM_TRY(check_tensor(router[i], rnames[i], 3));
    RLM_TRY(check_dim(router[i], rnames[i], 0, M));
    RLM_TRY(check_dim(router[i], rnames[i], 1, T));
    RLM_TRY(check_dim(router[i], rnames[i], 2, D));
  }
  const char* snames[4] = {"anchor_mean", "anchor_std", "partner_mean", "partner_std"};
  int64_t nb = -1;
  for (int i = 0; i < 4; ++i) {
    const rlm_tensor* st = router[4 + i];
    RLM_TRY(check_tensor(st, snames[i], st->ndim));
    int64_t per_block = 1;
    for (int d = 2; d < st->ndim; ++d) per_block *= st->shape[d];
    RLM_REQUIRE(st->shape[0] == M && per_block == D,
                "%s: expected [B=%lld, blocks, ...] with %lld values per block", snames[i],
                (long long)M, (long long)D);
    RLM_REQUIRE(nb < 0 || st->shape[1] == nb, "router statistics must all have the same number of blocks");
    nb = st->shape[1];
  }
  for (int i = 0; i < 2; ++i) {
    const char* wn = i == 0 ? "anchor_conv_weight" : "partner_conv_weight";
    RLM_TRY(check_tensor(router[8 + i], wn, 2));
    RLM_TRY(check_dim(router[8 + i], wn, 0, D));
    RLM_TRY(check_dim(router[8 + i], wn, 1, 3));
  }
  if (ring)
    RLM_REQUIRE(T > 0 && (T & (T - 1)) == 0 && nb * block_size == T,
                "ring-buffer caches need a power-of-two cache length equal to blocks * "
                "block_size (cache length %lld, %lld blocks of %lld)",
                (long long)T, (long long)nb, (long long)block_size);
  RLM_TRY(check_tensor(router_out, "router_out", 3));
  RLM_TRY(check_dtype_is(router_out, "router_out", RLM_F32));
  RLM_TRY(check_dim(router_out, "router_out", 0, M));
  RLM_TRY(check_dim(router_out, "router_out", 1, 2));
  RLM_TRY(check_dim(router_out, "router_out", 2, D));
  const int64_t es = dtype_size(memory->dtype);
  const int64_t lda = M > 1 ? memory->stride[0] : K;
  RLM_REQUIRE(((M - 1) * lda + K) * es < (int64_t(1) << 31) && N * K * es < (int64_t(1) << 31) &&
                  T * D * dtype_size(anchor_conv_cache->dtype) < (int64_t(1) << 31),
              "packed_projection_router_update: operands must be below 2 GiB");
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.Nmain = static_cast<int>(lo);
  p.D = static_cast<int>(D);
  p.lda = lda;
  p.a = memory->data;
  p.w = weight->data;
  p.out = out->data;
  p.a_bytes = static_cast<uint32_t>(((M - 1) * lda + K) * es);
  p.w_bytes = static_cast<uint32_t>(N * K * es);
  p.pos = position->data;
  p.pos_dtype = position->dtype;
  p.T = static_cast<int>(T);
  p.NB = static_cast<int>(nb);
  for (int s = 0; s < 2; ++s) {
    p.raw_cache[s] = router[s]->data;
    p.conv_cache[s] = router[2 + s]->data;
    p.mean[s] = router[4 + 2 * s]->data;
    p.stdev[s] = router[5 + 2 * s]->data;
    p.cweight[s] = router[8 + s]->data;
  }
  p.rout = static_cast<float*>(router_out->data);
  const bool tc32 = anchor_raw_cache->dtype == RLM_F32;
  const int bs = static_cast<int>(block_size);
  if (memory->dtype == RLM_BF16)
    return tc32 ? launch_pr<bf16, float>(p, bs, ring, stream) : launch_pr<bf16, bf16>(p, bs, ring, stream);
  return tc32 ? launch_pr<f16, float>(p, bs, ring, stream) : launch_pr<f16, bf16>(p, bs, ring, stream);
}

// Fused relation reduce for gfx950, sequence form: relation hidden -> second
// linear -> LayerNorm / active-K softmax / partner sum in one kernel.
//
// The reference runs the chain as three launches with fp32 intermediates in
// memory (relation_hidden_cached relation_reduce.py:149-183, F.linear,
// relation_norm_reduce relation_reduce.py:420-450; the call sequence of
// benchmarks/benchmark_relation_reduce.py:55-64).  Here the [K,H] hidden and
// [K,D] raw rows of a query never leave the CU.
//
// Mapping: a workgroup of 8 waves (2 per SIMD) owns 128 consecutive
// (query, partner) rows, so it holds whole queries (K in {1, 2, 4, 8, 16}).
//   set-up   the exact hi/lo bf16 split of every row's operand product
//            (op[anchor] * op[partner], exact in fp32) goes to LDS, and the
//            row's active-K softmax weight is computed once.
//   phase 1  per 128-column chunk of the hidden dimension, wave w forms
//            hidden^T[64 cols x 32 rows] = W_m[chunk cols] . P^T on the matrix
//            cores (A = W_m rows streamed from L2, B = P hi and lo from LDS),
//            starting from the gathered expanded-cache halves, applies GELU and
//            rounds to bf16 -- the operand the unfused path's bf16 second
//            linear sees -- into a double-buffered LDS hidden chunk.  The
//            transposed product leaves 4 consecutive hidden columns of one row
//            in a lane, so the gathers are 8-byte loads and the LDS writes
//            ds_write_b64.
//   phase 2  raw[128 rows x D/8 cols of wave w] += hidden chunk . W2^T; the
//            hidden fragments come from LDS, W2 fragments from L2, and the raw
//            accumulators stay in registers for the whole kernel.
// Epilogue: + b2, LayerNorm per row (moments combined across the 8 waves in
// LDS), partner weights, sum over the query's rows (in-lane, then the
// neighbouring 16-lane groups), fp32 store.
#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kRows = 128;                 // (query, partner) rows per workgroup
constexpr int kRowTiles = kRows / 16;
constexpr int kHC = 128;                   // hidden columns per chunk
constexpr int kMaxR = 128;                 // relation dim held in LDS
constexpr int kLd = 136;                   // LDS row stride (bf16): 128 + 8, conflict-free b128 reads
constexpr int kTileElems = kRows * kLd;    // one [128 x kLd] bf16 LDS tile
constexpr size_t kLdsBytes =
    static_cast<size_t>(4 * kTileElems) * 2 + (kRows + 2 * kRows + kWaves * kRows) * 4;

struct FusedParams {
  int64_t B, Tq, T;
  int R, H, D, K;
  int64_t rows;        // B*Tq*K
  int64_t queries;     // B*Tq
  const void* expanded;   // [B,T,2H] bf16
  const void* operand;    // [B,T,R] bf16
  const void* anchor;     // [B*Tq]
  const void* partner;    // [B*Tq*K]
  int index_dtype_a, index_dtype_p;
  const void* wm;         // [H,R] bf16
  const void* w2;         // [D,H] bf16
  const void* b2;         // [D]
  int b2_dtype;
  const float* scores;    // [B*Tq*K]
  const void* gamma;      // [D]
  const void* beta;       // [D]
  int gamma_dtype, beta_dtype;
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  float eps;
  float* out;             // [B*Tq, D]
  uint32_t expanded_bytes, operand_bytes, wm_bytes, w2_bytes;
};

__device__ __forceinline__ f32x4 mfma_bf16(const u16x8& a, const u16x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ u16x8 lds_frag(const uint16_t* p) {
  return *reinterpret_cast<const u16x8*>(p);
}

__device__ __forceinline__ u16x8 as_frag(uint4 v) { return __builtin_bit_cast(u16x8, v); }

// Row sum over the 16 lanes of a DPP row (every lane gets the same bits).
__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v)));
  return v;
}

// Weight p_k of row `grow` in its query's partner mixture: softmax over the
// active partners (rank < k_limit, score > -1e30; inactive scores -1e4),
// renormalised by max(sum, 1e-9) -- relation_reduce.py:399-411.
__device__ float row_weight(const FusedParams& p, int64_t grow) {
  if (grow >= p.rows) return 0.0f;
  const int K = p.K;
  const int64_t q = grow / K;
  const int k = static_cast<int>(grow - q * K);
  const int64_t b = q / p.Tq;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + (q - b * p.Tq) * p.pos_sq);
  const int64_t n = t + 1;
  int k_limit = n > 0 ? 64 - __clzll(static_cast<unsigned long long>(n)) : 0;  // ceil(log2(t+2))
  k_limit = k_limit < 1 ? 1 : (k_limit > K ? K : k_limit);
  const float* sq = p.scores + q * K;
  float m = -INFINITY;
  for (int c = 0; c < K; ++c) {
    const float sc = sq[c];
    m = fmaxf(m, (c < k_limit && sc > -1.0e30f) ? sc : -1.0e4f);
  }
  float total = 0.0f, mine = 0.0f;
  for (int c = 0; c < K; ++c) {
    const float sc = sq[c];
    const float pc = (c < k_limit && sc > -1.0e30f) ? expf(sc - m) : 0.0f;
    total += pc;
    mine = c == k ? pc : mine;
  }
  return mine / fmaxf(total, 1.0e-9f);
}

struct RowIndex {
  int32_t b, a, p;  // a / p = -1 when out of range
};

__device__ __forceinline__ RowIndex row_index(const FusedParams& p, int64_t grow) {
  RowIndex r{0, -1, -1};
  if (grow < p.rows) {
    const int64_t q = grow / p.K;
    r.b = static_cast<int32_t>(q / p.Tq);
    const int64_t ai = load_any_i(p.anchor, p.index_dtype_a, q);
    const int64_t pi = load_any_i(p.partner, p.index_dtype_p, grow);
    r.a = (ai >= 0 && ai < p.T) ? static_cast<int32_t>(ai) : -1;
    r.p = (pi >= 0 && pi < p.T) ? static_cast<int32_t>(pi) : -1;
  }
  return r;
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

template <int DT, int KS1>
__global__ void __launch_bounds__(kThreads) fused_reduce_kernel(const FusedParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* phi = reinterpret_cast<uint16_t*>(smem);   // [kRows][kLd] products, bf16 high part
  uint16_t* plo = phi + kTileElems;                     // low part
  uint16_t* hid0 = plo + kTileElems;                    // two [kRows][kLd] hidden chunks
  float* wts = reinterpret_cast<float*>(hid0 + 2 * kTileElems);  // [kRows]
  float* mom = wts + kRows;                             // [2][kRows] mean, rstd
  float* part = mom + 2 * kRows;                        // [kWaves][kRows]

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wmr = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t w2r = make_rsrc(p.w2, p.w2_bytes);
  const int R = KS1 * 32, H = p.H;

  // ---- Set-up: partner weights and the hi/lo operand products.
  if (tid < kRows) wts[tid] = row_weight(p, row0 + tid);
  {
    constexpr int cpr = KS1 * 4;  // 16-byte chunks per row
    for (int i = tid; i < kRows * cpr; i += kThreads) {
      const int r = i / cpr;
      const int c = i % cpr;
      const RowIndex ix = row_index(p, row0 + r);
      const bool ok = ix.a >= 0 && ix.p >= 0;
      const uint32_t base = static_cast<uint32_t>(ix.b) * static_cast<uint32_t>(p.T);
      const uint32_t oa = ok ? ((base + ix.a) * R + 8 * c) * 2u : kNoOffset;
      const uint32_t op = ok ? ((base + ix.p) * R + 8 * c) * 2u : kNoOffset;
      const uint4 va = buf_load_b128(opr, oa);
      const uint4 vp = buf_load_b128(opr, op);
      const uint32_t wa[4] = {va.x, va.y, va.z, va.w};
      const uint32_t wp[4] = {vp.x, vp.y, vp.z, vp.w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = bf16_lo(wp[k]) * bf16_lo(wa[k]);  // exact: 8-bit x 8-bit significands
        const float x1 = bf16_hi(wp[k]) * bf16_hi(wa[k]);
        h[k] = pack_bf16x2(x0, x1);
        l[k] = pack_bf16x2(x0 - bf16_lo(h[k]), x1 - bf16_hi(h[k]));
      }
      *reinterpret_cast<uint4*>(phi + r * kLd + 8 * c) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(plo + r * kLd + 8 * c) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }

  // Phase-1 roles: row tiles 2*rg, 2*rg+1 and chunk columns [64*cg, 64*cg+64).
  const int rg = wave >> 1, cg = wave & 1;
  uint32_t xa_off[2], xp_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const RowIndex ix = row_index(p, row0 + 32 * rg + 16 * i + r16);
    const uint32_t base = static_cast<uint32_t>(ix.b) * static_cast<uint32_t>(p.T);
    xa_off[i] = ix.a >= 0 ? (base + ix.a) * (4u * H) : kNoOffset;           // anchor row, first half
    xp_off[i] = ix.p >= 0 ? (base + ix.p) * (4u * H) + 2u * H : kNoOffset;  // partner row, second half
  }
  // W_m fragments (A operand of phase 1): rows chunk*128 + 64cg + 16j + r16, k = 32s + 8g.
  const uint32_t wm_lane = (static_cast<uint32_t>(64 * cg + r16) * R + 8 * g) * 2u;
  auto load_wm = [&](u16x8 (&w)[4], int chunk, int s) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = as_frag(buf_load_b128(
          wmr, wm_lane + (static_cast<uint32_t>(chunk * kHC + 16 * j) * R + 32 * s) * 2u));
  };
  // W2 fragments (B operand of phase 2): rows dcol0 + 16j + r16, k = chunk*128 + 32s + 8g.
  const int dcol0 = wave * DT * 16;    // this wave's phase-2 output columns
  const uint32_t w2_lane = (static_cast<uint32_t>(dcol0 + r16) * H + 8 * g) * 2u;
  auto load_w2 = [&](u16x8 (&w)[DT], int chunk, int s) {
#pragma unroll
    for (int j = 0; j < DT; ++j)
      w[j] = as_frag(buf_load_b128(
          w2r, w2_lane + (static_cast<uint32_t>(16 * j) * H + chunk * kHC + 32 * s) * 2u));
  };

  f32x4 raw[kRowTiles][DT];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int j = 0; j < DT; ++j) raw[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nchunks = H / kHC;
  u16x8 wa[4];
  load_wm(wa, 0, 0);
  __syncthreads();  // products and weights visible

  for (int c = 0; c < nchunks; ++c) {
    uint16_t* hid = hid0 + (c & 1) * kTileElems;
    u16x8 b[DT];
    // ---- Phase 1: hidden^T[chunk cols 64*cg.. x rows 32*rg..] on the matrix cores.
    {
      // Expanded-cache halves of this lane's hidden entries (added after the products).
      uint2 ga[2][4], gp[2][4];
      const uint32_t col = 2u * static_cast<uint32_t>(c * kHC + 64 * cg + 4 * g);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ga[i][j] = buf_load_b64(xr, xa_off[i] == kNoOffset ? kNoOffset : xa_off[i] + col + 32u * j);
          gp[i][j] = buf_load_b64(xr, xp_off[i] == kNoOffset ? kNoOffset : xp_off[i] + col + 32u * j);
        }
      f32x4 acc[2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS1; ++s) {
        u16x8 wn[4];
        if (s + 1 < KS1) load_wm(wn, c, s + 1);
        else load_w2(b, c, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int m = 32 * rg + 16 * i + r16;
          const u16x8 bh = lds_frag(phi + m * kLd + 32 * s + 8 * g);
          const u16x8 bl = lds_frag(plo + m * kLd + 32 * s + 8 * g);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][j] = mfma_bf16(wa[j], bh, acc[i][j]);
            acc[i][j] = mfma_bf16(wa[j], bl, acc[i][j]);
          }
        }
        if (s + 1 < KS1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) wa[j] = wn[j];
        }
      }
      // acc[i][j][e] = hidden[row 32rg+16i+r16][col 64cg+16j+4g+e]
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float h0 = acc[i][j][0] + (bf16_lo(ga[i][j].x) + bf16_lo(gp[i][j].x));
          const float h1 = acc[i][j][1] + (bf16_hi(ga[i][j].x) + bf16_hi(gp[i][j].x));
          const float h2 = acc[i][j][2] + (bf16_lo(ga[i][j].y) + bf16_lo(gp[i][j].y));
          const float h3 = acc[i][j][3] + (bf16_hi(ga[i][j].y) + bf16_hi(gp[i][j].y));
          const uint32_t lo = pack_bf16x2(gelu_erf(h0), gelu_erf(h1));
          const uint32_t hi = pack_bf16x2(gelu_erf(h2), gelu_erf(h3));
          *reinterpret_cast<uint2*>(hid + (32 * rg + 16 * i + r16) * kLd + 64 * cg + 16 * j +
                                    4 * g) = make_uint2(lo, hi);
        }
    }
    __syncthreads();  // hidden chunk complete; the other buffer is free for chunk c+1
    // ---- Phase 2: raw[128 x 16*DT] += hidden chunk . W2[cols, chunk]^T.
#pragma unroll
    for (int s = 0; s < kHC / 32; ++s) {
      u16x8 bn[DT];
      if (s + 1 < kHC / 32) load_w2(bn, c, s + 1);
      else if (c + 1 < nchunks) load_wm(wa, c + 1, 0);
      u16x8 a[kRowTiles];
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i) a[i] = lds_frag(hid + (16 * i + r16) * kLd + 32 * s + 8 * g);
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
        for (int j = 0; j < DT; ++j) raw[i][j] = mfma_bf16(a[i], b[j], raw[i][j]);
      if (s + 1 < kHC / 32) {
#pragma unroll
        for (int j = 0; j < DT; ++j) b[j] = bn[j];
      }
    }
  }

  // ---- Epilogue.  raw[i][j][e] = row 16i+4g+e, column dcol0+16j+r16.
  const float inv_d = 1.0f / static_cast<float>(p.D);
#pragma unroll
  for (int j = 0; j < DT; ++j) {
    const float bias = load_any_f(p.b2, p.b2_dtype, dcol0 + 16 * j + r16);
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) raw[i][j][e] += bias;
  }
  // Mean: per-wave partial row sums, combined per row by threads 0..127.
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < DT; ++j) sum += raw[i][j][e];
      sum = row16_sum(sum);
      if (r16 == 0) part[wave * kRows + 16 * i + 4 * g + e] = sum;
    }
  __syncthreads();
  if (tid < kRows) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum += part[w * kRows + tid];
    mom[tid] = sum * inv_d;
  }
  __syncthreads();
  float4 mean[kRowTiles];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i) mean[i] = *reinterpret_cast<const float4*>(mom + 16 * i + 4 * g);
  // Biased variance from the centred values.
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i) {
    const float mu[4] = {mean[i].x, mean[i].y, mean[i].z, mean[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        const float d = raw[i][j][e] - mu[e];
        sum += d * d;
      }
      sum = row16_sum(sum);
      if (r16 == 0) part[wave * kRows + 16 * i + 4 * g + e] = sum;
    }
  }
  __syncthreads();
  if (tid < kRows) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum += part[w * kRows + tid];
    mom[kRows + tid] = rsqrtf(sum * inv_d + p.eps);
  }
  __syncthreads();
  // LayerNorm, weights, sum over each query's K consecutive rows, store.
  const int K = p.K;
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i) {
    const float4 m4 = mean[i];
    const float4 r4 = *reinterpret_cast<const float4*>(mom + kRows + 16 * i + 4 * g);
    const float4 w4 = *reinterpret_cast<const float4*>(wts + 16 * i + 4 * g);
    const float mu[4] = {m4.x, m4.y, m4.z, m4.w};
    const float rs[4] = {r4.x, r4.y, r4.z, r4.w};
    const float wt[4] = {w4.x, w4.y, w4.z, w4.w};
    const int64_t trow = row0 + 16 * i + 4 * g;  // first row of this lane group
#pragma unroll
    for (int j = 0; j < DT; ++j) {
      const int n = dcol0 + 16 * j + r16;
      const float gm = load_any_f(p.gamma, p.gamma_dtype, n);
      const float bt = load_any_f(p.beta, p.beta_dtype, n);
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y[e] = wt[e] > 0.0f ? ((raw[i][j][e] - mu[e]) * rs[e] * gm + bt) * wt[e] : 0.0f;
      if (K >= 4) {
        // Rows of one query: K = 4 -> this group, K = 8 -> groups {0,1} / {2,3}, K = 16 -> all.
        float v = (y[0] + y[1]) + (y[2] + y[3]);
        if (K >= 8) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
        if (K >= 16) v += __shfl_xor(v, 32, kWave);
        const int lead = (g * 4 / K) * K / 4;
        const int64_t q = trow / K;
        if (g == lead && q < p.queries) p.out[q * p.D + n] = v;
      } else if (K == 2) {
        const int64_t q0 = trow / 2;
        if (q0 < p.queries) p.out[q0 * p.D + n] = y[0] + y[1];
        if (q0 + 1 < p.queries) p.out[(q0 + 1) * p.D + n] = y[2] + y[3];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (trow + e < p.queries) p.out[(trow + e) * p.D + n] = y[e];
      }
    }
  }
}

template <int DT, int KS1>
hipError_t launch_fused(const FusedParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((p.rows + kRows - 1) / kRows));
  static bool attr_set = false;  // the LDS opt-in is a per-process function attribute
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&fused_reduce_kernel<DT, KS1>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
    if (e != hipSuccess) {
      set_error("relation_reduce_fused: cannot reserve %zu bytes of LDS: %s", kLdsBytes,
                hipGetErrorString(e));
      return e;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((fused_reduce_kernel<DT, KS1>), grid, dim3(kThreads), kLdsBytes, stream, p);
  return launch_status("relation_reduce_fused");
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_relation_reduce_fused_seq(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight,
    const rlm_tensor* second_bias, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias, const rlm_tensor* positions,
    double norm_eps, const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(operand_cache, "operand_cache", 3));
  RLM_TRY(check_tensor(expanded_cache, "expanded_cache", 3));
  RLM_TRY(check_tensor(product_weight, "product_weight", 2));
  RLM_TRY(check_tensor(second_weight, "second_weight", 2));
  RLM_TRY(check_dtype_is(operand_cache, "operand_cache", RLM_BF16));
  RLM_TRY(check_dtype_is(expanded_cache, "expanded_cache", RLM_BF16));
  RLM_TRY(check_dtype_is(product_weight, "product_weight", RLM_BF16));
  RLM_TRY(check_dtype_is(second_weight, "second_weight", RLM_BF16));
  const int64_t B = operand_cache->shape[0], T = operand_cache->shape[1];
  const int64_t R = operand_cache->shape[2], H = product_weight->shape[0];
  const int64_t D = second_weight->shape[0];
  RLM_TRY(check_dim(product_weight, "product_weight", 1, R));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 0, B));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 1, T));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 2, 2 * H));
  RLM_TRY(check_dim(second_weight, "second_weight", 1, H));
  RLM_TRY(check_tensor(anchor_index, "anchor_index", 2));
  RLM_TRY(check_tensor(partner_index, "partner_index", 3));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype) && is_index_dtype(partner_index->dtype),
              "anchor_index/partner_index must be int32 or int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, B));
  const int64_t Tq = anchor_index->shape[1];
  RLM_TRY(check_dim(partner_index, "partner_index", 0, B));
  RLM_TRY(check_dim(partner_index, "partner_index", 1, Tq));
  const int64_t K = partner_index->shape[2];
  RLM_REQUIRE(K == 1 || K == 2 || K == 4 || K == 8 || K == 16,
              "fused relation reduce supports K in {1, 2, 4, 8, 16}, got %lld", (long long)K);
  RLM_REQUIRE(R == 32 || R == 64 || R == 128,
              "fused relation reduce needs relation dim 32, 64 or 128, got %lld", (long long)R);
  RLM_REQUIRE(H % kHC == 0 && H > 0, "fused relation reduce needs hidden dim a multiple of %d",
              kHC);
  RLM_TRY(check_tensor(second_bias, "second_bias", 1));
  RLM_TRY(check_dtype_float(second_bias, "second_bias"));
  RLM_TRY(check_dim(second_bias, "second_bias", 0, D));
  RLM_TRY(check_tensor(partner_scores, "partner_scores", 3));
  RLM_TRY(check_dtype_is(partner_scores, "partner_scores", RLM_F32));
  RLM_TRY(check_dim(partner_scores, "partner_scores", 0, B));
  RLM_TRY(check_dim(partner_scores, "partner_scores", 1, Tq));
  RLM_TRY(check_dim(partner_scores, "partner_scores", 2, K));
  RLM_TRY(check_tensor(norm_weight, "norm_weight", 1));
  RLM_TRY(check_dtype_float(norm_weight, "norm_weight"));
  RLM_TRY(check_dim(norm_weight, "norm_weight", 0, D));
  RLM_TRY(check_tensor(norm_bias, "norm_bias", 1));
  RLM_TRY(check_dtype_float(norm_bias, "norm_bias"));
  RLM_TRY(check_dim(norm_bias, "norm_bias", 0, D));
  RLM_TRY(check_tensor(out, "out", 3));
  RLM_TRY(check_dtype_is(out, "out", RLM_F32));
  RLM_TRY(check_dim(out, "out", 0, B));
  RLM_TRY(check_dim(out, "out", 1, Tq));
  RLM_TRY(check_dim(out, "out", 2, D));
  FusedParams p{};
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
  constexpr int64_t kMaxBytes = int64_t(1) << 31;
  RLM_REQUIRE(B * T * 2 * H * 2 < kMaxBytes && B * T * R * 2 < kMaxBytes && D * H * 2 < kMaxBytes,
              "caches and weights must each be smaller than 2 GiB");
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "operand_cache, product_weight and second_weight must be 16-byte aligned");
  p.B = B;
  p.Tq = Tq;
  p.T = T;
  p.R = static_cast<int>(R);
  p.H = static_cast<int>(H);
  p.D = static_cast<int>(D);
  p.K = static_cast<int>(K);
  p.rows = B * Tq * K;
  p.queries = B * Tq;
  p.expanded = expanded_cache->data;
  p.operand = operand_cache->data;
  p.anchor = anchor_index->data;
  p.partner = partner_index->data;
  p.index_dtype_a = anchor_index->dtype;
  p.index_dtype_p = partner_index->dtype;
  p.wm = product_weight->data;
  p.w2 = second_weight->data;
  p.b2 = second_bias->data;
  p.b2_dtype = second_bias->dtype;
  p.scores = static_cast<const float*>(partner_scores->data);
  p.gamma = norm_weight->data;
  p.beta = norm_bias->data;
  p.gamma_dtype = norm_weight->dtype;
  p.beta_dtype = norm_bias->dtype;
  p.pos = positions->data;
  p.pos_dtype = positions->dtype;
  p.eps = static_cast<float>(norm_eps);
  p.out = static_cast<float*>(out->data);
  p.expanded_bytes = static_cast<uint32_t>(B * T * 2 * H * 2);
  p.operand_bytes = static_cast<uint32_t>(B * T * R * 2);
  p.wm_bytes = static_cast<uint32_t>(H * R * 2);
  p.w2_bytes = static_cast<uint32_t>(D * H * 2);
  if (p.rows == 0) return hipSuccess;
  const int ks1 = static_cast<int>(R / 32);
#define RLM_FUSED_CASE(DT)                                          \
  if (D == 128 * DT) {                                              \
    if (ks1 == 1) return launch_fused<DT, 1>(p, stream);            \
    if (ks1 == 2) return launch_fused<DT, 2>(p, stream);            \
    return launch_fused<DT, 4>(p, stream);                          \
  }
  RLM_FUSED_CASE(1)
  RLM_FUSED_CASE(2)
  RLM_FUSED_CASE(3)
  RLM_FUSED_CASE(4)
#undef RLM_FUSED_CASE
  set_error("fused relation reduce supports d_model in {128, 256, 384, 512} (a wave keeps "
            "[128, d_model/8] accumulators in registers), got %lld; use the unfused "
            "relation_hidden_cached_seq / relation_linear / relation_norm_reduce_seq chain",
            (long long)D);
  return hipErrorInvalidValue;
}

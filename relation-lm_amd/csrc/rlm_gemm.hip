// Dense projections for gfx950: out[M,N] = A[M,K] @ W[N,K]^T (+ bias[N]).
//
// Serves the packed 576->512 sparse-cache projection
// (src/relation_lm/inference/packed_cache.py:52-57), the expanded-cache
// projection and the relation MLP's second linear of the reference's callers.
//
// 16-bit weights (bf16/f16): v_mfma_f32_16x16x32_{bf16,f16}, fp32 accumulation.
// A may be fp32 (the relation hidden); it is rounded to the weight type while
// it is staged, so the MFMA sees the same operand a bf16 F.linear would.
//
//   tile_kernel   (M > 64)   BMxBN workgroup tile (128x128 or 64x128), four
//                 waves in 2x2, each a (BM/2)x(BN/2) grid of 16x16 MFMA tiles.
//                 A and W k-slices of 32 are double-buffered in LDS: the
//                 global loads of slice k+1 are in flight while slice k runs
//                 on the matrix cores.  Workgroups are renumbered so that the
//                 tiles sharing an A row-block run on the same XCD (one L2),
//                 which keeps A's HBM traffic at one read.
//   smallk_kernel (M > 64, K in {32, 64, 96, 128})  e.g. the expanded-cache
//                 projection (K = relation dim).  Each wave owns a 64x64 output
//                 tile and loads all of its A and W fragments for the whole K
//                 straight from L2 in MFMA operand layout -- one round trip,
//                 no LDS staging and no barriers.
//   skinny_kernel (M <= 64)  decode shapes.  A workgroup owns one 16x16 output
//                 tile; its eight waves split K, each issuing the W and A
//                 fragment loads of up to six 32-wide slices at once straight
//                 from global memory in MFMA operand layout, and the partial
//                 tiles meet once in LDS.
//
// fp32 weights: f32_tile_kernel, 64x64 tiles on v_mfma_f32_16x16x4f32 (fp32
// operands, fp32 accumulation), so fp32 mode never passes through reduced
// precision.
#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kBK = 32;   // k-slice of the 16-bit path
constexpr int kPad = 8;   // 16-bit elements of padding per LDS row (conflict-free b128 reads)
constexpr int kSkinnyM = 64;

constexpr int kMaxSegments = 4;

struct GemmParams {
  int64_t M, N, K;
  int64_t lda;  // input row stride in elements (>= K)
  const void* a;
  const void* w;
  const void* bias;
  int bias_dtype;
  void* out;
  // Optional cache-row scatter (decode projection, skinny kernel only): output
  // columns [seg_lo[s], seg_hi[s]) of row m also go to row `position` of cache
  // s ([M, seg_rows[s], seg_hi[s] - seg_lo[s]], the output dtype); ring caches
  // take row position mod seg_rows[s] (a power of two).
  int nseg;
  int64_t seg_lo[kMaxSegments], seg_hi[kMaxSegments], seg_rows[kMaxSegments];
  void* seg_dst[kMaxSegments];
  const void* pos;
  int pos_dtype;
  int ring;
};

// 16-bit bit pattern of v in the MFMA input type W (bf16 or f16).
template <typename W>
__device__ __forceinline__ uint16_t to_bits(float v);
template <>
__device__ __forceinline__ uint16_t to_bits<f16>(float v) {
  const f16 h = static_cast<f16>(v);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

// Eight consecutive elements starting at row[k] as W bit patterns.  The
// caller guarantees k + 8 <= K and 16-byte alignment of 16-bit rows.
template <typename TA, typename W>
__device__ __forceinline__ uint4 load8(const TA* row, int64_t k) {
  if constexpr (sizeof(TA) == 2) {
    return *reinterpret_cast<const uint4*>(row + k);
  } else if constexpr (__is_same(W, bf16)) {
    const float4 x = *reinterpret_cast<const float4*>(row + k);
    const float4 y = *reinterpret_cast<const float4*>(row + k + 4);
    return make_uint4(pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w), pack_bf16x2(y.x, y.y),
                      pack_bf16x2(y.z, y.w));
  } else {
    const float4 x = *reinterpret_cast<const float4*>(row + k);
    const float4 y = *reinterpret_cast<const float4*>(row + k + 4);
    return make_uint4(pack2(to_bits<W>(x.x), to_bits<W>(x.y)), pack2(to_bits<W>(x.z), to_bits<W>(x.w)),
                      pack2(to_bits<W>(y.x), to_bits<W>(y.y)), pack2(to_bits<W>(y.z), to_bits<W>(y.w)));
  }
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

// Renumbers workgroup `i` of `count` so that each XCD (the hardware deals
// workgroups round-robin over 8 XCDs) receives a contiguous range of logical
// tile ids.
__device__ __forceinline__ int64_t xcd_tile(int64_t i, int64_t count) {
  constexpr int kXcd = 8;
  const int64_t per = count / kXcd, rem = count % kXcd;
  const int64_t x = i % kXcd;
  return x * per + (x < rem ? x : rem) + i / kXcd;
}

// Stores one 16x16 MFMA accumulator (lane holds rows 4*(lane/16)+e of column
// lane%16) plus bias.
template <typename TO>
__device__ __forceinline__ void store_tile(const GemmParams& p, const f32x4& acc, int64_t m_base,
                                           int64_t n, float bv, int lane) {
  if (n >= p.N) return;
  TO* out = static_cast<TO*>(p.out);
  const int64_t m0 = m_base + (lane >> 4) * 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t m = m0 + e;
    if (m < p.M) out[m * p.N + n] = from_f32<TO>(acc[e] + bv);
  }
}

// The cache-row scatter of one 16x16 accumulator (see GemmParams): column n's
// four rows also go to their caches' row `position`.  A position outside the
// cache (linear caches: t >= rows; any: t < 0) writes nothing.
template <typename TO>
__device__ __forceinline__ void scatter_tile(const GemmParams& p, const f32x4& acc,
                                             int64_t m_base, int64_t n, float bv, int lane) {
  if (p.nseg == 0 || n >= p.N) return;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, 0);
  const int64_t m0 = m_base + (lane >> 4) * 4;
#pragma unroll
  for (int s = 0; s < kMaxSegments; ++s) {
    if (s >= p.nseg || n < p.seg_lo[s] || n >= p.seg_hi[s]) continue;
    const int64_t rows = p.seg_rows[s];
    if (t < 0 || (!p.ring && t >= rows)) continue;
    const int64_t row = p.ring ? (t & (rows - 1)) : t;
    const int64_t width = p.seg_hi[s] - p.seg_lo[s];
    TO* dst = static_cast<TO*>(p.seg_dst[s]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t m = m0 + e;
      if (m < p.M) dst[(m * rows + row) * width + (n - p.seg_lo[s])] = from_f32<TO>(acc[e] + bv);
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit weights, large M
// ---------------------------------------------------------------------------

template <typename TA, typename W, typename TO, int BM, int BN>
__global__ void __launch_bounds__(256) tile_kernel(const GemmParams p) {
  constexpr int TM = BM / 32;              // 16-row MFMA tiles per wave
  constexpr int TN = BN / 32;              // 16-col MFMA tiles per wave
  constexpr int AE = BM * kBK / 256;       // A elements each thread stages per slice
  constexpr int BE = BN * kBK / 256;
  static_assert(AE % 8 == 0 && BE % 8 == 0, "stage in 8-element chunks");
  __shared__ __align__(16) uint16_t As[2][BM][kBK + kPad];
  __shared__ __align__(16) uint16_t Bs[2][BN][kBK + kPad];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t tiles_n = (p.N + BN - 1) / BN;
  const int64_t tiles = tiles_n * ((p.M + BM - 1) / BM);
  const int64_t tile = xcd_tile(blockIdx.x, tiles);
  const int64_t m0 = (tile / tiles_n) * BM;
  const int64_t n0 = (tile % tiles_n) * BN;
  const int wm = (wave >> 1) * (BM / 2);
  const int wn = (wave & 1) * (BN / 2);
  const TA* A = static_cast<const TA*>(p.a);
  const W* Wt = static_cast<const W*>(p.w);

  // Staging assignment: thread -> (row, 8-element chunks along k).
  const int a_row = tid / (kBK / AE);
  const int a_k = (tid % (kBK / AE)) * AE;
  const int b_row = tid / (kBK / BE);
  const int b_k = (tid % (kBK / BE)) * BE;
  const bool a_ok = m0 + a_row < p.M;
  const bool b_ok = n0 + b_row < p.N;
  const TA* a_src = A + (a_ok ? (m0 + a_row) * p.lda : 0);
  const W* b_src = Wt + (b_ok ? (n0 + b_row) * p.K : 0);

  uint4 ra[AE / 8], rb[BE / 8];
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < AE / 8; ++c) {
      const int64_t k = k0 + a_k + 8 * c;
      ra[c] = (a_ok && k < p.K) ? load8<TA, W>(a_src, k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < BE / 8; ++c) {
      const int64_t k = k0 + b_k + 8 * c;
      rb[c] = (b_ok && k < p.K) ? load8<W, W>(b_src, k) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int c = 0; c < AE / 8; ++c) *reinterpret_cast<uint4*>(&As[buf][a_row][a_k + 8 * c]) = ra[c];
#pragma unroll
    for (int c = 0; c < BE / 8; ++c) *reinterpret_cast<uint4*>(&Bs[buf][b_row][b_k + 8 * c]) = rb[c];
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t slices = (p.K + kBK - 1) / kBK;
  fetch(0);
  stage(0);
  __syncthreads();
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  for (int64_t s = 0; s < slices; ++s) {
    const int cur = static_cast<int>(s & 1);
    if (s + 1 < slices) fetch((s + 1) * kBK);
    u16x8 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
      a[i] = *reinterpret_cast<const u16x8*>(&As[cur][wm + i * 16 + r16][kq]);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      b[j] = *reinterpret_cast<const u16x8*>(&Bs[cur][wn + j * 16 + r16][kq]);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma16<W>(a[i], b[j], acc[i][j]);
    if (s + 1 < slices) stage(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + wn + j * 16 + r16;
    const float bv = (p.bias && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) store_tile<TO>(p, acc[i][j], m0 + wm + i * 16, n, bv, lane);
  }
}

// ---------------------------------------------------------------------------
// 16-bit weights, small K (K = 32*KS, KS <= 4)
// ---------------------------------------------------------------------------

template <typename TA, typename W, typename TO, int KS>
__global__ void __launch_bounds__(256) smallk_kernel(const GemmParams p) {
  constexpr int kLdo = 64 + 16 / static_cast<int>(sizeof(TO));  // staged row stride (elements)
  __shared__ __align__(16) TO stage[4][64 * kLdo];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t tiles_n = (p.N + 127) / 128;
  const int64_t tiles = tiles_n * ((p.M + 127) / 128);
  const int64_t tile = xcd_tile(blockIdx.x, tiles);
  const int64_t m0 = (tile / tiles_n) * 128 + (wave >> 1) * 64;
  const int64_t n0 = (tile % tiles_n) * 128 + (wave & 1) * 64;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int kq = g * 8;
  const TA* A = static_cast<const TA*>(p.a);
  const W* Wt = static_cast<const W*>(p.w);

  u16x8 a[KS][4], b[KS][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + 16 * i + r16;
    const int64_t n = n0 + 16 * i + r16;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      a[s][i] = __builtin_bit_cast(
          u16x8, m < p.M ? load8<TA, W>(A + m * p.lda, 32 * s + kq) : make_uint4(0, 0, 0, 0));
      b[s][i] = __builtin_bit_cast(
          u16x8, n < p.N ? load8<W, W>(Wt + n * p.K, 32 * s + kq) : make_uint4(0, 0, 0, 0));
    }
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<W>(a[s][i], b[s][j], acc[i][j]);

  float bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + 16 * j + r16;
    bv[j] = (p.bias && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
  }
  TO* out = static_cast<TO*>(p.out);
  constexpr int kVec = 16 / static_cast<int>(sizeof(TO));  // elements per 16-byte store
  const bool full = m0 + 64 <= p.M && n0 + 64 <= p.N && p.N % kVec == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  if (!full) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) store_tile<TO>(p, acc[i][j], m0 + 16 * i, n0 + 16 * j + r16, bv[j], lane);
    return;
  }
  // Stage the wave's 64x64 tile in LDS, then write whole 16-byte row pieces.
  TO* st = stage[wave];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        st[(16 * i + 4 * g + e) * kLdo + 16 * j + r16] = from_f32<TO>(acc[i][j][e] + bv[j]);
  wave_sync();
  constexpr int kPieces = 64 * 64 / kVec;
#pragma unroll
  for (int t = 0; t < kPieces / kWave; ++t) {
    const int piece = t * kWave + lane;
    const int row = piece / (64 / kVec);
    const int col = (piece % (64 / kVec)) * kVec;
    *reinterpret_cast<uint4*>(out + (m0 + row) * p.N + n0 + col) =
        *reinterpret_cast<const uint4*>(st + row * kLdo + col);
  }
}

// ---------------------------------------------------------------------------
// 16-bit weights, M <= 64 (decode)
// ---------------------------------------------------------------------------

constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyBatch = 9;  // k-slices whose loads a wave issues together (K = 2304: one round trip)

// One 16x16 output tile per workgroup (grid: N/16 x M/16).  The 8 waves split
// K into 32-wide slices (wave w takes slices w, w+8, ...); each wave issues
// the A and W fragment loads of up to kSkinnyBatch slices at once, so a wave
// pays about one memory round trip per batch, and the 8 partial tiles are
// summed in LDS in a fixed order.
template <typename TA, typename W, typename TO>
__global__ void __launch_bounds__(kSkinnyWaves * kWave) skinny_kernel(const GemmParams p) {
  __shared__ f32x4 part[kSkinnyWaves][kWave];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 16;
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  const TA* A = static_cast<const TA*>(p.a);
  const W* Wt = static_cast<const W*>(p.w);
  const bool n_ok = n0 + r16 < p.N;
  const bool m_ok = m0 + r16 < p.M;
  const W* wrow = Wt + (n_ok ? (n0 + r16) * p.K : 0);
  const TA* arow = A + (m_ok ? (m0 + r16) * p.lda : 0);
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t slices = (p.K + kBK - 1) / kBK;
  for (int64_t s0 = wave; s0 < slices; s0 += kSkinnyWaves * kSkinnyBatch) {
    uint4 a[kSkinnyBatch], b[kSkinnyBatch];
#pragma unroll
    for (int u = 0; u < kSkinnyBatch; ++u) {
      // K is a multiple of 8, so an 8-element chunk is either wholly inside or past K.
      const int64_t k = (s0 + u * kSkinnyWaves) * kBK + kq;
      const bool in = k < p.K;
      b[u] = (n_ok && in) ? load8<W, W>(wrow, k) : make_uint4(0, 0, 0, 0);
      a[u] = (m_ok && in) ? load8<TA, W>(arow, k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kSkinnyBatch; ++u)
      acc = mfma16<W>(__builtin_bit_cast(u16x8, a[u]), __builtin_bit_cast(u16x8, b[u]), acc);
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 sum = part[0][lane];
#pragma unroll
  for (int w = 1; w < kSkinnyWaves; ++w) sum += part[w][lane];
  const int64_t n = n0 + r16;
  const float bv = (p.bias && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
  store_tile<TO>(p, sum, m0, n, bv, lane);
  scatter_tile<TO>(p, sum, m0, n, bv, lane);
}

// ---------------------------------------------------------------------------
// fp32 weights (fp32 MFMA, K steps of 4 per instruction)
// ---------------------------------------------------------------------------

// 64x64 workgroup tile, 2x2 waves of 32x32; 16-element k-slices in LDS.
template <typename TO>
__global__ void __launch_bounds__(256) f32_tile_kernel(const GemmParams p) {
  constexpr int BM = 64, BN = 64, BKF = 16;
  __shared__ float As[BKF][BM + 4];
  __shared__ float Bs[BKF][BN + 4];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t tiles_n = (p.N + BN - 1) / BN;
  const int64_t tiles = tiles_n * ((p.M + BM - 1) / BM);
  const int64_t tile = xcd_tile(blockIdx.x, tiles);
  const int64_t m0 = (tile / tiles_n) * BM;
  const int64_t n0 = (tile % tiles_n) * BN;
  const int wm = (wave >> 1) * 32;
  const int wn = (wave & 1) * 32;
  const float* A = static_cast<const float*>(p.a);
  const float* Wt = static_cast<const float*>(p.w);
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int row = tid >> 2;        // 0..63
  const int kc = (tid & 3) * 4;    // 0,4,8,12
  const int r16 = lane & 15;
  const int k4 = lane >> 4;
  for (int64_t k0 = 0; k0 < p.K; k0 += BKF) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t k = k0 + kc + e;
      const int64_t m = m0 + row, n = n0 + row;
      As[kc + e][row] = (m < p.M && k < p.K) ? A[m * p.lda + k] : 0.0f;
      Bs[kc + e][row] = (n < p.N && k < p.K) ? Wt[n * p.K + k] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BKF; kk += 4) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float av = As[kk + k4][wm + i * 16 + r16];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float bv = Bs[kk + k4][wn + j * 16 + r16];
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i][j], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t n = n0 + wn + j * 16 + r16;
    const float bv = (p.bias && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) store_tile<TO>(p, acc[i][j], m0 + wm + i * 16, n, bv, lane);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

template <typename TA, typename W, typename TO>
hipError_t launch_typed(const GemmParams& p, hipStream_t s) {
  if (p.M <= kSkinnyM) {
    const dim3 grid(static_cast<unsigned>((p.N + 15) / 16), static_cast<unsigned>((p.M + 15) / 16));
    hipLaunchKernelGGL((skinny_kernel<TA, W, TO>), grid, dim3(kSkinnyWaves * kWave), 0, s, p);
    return launch_status("linear");
  }
  const int64_t big = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (p.K <= 128 && p.K % 32 == 0) {
    const dim3 grid(static_cast<unsigned>(big));
    switch (p.K / 32) {
      case 1: hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 1>), grid, dim3(256), 0, s, p); break;
      case 2: hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 2>), grid, dim3(256), 0, s, p); break;
      case 3: hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 3>), grid, dim3(256), 0, s, p); break;
      default: hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 4>), grid, dim3(256), 0, s, p); break;
    }
    return launch_status("linear");
  }
  if (big >= 256) {
    hipLaunchKernelGGL((tile_kernel<TA, W, TO, 128, 128>), dim3(static_cast<unsigned>(big)),
                       dim3(256), 0, s, p);
  } else {
    const int64_t small = ((p.M + 63) / 64) * ((p.N + 127) / 128);
    hipLaunchKernelGGL((tile_kernel<TA, W, TO, 64, 128>), dim3(static_cast<unsigned>(small)),
                       dim3(256), 0, s, p);
  }
  return launch_status("linear");
}

template <typename TA, typename W>
hipError_t launch_out(const GemmParams& p, int out_dtype, hipStream_t s) {
  if (out_dtype == RLM_F32) return launch_typed<TA, W, float>(p, s);
  if (out_dtype == RLM_BF16) return launch_typed<TA, W, bf16>(p, s);
  return launch_typed<TA, W, f16>(p, s);
}

hipError_t linear_impl(const rlm_tensor* input, const rlm_tensor* weight, const rlm_tensor* bias,
                       const rlm_tensor* out, hipStream_t stream, const char* what,
                       const GemmParams* scatter = nullptr) {
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
  if (scatter != nullptr) {
    RLM_REQUIRE(M <= kSkinnyM && weight->dtype != RLM_F32,
                "%s: the cache-row scatter takes at most %d rows and 16-bit weights", what,
                kSkinnyM);
    p.nseg = scatter->nseg;
    for (int s = 0; s < kMaxSegments; ++s) {
      p.seg_lo[s] = scatter->seg_lo[s];
      p.seg_hi[s] = scatter->seg_hi[s];
      p.seg_rows[s] = scatter->seg_rows[s];
      p.seg_dst[s] = scatter->seg_dst[s];
    }
    p.pos = scatter->pos;
    p.pos_dtype = scatter->pos_dtype;
    p.ring = scatter->ring;
  }
  if (M == 0 || N == 0) return hipSuccess;
  RLM_REQUIRE(((M + 63) / 64) * ((N + 63) / 64) <= 0x7fffffff, "%s: problem too large", what);
  if (weight->dtype == RLM_F32) {
    RLM_REQUIRE(input->dtype == RLM_F32, "%s: fp32 weights need fp32 input (got %s)", what,
                dtype_name(input->dtype));
    const dim3 grid(static_cast<unsigned>(((M + 63) / 64) * ((N + 63) / 64)));
    if (out->dtype == RLM_F32)
      hipLaunchKernelGGL((f32_tile_kernel<float>), grid, dim3(256), 0, stream, p);
    else if (out->dtype == RLM_BF16)
      hipLaunchKernelGGL((f32_tile_kernel<bf16>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((f32_tile_kernel<f16>), grid, dim3(256), 0, stream, p);
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
    if (input->dtype == RLM_F32) return launch_out<float, bf16>(p, out->dtype, stream);
    return launch_out<bf16, bf16>(p, out->dtype, stream);
  }
  if (input->dtype == RLM_F32) return launch_out<float, f16>(p, out->dtype, stream);
  return launch_out<f16, f16>(p, out->dtype, stream);
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

extern "C" hipError_t rlm_packed_projection_to_caches(
    const rlm_tensor* memory, const rlm_tensor* weight, const rlm_tensor* out,
    const rlm_tensor* anchor_keys, const rlm_tensor* partner_keys,
    const rlm_tensor* operand_cache, const rlm_tensor* partner_anchor_cache,
    const rlm_tensor* position, int32_t ring, hipStream_t stream) {
  clear_error();
  const char* what = "packed_projection_to_caches";
  RLM_REQUIRE(memory != nullptr && out != nullptr && memory->dtype == out->dtype,
              "%s: output dtype must equal the memory dtype", what);
  RLM_TRY(check_tensor(out, "out", 2));
  const int64_t M = out->shape[0], N = out->shape[1];
  const rlm_tensor* caches[kMaxSegments] = {anchor_keys, partner_keys, operand_cache,
                                            partner_anchor_cache};
  const char* names[kMaxSegments] = {"anchor_keys", "partner_keys", "operand_cache",
                                     "partner_anchor_cache"};
  GemmParams sc{};
  sc.nseg = kMaxSegments;
  int64_t lo = 0;
  for (int s = 0; s < kMaxSegments; ++s) {
    RLM_TRY(check_tensor(caches[s], names[s], 3));
    RLM_TRY(check_dtype_is(caches[s], names[s], out->dtype));
    RLM_TRY(check_dim(caches[s], names[s], 0, M));
    const int64_t rows = caches[s]->shape[1], width = caches[s]->shape[2];
    RLM_REQUIRE(rows >= 1, "%s: empty cache", names[s]);
    if (ring)
      RLM_REQUIRE((rows & (rows - 1)) == 0,
                  "%s: ring-buffer caches need a power-of-two length, got %lld", names[s],
                  (long long)rows);
    sc.seg_lo[s] = lo;
    sc.seg_hi[s] = lo + width;
    sc.seg_rows[s] = rows;
    sc.seg_dst[s] = caches[s]->data;
    lo += width;
  }
  RLM_REQUIRE(lo <= N,
              "%s: the four cache widths (%lld in total) exceed the projection width %lld", what,
              (long long)lo, (long long)N);
  RLM_REQUIRE(position != nullptr && position->ndim == 0 && is_index_dtype(position->dtype) &&
                  position->data != nullptr,
              "position: expected a 0-d int32/int64 device tensor");
  sc.pos = position->data;
  sc.pos_dtype = position->dtype;
  sc.ring = ring ? 1 : 0;
  return linear_impl(memory, weight, nullptr, out, stream, what, &sc);
}

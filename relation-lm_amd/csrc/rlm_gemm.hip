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
//   dma_tile_kernel (M > 64, A of the weight's 16-bit type, K % 64 == 0)
//                 256x256 workgroup tiles of eight waves (128x128 of four
//                 waves, two workgroups per CU, for problems under one tile
//                 per CU) on v_mfma_f32_32x32x16; A and W k-slices of 64 go
//                 from global memory straight into LDS (two stages), the
//                 output is restaged through LDS into whole row segments.
//   tile_kernel   (M > 64, the other cases: fp32 A, K % 64 != 0)
//                 BMxBN workgroup tile (128x128 or 64x128), four
//                 waves in 2x2, each a (BM/2)x(BN/2) grid of 16x16 MFMA tiles.
//                 A and W k-slices of 32 are double-buffered in LDS: the
//                 global loads of slice k+1 are in flight while slice k runs
//                 on the matrix cores.  Workgroups are renumbered so that the
//                 tiles sharing an A row-block run on the same XCD (one L2),
//                 which keeps A's HBM traffic at one read.
//   smallk_kernel (M > 64, K in {32, 64, 96, 128})  e.g. the expanded-cache
//                 projection (K = relation dim).  A workgroup loads its 128-row
//                 A and W tiles for the whole K once, in one round of
//                 branch-free buffer loads, into swizzled LDS; each wave then
//                 forms a 64x64 output tile as (W . A^T) so that a lane holds
//                 four consecutive columns of a row (16-byte stores for fp32
//                 output, 8-byte LDS staging then 16-byte row pieces for 16-bit).
//   skinny_kernel (M <= 64)  decode shapes.  A workgroup owns one 16x16 output
//                 tile; its eight waves split K, each issuing the W and A
//                 fragment loads of up to six 32-wide slices at once straight
//                 from global memory in MFMA operand layout, and the partial
//                 tiles meet once in LDS.
//
// fp32 weights: f32_tile_kernel, 64x64 tiles on v_mfma_f32_16x16x4f32 (fp32
// operands, fp32 accumulation), and f32_skinny_kernel (M <= 64: fp32 FMA dot
// products split over a wave), so fp32 mode never passes through reduced
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
  int64_t ldo;  // output row stride in elements (>= N)
  uint32_t a_bytes, w_bytes;  // descriptor sizes of A and W (smallk_kernel; < 2 GiB)
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
  // Optional split-K (skinny kernel only): grid.z = splits, split z takes
  // slices [z * split_slices, (z + 1) * split_slices) and writes its fp32
  // partial tile, without bias, to part[z][M][N] (the consumer adds the splits).
  int64_t split_slices;
  float* part;
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
    if (m < p.M) out[m * p.ldo + n] = from_f32<TO>(acc[e] + bv);
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

// Eight consecutive elements at element offset `elem` of a TA buffer, as W
// bit patterns, through a range-checked descriptor (`valid` false reads
// zeros): no branch, so a wave's loads all issue back to back.
template <typename TA, typename W>
__device__ __forceinline__ uint4 load8_buf(rsrc_t r, uint32_t elem, bool valid) {
  if constexpr (sizeof(TA) == 2) {
    return buf_load_b128(r, valid ? elem * 2u : kNoOffset);
  } else {
    const uint4 x = buf_load_b128(r, valid ? elem * 4u : kNoOffset);
    const uint4 y = buf_load_b128(r, valid ? elem * 4u + 16u : kNoOffset);
    const float f[8] = {__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                        __uint_as_float(x.w), __uint_as_float(y.x), __uint_as_float(y.y),
                        __uint_as_float(y.z), __uint_as_float(y.w)};
    if constexpr (__is_same(W, bf16)) {
      return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                        pack_bf16x2(f[6], f[7]));
    } else {
      return make_uint4(pack2(to_bits<W>(f[0]), to_bits<W>(f[1])), pack2(to_bits<W>(f[2]), to_bits<W>(f[3])),
                        pack2(to_bits<W>(f[4]), to_bits<W>(f[5])), pack2(to_bits<W>(f[6]), to_bits<W>(f[7])));
    }
  }
}

// LDS of smallk_kernel: the workgroup's A and W tiles, 128 rows x K 16-bit
// elements each, 16-byte piece q of row r stored at piece q ^ (r % SW) (SW
// the largest of 16, 8, 4 dividing K/8) so that the rows of an MFMA fragment
// read spread over the banks.  16-bit outputs are
// staged after the tiles (4 waves x 64 rows x 72), so no wave waits for the
// others before staging.
template <typename TO, int KS>
constexpr size_t smallk_tiles_bytes() {
  return static_cast<size_t>(2 * 128 * 32 * KS * 2);
}
template <typename TO, int KS>
constexpr size_t smallk_lds_bytes() {
  return smallk_tiles_bytes<TO, KS>() + (sizeof(TO) == 2 ? 4 * 64 * 72 * 2 : 0);
}

template <typename TA, typename W, typename TO, int KS>
__global__ void __launch_bounds__(256) smallk_kernel(const GemmParams p) {
  constexpr int K = 32 * KS;
  constexpr int QPR = K / 8;                                // 16-byte pieces per tile row
  // XOR swizzle width: a power of two dividing QPR (and 16), so that piece
  // q ^ (row % SW) stays inside the row and a fragment's rows r16 use r16 % SW.
  constexpr int SW = QPR % 16 == 0 ? 16 : (QPR % 8 == 0 ? 8 : 4);
  constexpr int kVec = 16 / static_cast<int>(sizeof(TO));  // outputs per 16-byte store
  constexpr int kLdo = 64 + kVec;                           // staged output row stride (elements)
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* tile_a = smem;
  unsigned char* tile_w = smem + 128 * K * 2;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t tiles_n = (p.N + 127) / 128;
  const int64_t tiles = tiles_n * ((p.M + 127) / 128);
  const int64_t tile = xcd_tile(blockIdx.x, tiles);
  const int64_t mt = (tile / tiles_n) * 128;
  const int64_t nt = (tile % tiles_n) * 128;
  const int64_t m0 = mt + (wave >> 1) * 64;
  const int64_t n0 = nt + (wave & 1) * 64;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const rsrc_t ar = make_rsrc(p.a, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.w, p.w_bytes);

  // The tiles, once per workgroup, all loads in flight together.
  constexpr int kPer = 128 * QPR / 256;  // pieces per thread per tile
  uint4 va[kPer], vw[kPer];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int piece = t * 256 + tid;
    const int row = piece / QPR, q = piece % QPR;
    const int64_t m = mt + row, n = nt + row;
    va[t] = load8_buf<TA, W>(ar, static_cast<uint32_t>(m * p.lda + 8 * q), m < p.M);
    vw[t] = load8_buf<W, W>(wr, static_cast<uint32_t>(n * K + 8 * q), n < p.N);
  }
  TO* out = static_cast<TO*>(p.out);
  const bool full = m0 + 64 <= p.M && n0 + 64 <= p.N && p.ldo % kVec == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  // Bias of this lane's output columns n0 + 16j + 4g .. +3 on full tiles: one
  // 16-byte (fp32) or 8-byte (16-bit) load per j, the other form out of range
  // (edge tiles load theirs after the products).
  const bool is32 = p.bias_dtype == RLM_F32;
  const bool vec_bias = full && p.bias != nullptr;
  const rsrc_t br = make_rsrc(p.bias, static_cast<uint32_t>(p.N * (is32 ? 4 : 2)));
  uint4 bq[4];
  uint2 bh[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t n = static_cast<uint32_t>(n0 + 16 * j + 4 * g);
    bq[j] = buf_load_b128(br, vec_bias && is32 ? 4u * n : kNoOffset);
    bh[j] = buf_load_b64(br, vec_bias && !is32 ? 2u * n : kNoOffset);
  }
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const int piece = t * 256 + tid;
    const int row = piece / QPR, q = piece % QPR;
    const int at = row * (2 * K) + 16 * (q ^ (row % SW));
    *reinterpret_cast<uint4*>(tile_a + at) = va[t];
    *reinterpret_cast<uint4*>(tile_w + at) = vw[t];
  }
  __syncthreads();

  // Transposed product: acc[i][j] = (W . A^T) tile, so lane (r16, g) holds
  // out[m0 + 16i + r16][n0 + 16j + 4g + e], four consecutive columns of a row.
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int ra = (wave >> 1) * 64 + r16, rw = (wave & 1) * 64 + r16;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int q = 4 * s + g;  // piece of k = 32s + 8g
    u16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = *reinterpret_cast<const u16x8*>(tile_a + (ra + 16 * i) * (2 * K) + 16 * (q ^ (r16 % SW)));
      b[i] = *reinterpret_cast<const u16x8*>(tile_w + (rw + 16 * i) * (2 * K) + 16 * (q ^ (r16 % SW)));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<W>(b[j], a[i], acc[i][j]);
  }

  float bv[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w16[4] = {bh[j].x & 0xffffu, bh[j].x >> 16, bh[j].y & 0xffffu, bh[j].y >> 16};
    const uint32_t w32[4] = {bq[j].x, bq[j].y, bq[j].z, bq[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (vec_bias) {
        bv[j][e] = decode_float(FloatWords{w32[e], w16[e]}, p.bias_dtype);
      } else {
        const int64_t n = n0 + 16 * j + 4 * g + e;
        bv[j][e] = (p.bias && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
      }
    }
  }
  if (!full) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + 16 * i + r16;
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t n = n0 + 16 * j + 4 * g + e;
          if (n < p.N) out[m * p.ldo + n] = from_f32<TO>(acc[i][j][e] + bv[j][e]);
        }
    }
    return;
  }
  if constexpr (sizeof(TO) == 4) {
    // fp32: a lane's four columns are one 16-byte store.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(out + (m0 + 16 * i + r16) * p.ldo + n0 + 16 * j + 4 * g) =
            make_float4(acc[i][j][0] + bv[j][0], acc[i][j][1] + bv[j][1], acc[i][j][2] + bv[j][2],
                        acc[i][j][3] + bv[j][3]);
  } else {
    // 16-bit: stage the wave's 64x64 tile in LDS (8-byte writes), then write
    // whole 16-byte row pieces.
    TO* st = reinterpret_cast<TO*>(smem + smallk_tiles_bytes<TO, KS>()) + wave * 64 * kLdo;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        put4<TO>(st + (16 * i + r16) * kLdo + 16 * j + 4 * g, acc[i][j][0] + bv[j][0],
                 acc[i][j][1] + bv[j][1], acc[i][j][2] + bv[j][2], acc[i][j][3] + bv[j][3]);
    wave_sync();
    constexpr int kPieces = 64 * 64 / kVec;
#pragma unroll
    for (int t = 0; t < kPieces / kWave; ++t) {
      const int piece = t * kWave + lane;
      const int row = piece / (64 / kVec);
      const int col = (piece % (64 / kVec)) * kVec;
      *reinterpret_cast<uint4*>(out + (m0 + row) * p.ldo + n0 + col) =
          *reinterpret_cast<const uint4*>(st + row * kLdo + col);
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit weights, M <= 64 (decode)
// ---------------------------------------------------------------------------

constexpr int kSkinnyWaves = 8;
// k-slices whose loads a wave issues together: 9 covers K = 2304 in one round
// trip; K <= 768 (the 576-wide packed projection) needs only 3 per wave.
constexpr int kSkinnyBatchLong = 9;
constexpr int kSkinnyBatchShort = 3;

// One 16x16 output tile per workgroup (grid: N/16 x M/16).  The 8 waves split
// K into 32-wide slices (wave w takes slices w, w+8, ...); each wave issues
// the A and W fragment loads of up to kSkinnyBatch slices at once, so a wave
// pays about one memory round trip per batch, and the 8 partial tiles are
// summed in LDS in a fixed order.
template <typename TA, typename W, typename TO, int kSkinnyBatch>
__global__ void __launch_bounds__(kSkinnyWaves * kWave) skinny_kernel(const GemmParams p) {
  __shared__ f32x4 part[kSkinnyWaves][kWave];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: scalar branches below
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 16;
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  const bool n_ok = n0 + r16 < p.N;
  const bool m_ok = m0 + r16 < p.M;
  const rsrc_t ar = make_rsrc(p.a, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  const uint32_t arow = static_cast<uint32_t>((m0 + r16) * p.lda * static_cast<int64_t>(sizeof(TA)));
  const uint32_t wrow = static_cast<uint32_t>((n0 + r16) * p.K * static_cast<int64_t>(sizeof(W)));
  // The bias of this lane's column, issued now (both dtype forms, one kept)
  // and used after the reduction: no load waits at the end on its own.
  const bool has_bias = p.bias != nullptr && n_ok && wave == 0;
  const FloatWords bias_w = issue_float(p.bias, p.bias_dtype, static_cast<uint32_t>(p.N),
                                        static_cast<uint32_t>(n_ok ? n0 + r16 : 0), has_bias);
  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t all_slices = (p.K + kBK - 1) / kBK;
  // Split-K: this workgroup's slices [s_lo, slices).
  const int64_t s_lo = p.part != nullptr ? static_cast<int64_t>(blockIdx.z) * p.split_slices : 0;
  const int64_t slices = p.part != nullptr ? min(all_slices, s_lo + p.split_slices) : all_slices;
  for (int64_t s0 = s_lo + wave; s0 < slices; s0 += kSkinnyWaves * kSkinnyBatch) {
    // All raw loads of the batch first (from clamped, valid addresses: no
    // branch), then the conversions and products, so the wave pays one memory
    // round trip per batch.  fp32 inputs are two 16-byte loads per fragment.
    constexpr int kAParts = sizeof(TA) == 4 ? 2 : 1;
    // Range-checked buffer loads: rows past M or N and slots past K get an
    // out-of-range offset (no memory access, zeros), so there is no branch and
    // no dummy traffic.
    uint4 araw[kSkinnyBatch][kAParts], braw[kSkinnyBatch];
#pragma unroll
    for (int u = 0; u < kSkinnyBatch; ++u) {
      // K is a multiple of 8, so an 8-element chunk is either wholly inside or past K.
      const int64_t su = s0 + u * kSkinnyWaves;
      const int64_t k = su * kBK + kq;
      const bool in = su < slices && k < p.K;
      const uint32_t kb = static_cast<uint32_t>(in ? k : 0);
      braw[u] = buf_load_b128(wr, n_ok && in ? wrow + kb * static_cast<uint32_t>(sizeof(W)) : kNoOffset);
#pragma unroll
      for (int h = 0; h < kAParts; ++h)
        araw[u][h] = buf_load_b128(
            ar, m_ok && in ? arow + (kb + 4 * h) * static_cast<uint32_t>(sizeof(TA)) : kNoOffset);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kSkinnyBatch; ++u) {
      uint4 av;
      if constexpr (kAParts == 1) {
        av = araw[u][0];
      } else {
        const uint4 x = araw[u][0], y = araw[u][1];
        if constexpr (__is_same(W, bf16)) {
          av = make_uint4(pack_bf16x2(__uint_as_float(x.x), __uint_as_float(x.y)),
                          pack_bf16x2(__uint_as_float(x.z), __uint_as_float(x.w)),
                          pack_bf16x2(__uint_as_float(y.x), __uint_as_float(y.y)),
                          pack_bf16x2(__uint_as_float(y.z), __uint_as_float(y.w)));
        } else {
          av = make_uint4(pack2(to_bits<W>(__uint_as_float(x.x)), to_bits<W>(__uint_as_float(x.y))),
                          pack2(to_bits<W>(__uint_as_float(x.z)), to_bits<W>(__uint_as_float(x.w))),
                          pack2(to_bits<W>(__uint_as_float(y.x)), to_bits<W>(__uint_as_float(y.y))),
                          pack2(to_bits<W>(__uint_as_float(y.z)), to_bits<W>(__uint_as_float(y.w))));
        }
      }
      // Out-of-range loads already read zeros.
      acc = mfma16<W>(__builtin_bit_cast(u16x8, av), __builtin_bit_cast(u16x8, braw[u]), acc);
    }
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 sum = part[0][lane];
#pragma unroll
  for (int w = 1; w < kSkinnyWaves; ++w) sum += part[w][lane];
  const int64_t n = n0 + r16;
  if (p.part != nullptr) {  // split-K partial: fp32, no bias
    if (n < p.N) {
      float* dst = p.part + static_cast<int64_t>(blockIdx.z) * p.M * p.N;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + (lane >> 4) * 4 + e;
        if (m < p.M) dst[m * p.N + n] = sum[e];
      }
    }
    return;
  }
  const float bv = has_bias ? decode_float(bias_w, p.bias_dtype) : 0.0f;
  store_tile<TO>(p, sum, m0, n, bv, lane);
  scatter_tile<TO>(p, sum, m0, n, bv, lane);
}

// ---------------------------------------------------------------------------
// fp32 weights, M <= 64 (decode)
// ---------------------------------------------------------------------------

constexpr int kF32SkinnyCols = 2;    // output columns per wave
constexpr int kF32SkinnyRows = 8;    // rows of A per workgroup (grid.y)
constexpr int kF32SkinnyPieces = 3;  // 4-element pieces per lane per pass (768 of K)

// One wave per pair of output columns, four waves per workgroup, eight rows
// of A per workgroup.  The lanes split K in 16-byte pieces; every load of a
// pass (both W rows, the A rows) is issued before the first product, through
// range-checked buffer loads (pieces past K, rows past M or N read zero, so
// there is no branch), then each of the 8 x 2 dot products is summed over the
// wave and lane 2r + c writes output (m0 + r, n0 + c).  fp32 FMA throughout:
// the fp32 path never passes through reduced precision.
template <typename TO>
__global__ void __launch_bounds__(256) f32_skinny_kernel(const GemmParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kF32SkinnyCols;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kF32SkinnyRows;
  const rsrc_t ar = make_rsrc(p.a, p.a_bytes);
  const rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  float acc[kF32SkinnyRows][kF32SkinnyCols];
#pragma unroll
  for (int r = 0; r < kF32SkinnyRows; ++r)
#pragma unroll
    for (int c = 0; c < kF32SkinnyCols; ++c) acc[r][c] = 0.0f;
  for (int64_t k0 = 0; k0 < p.K; k0 += kWave * 4 * kF32SkinnyPieces) {
    uint4 wv[kF32SkinnyCols][kF32SkinnyPieces], av[kF32SkinnyRows][kF32SkinnyPieces];
#pragma unroll
    for (int j = 0; j < kF32SkinnyPieces; ++j) {
      const int64_t k = k0 + (j * kWave + lane) * 4;
#pragma unroll
      for (int c = 0; c < kF32SkinnyCols; ++c) {
        const int64_t n = n0 + c;
        wv[c][j] = buf_load_b128(wr, n < p.N && k < p.K ? static_cast<uint32_t>((n * p.K + k) * 4)
                                                        : kNoOffset);
      }
#pragma unroll
      for (int r = 0; r < kF32SkinnyRows; ++r) {
        const int64_t m = m0 + r;
        av[r][j] = buf_load_b128(ar, m < p.M && k < p.K ? static_cast<uint32_t>((m * p.lda + k) * 4)
                                                        : kNoOffset);
      }
    }
#pragma unroll
    for (int j = 0; j < kF32SkinnyPieces; ++j)
#pragma unroll
      for (int r = 0; r < kF32SkinnyRows; ++r)
#pragma unroll
        for (int c = 0; c < kF32SkinnyCols; ++c) {
          float s = acc[r][c];
          s = fmaf(__uint_as_float(av[r][j].x), __uint_as_float(wv[c][j].x), s);
          s = fmaf(__uint_as_float(av[r][j].y), __uint_as_float(wv[c][j].y), s);
          s = fmaf(__uint_as_float(av[r][j].z), __uint_as_float(wv[c][j].z), s);
          acc[r][c] = fmaf(__uint_as_float(av[r][j].w), __uint_as_float(wv[c][j].w), s);
        }
  }
  TO* out = static_cast<TO*>(p.out);
#pragma unroll
  for (int r = 0; r < kF32SkinnyRows; ++r)
#pragma unroll
    for (int c = 0; c < kF32SkinnyCols; ++c) {
      const float sum = wave_sum_f32(acc[r][c]);
      const int64_t m = m0 + r, n = n0 + c;
      if (lane == r * kF32SkinnyCols + c && m < p.M && n < p.N) {
        const float bv = p.bias ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
        out[m * p.ldo + n] = from_f32<TO>(sum + bv);
      }
    }
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
// 16-bit A and W, large M, K % BK == 0: macro tiles fed by LDS DMA
// ---------------------------------------------------------------------------
//
// A workgroup of WM x WN waves owns a BM x BN output tile; each wave a
// (BM/WM) x (BN/WN) grid of 32x32 blocks on v_mfma_f32_32x32x16_{bf16,f16}.
// k advances in BK-wide slices (32 or 64).  A slice's A and W rows go from
// global memory straight into LDS (lds_dma16: no VGPRs, no LDS write
// instructions) into one of NS stages; the DMA of slice s + NS is issued as
// soon as every wave has read slice s, so a DMA has NS - 1 slices of matrix
// work to land (global-memory latency under load is a few thousand cycles,
// one 256x256x32 slice about a thousand).  Within a slice the fragments of
// the next 16-wide k-group are read while the current group's MFMAs run, and
// the barrier that publishes the next slice sits before the slice's last
// MFMA group, so its first fragment reads overlap matrix work too.
//
// LDS tile rows are BK*2 bytes; 16-byte piece q of row r is stored at piece
// q ^ swz(r): the 16 rows a fragment read serves together land on 16 distinct
// 16-byte bank groups, whether the LDS serves 8 or 16 lanes of a 16-byte read
// per cycle.  A DMA instruction writes 64 consecutive 16-byte pieces, so the
// swizzle is applied on the global side: each lane fetches the piece that
// belongs at its LDS position.
//
// The product is computed transposed, out^T = W . A^T, so that a lane holds
// four consecutive columns of one output row (16-byte fp32 stores).

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename W>
__device__ __forceinline__ f32x16 mfma32(const u16x8& a, const u16x8& b, const f32x16& c);
template <>
__device__ __forceinline__ f32x16 mfma32<bf16>(const u16x8& a, const u16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<f16>(const u16x8& a, const u16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Piece swizzle of tile row r (only r % 16 matters) for BK-wide rows.
template <int BK>
__device__ __forceinline__ int dma_swz(int r) {
  if constexpr (BK == 64) return (r & 7) ^ ((r >> 3) & 1);   // 8 pieces per row
  else return ((r >> 1) & 3) ^ ((r >> 3) & 1);              // 4 pieces per row
}

// NS stages of the A and W tiles, then the tile's BN bias columns (fp32).
constexpr int kDmaSliceK = 64;  // k-slice of the production configurations

template <int BM, int BN, int NS, int BK>
constexpr size_t dma_lds_bytes() {
  return static_cast<size_t>(NS) * (BM + BN) * BK * 2 + BN * 4;
}

// Epilogue of the DMA tile kernels.  Lane holds out[m][n .. n+3] of block
// (j, i) for m = m0 + wm0 + 32i + (lane & 31), n = n0 + wn0 + 32j + 8q +
// 4 (lane >> 5), q = 0..3 (acc elements 4q .. 4q+3); the bias of the tile's
// columns comes from LDS (bias_lds[c] = bias[n0 + c], zero past N or without
// a bias).  Each wave restages one 32-row block at a time in its own LDS
// region (rows padded by 16 bytes) and writes it back as whole 16-byte pieces
// of consecutive columns, so a store instruction covers two or more complete
// row segments instead of 32 rows x 32 bytes.  The caller has passed a
// barrier after the last LDS read of the main loop.
template <typename TO, int TMB, int TNB>
__device__ __forceinline__ void dma_epilogue(const GemmParams& p, const f32x16 (&acc)[TNB][TMB],
                                             const float* bias_lds, unsigned char* stage,
                                             int64_t m0, int64_t n0, int wm0, int wn0, int lane) {
  constexpr int kSz = static_cast<int>(sizeof(TO));
  constexpr int WC = 32 * TNB;                 // columns of the wave's block
  constexpr int RS = WC * kSz + 16;            // staged row stride (bytes)
  constexpr int kPiecesRow = WC * kSz / 16;    // 16-byte pieces per staged row
  constexpr int kVec = 16 / kSz;               // outputs per piece
  static_assert((32 * kPiecesRow) % kWave == 0, "whole store rounds");
  float4 bv[TNB][4];
#pragma unroll
  for (int j = 0; j < TNB; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      bv[j][q] = *reinterpret_cast<const float4*>(bias_lds + wn0 + 32 * j + 8 * q + 4 * (lane >> 5));
  TO* out = static_cast<TO*>(p.out);
#pragma unroll
  for (int i = 0; i < TMB; ++i) {
#pragma unroll
    for (int j = 0; j < TNB; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        put4<TO>(reinterpret_cast<TO*>(stage + (lane & 31) * RS +
                                       (32 * j + 8 * q + 4 * (lane >> 5)) * kSz),
                 acc[j][i][4 * q] + bv[j][q].x, acc[j][i][4 * q + 1] + bv[j][q].y,
                 acc[j][i][4 * q + 2] + bv[j][q].z, acc[j][i][4 * q + 3] + bv[j][q].w);
    wave_sync();
#pragma unroll
    for (int t = 0; t < 32 * kPiecesRow / kWave; ++t) {
      const int piece = t * kWave + lane;
      const int row = piece / kPiecesRow, col = (piece % kPiecesRow) * kVec;
      const int64_t m = m0 + wm0 + 32 * i + row;
      const int64_t n = n0 + wn0 + col;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + row * RS + col * kSz);
      if (m < p.M) {
        TO* dst = out + m * p.ldo + n;
        if (n + kVec <= p.N) {
          *reinterpret_cast<uint4*>(dst) = v;
        } else {
          const TO* e = reinterpret_cast<const TO*>(&v);
#pragma unroll
          for (int k = 0; k < kVec; ++k)
            if (n + k < p.N) dst[k] = e[k];
        }
      }
    }
    wave_sync();
  }
}

// Bytes of one wave's epilogue staging region.
template <typename TO, int TNB>
constexpr int dma_stage_region() {
  return 32 * (32 * TNB * static_cast<int>(sizeof(TO)) + 16);
}

// Bias of tile columns n0 .. n0 + BN - 1 into LDS (threads t < BN, one column
// each); the caller's next barrier publishes it.
template <int BN>
__device__ __forceinline__ void dma_stage_bias(const GemmParams& p, float* bias_lds, int64_t n0) {
  const int t = threadIdx.x;
  if (t < BN) {
    const int64_t n = n0 + t;
    bias_lds[t] = (p.bias != nullptr && n < p.N) ? load_any_f(p.bias, p.bias_dtype, n) : 0.0f;
  }
}

template <typename W, typename TO, int BM, int BN, int WM, int WN, int NS, int BK>
__global__ void __launch_bounds__(WM * WN * kWave) dma_tile_kernel(const GemmParams p) {
  constexpr int kWaves = WM * WN;
  constexpr int TMB = BM / WM / 32;         // 32-row blocks of A per wave
  constexpr int TNB = BN / WN / 32;         // 32-row blocks of W per wave
  constexpr int KK = BK / 16;               // MFMA k-groups per slice
  constexpr int RB = BK * 2;                // bytes per LDS tile row
  constexpr int PR = BK / 8;                // 16-byte pieces per row
  constexpr int RPI = kWave / PR;           // rows per DMA instruction
  constexpr int kStage = (BM + BN) * RB;
  constexpr int kLoadsA = BM / RPI / kWaves;  // DMA instructions per wave per slice
  constexpr int kLoadsB = BN / RPI / kWaves;
  constexpr int L = kLoadsA + kLoadsB;
  static_assert(BK == 32 || BK == 64, "32- or 64-wide k-slices");
  static_assert(BM % (RPI * kWaves) == 0 && BN % (RPI * kWaves) == 0, "whole DMA row groups per wave");
  static_assert(NS >= 2 && (NS - 1) * L <= 63, "stages within the vmcnt range");
  static_assert(KK % 2 == 0, "fragment double buffer alternates within a slice");
  static_assert(WM * WN * kWave >= BN, "one thread per bias column");
  static_assert(kWaves * dma_stage_region<TO, TNB>() <= NS * kStage, "epilogue staging fits the stages");
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int64_t tiles_n = (p.N + BN - 1) / BN;
  const int64_t tiles = tiles_n * ((p.M + BM - 1) / BM);
  const int64_t tile = xcd_tile(blockIdx.x, tiles);
  const int64_t m0 = (tile / tiles_n) * BM;
  const int64_t n0 = (tile % tiles_n) * BN;

  // Descriptors based at the tile's first row; their sizes end with the
  // matrices' last elements (clipped below 2 GiB: the host checks that a
  // tile's rows lie within that), so rows past M or N read zeros.
  const int64_t a_left = ((p.M - 1 - m0) * p.lda + p.K) * 2;
  const int64_t w_left = (p.N - n0) * p.K * 2;
  const rsrc_t ar = make_rsrc(static_cast<const unsigned char*>(p.a) + m0 * p.lda * 2,
                              static_cast<uint32_t>(a_left < 0x7fffffff ? a_left : 0x7fffffff));
  const rsrc_t wr = make_rsrc(static_cast<const unsigned char*>(p.w) + n0 * p.K * 2,
                              static_cast<uint32_t>(w_left < 0x7fffffff ? w_left : 0x7fffffff));
  const uint32_t a_row_bytes = static_cast<uint32_t>(p.lda * 2);
  const uint32_t w_row_bytes = static_cast<uint32_t>(p.K * 2);

  // DMA lane roles: row (lane / PR) of a RPI-row group, LDS piece (lane % PR).
  // The group's row offset modulo 16 is 0 or 8 (h, for 8-row groups).
  const int sub = lane / PR, pc = lane % PR;
  uint32_t a_off[2], w_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t q = static_cast<uint32_t>(pc ^ dma_swz<BK>(8 * h + sub)) << 4;
    a_off[h] = sub * a_row_bytes + q;
    w_off[h] = sub * w_row_bytes + q;
  }
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  auto issue = [&](int stage, int slice) {
    const uint32_t st = lds0 + stage * kStage;
    const uint32_t kb = static_cast<uint32_t>(slice) * RB;
#pragma unroll
    for (int j = 0; j < kLoadsA; ++j) {
      const int g = wave * kLoadsA + j;
      lds_dma16(ar, st + g * RPI * RB, a_off[(g * RPI / 8) & 1], kb + g * RPI * a_row_bytes);
    }
#pragma unroll
    for (int j = 0; j < kLoadsB; ++j) {
      const int g = wave * kLoadsB + j;
      lds_dma16(wr, st + (BM + g * RPI) * RB, w_off[(g * RPI / 8) & 1], kb + g * RPI * w_row_bytes);
    }
  };

  // Fragment roles: row (lane & 31) of a 32-row block, k-half (lane >> 5).
  const int wm0 = (wave / WN) * (BM / WM);
  const int wn0 = (wave % WN) * (BN / WN);
  const int swz = dma_swz<BK>(lane & 15);
  int frag_off[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) frag_off[kk] = (lane & 31) * RB + (((2 * kk + (lane >> 5)) ^ swz) << 4);

  u16x8 fa[2][TMB], fw[2][TNB];
  auto read_frags = [&](int buf, int stage, int kk) {
    const unsigned char* st = smem + stage * kStage;
#pragma unroll
    for (int i = 0; i < TMB; ++i)
      fa[buf][i] = *reinterpret_cast<const u16x8*>(st + (wm0 + 32 * i) * RB + frag_off[kk]);
#pragma unroll
    for (int j = 0; j < TNB; ++j)
      fw[buf][j] = *reinterpret_cast<const u16x8*>(st + (BM + wn0 + 32 * j) * RB + frag_off[kk]);
  };

  f32x16 acc[TNB][TMB];
#pragma unroll
  for (int j = 0; j < TNB; ++j)
#pragma unroll
    for (int i = 0; i < TMB; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.0f;

  const int slices = static_cast<int>(p.K / BK);
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (s < slices) issue(s, s);
  float* bias_lds = reinterpret_cast<float*>(smem + NS * kStage);
  dma_stage_bias<BN>(p, bias_lds, n0);
  if (slices >= NS) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 1) * L));
  } else {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  }
  __syncthreads();
  read_frags(0, 0, 0);
  int stage = 0;
  for (int s = 0; s < slices; ++s) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) {
        read_frags((kk + 1) & 1, stage, kk + 1);
      } else if (s + 1 < slices) {
        // Slice s + 1 has landed once this wave's DMAs up to it are done
        // and every wave has passed the barrier; after the barrier no wave
        // reads slice s again, so its stage takes slice s + NS.
        if (s + NS - 1 < slices) {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * L));
        } else {
          __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        __syncthreads();
        if (s + NS < slices) issue(stage, s + NS);
        stage = stage + 1 == NS ? 0 : stage + 1;
        read_frags(0, stage, 0);
      }
#pragma unroll
      for (int j = 0; j < TNB; ++j)
#pragma unroll
        for (int i = 0; i < TMB; ++i) acc[j][i] = mfma32<W>(fw[kk & 1][j], fa[kk & 1][i], acc[j][i]);
    }
  }

  __syncthreads();  // every wave has read its last fragments: the stages are free
  dma_epilogue<TO, TMB, TNB>(p, acc, bias_lds, smem + wave * dma_stage_region<TO, TNB>(), m0, n0,
                             wm0, wn0, lane);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// The DMA tile kernel at one configuration: LDS above 64 KiB is a
// per-process function attribute, set on first use.
template <typename W, typename TO, int BM, int BN, int WM, int WN, int NS, int BK>
hipError_t launch_dma(const GemmParams& p, hipStream_t s) {
  constexpr size_t lds = dma_lds_bytes<BM, BN, NS, BK>();
  auto kernel = &dma_tile_kernel<W, TO, BM, BN, WM, WN, NS, BK>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(lds));
  if (attr != hipSuccess) {
    set_error("linear: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
    return attr;
  }
  const int64_t tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(tiles)), dim3(WM * WN * kWave), lds, s, p);
  return launch_status("linear");
}

// Whether the DMA tile kernel takes this problem: 16-bit A of the weight's
// type, whole 64-wide k-slices, 16-byte aligned rows of A, W and out, and a
// tile's rows of A and W within the 2 GiB its descriptors address.
template <typename TA, typename W, typename TO>
bool dma_fits(const GemmParams& p) {
  if constexpr (!__is_same(TA, W)) {
    return false;
  } else {
    constexpr int64_t kLimit = int64_t(1) << 31;
    return p.K % kDmaSliceK == 0 && p.lda % 8 == 0 &&
           (p.ldo * static_cast<int64_t>(sizeof(TO))) % 16 == 0 &&
           (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0 && 256 * p.lda * 2 < kLimit &&
           256 * p.K * 2 < kLimit;
  }
}

template <typename TA, typename W, typename TO>
hipError_t launch_typed(const GemmParams& p, hipStream_t s) {
  if (p.M <= kSkinnyM && p.a_bytes != 0) {
    const dim3 grid(static_cast<unsigned>((p.N + 15) / 16), static_cast<unsigned>((p.M + 15) / 16));
    if (p.K <= kSkinnyWaves * kSkinnyBatchShort * kBK)
      hipLaunchKernelGGL((skinny_kernel<TA, W, TO, kSkinnyBatchShort>), grid,
                         dim3(kSkinnyWaves * kWave), 0, s, p);
    else
      hipLaunchKernelGGL((skinny_kernel<TA, W, TO, kSkinnyBatchLong>), grid,
                         dim3(kSkinnyWaves * kWave), 0, s, p);
    return launch_status("linear");
  }
  const int64_t big = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (p.K <= 128 && p.K % 32 == 0 && p.a_bytes != 0) {
    const dim3 grid(static_cast<unsigned>(big));
    switch (p.K / 32) {
      case 1: {
        constexpr size_t lds = smallk_lds_bytes<TO, 1>();
        // The LDS opt-in above 64 KiB is a per-process function attribute.
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&smallk_kernel<TA, W, TO, 1>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr != hipSuccess) {
          set_error("linear: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
          return attr;
        }
        hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 1>), grid, dim3(256), lds, s, p);
        break;
      }
      case 2: {
        constexpr size_t lds = smallk_lds_bytes<TO, 2>();
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&smallk_kernel<TA, W, TO, 2>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr != hipSuccess) {
          set_error("linear: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
          return attr;
        }
        hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 2>), grid, dim3(256), lds, s, p);
        break;
      }
      case 3: {
        constexpr size_t lds = smallk_lds_bytes<TO, 3>();
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&smallk_kernel<TA, W, TO, 3>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr != hipSuccess) {
          set_error("linear: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
          return attr;
        }
        hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 3>), grid, dim3(256), lds, s, p);
        break;
      }
      default: {
        constexpr size_t lds = smallk_lds_bytes<TO, 4>();
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&smallk_kernel<TA, W, TO, 4>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr != hipSuccess) {
          set_error("linear: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
          return attr;
        }
        hipLaunchKernelGGL((smallk_kernel<TA, W, TO, 4>), grid, dim3(256), lds, s, p);
        break;
      }
    }
    return launch_status("linear");
  }
  if (dma_fits<TA, W, TO>(p)) {
    // 256x256 tiles (eight waves of 128x64) once they fill the chip; 128x128
    // (four waves, two workgroups per CU) below that.
    if (((p.M + 255) / 256) * ((p.N + 255) / 256) >= 256)
      return launch_dma<W, TO, 256, 256, 2, 4, 2, kDmaSliceK>(p, s);
    return launch_dma<W, TO, 128, 128, 2, 2, 2, kDmaSliceK>(p, s);
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
  RLM_TRY(check_rows(out, "out"));
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
  p.ldo = M > 1 ? out->stride[0] : N;
  {
    // Byte extents of A (last row counts K elements) and W; 0 marks "too large
    // for 32-bit buffer offsets" (the tile kernels take it then).
    const int64_t ab = M > 0 ? ((M - 1) * p.lda + K) * dtype_size(input->dtype) : 0;
    const int64_t wb = N * K * dtype_size(weight->dtype);
    const bool fits = ab < (int64_t(1) << 31) && wb < (int64_t(1) << 31);
    p.a_bytes = fits ? static_cast<uint32_t>(ab) : 0u;
    p.w_bytes = fits ? static_cast<uint32_t>(wb) : 0u;
  }
  if (scatter != nullptr) {
    RLM_REQUIRE(p.a_bytes != 0, "%s: the cache-row scatter needs the input within 2 GiB", what);
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
    if (M <= kSkinnyM && p.a_bytes != 0 && K % 4 == 0 && p.lda % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(input->data) & 15u) == 0 &&
        (reinterpret_cast<uintptr_t>(weight->data) & 15u) == 0) {
      const dim3 grid(static_cast<unsigned>((N + 4 * kF32SkinnyCols - 1) / (4 * kF32SkinnyCols)),
                      static_cast<unsigned>((M + kF32SkinnyRows - 1) / kF32SkinnyRows));
      if (out->dtype == RLM_F32)
        hipLaunchKernelGGL((f32_skinny_kernel<float>), grid, dim3(256), 0, stream, p);
      else if (out->dtype == RLM_BF16)
        hipLaunchKernelGGL((f32_skinny_kernel<bf16>), grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL((f32_skinny_kernel<f16>), grid, dim3(256), 0, stream, p);
      return launch_status(what);
    }
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

// Split-K partial products of the skinny GEMM: part[z] = input @ weight^T over
// reduction slices [z * split_slices * 32, ...), fp32, no bias (declared in
// rlm_common.hpp; the consumer sums the splits).  input [M<=64, K] fp32 or
// 16-bit, weight [N, K] bf16/f16, part [splits, M, N] fp32.
hipError_t linear_partials_impl(const rlm_tensor* input, const rlm_tensor* weight,
                                const rlm_tensor* part, hipStream_t stream) {
  const char* what = "linear partials";
  RLM_TRY(check_rows(input, "input"));
  RLM_TRY(check_tensor(weight, "weight", 2));
  RLM_TRY(check_tensor(part, "partials", 3));
  RLM_TRY(check_dtype_is(part, "partials", RLM_F32));
  const int64_t M = input->shape[0], K = input->shape[1], N = weight->shape[0];
  const int64_t splits = part->shape[0];
  RLM_TRY(check_dim(weight, "weight", 1, K));
  RLM_TRY(check_dim(part, "partials", 1, M));
  RLM_TRY(check_dim(part, "partials", 2, N));
  RLM_REQUIRE(weight->dtype == RLM_BF16 || weight->dtype == RLM_F16,
              "%s: 16-bit weights required", what);
  RLM_REQUIRE(input->dtype == RLM_F32 || input->dtype == weight->dtype,
              "%s: input must be fp32 or share the weight dtype", what);
  RLM_REQUIRE(M >= 1 && M <= kSkinnyM && splits >= 1 && splits <= 64,
              "%s: 1..%d rows and 1..64 splits", what, kSkinnyM);
  const int64_t lda = M > 1 ? input->stride[0] : K;
  RLM_REQUIRE(K % 8 == 0 && lda % 8 == 0, "%s: reduction dim and row stride must be multiples of 8", what);
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(input->data) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(weight->data) & 15u) == 0,
              "%s: input and weight must be 16-byte aligned", what);
  const int64_t ab = ((M - 1) * lda + K) * dtype_size(input->dtype);
  const int64_t wb = N * K * dtype_size(weight->dtype);
  RLM_REQUIRE(ab < (int64_t(1) << 31) && wb < (int64_t(1) << 31), "%s: operands over 2 GiB", what);
  GemmParams p{};
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.a = input->data;
  p.w = weight->data;
  p.bias_dtype = RLM_F32;
  p.out = part->data;
  p.ldo = N;
  p.a_bytes = static_cast<uint32_t>(ab);
  p.w_bytes = static_cast<uint32_t>(wb);
  const int64_t slices = (K + kBK - 1) / kBK;
  p.split_slices = (slices + splits - 1) / splits;
  p.part = static_cast<float*>(part->data);
  if (N == 0) return hipSuccess;
  RLM_REQUIRE(p.split_slices <= kSkinnyWaves * kSkinnyBatchLong,
              "%s: %lld slices per split exceed one round of loads", what,
              (long long)p.split_slices);
  const dim3 grid(static_cast<unsigned>((N + 15) / 16), static_cast<unsigned>((M + 15) / 16),
                  static_cast<unsigned>(splits));
  const bool short_batch = p.split_slices <= kSkinnyWaves * kSkinnyBatchShort;
#define RLM_PART_CASE(TA, W)                                                                   \
  if (short_batch)                                                                             \
    hipLaunchKernelGGL((skinny_kernel<TA, W, float, kSkinnyBatchShort>), grid,                \
                       dim3(kSkinnyWaves * kWave), 0, stream, p);                              \
  else                                                                                         \
    hipLaunchKernelGGL((skinny_kernel<TA, W, float, kSkinnyBatchLong>), grid,                 \
                       dim3(kSkinnyWaves * kWave), 0, stream, p);
  if (weight->dtype == RLM_BF16) {
    if (input->dtype == RLM_F32) { RLM_PART_CASE(float, bf16) } else { RLM_PART_CASE(bf16, bf16) }
  } else {
    if (input->dtype == RLM_F32) { RLM_PART_CASE(float, f16) } else { RLM_PART_CASE(f16, f16) }
  }
#undef RLM_PART_CASE
  return launch_status(what);
}

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

// Relation reduce for gfx950: factorized relation hidden (gather + product
// GEMM + GELU), the fused current-row cache update, and the fused LayerNorm /
// active-K softmax / partner sum.
//
// Reference semantics: src/relation_lm/kernels/relation_reduce.py:72-450.
//
// Relation hidden, hidden[row, n] = GELU(W_m[n] . (op[a] * op[p]) + X[a,n] + X[p,H+n])
// for every (query, partner) row, is a GEMM whose A operand is gathered.  A
// workgroup owns 64 rows x BN hidden columns.  It gathers the operand rows of
// its rows' anchors and partners, forms the products in fp32 and stages them
// in LDS together with the W_m tile; the matrix cores do the product term and
// the epilogue adds the gathered expanded-cache halves and applies erf-GELU.
//   * 16-bit bf16 caches: a bf16 x bf16 product is exact in fp32 and splits
//     exactly into hi = bf16(x) and lo = x - hi (lo has at most 8 significant
//     bits), so two v_mfma_f32_16x16x32_bf16 passes (hi and lo against the
//     bf16 W_m) give exact products with fp32 accumulation: the numerics of the
//     reference's fp32 "ieee" dot, at bf16 matrix-core rate.
//   * fp32 (and fp16) caches: fp32 products, v_mfma_f32_16x16x4f32.
// Out-of-range indices read zero rows instead of faulting.
// norm_reduce_kernel: one wavefront per query; each lane owns D/64 columns,
//   LayerNorm moments are wave64 reductions, the K softmax weights live in
//   lanes 0..K-1 and are broadcast by shuffles.
#include <mutex>

#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 64;   // (query, partner) rows per workgroup
constexpr int kRC16 = 128;  // relation-dim chunk staged in LDS, 16-bit path
constexpr int kRC32 = 64;   // relation-dim chunk staged in LDS, fp32 path
constexpr int kPad16 = 8;   // 16-bit elements of row padding (conflict-free b128 reads)
constexpr int kPad32 = 4;

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
  int ring;               // ring-buffer caches: position p in row p mod T
  void* expanded_out;     // same buffer as expanded (mutated)
  float* out;             // [rows, H]
  // Byte sizes of the buffers addressed through range-checked descriptors.
  uint32_t expanded_bytes, operand_bytes, wm_bytes, out_bytes;
  int out_bf16;           // hidden stored as bf16 (round to nearest even), else fp32
};


// Per-row bookkeeping of a workgroup's 64 (query, partner) rows, in LDS.
// Offsets are byte offsets into the caches; kNoOffset marks an index outside
// [0, T) (the row then gathers zeros) or a padding row past the end.
template <int NR>
struct RowTableN {
  int32_t b[NR];      // batch row
  int32_t a[NR];      // anchor index (-1 if out of range)
  int32_t p[NR];      // partner index (-1 if out of range)
  uint32_t op_a[NR];  // operand row of the anchor (kNoOffset unless both indices are valid)
  uint32_t op_p[NR];  // operand row of the partner (same validity)
  uint32_t x_a[NR];   // anchor half of the anchor's expanded row
  uint32_t x_p[NR];   // partner half of the partner's expanded row
};
using RowTable = RowTableN<kRows>;

template <typename T, int NR = kRows>
__device__ __forceinline__ void load_rows(const HiddenParams& p, int64_t r0, RowTableN<NR>& rt) {
  const int tid = threadIdx.x;
  if (tid < NR) {
    const int64_t row = r0 + tid;
    // Unconditional loads (padding rows read row 0, the position a stand-in
    // when there is none), decoded by selects: one round trip.
    const bool live = row < p.rows;
    const int64_t rowc = live ? row : 0;
    const int64_t q = rowc / p.K;
    const int32_t b = live ? static_cast<int32_t>(q / p.Tq) : 0;
    const int64_t ai = index_at(p.anchor, p.index_dtype_a, q);
    const int64_t pi = index_at(p.partner, p.index_dtype_p, rowc);
    const bool has_pos = p.pos != nullptr;
    const int64_t tp = index_at(has_pos ? p.pos : p.anchor, has_pos ? p.pos_dtype : p.index_dtype_a, 0);
    // Valid index range [lo, hi).  Ring caches (row p mod T): any position
    // below 2^31, and in the update form only the resident [t-T+1, t] --
    // an older index would alias the row this launch rewrites.
    int64_t lo = 0, hi = p.T;
    if (p.ring) {
      hi = int64_t(1) << 31;
      if (has_pos) {
        lo = tp - p.T + 1 > 0 ? tp - p.T + 1 : 0;
        hi = tp + 1 < hi ? tp + 1 : hi;
      }
    }
    const int32_t a = (live && ai >= lo && ai < hi) ? static_cast<int32_t>(ai) : -1;
    const int32_t pp = (live && pi >= lo && pi < hi) ? static_cast<int32_t>(pi) : -1;
    const uint32_t base = static_cast<uint32_t>(b) * static_cast<uint32_t>(p.T);
    const uint32_t mask = p.ring ? static_cast<uint32_t>(p.T - 1) : 0xffffffffu;
    const uint32_t ra = static_cast<uint32_t>(a) & mask, rp = static_cast<uint32_t>(pp) & mask;
    const bool ok = a >= 0 && pp >= 0;
    constexpr uint32_t es = sizeof(T);
    rt.b[tid] = b;
    rt.a[tid] = a;
    rt.p[tid] = pp;
    rt.op_a[tid] = ok ? (base + ra) * p.R * es : kNoOffset;
    rt.op_p[tid] = ok ? (base + rp) * p.R * es : kNoOffset;
    rt.x_a[tid] = a >= 0 ? (base + ra) * (2 * p.H) * es : kNoOffset;
    rt.x_p[tid] = pp >= 0 ? ((base + rp) * (2 * p.H) + p.H) * es : kNoOffset;
  }
}

// Update form (relation_reduce.py:215-251): the fresh expanded row t of every
// batch row the tile touches, for the tile's columns: half 0 = W_a op[t] + b1,
// half 1 = W_p op[t], fp32.  Eight lanes share one dot (16-byte loads, three
// shuffle steps).  The tile holding row (b, k=0) then stores batch b's row.
// fresh[(bi * 2 + half) * cols + c] for bi = b - b_first.
template <typename T>
__device__ void fresh_rows(const HiddenParams& p, int64_t t, int64_t r0, int64_t b_first, int nb,
                           int n0, int cols, float* fresh) {
  // Eight lanes share one dot; a lane takes 8-element chunks j, j+8, ...
  // Every weight, operand-row and bias load of kIB items is issued before any
  // is used (unconditional, from clamped addresses), so the items cost one
  // memory round trip instead of one per chunk.
  constexpr int EW = sizeof(T) == 4 ? 2 : 1;  // 16-byte pieces per 8-element chunk
  constexpr int kIB = 4;                      // items per group in flight together
  constexpr int kCH = 2;                      // chunks per lane per pass (R <= 128: one pass)
  const int tid = threadIdx.x;
  const int j = tid & 7;
  const int group = tid >> 3;
  const int groups = blockDim.x >> 3;
  const int items = nb * 2 * cols;
  const int chunks = p.R / 8;
  const int64_t row = p.ring ? (t & (p.T - 1)) : t;
  for (int base = 0; base < items; base += groups * kIB) {
    const unsigned char* wrow[kIB];
    const unsigned char* orow[kIB];
    bool ok[kIB];
    int half[kIB];
    float bias[kIB], acc[kIB];
#pragma unroll
    for (int ib = 0; ib < kIB; ++ib) {
      const int item = base + group + groups * ib;
      const int it = item < items ? item : 0;
      const int c = it % cols;
      half[ib] = (it / cols) % 2;
      const int bi = it / (2 * cols);
      const int n = n0 + c;
      ok[ib] = item < items && n < p.H;
      const int nc = n < p.H ? n : 0;
      wrow[ib] = static_cast<const unsigned char*>(half[ib] == 0 ? p.wa : p.wp) +
                 static_cast<int64_t>(nc) * p.R * sizeof(T);
      orow[ib] = static_cast<const unsigned char*>(p.operand) +
                 ((b_first + bi) * p.T + row) * p.R * sizeof(T);
      bias[ib] = to_f32(static_cast<const T*>(p.b1)[nc]);
      acc[ib] = 0.0f;
    }
    for (int c0 = 0; c0 < chunks; c0 += 8 * kCH) {
      uint4 wv[kIB][kCH][EW], ov[kIB][kCH][EW];
#pragma unroll
      for (int ib = 0; ib < kIB; ++ib)
#pragma unroll
        for (int cc = 0; cc < kCH; ++cc) {
          const int ch = c0 + j + 8 * cc;
          const int chc = ch < chunks ? ch : 0;
#pragma unroll
          for (int e = 0; e < EW; ++e) {
            wv[ib][cc][e] = *reinterpret_cast<const uint4*>(wrow[ib] + (chc * EW + e) * 16);
            ov[ib][cc][e] = *reinterpret_cast<const uint4*>(orow[ib] + (chc * EW + e) * 16);
          }
        }
#pragma unroll
      for (int ib = 0; ib < kIB; ++ib)
#pragma unroll
        for (int cc = 0; cc < kCH; ++cc) {
          const bool in = ok[ib] && c0 + j + 8 * cc < chunks;
          float d = 0.0f;
          if constexpr (EW == 1) {
            const uint32_t w4[4] = {wv[ib][cc][0].x, wv[ib][cc][0].y, wv[ib][cc][0].z, wv[ib][cc][0].w};
            const uint32_t o4[4] = {ov[ib][cc][0].x, ov[ib][cc][0].y, ov[ib][cc][0].z, ov[ib][cc][0].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              d += __uint_as_float(w4[k] << 16) * __uint_as_float(o4[k] << 16);
              d += __uint_as_float(w4[k] & 0xffff0000u) * __uint_as_float(o4[k] & 0xffff0000u);
            }
          } else {
#pragma unroll
            for (int e = 0; e < EW; ++e) {
              const uint4 w4 = wv[ib][cc][e], o4 = ov[ib][cc][e];
              d += __uint_as_float(w4.x) * __uint_as_float(o4.x) + __uint_as_float(w4.y) * __uint_as_float(o4.y);
              d += __uint_as_float(w4.z) * __uint_as_float(o4.z) + __uint_as_float(w4.w) * __uint_as_float(o4.w);
            }
          }
          acc[ib] += in ? d : 0.0f;
        }
    }
#pragma unroll
    for (int ib = 0; ib < kIB; ++ib) {
      float v = acc[ib];
      v += __shfl_xor(v, 1, 8);
      v += __shfl_xor(v, 2, 8);
      v += __shfl_xor(v, 4, 8);
      const int item = base + group + groups * ib;
      if (ok[ib] && j == 0) fresh[item] = half[ib] == 0 ? v + bias[ib] : v;
    }
  }
  __syncthreads();
  const int64_t QK = p.Tq * p.K;
  const int64_t b_lo = (r0 + QK - 1) / QK;
  int64_t b_hi = (r0 + kRows - 1) / QK;
  if (b_hi > p.B - 1) b_hi = p.B - 1;
  for (int item = tid; item < items; item += blockDim.x) {
    const int c = item % cols;
    const int half = (item / cols) % 2;
    const int64_t b = b_first + item / (2 * cols);
    const int n = n0 + c;
    if (b < b_lo || b > b_hi || n >= p.H) continue;
    const int64_t row = p.ring ? (t & (p.T - 1)) : t;
    T* dst = static_cast<T*>(p.expanded_out) + (b * p.T + row) * (2 * static_cast<int64_t>(p.H)) +
             static_cast<int64_t>(half) * p.H + n;
    *dst = from_f32<T>(fresh[item]);
  }
}

// Largest number of batch rows one 64-row tile can touch in the update form.
__host__ __device__ constexpr int fresh_batches() { return kRows; }

// Anchor + partner halves of the expanded cache for the lane's accumulator
// elements (rows 4*(lane/16)+e of column n), gathered before the matrix-core
// work so their latency overlaps it.  Row t of the update form is taken from
// `fresh` instead of the cache row this launch rewrites.
template <typename T, bool UPDATE>
__device__ __forceinline__ void gather_bases(const HiddenParams& p, rsrc_t xr, const RowTable& rt,
                                             int mrow, int n, int c, int64_t t, int64_t b_first,
                                             const float* fresh, int cols, int lane,
                                             float (&xs)[4]) {
  // Branch-free: every row-table and `fresh` read is unconditional and the
  // conditions only select between registers, so all the gathers are in
  // flight together (a branch would make the compiler wait for each pair of
  // loads at its join).
  const bool in = n < p.H;
  const uint32_t col = (in ? static_cast<uint32_t>(n) : 0u) * sizeof(T);
  float xa[4], xp[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = mrow + (lane >> 4) * 4 + e;
    const uint32_t xam = rt.x_a[m], xpm = rt.x_p[m];
    xa[e] = buf_load_elem<T>(xr, (in ? xam : kNoOffset) + col);
    xp[e] = buf_load_elem<T>(xr, (in ? xpm : kNoOffset) + col);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a = xa[e], b = xp[e];
    if constexpr (UPDATE) {
      // Row t comes from `fresh` (clamped index: always a valid LDS read).
      const int m = mrow + (lane >> 4) * 4 + e;
      const int32_t am = rt.a[m], pm = rt.p[m];
      int64_t bi = rt.b[m] - b_first;
      bi = bi < 0 ? 0 : (bi >= fresh_batches() ? fresh_batches() - 1 : bi);
      const float fa = fresh[(bi * 2 + 0) * cols + c];
      const float fp = fresh[(bi * 2 + 1) * cols + c];
      const bool use = (t >= 0) & in;
      a = (use & (am == t)) ? fa : a;
      b = (use & (pm == t)) ? fp : b;
    }
    xs[e] = a + b;
  }
}

// GELU(acc + bases) for the lane's four rows of column n; rows past the end
// fall outside the output descriptor and are dropped.  A bf16 output holds
// the value a bf16 consumer would round the fp32 one to (the same conversion).
__device__ __forceinline__ void store_hidden(const HiddenParams& p, rsrc_t outr, const f32x4& acc,
                                             const float (&xs)[4], int64_t r0, int mrow, int n,
                                             int lane) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t grow = static_cast<uint32_t>(r0 + mrow + (lane >> 4) * 4 + e);
    const uint32_t idx = grow * static_cast<uint32_t>(p.H) + n;
    const float v = gelu_erf(acc[e] + xs[e]);
    if (p.out_bf16)  // uniform
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(pack_bf16x2(v, 0.0f)), outr,
                                            n < p.H ? idx * 2u : kNoOffset, 0, 0);
    else
      buf_store_f32(v, outr, n < p.H ? idx * 4u : kNoOffset);
  }
}

// Update-form set-up shared by both kernels: position, the batch range of the
// tile and the fresh rows (computed, and stored to the cache by the owning tile).
template <typename T, bool UPDATE>
__device__ __forceinline__ int64_t update_setup(const HiddenParams& p, int64_t t, int64_t r0,
                                                int n0, int cols, int64_t& b_first, float* fresh) {
  // t: the position, loaded by the caller before the row table.
  b_first = 0;
  if (!UPDATE) return -1;
  // Out-of-range position: nothing to write or reuse (ring caches: t < 0 only).
  if (t < 0 || (!p.ring && t >= p.T) || t >= (int64_t(1) << 31)) t = -1;
  const int64_t QK = p.Tq * p.K;
  b_first = r0 / QK;
  int64_t b_last = (r0 + kRows - 1) / QK;
  if (b_last > p.B - 1) b_last = p.B - 1;
  if (t >= 0) fresh_rows<T>(p, t, r0, b_first, static_cast<int>(b_last - b_first + 1), n0, cols, fresh);
  return t;
}

// bf16 caches: exact hi/lo split products on bf16 MFMA.  BN hidden columns
// per workgroup (64 or 128); waves in 2x2, each 32 rows x BN/2 columns.
template <bool UPDATE, int BN>
__global__ void __launch_bounds__(256) hidden_bf16_kernel(const HiddenParams p) {
  constexpr int TN = BN / 32;
  constexpr int LD = kRC16 + kPad16;
  constexpr int kAChunks = kRows * (kRC16 / 8) / 256;   // product chunks staged per thread
  constexpr int kWChunks = BN * (kRC16 / 8) / 256;      // W_m chunks staged per thread
  __shared__ __align__(16) uint16_t a_hi[kRows][LD];
  __shared__ __align__(16) uint16_t a_lo[kRows][LD];
  __shared__ __align__(16) uint16_t w_t[BN][LD];
  __shared__ RowTable rt;
  __shared__ float fresh[UPDATE ? fresh_batches() * 2 * BN : 1];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  // Row tiles of one batch row run on one XCD (one L2 for the rows they gather).
  const int64_t wg = xcd_tile(static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x,
                              static_cast<int64_t>(gridDim.x) * gridDim.y);
  const int64_t r0 = wg / gridDim.x * kRows;
  const int n0 = static_cast<int>(wg % gridDim.x) * BN;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wr_ = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t outr = make_rsrc(p.out, p.out_bytes);
  const int64_t t_pos = UPDATE ? index_at(p.pos, p.pos_dtype, 0) : -1;  // beside the row loads
  load_rows<bf16>(p, r0, rt);
  int64_t b_first;
  const int64_t t = update_setup<bf16, UPDATE>(p, t_pos, r0, n0, BN, b_first, fresh);
  __syncthreads();

  const int wr = (wave >> 1) * 32;
  const int wc = (wave & 1) * (BN / 2);
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  float xs[2][TN][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      gather_bases<bf16, UPDATE>(p, xr, rt, wr + i * 16, n0 + wc + j * 16 + r16,
                                 wc + j * 16 + r16, t, b_first, fresh, BN, lane, xs[i][j]);

  f32x4 acc[2][TN];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int rc = 0; rc < p.R; rc += kRC16) {
    if (rc) __syncthreads();
    // Gather first (every load in flight), then form and stage the products.
    uint4 va[kAChunks], vp[kAChunks], vw[kWChunks];
#pragma unroll
    for (int c = 0; c < kAChunks; ++c) {
      const int idx = tid + 256 * c;
      const int row = idx / (kRC16 / 8);
      const int r = rc + (idx % (kRC16 / 8)) * 8;
      const bool in = r < p.R;
      va[c] = buf_load_b128(opr, in ? rt.op_a[row] + 2u * r : kNoOffset);
      vp[c] = buf_load_b128(opr, in ? rt.op_p[row] + 2u * r : kNoOffset);
    }
#pragma unroll
    for (int c = 0; c < kWChunks; ++c) {
      const int idx = tid + 256 * c;
      const int n = n0 + idx / (kRC16 / 8);
      const int r = rc + (idx % (kRC16 / 8)) * 8;
      vw[c] = buf_load_b128(wr_, (n < p.H && r < p.R)
                                      ? 2u * (static_cast<uint32_t>(n) * p.R + r)
                                      : kNoOffset);
    }
#pragma unroll
    for (int c = 0; c < kAChunks; ++c) {
      const int idx = tid + 256 * c;
      const int row = idx / (kRC16 / 8);
      const int r = (idx % (kRC16 / 8)) * 8;
      const uint32_t wa[4] = {va[c].x, va[c].y, va[c].z, va[c].w};
      const uint32_t wp[4] = {vp[c].x, vp[c].y, vp[c].z, vp[c].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // Exact fp32 products of the two bf16 pairs in this word.
        const float x0 = __uint_as_float(wp[q] << 16) * __uint_as_float(wa[q] << 16);
        const float x1 = __uint_as_float(wp[q] & 0xffff0000u) * __uint_as_float(wa[q] & 0xffff0000u);
        h[q] = pack_bf16x2(x0, x1);
        l[q] = pack_bf16x2(x0 - __uint_as_float(h[q] << 16), x1 - __uint_as_float(h[q] & 0xffff0000u));
      }
      *reinterpret_cast<uint4*>(&a_hi[row][r]) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(&a_lo[row][r]) = make_uint4(l[0], l[1], l[2], l[3]);
    }
#pragma unroll
    for (int c = 0; c < kWChunks; ++c) {
      const int idx = tid + 256 * c;
      *reinterpret_cast<uint4*>(&w_t[idx / (kRC16 / 8)][(idx % (kRC16 / 8)) * 8]) = vw[c];
    }
    __syncthreads();
    const int rlen = p.R - rc < kRC16 ? p.R - rc : kRC16;
    for (int kk = 0; kk < rlen; kk += 32) {
      u16x8 ah[2], al[2], bw[TN];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ah[i] = *reinterpret_cast<const u16x8*>(&a_hi[wr + i * 16 + r16][kk + kq]);
        al[i] = *reinterpret_cast<const u16x8*>(&a_lo[wr + i * 16 + r16][kk + kq]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[j] = *reinterpret_cast<const u16x8*>(&w_t[wc + j * 16 + r16][kk + kq]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, ah[i]), __builtin_bit_cast(bf16x8, bw[j]), acc[i][j], 0,
              0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, al[i]), __builtin_bit_cast(bf16x8, bw[j]), acc[i][j], 0,
              0, 0);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      store_hidden(p, outr, acc[i][j], xs[i][j], r0, wr + i * 16, n0 + wc + j * 16 + r16, lane);
}

// bf16 caches, sequence form with many rows: a workgroup of four waves owns
// 64 rows and walks every 256-column tile of the hidden dimension, so the
// rows' indices and operand products are read and formed once per row tile.
//   set-up  the row table, then the rows' exact operand products op[a] *
//           op[p] (fp32, split into hi + lo bf16 as hidden_bf16_kernel does)
//           into LDS;
//   per column tile (wave w: columns n0 + 64w .. + 63)
//     - hidden^T = W_m . P^T on v_mfma_f32_32x32x16_bf16 (hi and lo; W_m
//       fragments straight from L2 in operand layout, loaded during the
//       second half of the previous column tile's epilogue);
//     - the fp32 sums are restaged through the wave's own LDS region one
//       32-row block at a time and read back row-contiguous: a lane takes
//       eight consecutive columns of one row, adds the expanded-cache halves
//       X[a, n..n+7] and X[p, H+n..H+n+7] (16-byte gathers, eight lanes per
//       128-byte row segment, issued one column tile ahead), applies GELU and
//       stores 8 outputs.
// Several workgroups share a CU, so one's load round trips overlap another's
// GELU and matrix work.  LDS rows of the products are R*2 bytes, 16-byte
// piece q of row r stored at piece q ^ swz(r) (conflict-free fragment reads).
constexpr int kTileRows = 64;
constexpr int kTileCols = 256;
constexpr int kTileThreads = 256;
constexpr int kStageRow = 64 * 4 + 16;                 // staged fp32 row stride (bytes)
constexpr int kStageBytes = 32 * kStageRow;            // one wave's 32-row block

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int PR>
__device__ __forceinline__ int tile_swz(int r) {
  if constexpr (PR == 16) return r & 15;
  else return (r & 7) ^ ((r >> 3) & 1);
}

// LDS: the hi / lo product tiles, the four waves' staging, the row table.
template <int R>
constexpr int hidden_tile_stage_offset() {
  return 2 * kTileRows * R * 2;
}
template <int R>
constexpr int hidden_tile_table_offset() {
  return hidden_tile_stage_offset<R>() + 4 * kStageBytes;
}
template <int R>
constexpr size_t hidden_tile_lds_bytes() {
  return static_cast<size_t>(hidden_tile_table_offset<R>()) + sizeof(RowTableN<kTileRows>);
}

// Eight consecutive outputs of one row.
template <typename TO>
__device__ __forceinline__ void put8(TO* dst, const float (&v)[8]) {
  if constexpr (sizeof(TO) == 4) {
    reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    *reinterpret_cast<uint4*>(dst) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
}

template <typename TO, int R>
__global__ void __launch_bounds__(kTileThreads, 2) hidden_tile_kernel(const HiddenParams p) {
  constexpr int PR = R / 8;                              // 16-byte pieces per LDS row
  constexpr int RB = R * 2;                              // bytes per LDS row
  constexpr int KK = R / 16;                             // MFMA k-steps
  constexpr int kPieces = kTileRows * PR / kTileThreads; // product pieces per thread
  static_assert(R == 64 || R == 128, "relation dim 64 or 128");
  static_assert(__is_same(TO, float) || __is_same(TO, bf16), "fp32 or bf16 hidden");
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* p_hi = smem;
  unsigned char* p_lo = smem + kTileRows * RB;
  auto& rt = *reinterpret_cast<RowTableN<kTileRows>*>(smem + hidden_tile_table_offset<R>());

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t row_tiles = (p.rows + kTileRows - 1) / kTileRows;
  // Row tiles of neighbouring queries run on one XCD (one L2 for their gathers).
  const int64_t r0 = xcd_tile(blockIdx.x, row_tiles) * kTileRows;
  const int col_tiles = (p.H + kTileCols - 1) / kTileCols;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wr = make_rsrc(p.wm, p.wm_bytes);
  unsigned char* stage = smem + hidden_tile_stage_offset<R>() + wave * kStageBytes;
  TO* out = reinterpret_cast<TO*>(p.out);

  // W_m fragments of column tile ct: block j of 32 hidden columns, k-step kk --
  // row n0 + 64 wave + 32j + (lane & 31), k = 16kk + 8 (lane >> 5) .. +7
  // (rows past H read zero).
  u16x8 fw[2][KK];
  auto load_w = [&](int ct) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = ct * kTileCols + wave * 64 + 32 * j + (lane & 31);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        fw[j][kk] = __builtin_bit_cast(
            u16x8, buf_load_b128(wr, n < p.H ? static_cast<uint32_t>(n * RB + 32 * kk + 16 * (lane >> 5))
                                             : kNoOffset));
    }
  };

  // Set-up: row table, then the products (every load of a thread issued first).
  load_rows<bf16, kTileRows>(p, r0, rt);
  __syncthreads();
  {
    uint4 va[kPieces], vp[kPieces];
#pragma unroll
    for (int c = 0; c < kPieces; ++c) {
      const int piece = c * kTileThreads + tid;
      const int row = piece / PR, q = piece % PR;
      va[c] = buf_load_b128(opr, rt.op_a[row] + 16u * q);
      vp[c] = buf_load_b128(opr, rt.op_p[row] + 16u * q);
    }
    load_w(0);
#pragma unroll
    for (int c = 0; c < kPieces; ++c) {
      const int piece = c * kTileThreads + tid;
      const int row = piece / PR, q = piece % PR;
      const uint32_t wa[4] = {va[c].x, va[c].y, va[c].z, va[c].w};
      const uint32_t wp[4] = {vp[c].x, vp[c].y, vp[c].z, vp[c].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_lo(wp[e]) * bf16_lo(wa[e]);
        const float x1 = bf16_hi(wp[e]) * bf16_hi(wa[e]);
        h[e] = pack_bf16x2(x0, x1);
        l[e] = pack_bf16x2(x0 - bf16_lo(h[e]), x1 - bf16_hi(h[e]));
      }
      const int at = row * RB + ((q ^ tile_swz<PR>(row)) << 4);
      *reinterpret_cast<uint4*>(p_hi + at) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(p_lo + at) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
  __syncthreads();
  const int swz = tile_swz<PR>(lane & 15);

  // Row-contiguous roles of the epilogue: piece t of block i is row
  // 32i + 8t + (lane >> 3), columns 8 (lane & 7) .. +7 of the wave's 64.
  const int c8 = 8 * (lane & 7);
  uint4 xa[2][4], xp[2][4];
  auto load_x = [&](int ct, int i) {
    const int n = ct * kTileCols + wave * 64 + c8;
    const bool in = n < p.H;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int m = 32 * i + 8 * t + (lane >> 3);
      xa[i][t] = buf_load_b128(xr, in ? rt.x_a[m] + 2u * n : kNoOffset);
      xp[i][t] = buf_load_b128(xr, in ? rt.x_p[m] + 2u * n : kNoOffset);
    }
  };
  load_x(0, 0);
  load_x(0, 1);

  for (int ct = 0; ct < col_tiles; ++ct) {
    const int wn0 = ct * kTileCols + wave * 64;
    f32x16 acc[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int off = (lane & 31) * RB + (((2 * kk + (lane >> 5)) ^ swz) << 4);
      u16x8 fh[2], fl[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fh[i] = *reinterpret_cast<const u16x8*>(p_hi + 32 * i * RB + off);
        fl[i] = *reinterpret_cast<const u16x8*>(p_lo + 32 * i * RB + off);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, fw[j][kk]), __builtin_bit_cast(bf16x8, fh[i]), acc[j][i], 0, 0, 0);
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, fw[j][kk]), __builtin_bit_cast(bf16x8, fl[i]), acc[j][i], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // The next tile's W_m fragments once block 0's accumulators are free.
      if (i == 1 && ct + 1 < col_tiles) load_w(ct + 1);
      // acc block i: lane holds row (lane & 31), columns 32j + 8q + 4 (lane >> 5) .. +3.
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<float4*>(stage + (lane & 31) * kStageRow + (32 * j + 8 * q + 4 * (lane >> 5)) * 4) =
              make_float4(acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                          acc[j][i][4 * q + 3]);
      wave_sync();
      // Wave-uniform: whole pieces inside the output, or the edge path.
      const bool full = r0 + 32 * i + 32 <= p.rows && wn0 + 64 <= p.H;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int row = 8 * t + (lane >> 3);
        const float4 s0 = *reinterpret_cast<const float4*>(stage + row * kStageRow + c8 * 4);
        const float4 s1 = *reinterpret_cast<const float4*>(stage + row * kStageRow + c8 * 4 + 16);
        const uint32_t a[4] = {xa[i][t].x, xa[i][t].y, xa[i][t].z, xa[i][t].w};
        const uint32_t b[4] = {xp[i][t].x, xp[i][t].y, xp[i][t].z, xp[i][t].w};
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = gelu_erf(sv[2 * e] + (bf16_lo(a[e]) + bf16_lo(b[e])));
          v[2 * e + 1] = gelu_erf(sv[2 * e + 1] + (bf16_hi(a[e]) + bf16_hi(b[e])));
        }
        const int64_t m = r0 + 32 * i + row;
        if (full) {
          put8<TO>(out + m * p.H + wn0 + c8, v);
        } else if (m < p.rows) {
          for (int k = 0; k < 8; ++k)
            if (wn0 + c8 + k < p.H) out[m * p.H + wn0 + c8 + k] = from_f32<TO>(v[k]);
        }
      }
      wave_sync();
      if (ct + 1 < col_tiles) load_x(ct + 1, i);
    }
  }
}

// ---------------------------------------------------------------------------
// Relation MLP, sequence form: the relation hidden and the second Linear in one
// kernel -- the multi-anchor block's relation MLP Linear -> GELU -> Linear
// (multi_relation_blocks.py:47-52,163) with its first Linear factorized
// (relation_hidden_cached, relation_reduce.py:149-183), bias-free:
//   raw[m, :] = W2 . bf16(GELU(W_m (op[a_m] * op[p_m]) + X[a_m, :H] + X[p_m, H:]))
// The [rows, H] hidden never reaches memory.  A workgroup of eight waves owns
// 64 rows and all D output columns and walks the hidden dimension in chunks of
// 128 columns:
//   phase 1  wave w forms the 32 x 32 block (rows 32 (w & 1).., chunk columns
//            32 (w >> 1)..) of the chunk's hidden with hidden_tile_kernel's
//            arithmetic -- the same MFMA sums over the exact hi / lo product
//            split, the same fp32 adds of the expanded-cache halves, GELU and
//            bf16 rounding -- into the LDS hidden tile (two buffers, so the
//            next chunk's phase 1 needs no barrier against this chunk's
//            phase 2);
//   phase 2  raw^T[D x 64] += W2[:, chunk] . hidden^T on 32x32x16 MFMAs, wave w
//            owning D columns [32 TNB w, 32 TNB (w + 1)), k ascending in
//            16-wide groups: the accumulation of relation_linear's tile kernel.
// So raw is bit-identical to relation_hidden_cached_seq (bf16 hidden) followed
// by relation_linear (fp32 output, no bias).  W_m fragments come from L2 into
// operand registers one chunk ahead, W2 fragments kMlpW2Ahead k-groups ahead;
// the expanded-cache halves are gathered one chunk ahead.  The output rows are
// restaged through LDS and stored as whole 16-byte row pieces.
constexpr int kMlpRows = 64;
constexpr int kMlpWaves = 8;
constexpr int kMlpThreads = kMlpWaves * kWave;
constexpr int kMlpChunk = 128;                  // hidden columns per chunk
constexpr int kMlpHidRow = kMlpChunk * 2 + 16;  // LDS hidden row (bytes): conflict-free 16-byte reads
constexpr int kMlpStageRow = 32 * 4 + 16;       // phase-1 restaged fp32 row (bytes)
constexpr int kMlpW2Ahead = 2;                  // W2 k-groups loaded ahead of their products

// Both weights arrive in MFMA fragment order (rlm_mfma_fragments): fragment
// (n-block nb, k-group g) of a [N, K] weight is 64 lanes x 8 consecutive k,
// lane l holding row 32 nb + (l & 31), k = 16 g + 8 (l >> 5) .. +7, stored
// as 1 KiB at ((nb * K/16 + g) * 64 + l) * 16 bytes -- so a wave reads a
// fragment as one contiguous 1 KiB instead of 32 rows of 32 bytes.
struct MlpParams {
  HiddenParams h;      // rows, caches, indices and W_m (fragment order; h.out unused)
  const void* w2;      // second Linear weight [D, H] in fragment order, bf16
  float* out;          // [rows, D]
  int D;
  uint32_t w2_bytes;
};

// LDS: the hi / lo product tiles, two hidden tiles, the waves' phase-1
// staging, the row table; after the main loop the output restaging reuses it
// from the start.
template <int R>
constexpr int mlp_hid_offset() {
  return 2 * kMlpRows * R * 2;
}
template <int R>
constexpr int mlp_stage_offset() {
  return mlp_hid_offset<R>() + 2 * kMlpRows * kMlpHidRow;
}
template <int R>
constexpr int mlp_table_offset() {
  return mlp_stage_offset<R>() + kMlpWaves * 32 * kMlpStageRow;
}
template <int TNB>
constexpr int mlp_out_row() {
  return 32 * TNB * 4 + 16;
}
template <int R, int TNB>
constexpr size_t mlp_lds_bytes() {
  constexpr size_t main_bytes = mlp_table_offset<R>() + sizeof(RowTableN<kMlpRows>);
  constexpr size_t out_bytes = static_cast<size_t>(kMlpWaves) * 32 * mlp_out_row<TNB>();
  return main_bytes > out_bytes ? main_bytes : out_bytes;
}

template <int R, int TNB>
__global__ void __launch_bounds__(kMlpThreads) relation_mlp_kernel(const MlpParams mp) {
  const HiddenParams& p = mp.h;
  constexpr int PR = R / 8;                               // 16-byte pieces per product row
  constexpr int RB = R * 2;                               // bytes per product row
  constexpr int KK = R / 16;                              // phase-1 k-steps
  constexpr int K2 = kMlpChunk / 16;                      // phase-2 k-groups per chunk
  constexpr int kPieces = kMlpRows * PR / kMlpThreads;    // product pieces per thread
  static_assert(R == 64 || R == 128, "relation dim 64 or 128");
  static_assert(kPieces * kMlpThreads == kMlpRows * PR, "whole product pieces per thread");
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* p_hi = smem;
  unsigned char* p_lo = smem + kMlpRows * RB;
  unsigned char* hid = smem + mlp_hid_offset<R>();
  auto& rt = *reinterpret_cast<RowTableN<kMlpRows>*>(smem + mlp_table_offset<R>());

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t row_tiles = (p.rows + kMlpRows - 1) / kMlpRows;
  // Row tiles of neighbouring queries run on one XCD (one L2 for their gathers).
  const int64_t r0 = xcd_tile(blockIdx.x, row_tiles) * kMlpRows;
  const int nchunks = p.H / kMlpChunk;
  const uint32_t H = static_cast<uint32_t>(p.H);
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wr = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t w2r = make_rsrc(mp.w2, mp.w2_bytes);
  unsigned char* stage = smem + mlp_stage_offset<R>() + wave * 32 * kMlpStageRow;

  // Phase-1 roles: row block i1 and column block j1 (32 hidden columns of the
  // chunk).  W_m fragment kk: rows c*128 + 32 j1 .. +31, k-group kk.
  const int i1 = wave & 1, j1 = wave >> 1;
  u16x8 fwm[KK];
  auto load_wm = [&](int c) {
    const uint32_t nb = static_cast<uint32_t>(c * (kMlpChunk / 32) + j1);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      fwm[kk] = __builtin_bit_cast(u16x8, buf_load_b128(wr, ((nb * KK + kk) * kWave + lane) * 16u));
  };
  // Row-contiguous roles of the phase-1 epilogue: piece t is row 16t + (lane >> 2)
  // of the block, columns 8 (lane & 3) .. +7 of its 32.  Rows outside the
  // caches have kNoOffset bases: their gathers read zeros.
  const int c8 = 8 * (lane & 3);
  uint4 xa[2], xp[2];
  auto load_x = [&](int c) {
    const uint32_t n = static_cast<uint32_t>(c * kMlpChunk + 32 * j1 + c8);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int m = 32 * i1 + 16 * t + (lane >> 2);
      xa[t] = buf_load_b128(xr, rt.x_a[m] + 2u * n);
      xp[t] = buf_load_b128(xr, rt.x_p[m] + 2u * n);
    }
  };

  // Set-up: row table, then the products (every load of a thread issued first).
  load_rows<bf16, kMlpRows>(p, r0, rt);
  __syncthreads();
  {
    uint4 va[kPieces], vp[kPieces];
#pragma unroll
    for (int c = 0; c < kPieces; ++c) {
      const int piece = c * kMlpThreads + tid;
      const int row = piece / PR, q = piece % PR;
      va[c] = buf_load_b128(opr, rt.op_a[row] + 16u * q);
      vp[c] = buf_load_b128(opr, rt.op_p[row] + 16u * q);
    }
    load_wm(0);
    load_x(0);
#pragma unroll
    for (int c = 0; c < kPieces; ++c) {
      const int piece = c * kMlpThreads + tid;
      const int row = piece / PR, q = piece % PR;
      const uint32_t wa[4] = {va[c].x, va[c].y, va[c].z, va[c].w};
      const uint32_t wp[4] = {vp[c].x, vp[c].y, vp[c].z, vp[c].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_lo(wp[e]) * bf16_lo(wa[e]);  // exact: 8-bit x 8-bit significands
        const float x1 = bf16_hi(wp[e]) * bf16_hi(wa[e]);
        h[e] = pack_bf16x2(x0, x1);
        l[e] = pack_bf16x2(x0 - bf16_lo(h[e]), x1 - bf16_hi(h[e]));
      }
      const int at = row * RB + ((q ^ tile_swz<PR>(row)) << 4);
      *reinterpret_cast<uint4*>(p_hi + at) = make_uint4(h[0], h[1], h[2], h[3]);
      *reinterpret_cast<uint4*>(p_lo + at) = make_uint4(l[0], l[1], l[2], l[3]);
    }
  }
  __syncthreads();
  const int swz = tile_swz<PR>(lane & 15);
  const int prod_off = (32 * i1 + (lane & 31)) * RB;

  // Phase-2 roles: D columns dw0 .. dw0 + 32 TNB - 1.  W2 fragment j of global
  // k-group g: n-block TNB w + j, k-group g.
  const int dw0 = 32 * TNB * wave;
  const uint32_t kgroups = H / 16u;
  auto load_w2 = [&](u16x8 (&w)[TNB], int g) {
#pragma unroll
    for (int j = 0; j < TNB; ++j)
      w[j] = __builtin_bit_cast(
          u16x8, buf_load_b128(w2r, ((static_cast<uint32_t>(TNB * wave + j) * kgroups + g) * kWave +
                                     lane) * 16u));
  };
  // Hidden-tile A fragments: row 32i + (lane & 31), k = 16s + 8 (lane >> 5) of the chunk.
  const int hid_lane = (lane & 31) * kMlpHidRow + 16 * (lane >> 5);

  f32x16 acc[TNB][2];
#pragma unroll
  for (int j = 0; j < TNB; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.0f;

  // Phase 1 of a chunk, one k-step: hidden^T block (columns 32 j1.., rows
  // 32 i1..) += W_m fragment kk . product fragments (hi, then lo).
  auto p1_step = [&](f32x16& hacc, int kk) {
    const int off = prod_off + (((2 * kk + (lane >> 5)) ^ swz) << 4);
    const u16x8 fh = *reinterpret_cast<const u16x8*>(p_hi + off);
    const u16x8 fl = *reinterpret_cast<const u16x8*>(p_lo + off);
    hacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fwm[kk]),
                                                   __builtin_bit_cast(bf16x8, fh), hacc, 0, 0, 0);
    hacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fwm[kk]),
                                                   __builtin_bit_cast(bf16x8, fl), hacc, 0, 0, 0);
  };
  // Its epilogue: + expanded-cache halves (xa / xp), GELU, bf16 into hidden
  // buffer hb.  hacc: lane holds hidden^T[column 8q + 4 (lane >> 5) + e][row lane & 31].
  auto p1_epilogue = [&](const f32x16& hacc, unsigned char* hb) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(stage + (lane & 31) * kMlpStageRow + (8 * q + 4 * (lane >> 5)) * 4) =
          make_float4(hacc[4 * q], hacc[4 * q + 1], hacc[4 * q + 2], hacc[4 * q + 3]);
    wave_sync();
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = 16 * t + (lane >> 2);
      const float4 s0 = *reinterpret_cast<const float4*>(stage + row * kMlpStageRow + c8 * 4);
      const float4 s1 = *reinterpret_cast<const float4*>(stage + row * kMlpStageRow + c8 * 4 + 16);
      const uint32_t a[4] = {xa[t].x, xa[t].y, xa[t].z, xa[t].w};
      const uint32_t b[4] = {xp[t].x, xp[t].y, xp[t].z, xp[t].w};
      const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = gelu_erf(sv[2 * e] + (bf16_lo(a[e]) + bf16_lo(b[e])));
        v[2 * e + 1] = gelu_erf(sv[2 * e + 1] + (bf16_hi(a[e]) + bf16_hi(b[e])));
      }
      put8<bf16>(reinterpret_cast<bf16*>(hb + (32 * i1 + row) * kMlpHidRow + (32 * j1 + c8) * 2), v);
    }
    wave_sync();  // the staging is read before it is written again
  };

  // Prologue: chunk 0's hidden, then the first W2 k-groups of chunk 0.
  u16x8 wq[K2][TNB];
  {
    f32x16 hacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) hacc[e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) p1_step(hacc, kk);
    if (nchunks > 1) load_wm(1);
#pragma unroll
    for (int s = 0; s < kMlpW2Ahead; ++s) load_w2(wq[s], s);
    p1_epilogue(hacc, hid);
    if (nchunks > 1) load_x(1);
  }
  __syncthreads();  // hidden chunk 0 complete

  // Iteration c: phase 2 of chunk c with phase 1's matrix work for chunk c + 1
  // interleaved (one k-step per k-group: independent of phase 2, it fills the
  // matrix pipeline around phase 2's products), then chunk c + 1's epilogue into
  // the other hidden buffer.  The last iteration's phase-1 products are
  // discarded (no branch in the k-loop).
  for (int c = 0; c < nchunks; ++c) {
    unsigned char* hb = hid + (c & 1) * (kMlpRows * kMlpHidRow);
    unsigned char* hn = hid + ((c + 1) & 1) * (kMlpRows * kMlpHidRow);
    f32x16 hacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) hacc[e] = 0.0f;
#pragma unroll
    for (int s = 0; s < K2; ++s) {
      if (s + kMlpW2Ahead < K2) load_w2(wq[s + kMlpW2Ahead], c * K2 + s + kMlpW2Ahead);
      u16x8 fa[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const u16x8*>(hb + 32 * i * kMlpHidRow + hid_lane + 32 * s);
#pragma unroll
      for (int j = 0; j < TNB; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, wq[s][j]), __builtin_bit_cast(bf16x8, fa[i]), acc[j][i], 0, 0, 0);
      if (s < KK) p1_step(hacc, s);
    }
    if (c + 1 < nchunks) {  // uniform
      if (c + 2 < nchunks) load_wm(c + 2);
#pragma unroll
      for (int s = 0; s < kMlpW2Ahead; ++s) load_w2(wq[s], (c + 1) * K2 + s);
      p1_epilogue(hacc, hn);
      if (c + 2 < nchunks) load_x(c + 2);
    }
    __syncthreads();  // phase 2 of chunk c read; hidden chunk c + 1 complete
  }

  // ---- Output: acc[j][i] holds raw[row 32i + (lane & 31)][columns dw0 + 32j +
  // 8q + 4 (lane >> 5) .. +3] in element 4q..4q+3.  Each wave restages one
  // 32-row block at a time and stores whole 16-byte row pieces.
  __syncthreads();  // every wave is done with the main loop's LDS
  constexpr int RS = mlp_out_row<TNB>();
  constexpr int kPiecesRow = 32 * TNB * 4 / 16;
  unsigned char* ost = smem + wave * 32 * RS;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < TNB; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(ost + (lane & 31) * RS + (32 * j + 8 * q + 4 * (lane >> 5)) * 4) =
            make_float4(acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                        acc[j][i][4 * q + 3]);
    wave_sync();
#pragma unroll
    for (int t = 0; t < 32 * kPiecesRow / kWave; ++t) {
      const int piece = t * kWave + lane;
      const int row = piece / kPiecesRow, col = (piece % kPiecesRow) * 4;
      const int64_t m = r0 + 32 * i + row;
      const uint4 v = *reinterpret_cast<const uint4*>(ost + row * RS + col * 4);
      if (m < p.rows) *reinterpret_cast<uint4*>(mp.out + m * mp.D + dw0 + col) = v;
    }
    wave_sync();
  }
}

// fp32 / fp16 caches: fp32 products on v_mfma_f32_16x16x4f32.  64 hidden
// columns per workgroup; waves in 2x2, each 32 x 32.
template <typename T, bool UPDATE>
__global__ void __launch_bounds__(256) hidden_f32_kernel(const HiddenParams p) {
  constexpr int BN = 64;
  constexpr int LD = kRC32 + kPad32;
  constexpr uint32_t es = sizeof(T);
  __shared__ float a_s[kRows][LD];
  __shared__ float w_s[BN][LD];
  __shared__ RowTable rt;
  __shared__ float fresh[UPDATE ? fresh_batches() * 2 * BN : 1];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  // Row tiles of one batch row run on one XCD (one L2 for the rows they gather).
  const int64_t wg = xcd_tile(static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x,
                              static_cast<int64_t>(gridDim.x) * gridDim.y);
  const int64_t r0 = wg / gridDim.x * kRows;
  const int n0 = static_cast<int>(wg % gridDim.x) * BN;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wr_ = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t outr = make_rsrc(p.out, p.out_bytes);
  const int64_t t_pos = UPDATE ? index_at(p.pos, p.pos_dtype, 0) : -1;  // beside the row loads
  load_rows<T>(p, r0, rt);
  int64_t b_first;
  const int64_t t = update_setup<T, UPDATE>(p, t_pos, r0, n0, BN, b_first, fresh);
  __syncthreads();

  const int wr = (wave >> 1) * 32;
  const int wc = (wave & 1) * 32;
  const int r16 = lane & 15;
  const int k4 = lane >> 4;
  float xs[2][2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      gather_bases<T, UPDATE>(p, xr, rt, wr + i * 16, n0 + wc + j * 16 + r16, wc + j * 16 + r16,
                              t, b_first, fresh, BN, lane, xs[i][j]);
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int rc = 0; rc < p.R; rc += kRC32) {
    if (rc) __syncthreads();
    for (int idx = tid; idx < kRows * kRC32; idx += 256) {
      const int row = idx / kRC32;
      const int r = rc + idx % kRC32;
      const bool in = r < p.R;
      const float oa = buf_load_elem<T>(opr, in ? rt.op_a[row] + es * r : kNoOffset);
      const float op = buf_load_elem<T>(opr, in ? rt.op_p[row] + es * r : kNoOffset);
      a_s[row][idx % kRC32] = op * oa;
    }
    for (int idx = tid; idx < BN * kRC32; idx += 256) {
      const int n = n0 + idx / kRC32;
      const int r = rc + idx % kRC32;
      w_s[idx / kRC32][idx % kRC32] = buf_load_elem<T>(
          wr_, (n < p.H && r < p.R) ? es * (static_cast<uint32_t>(n) * p.R + r) : kNoOffset);
    }
    __syncthreads();
    const int rlen = p.R - rc < kRC32 ? p.R - rc : kRC32;
    for (int kk = 0; kk < rlen; kk += 4) {
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = a_s[wr + i * 16 + r16][kk + k4];
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = w_s[wc + j * 16 + r16][kk + k4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      store_hidden(p, outr, acc[i][j], xs[i][j], r0, wr + i * 16, n0 + wc + j * 16 + r16, lane);
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
  // Output-head preparation (relation_lm.py:203-206), when `prep` is set:
  //   final = LayerNorm_out(query + sigmoid(mix) * context), in the query's dtype.
  // Unset, every pointer below aliases `w` (D elements of w_dtype), so the
  // epilogue's loads stay unconditional and in bounds.
  int prep;
  const void* query;    // [Q,D]
  const void* mix;      // 0-d mix logit
  const void* ow;       // [D] output_norm weight
  const void* ob;       // [D] output_norm bias
  int query_dtype, mix_dtype, ow_dtype, ob_dtype;
  float out_eps;
  void* final;          // [Q,D], query_dtype
  // Raw rows given as split-K partial products (the per-query kernel only):
  // raw = sum_z parts[z] + b2, the splits added in order.
  const float* parts;   // [nparts][Q*K][D] fp32
  int nparts;           // 1 .. the kernel's NP
  const void* b2;       // [D]
  int b2_dtype;
};

__device__ __forceinline__ void store_any4(void* base, int dtype, int64_t i4, float4 v) {
  if (dtype == RLM_F32) {
    reinterpret_cast<float4*>(base)[i4] = v;
  } else if (dtype == RLM_BF16) {
    reinterpret_cast<uint2*>(base)[i4] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
  } else {
    f16* h = static_cast<f16*>(base) + 4 * i4;
    h[0] = static_cast<f16>(v.x);
    h[1] = static_cast<f16>(v.y);
    h[2] = static_cast<f16>(v.z);
    h[3] = static_cast<f16>(v.w);
  }
}
__device__ __forceinline__ void store_any(void* base, int dtype, int64_t i, float v) {
  if (dtype == RLM_F32)
    static_cast<float*>(base)[i] = v;
  else if (dtype == RLM_BF16)
    static_cast<bf16*>(base)[i] = f32_to_bf16(v);
  else
    static_cast<f16*>(base)[i] = static_cast<f16>(v);
}

// Softmax weight of partner `lane` (lanes 0..K-1; K <= 64) for the query at
// position t: k_limit = clamp(ceil(log2(t + 2)), 1, K) == clamp(bit_length(t + 1), 1, K),
// active = rank < k_limit and score > -1e30, p = softmax(where(active, s, -1e4)) * active,
// renormalised by max(sum, 1e-9) (relation_reduce.py:399-411).
__device__ __forceinline__ float partner_score(const NormParams& p, int64_t q, int lane) {
  const float s = p.scores[q * p.K + (lane < p.K ? lane : 0)];  // unconditional: no branch
  return lane < p.K ? s : -INFINITY;
}

// s: this lane's partner score (partner_score), loaded by the caller.
__device__ __forceinline__ float partner_weight(const NormParams& p, float s, int64_t t,
                                                int lane) {
  const int64_t n = t + 1;
  int k_limit = n > 0 ? 64 - __clzll(static_cast<unsigned long long>(n)) : 0;
  k_limit = k_limit < 1 ? 1 : (k_limit > p.K ? p.K : k_limit);
  const bool active = lane < p.K && lane < k_limit && s > -1.0e30f;
  const float safe = active ? s : -1.0e4f;
  const float m = wave_max_f32(lane < p.K ? safe : -INFINITY);
  const float prob = active ? expf(safe - m) : 0.0f;
  const float total = wave_sum_f32(prob);
  return prob / fmaxf(total, 1.0e-9f);
}

// Four consecutive raw elements as floats.
__device__ __forceinline__ float4 load_raw4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ float4 load_raw4(const bf16* p) { return load4(p); }
__device__ __forceinline__ float4 load_raw4(const f16* p) {
  const uint2 raw = *reinterpret_cast<const uint2*>(p);
  const f16* h = reinterpret_cast<const f16*>(&raw);
  return make_float4(static_cast<float>(h[0]), static_cast<float>(h[1]),
                     static_cast<float>(h[2]), static_cast<float>(h[3]));
}

// D % 4 == 0: lane owns column groups g = lane + 64*i (columns 4g..4g+3), so
// every raw row is read with 16-byte (fp32) or 8-byte (16-bit) coalesced
// loads.  KB partner rows are loaded before any of them is reduced, which puts
// the whole query's traffic in flight at once.
template <typename TR, int G, int KB>
__global__ void __launch_bounds__(256) norm_reduce_vec_kernel(const NormParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (q >= p.Q) return;
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  // Every load of the query is issued before any is used: position, scores,
  // gamma / beta, and the first KB partner rows (one memory round trip; the
  // loads are unconditional, from in-bounds addresses, so none waits at a branch).
  const int64_t t = index_at(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  const float score = partner_score(p, q, lane);
  const int groups = p.D >> 2;
  const TR* raw = static_cast<const TR*>(p.raw) + q * p.K * static_cast<int64_t>(p.D);

  F4Words gw[G], bw[G], qw[G], ow[G], obw[G];
  const int64_t qoff = p.prep ? q * (p.D >> 2) : 0;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    const int gs = g < groups ? g : 0;
    gw[i] = f4_issue(p.w, p.w_dtype, gs);
    bw[i] = f4_issue(p.bias, p.b_dtype, gs);
    qw[i] = f4_issue(p.query, p.query_dtype, qoff + gs);
    ow[i] = f4_issue(p.ow, p.ow_dtype, gs);
    obw[i] = f4_issue(p.ob, p.ob_dtype, gs);
  }
  const FloatWords mixw = issue_float(p.mix, p.mix_dtype, 1, 0, p.prep != 0);
  // Partner rows in batches of KB; the first batch is issued before anything
  // is decoded, so position, scores, gamma / beta and these rows share one
  // memory round trip.
  float4 x[KB][G];
  auto load_batch = [&](int k0) {
#pragma unroll
    for (int kk = 0; kk < KB; ++kk)
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const int g = lane + kWave * i;
        const bool in = k0 + kk < p.K && g < groups;
        const float4 v = load_raw4(raw + static_cast<int64_t>(in ? k0 + kk : 0) * p.D + 4 * (in ? g : 0));
        x[kk][i] = in ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  };
  load_batch(0);
  float4 gam[G], bet[G], ctx[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    gam[i] = g < groups ? f4_decode(gw[i], p.w_dtype) : zero;
    bet[i] = g < groups ? f4_decode(bw[i], p.b_dtype) : zero;
    ctx[i] = zero;
  }
  const float inv_d = 1.0f / static_cast<float>(p.D);
  const float prob = partner_weight(p, score, t, lane);
  for (int k0 = 0; k0 < p.K; k0 += KB) {
    if (k0 > 0) load_batch(k0);
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
      if (k0 + kk >= p.K) break;
      const float pk = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(prob), k0 + kk));
      if (pk == 0.0f) continue;  // wave-uniform: inactive rows contribute exactly 0
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < G; ++i) sum += (x[kk][i].x + x[kk][i].y) + (x[kk][i].z + x[kk][i].w);
      const float mean = wave_sum_f32(sum) * inv_d;
      float sq = 0.0f;
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const bool in = lane + kWave * i < groups;
        float4& v = x[kk][i];
        v.x = in ? v.x - mean : 0.0f;
        v.y = in ? v.y - mean : 0.0f;
        v.z = in ? v.z - mean : 0.0f;
        v.w = in ? v.w - mean : 0.0f;
        sq += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      }
      const float inv_std = rsqrtf(wave_sum_f32(sq) * inv_d + p.eps);
#pragma unroll
      for (int i = 0; i < G; ++i) {
        ctx[i].x += (x[kk][i].x * inv_std * gam[i].x + bet[i].x) * pk;
        ctx[i].y += (x[kk][i].y * inv_std * gam[i].y + bet[i].y) * pk;
        ctx[i].z += (x[kk][i].z * inv_std * gam[i].z + bet[i].z) * pk;
        ctx[i].w += (x[kk][i].w * inv_std * gam[i].w + bet[i].w) * pk;
      }
    }
  }
  float* out = p.out + q * static_cast<int64_t>(p.D);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = lane + kWave * i;
    if (g < groups) *reinterpret_cast<float4*>(out + 4 * g) = ctx[i];
  }
  if (p.prep) {  // wave-uniform
    // Output-head preparation: LayerNorm_out(query + sigmoid(mix) * context).
    const float gate = 1.0f / (1.0f + expf(-decode_float(mixw, p.mix_dtype)));
    float4 y[G];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const bool in = lane + kWave * i < groups;
      const float4 qv = f4_decode(qw[i], p.query_dtype);
      y[i] = in ? make_float4(fmaf(gate, ctx[i].x, qv.x), fmaf(gate, ctx[i].y, qv.y),
                              fmaf(gate, ctx[i].z, qv.z), fmaf(gate, ctx[i].w, qv.w))
                : make_float4(0.f, 0.f, 0.f, 0.f);
      sum += (y[i].x + y[i].y) + (y[i].z + y[i].w);
    }
    const float mean = wave_sum_f32(sum) * inv_d;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if (lane + kWave * i < groups) {
        const float dx = y[i].x - mean, dy = y[i].y - mean, dz = y[i].z - mean, dw = y[i].w - mean;
        sq += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float rstd = rsqrtf(wave_sum_f32(sq) * inv_d + p.out_eps);
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int g = lane + kWave * i;
      if (g >= groups) continue;
      const float4 w4 = f4_decode(ow[i], p.ow_dtype);
      const float4 b4 = f4_decode(obw[i], p.ob_dtype);
      store_any4(p.final, p.query_dtype, q * (p.D >> 2) + g,
                 make_float4(fmaf((y[i].x - mean) * rstd, w4.x, b4.x),
                             fmaf((y[i].y - mean) * rstd, w4.y, b4.y),
                             fmaf((y[i].z - mean) * rstd, w4.z, b4.z),
                             fmaf((y[i].w - mean) * rstd, w4.w, b4.w)));
    }
  }
}

// Decode shapes (a few queries): one workgroup of four waves per query, so
// that the query's latency chain is short.  Wave w normalises partner rows w,
// w + 4, ... (RPW of them side by side, so their reductions interleave); the
// parameter vectors (norm weight and bias, and for the output-head
// preparation the query, output weight and bias) are loaded as one 4-element
// chunk per thread and staged in LDS as fp32; the waves' weighted row sums
// meet in LDS:  context = gamma * sum_k p_k xhat_k + beta * sum_k p_k.
// fp32 raw rows, D % 4 == 0, D <= 256 * GI.
constexpr int kQWaves = 4;
constexpr int kQMaxD = 1024;
constexpr int64_t kQueryKernelMaxQ = 256;  // queries below which a workgroup per query pays
constexpr int kMaxParts = 4;                // split-K partial products summed on load

// Four consecutive elements c*4.. of a parameter vector of `dtype`: a 16-byte
// and an 8-byte load are both issued, the one that does not match the dtype
// out of range (no memory access).
struct Chunk4 {
  uint4 w32;
  uint2 w16;
};
__device__ __forceinline__ Chunk4 chunk4_issue(const void* base, int dtype, int D, int c, bool live) {
  const bool is32 = dtype == RLM_F32;
  const rsrc_t r = make_rsrc(base, static_cast<uint32_t>(D) * (is32 ? 4u : 2u));
  return {buf_load_b128(r, live && is32 ? 16u * c : kNoOffset),
          buf_load_b64(r, live && !is32 ? 8u * c : kNoOffset)};
}
__device__ __forceinline__ float4 chunk4_decode(const Chunk4& v, int dtype) {
  if (dtype == RLM_F32)
    return make_float4(__uint_as_float(v.w32.x), __uint_as_float(v.w32.y),
                       __uint_as_float(v.w32.z), __uint_as_float(v.w32.w));
  const uint32_t e[4] = {v.w16.x & 0xffffu, v.w16.x >> 16, v.w16.y & 0xffffu, v.w16.y >> 16};
  float f[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    f[k] = dtype == RLM_BF16
               ? __uint_as_float(e[k] << 16)
               : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(e[k])));
  return make_float4(f[0], f[1], f[2], f[3]);
}

// NP > 0: the raw rows are the sum of NP split-K partial products plus b2.
// Query q on threads 0 .. NW*64-1 of the workgroup (any further waves of the
// workgroup must have exited: the barriers below count the threads that remain).
// Row k is wave k mod NW's row k / NW.  With NW = 8 the rows' weighted sum keeps
// the four-wave grouping: wave w < 4 of a four-wave run adds rows w and w + 4,
// and the eight-wave run adds waves w and w + 4 in the same place.
// Cache policy of a device-coherent access (SC1): what agent-scope atomic loads and
// stores use, so data another workgroup (on any XCD) publishes this way is read
// without stale cache lines, with no whole-cache writeback or invalidation.
constexpr int kCpolDevice = 16;

template <int RPW, int GI, int NP, bool COHERENT = false, int NW = kQWaves>
__device__ __forceinline__ void norm_query(const NormParams& p, int64_t q) {
  static_assert(NW == kQWaves || NW == 2 * kQWaves, "four or eight waves");
  static_assert(NW == kQWaves || RPW == 1, "eight waves take one row each");
  __shared__ float4 par[5][kQMaxD / 4];    // w, b, query, ow, ob as fp32
  __shared__ float4 part[NW][kQMaxD / 4];  // each wave's sum_k p_k xhat_k
  __shared__ float red[2][kQWaves];        // columns live on waves 0..3 (D <= 1024)
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  const int groups = p.D >> 2;
  // ---- Every load of the query at once: position, scores, mix logit, the
  // wave's partner rows and one chunk of each parameter vector per thread.
  const int64_t t = index_at(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  const float score = partner_score(p, q, lane);
  const FloatWords mixw = issue_float(p.mix, p.mix_dtype, 1, 0, p.prep != 0);
  const float* raw = static_cast<const float*>(p.raw) + q * p.K * static_cast<int64_t>(p.D);
  // The parameter chunks go first: the row statistics below wait for the rows,
  // and with the chunks already in flight that wait covers them too.
  const bool cl = tid < groups;
  const Chunk4 cw = chunk4_issue(p.w, p.w_dtype, p.D, tid, cl);
  const Chunk4 cb = chunk4_issue(p.bias, p.b_dtype, p.D, tid, cl);
  const Chunk4 cq = chunk4_issue(static_cast<const unsigned char*>(p.query) +
                                     (p.prep ? q * p.D * (p.query_dtype == RLM_F32 ? 4 : 2) : 0),
                                 p.query_dtype, p.D, tid, cl);
  const Chunk4 cow = chunk4_issue(p.ow, p.ow_dtype, p.D, tid, cl);
  const Chunk4 cob = chunk4_issue(p.ob, p.ob_dtype, p.D, tid, cl);
  float4 x[RPW][GI];
  if constexpr (NP > 0) {
    // raw = (sum of the split-K partial products, in split order) + b2.  Every
    // partial of the wave's rows is loaded before any is added, so the
    // partials cost one memory round trip.
    const uint32_t pstride = static_cast<uint32_t>(p.Q * p.K * p.D) * 4u;  // bytes per split
    const rsrc_t prs = make_rsrc(p.parts, pstride * static_cast<uint32_t>(p.nparts));
    const uint32_t qoff = static_cast<uint32_t>(q * p.K * p.D) * 4u;
    F4Words bw[GI];
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      const int g = lane + kWave * i;
      bw[i] = f4_issue(p.b2, p.b2_dtype, g < groups ? g : 0);
    }
    uint4 w[RPW][GI][NP];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int i = 0; i < GI; ++i) {
        const int k = wave + NW * r;
        const int g = lane + kWave * i;
        const bool in = k < p.K && g < groups;
        // Lanes past the row and rows past K read nothing.
        const uint32_t off = qoff + static_cast<uint32_t>((in ? k : 0) * p.D + 4 * (in ? g : 0)) * 4u;
#pragma unroll
        for (int z = 0; z < NP; ++z)
          w[r][i][z] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, in && z < p.nparts ? off + z * pstride : kNoOffset, 0,
                         COHERENT ? kCpolDevice : 0));
      }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int i = 0; i < GI; ++i) {
        const int k = wave + NW * r;
        const int g = lane + kWave * i;
        const bool in = k < p.K && g < groups;
        float4 v = make_float4(__uint_as_float(w[r][i][0].x), __uint_as_float(w[r][i][0].y),
                               __uint_as_float(w[r][i][0].z), __uint_as_float(w[r][i][0].w));
#pragma unroll
        for (int z = 1; z < NP; ++z) {
          const bool use = z < p.nparts;  // at most NP partial products, nparts of them given
          v.x = use ? v.x + __uint_as_float(w[r][i][z].x) : v.x;
          v.y = use ? v.y + __uint_as_float(w[r][i][z].y) : v.y;
          v.z = use ? v.z + __uint_as_float(w[r][i][z].z) : v.z;
          v.w = use ? v.w + __uint_as_float(w[r][i][z].w) : v.w;
        }
        const float4 b4 = f4_decode(bw[i], p.b2_dtype);
        x[r][i] = in ? make_float4(v.x + b4.x, v.y + b4.y, v.z + b4.z, v.w + b4.w)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  } else {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int i = 0; i < GI; ++i) {
        const int k = wave + NW * r;
        const int g = lane + kWave * i;
        const bool in = k < p.K && g < groups;
        const float4 v = *reinterpret_cast<const float4*>(raw + static_cast<int64_t>(in ? k : 0) * p.D +
                                                          4 * (in ? g : 0));
        x[r][i] = in ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  }

  // ---- Partner weights (every wave computes the same ones).
  const float prob = partner_weight(p, score, t, lane);
  const float psum = wave_sum_f32(prob);
  const float inv_d = 1.0f / static_cast<float>(p.D);
  // ---- Row statistics, the wave's rows side by side.
  float mean[RPW], rstd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < GI; ++i) s += (x[r][i].x + x[r][i].y) + (x[r][i].z + x[r][i].w);
    mean[r] = wave_sum_f32(s) * inv_d;
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      const bool in = lane + kWave * i < groups;
      float4& v = x[r][i];
      v.x = in ? v.x - mean[r] : 0.0f;
      v.y = in ? v.y - mean[r] : 0.0f;
      v.z = in ? v.z - mean[r] : 0.0f;
      v.w = in ? v.w - mean[r] : 0.0f;
      sq += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    rstd[r] = rsqrtf(wave_sum_f32(sq) * inv_d + p.eps);
  }
  // Weighted sum of the wave's normalised rows; an inactive row (weight 0)
  // adds exactly 0.
  float4 acc[GI];
#pragma unroll
  for (int i = 0; i < GI; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int k = wave + NW * r;
    const float pk = __uint_as_float(
        __builtin_amdgcn_readlane(__float_as_uint(prob), k < p.K ? k : 0));
    const bool use = k < p.K && pk != 0.0f;
#pragma unroll
    for (int i = 0; i < GI; ++i) {
      acc[i].x += use ? pk * (x[r][i].x * rstd[r]) : 0.0f;
      acc[i].y += use ? pk * (x[r][i].y * rstd[r]) : 0.0f;
      acc[i].z += use ? pk * (x[r][i].z * rstd[r]) : 0.0f;
      acc[i].w += use ? pk * (x[r][i].w * rstd[r]) : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < GI; ++i) {
    const int g = lane + kWave * i;
    if (g < groups) part[wave][g] = acc[i];
  }
  if (cl) {
    par[0][tid] = chunk4_decode(cw, p.w_dtype);
    par[1][tid] = chunk4_decode(cb, p.b_dtype);
    par[2][tid] = chunk4_decode(cq, p.query_dtype);
    par[3][tid] = chunk4_decode(cow, p.ow_dtype);
    par[4][tid] = chunk4_decode(cob, p.ob_dtype);
  }
  __syncthreads();
  // ---- Column phase: thread tid owns columns 4 tid .. 4 tid + 3.
  float4 ctx = make_float4(0.f, 0.f, 0.f, 0.f);
  if (cl) {
    // Wave w's rows of a four-wave run: rows w and w + 4.
    auto rows_of = [&](int w) {
      float4 v = part[w][tid];
      if constexpr (NW > kQWaves) {
        const float4 o = part[w + kQWaves][tid];
        v = make_float4(v.x + o.x, v.y + o.y, v.z + o.z, v.w + o.w);
      }
      return v;
    };
    float4 s = rows_of(0);
#pragma unroll
    for (int w = 1; w < kQWaves; ++w) {
      const float4 o = rows_of(w);
      s.x += o.x;
      s.y += o.y;
      s.z += o.z;
      s.w += o.w;
    }
    const float4 gm = par[0][tid], bt = par[1][tid];
    ctx = make_float4(fmaf(gm.x, s.x, bt.x * psum), fmaf(gm.y, s.y, bt.y * psum),
                      fmaf(gm.z, s.z, bt.z * psum), fmaf(gm.w, s.w, bt.w * psum));
    reinterpret_cast<float4*>(p.out + q * static_cast<int64_t>(p.D))[tid] = ctx;
  }
  if (!p.prep) return;  // uniform
  // ---- Output-head preparation: LayerNorm_out(query + sigmoid(mix) * context).
  const float gate = 1.0f / (1.0f + expf(-decode_float(mixw, p.mix_dtype)));
  float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
  if (cl) {
    const float4 qv = par[2][tid];
    y = make_float4(fmaf(gate, ctx.x, qv.x), fmaf(gate, ctx.y, qv.y), fmaf(gate, ctx.z, qv.z),
                    fmaf(gate, ctx.w, qv.w));
  }
  float s = wave_sum_f32((y.x + y.y) + (y.z + y.w));
  if (lane == 0 && wave < kQWaves) red[0][wave] = s;
  __syncthreads();
  const float ymean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) * inv_d;
  const float4 dy = cl ? make_float4(y.x - ymean, y.y - ymean, y.z - ymean, y.w - ymean)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
  s = wave_sum_f32((dy.x * dy.x + dy.y * dy.y) + (dy.z * dy.z + dy.w * dy.w));
  if (lane == 0 && wave < kQWaves) red[1][wave] = s;
  __syncthreads();
  const float yrstd =
      rsqrtf(((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) * inv_d + p.out_eps);
  if (cl) {
    const float4 w4 = par[3][tid], b4 = par[4][tid];
    store_any4(p.final, p.query_dtype, q * groups + tid,
               make_float4(fmaf(dy.x * yrstd, w4.x, b4.x), fmaf(dy.y * yrstd, w4.y, b4.y),
                           fmaf(dy.z * yrstd, w4.z, b4.z), fmaf(dy.w * yrstd, w4.w, b4.w)));
  }
}

template <int RPW, int GI, int NP>
__global__ void __launch_bounds__(kQWaves * kWave) __attribute__((amdgpu_waves_per_eu(1, 1)))
norm_reduce_query_kernel(const NormParams p) {
  norm_query<RPW, GI, NP>(p, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Decode relation tail in one launch: relation hidden -> second linear ->
// norm-reduce with the output-head preparation, for a few queries (one per
// batch row) of K <= 16 partner rows each.
//
// Workgroup (s, q) owns hidden columns [64 s, 64 s + 64) of query q's K rows:
//   1. hidden^T[64 x 16 rows] = W_m[slice] . P^T on v_mfma_f32_16x16x32_bf16
//      (P = op[a] * op[p], exact in fp32, as an exact hi + lo bf16 pair), plus
//      the expanded-cache halves X[a, n] + X[p, H + n], erf-GELU, rounded to
//      bf16 (the operand the two-launch linear sees) into LDS; waves 0..3, one
//      16-column tile each.  Invalid indices gather zero rows, as
//      relation_hidden_cached(_ring) does.
//   2. partial^T[D x 16 rows] = W2[:, slice] . hidden^T over the slice's 64
//      columns (all 8 waves, 16-row tiles of D; the W2 fragments are loaded at
//      entry), stored fp32 to partials[s][q K + k][:].
//   3. The slices are counted in groups of `spg`: each workgroup stores its
//      partials with device-coherent (SC1) stores, waits for their
//      acknowledgement and adds one to its group's counter with a vector
//      atomic; the workgroup that brings the count to the group's size reads
//      them back with device-coherent loads (no whole-L2 writeback or
//      invalidation, which every workgroup would otherwise pay) and sums the
//      group's partials in slice order into gsum[group], then
//      counts on the query's counter; the last group's workgroup runs the
//      per-query norm-reduce and output head (norm_query, on all eight waves:
//      one partner row each) on the group sums plus b2, in group order.  Every sum has a fixed order: the result does
//      not depend on which workgroup arrives last.  Nothing waits for another
//      workgroup; the last arrival of each level does the next step.  Each
//      counter is reset to zero by that last arrival, so the next launch (and a
//      graph replay) starts from zero.
// ---------------------------------------------------------------------------
constexpr int kDecSlice = 64;                  // hidden columns per workgroup
constexpr int kDecWaves = 8;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kDecMaxK = 8;                    // partner rows per query (rows of one 16-row tile)
constexpr int kDecMaxD = 768;                  // d_model: norm_query with GI <= 3
constexpr int kDecMaxDT = 6;                   // 16-row tiles of D per wave (D <= 768)
constexpr int kDecMaxSpg = 12;                 // slices per group
constexpr int kDecGroups = kMaxParts;          // groups per query (norm_query's NP)
constexpr int kDecHidLd = kDecSlice + 8;       // bf16 per hidden row in LDS (conflict-free b128)
constexpr int kDecSumBatch = 3;                // float4 elements per thread per level-1 round
static_assert(kDecMaxK <= kDecWaves, "norm_query takes one partner row per wave");

struct DecodeParams {
  NormParams n;            // level 2: parts = gsum, nparts = groups, b2, output head
  int64_t T;               // cache rows
  int B, K, R, H, D;
  int S, G, spg;           // slices, groups, slices per group
  int ring;                // ring caches: index i lives in row i mod T, any i < 2^31
  const void* expanded;    // [B,T,2H] bf16
  const void* operand;     // [B,T,R] bf16
  const void* anchor;      // [B]
  const void* partner;     // [B,K]
  int index_dtype_a, index_dtype_p;
  const void* wm;          // [H,R] bf16
  const void* w2;          // [D,H] bf16
  float* partials;         // [S][B*K][D]
  float* gsum;             // [G][B*K][D]
  uint32_t* counters;      // [B*G] group counters, then [B] query counters
  uint32_t expanded_bytes, operand_bytes, wm_bytes, w2_bytes, partials_bytes, gsum_bytes;
};

template <int KS, int GI>
__global__ void __launch_bounds__(kDecThreads) decode_relation_kernel(const DecodeParams p) {
  __shared__ __align__(16) uint16_t hid[16][kDecHidLd];
  __shared__ int last;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r16 = lane & 15, g = lane >> 4;
  const int s = blockIdx.x, q = blockIdx.y;
  const int h0 = s * kDecSlice;
  const uint32_t H = static_cast<uint32_t>(p.H), R = static_cast<uint32_t>(p.R);
  const rsrc_t wmr = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t w2r = make_rsrc(p.w2, p.w2_bytes);
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);

  // ---- Loads that need no index, all issued at entry.  W2 fragments of this
  // wave's D tiles (A operand: row d = 16 dt + r16, k = 32 ks + 8 g of the slice).
  u16x8 w2f[kDecMaxDT][2];
#pragma unroll
  for (int i = 0; i < kDecMaxDT; ++i) {
    const int d = (wave + kDecWaves * i) * 16 + r16;
    const bool in = d < p.D;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      w2f[i][ks] = __builtin_bit_cast(
          u16x8, buf_load_b128(w2r, in ? (static_cast<uint32_t>(d) * H + h0 + 32 * ks + 8 * g) * 2u
                                       : kNoOffset));
  }
  // W_m fragments of the hidden tile of waves 0..3: columns h0 + 16 wave + r16.
  const bool hw = wave < 4;
  u16x8 wmf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    wmf[ks] = __builtin_bit_cast(
        u16x8, buf_load_b128(wmr, hw ? ((h0 + 16u * wave + r16) * R + 32 * ks + 8 * g) * 2u
                                     : kNoOffset));
  // Row m = r16 of the tile is partner m of query q (m < K).
  const bool live = r16 < p.K;
  const int64_t ai = index_at(p.anchor, p.index_dtype_a, q);
  const int64_t pi = index_at(p.partner, p.index_dtype_p, static_cast<int64_t>(q) * p.K + (live ? r16 : 0));
  const int64_t hi_idx = p.ring ? (int64_t(1) << 31) : p.T;
  const int32_t a = (ai >= 0 && ai < hi_idx) ? static_cast<int32_t>(ai) : -1;
  const int32_t pp = (live && pi >= 0 && pi < hi_idx) ? static_cast<int32_t>(pi) : -1;
  const uint32_t mask = p.ring ? static_cast<uint32_t>(p.T - 1) : 0xffffffffu;
  const uint32_t base = static_cast<uint32_t>(q) * static_cast<uint32_t>(p.T);
  const uint32_t ra = base + (static_cast<uint32_t>(a) & mask);
  const uint32_t rp = base + (static_cast<uint32_t>(pp) & mask);
  const bool both = a >= 0 && pp >= 0;

  // ---- 1. Hidden tile (waves 0..3).
  if (hw) {
    uint4 va[KS], vp[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      va[ks] = buf_load_b128(opr, both ? (ra * R + 32 * ks + 8 * g) * 2u : kNoOffset);
      vp[ks] = buf_load_b128(opr, both ? (rp * R + 32 * ks + 8 * g) * 2u : kNoOffset);
    }
    const uint32_t col = h0 + 16u * wave + 4u * g;
    const uint2 xa = buf_load_b64(xr, (live && a >= 0) ? (ra * 2u * H + col) * 2u : kNoOffset);
    const uint2 xp = buf_load_b64(xr, pp >= 0 ? (rp * 2u * H + H + col) * 2u : kNoOffset);
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint32_t wa[4] = {va[ks].x, va[ks].y, va[ks].z, va[ks].w};
      const uint32_t wp[4] = {vp[ks].x, vp[ks].y, vp[ks].z, vp[ks].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = bf16_lo(wp[k]) * bf16_lo(wa[k]);  // exact: 8-bit x 8-bit significands
        const float x1 = bf16_hi(wp[k]) * bf16_hi(wa[k]);
        h[k] = pack_bf16x2(x0, x1);
        l[k] = pack_bf16x2(x0 - bf16_lo(h[k]), x1 - bf16_hi(h[k]));
      }
      const uint4 hv = make_uint4(h[0], h[1], h[2], h[3]), lv = make_uint4(l[0], l[1], l[2], l[3]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wmf[ks]),
                                                    __builtin_bit_cast(bf16x8, hv), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wmf[ks]),
                                                    __builtin_bit_cast(bf16x8, lv), acc, 0, 0, 0);
    }
    // acc[e] = hidden^T[column col + e][row r16].
    const float xs[4] = {bf16_lo(xa.x) + bf16_lo(xp.x), bf16_hi(xa.x) + bf16_hi(xp.x),
                         bf16_lo(xa.y) + bf16_lo(xp.y), bf16_hi(xa.y) + bf16_hi(xp.y)};
    *reinterpret_cast<uint2*>(&hid[r16][16 * wave + 4 * g]) =
        make_uint2(pack_bf16x2(gelu_erf(acc[0] + xs[0]), gelu_erf(acc[1] + xs[1])),
                   pack_bf16x2(gelu_erf(acc[2] + xs[2]), gelu_erf(acc[3] + xs[3])));
  }
  __syncthreads();

  // ---- 2. Partial products of the slice: partial^T[d][row] over 64 columns.
  const int BK = p.B * p.K;
  const rsrc_t pr = make_rsrc(p.partials, p.partials_bytes);
  {
    u16x8 hb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) hb[ks] = *reinterpret_cast<const u16x8*>(&hid[r16][32 * ks + 8 * g]);
    const uint32_t row_off = (static_cast<uint32_t>(s) * BK + static_cast<uint32_t>(q) * p.K + r16) *
                             static_cast<uint32_t>(p.D);
#pragma unroll
    for (int i = 0; i < kDecMaxDT; ++i) {
      const int d0 = (wave + kDecWaves * i) * 16;
      if (d0 >= p.D) break;  // uniform
      f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w2f[i][ks]),
                                                      __builtin_bit_cast(bf16x8, hb[ks]), acc, 0, 0, 0);
      // acc[e] = partial^T[d0 + 4 g + e][row r16]; D % 4 == 0.
      const int d = d0 + 4 * g;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), pr,
                                             (live && d < p.D) ? (row_off + d) * 4u : kNoOffset,
                                             0, kCpolDevice);
    }
  }

  // ---- 3a. Group count: the group's last workgroup sums its partials.
  const int grp = s / p.spg;
  const int s_lo = grp * p.spg;
  const int n_grp = min(p.S - s_lo, p.spg);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are acknowledged
  __syncthreads();
  if (tid == 0) {
    uint32_t* ctr = p.counters + q * p.G + grp;
    last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           static_cast<uint32_t>(n_grp - 1);
  }
  __syncthreads();
  if (!last) return;  // uniform
  if (tid == 0) __hip_atomic_store(p.counters + q * p.G + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  {
    const rsrc_t gr = make_rsrc(p.gsum, p.gsum_bytes);
    const uint32_t n4 = static_cast<uint32_t>(p.K * p.D / 4);       // float4 of the query's rows
    const uint32_t q4 = static_cast<uint32_t>(q) * n4;               // the query's first float4
    const uint32_t split4 = static_cast<uint32_t>(BK * p.D / 4);     // float4 per slice
    for (uint32_t e0 = 0; e0 < n4; e0 += kDecThreads * kDecSumBatch) {
      uint4 v[kDecSumBatch][kDecMaxSpg];
#pragma unroll
      for (int u = 0; u < kDecSumBatch; ++u) {
        const uint32_t e = e0 + tid + kDecThreads * u;
#pragma unroll
        for (int z = 0; z < kDecMaxSpg; ++z)
          v[u][z] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(
                         pr, (e < n4 && z < n_grp) ? ((s_lo + z) * split4 + q4 + e) * 16u
                                                   : kNoOffset,
                         0, kCpolDevice));
      }
#pragma unroll
      for (int u = 0; u < kDecSumBatch; ++u) {
        const uint32_t e = e0 + tid + kDecThreads * u;
        float4 acc = make_float4(__uint_as_float(v[u][0].x), __uint_as_float(v[u][0].y),
                                 __uint_as_float(v[u][0].z), __uint_as_float(v[u][0].w));
#pragma unroll
        for (int z = 1; z < kDecMaxSpg; ++z) {
          const bool use = z < n_grp;
          acc.x = use ? acc.x + __uint_as_float(v[u][z].x) : acc.x;
          acc.y = use ? acc.y + __uint_as_float(v[u][z].y) : acc.y;
          acc.z = use ? acc.z + __uint_as_float(v[u][z].z) : acc.z;
          acc.w = use ? acc.w + __uint_as_float(v[u][z].w) : acc.w;
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), gr,
                                               e < n4 ? (grp * split4 + q4 + e) * 16u : kNoOffset,
                                               0, kCpolDevice);
      }
    }
  }

  // ---- 3b. Query count: the last group's workgroup runs the norm-reduce.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's group sums are acknowledged
  __syncthreads();
  if (tid == 0) {
    uint32_t* ctr = p.counters + p.B * p.G + q;
    last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           static_cast<uint32_t>(p.G - 1);
  }
  __syncthreads();
  if (!last) return;  // uniform
  if (tid == 0) __hip_atomic_store(p.counters + p.B * p.G + q, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  norm_query<1, GI, kDecGroups, true, kDecWaves>(p.n, q);
}

// Slices, groups and slices per group for hidden dim H (a multiple of 64).
struct DecodeShape {
  int S, G, spg;
};
inline DecodeShape decode_shape(int64_t H) {
  const int S = static_cast<int>(H / kDecSlice);
  const int G = S < kDecGroups ? S : kDecGroups;
  return {S, G, G > 0 ? (S + G - 1) / G : 0};
}
inline bool decode_fits_shape(int64_t B, int64_t K, int64_t R, int64_t H, int64_t D) {
  if (!(R == 64 || R == 128) || H <= 0 || H % kDecSlice != 0) return false;
  return B >= 1 && B <= 65535 && K >= 1 && K <= kDecMaxK && D >= 4 && D % 4 == 0 &&
         D <= kDecMaxD && decode_shape(H).spg <= kDecMaxSpg;
}

template <int KS>
hipError_t launch_decode_ks(const DecodeParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.S), static_cast<unsigned>(p.B));
  const int gi = (p.D / 4 + kWave - 1) / kWave;
  if (gi <= 1)
    hipLaunchKernelGGL((decode_relation_kernel<KS, 1>), grid, dim3(kDecThreads), 0, stream, p);
  else if (gi <= 2)
    hipLaunchKernelGGL((decode_relation_kernel<KS, 2>), grid, dim3(kDecThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_relation_kernel<KS, 3>), grid, dim3(kDecThreads), 0, stream, p);
  return launch_status("relation_hidden_linear_norm_reduce_output");
}

hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
  return p.R == 128 ? launch_decode_ks<4>(p, stream) : launch_decode_ks<2>(p, stream);
}

template <typename TR, int VPL>
__global__ void __launch_bounds__(256) norm_reduce_kernel(const NormParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (q >= p.Q) return;
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  const float prob = partner_weight(p, partner_score(p, q, lane), t, lane);

  float gam[VPL], bet[VPL], ctx[VPL], qv[VPL], ow[VPL], obv[VPL];
  const int64_t qoff = p.prep ? q * p.D : 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int d = lane + kWave * i;
    const int ds = d < p.D ? d : 0;
    gam[i] = d < p.D ? load_any_f(p.w, p.w_dtype, d) : 0.0f;
    bet[i] = d < p.D ? load_any_f(p.bias, p.b_dtype, d) : 0.0f;
    qv[i] = load_any_f(p.query, p.query_dtype, qoff + ds);
    ow[i] = load_any_f(p.ow, p.ow_dtype, ds);
    obv[i] = load_any_f(p.ob, p.ob_dtype, ds);
    ctx[i] = 0.0f;
  }
  const FloatWords mixw = issue_float(p.mix, p.mix_dtype, 1, 0, p.prep != 0);
  const float inv_d = 1.0f / static_cast<float>(p.D);
  const TR* raw = static_cast<const TR*>(p.raw) + q * p.K * static_cast<int64_t>(p.D);
  for (int k = 0; k < p.K; ++k) {
    const float pk = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(prob), k));
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
  if (p.prep) {  // wave-uniform: output-head preparation, as the vector kernel
    const float gate = 1.0f / (1.0f + expf(-decode_float(mixw, p.mix_dtype)));
    float y[VPL], sum = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      y[i] = lane + kWave * i < p.D ? fmaf(gate, ctx[i], qv[i]) : 0.0f;
      sum += y[i];
    }
    const float mean = wave_sum_f32(sum) * inv_d;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const float dv = lane + kWave * i < p.D ? y[i] - mean : 0.0f;
      sq += dv * dv;
    }
    const float rstd = rsqrtf(wave_sum_f32(sq) * inv_d + p.out_eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int d = lane + kWave * i;
      if (d < p.D) store_any(p.final, p.query_dtype, q * p.D + d, fmaf((y[i] - mean) * rstd, ow[i], obv[i]));
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

hipError_t launch_hidden(HiddenParams& p, int dtype, bool update, hipStream_t stream) {
  if (p.rows == 0 || p.H == 0) return hipSuccess;
  const unsigned row_tiles = static_cast<unsigned>((p.rows + kRows - 1) / kRows);
  RLM_REQUIRE(row_tiles <= 65535u * 1024u, "too many relation rows");
  if (dtype == RLM_BF16) {
    // Sequence form with many rows, relation dim 64 or 128: a 64-row tile of
    // four waves per workgroup over every column (the same arithmetic for
    // fp32 and bf16 outputs).  Otherwise 128-column tiles when there are enough rows
    // to fill the chip, else 64 (always 64 in the update form, whose fresh
    // rows live in LDS too).
    if (!update && p.rows >= 4096 && (p.R == 128 || p.R == 64) && p.H % 8 == 0 &&
        (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0) {
      const int64_t tiles = (p.rows + kTileRows - 1) / kTileRows;
      RLM_REQUIRE(tiles <= 0x7fffffff, "too many relation rows");
#define RLM_TILE_CASE(TO, R)                                                                    \
  {                                                                                             \
    constexpr size_t lds = hidden_tile_lds_bytes<R>();                                          \
    static const hipError_t attr = hipFuncSetAttribute(                                         \
        reinterpret_cast<const void*>(&hidden_tile_kernel<TO, R>),                              \
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));                     \
    if (attr != hipSuccess) {                                                                   \
      set_error("relation_hidden: cannot reserve %zu bytes of LDS: %s", lds,                   \
                hipGetErrorString(attr));                                                       \
      return attr;                                                                              \
    }                                                                                           \
    hipLaunchKernelGGL((hidden_tile_kernel<TO, R>), dim3(static_cast<unsigned>(tiles)),         \
                       dim3(kTileThreads), lds, stream, p);                                     \
  }
      if (p.out_bf16) {
        if (p.R == 128) RLM_TILE_CASE(bf16, 128) else RLM_TILE_CASE(bf16, 64)
      } else {
        if (p.R == 128) RLM_TILE_CASE(float, 128) else RLM_TILE_CASE(float, 64)
      }
#undef RLM_TILE_CASE
      return launch_status("relation_hidden");
    }
    if (update) {
      const dim3 grid(static_cast<unsigned>((p.H + 63) / 64), row_tiles);
      hipLaunchKernelGGL((hidden_bf16_kernel<true, 64>), grid, dim3(256), 0, stream, p);
    } else if (p.rows >= 4096) {
      const dim3 grid(static_cast<unsigned>((p.H + 127) / 128), row_tiles);
      hipLaunchKernelGGL((hidden_bf16_kernel<false, 128>), grid, dim3(256), 0, stream, p);
    } else {
      const dim3 grid(static_cast<unsigned>((p.H + 63) / 64), row_tiles);
      hipLaunchKernelGGL((hidden_bf16_kernel<false, 64>), grid, dim3(256), 0, stream, p);
    }
    return launch_status("relation_hidden");
  }
  const dim3 grid(static_cast<unsigned>((p.H + 63) / 64), row_tiles);
#define RLM_HIDDEN_CASE(ID, T)                                                             \
  if (dtype == ID) {                                                                       \
    if (update)                                                                            \
      hipLaunchKernelGGL((hidden_f32_kernel<T, true>), grid, dim3(256), 0, stream, p);     \
    else                                                                                   \
      hipLaunchKernelGGL((hidden_f32_kernel<T, false>), grid, dim3(256), 0, stream, p);    \
    return launch_status("relation_hidden");                                               \
  }
  RLM_HIDDEN_CASE(RLM_F32, float)
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
  RLM_REQUIRE(R >= 8 && R <= 4096 && R % 8 == 0 && H <= (1 << 20) && K <= 4096,
              "relation dim must be a multiple of 8 in [8, 4096]; hidden dim and partner count "
              "out of range otherwise");
  const int64_t es = operand_cache->dtype == RLM_F32 ? 4 : 2;
  constexpr int64_t kMaxBytes = int64_t(1) << 31;
  RLM_REQUIRE(B * T * 2 * H * es < kMaxBytes && B * T * R * es < kMaxBytes &&
                  H * R * es < kMaxBytes,
              "expanded_cache, operand_cache and product_weight must each be smaller than 2 GiB");
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(operand_cache->data) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(product_weight->data) & 15u) == 0,
              "operand_cache and product_weight must be 16-byte aligned");
  RLM_TRY(check_tensor(out, "out", qd + 2));
  RLM_REQUIRE(out->dtype == RLM_F32 || out->dtype == RLM_BF16, "out must be float32 or bfloat16");
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
  p.out_bf16 = out->dtype == RLM_BF16 ? 1 : 0;
  const int64_t os = p.out_bf16 ? 2 : 4;
  RLM_REQUIRE(p.rows * H * os + 64 * H * 4 < kMaxBytes,
              "relation hidden output must be smaller than 2 GiB");
  p.expanded_bytes = static_cast<uint32_t>(B * T * 2 * H * es);
  p.operand_bytes = static_cast<uint32_t>(B * T * R * es);
  p.wm_bytes = static_cast<uint32_t>(H * R * es);
  p.out_bytes = static_cast<uint32_t>(p.rows * H * os);
  return hipSuccess;
}

template <int G, int KB>
hipError_t launch_norm_vec(const NormParams& p, int dtype, hipStream_t stream) {
  const int waves = 4;
  const dim3 grid(static_cast<unsigned>((p.Q + waves - 1) / waves));
#define RLM_NORM_CASE(ID, T)                                                                   \
  if (dtype == ID) {                                                                           \
    hipLaunchKernelGGL((norm_reduce_vec_kernel<T, G, KB>), grid, dim3(waves * kWave), 0, stream, \
                       p);                                                                     \
    return launch_status("relation_norm_reduce");                                             \
  }
  RLM_NORM_CASE(RLM_F32, float)
  RLM_NORM_CASE(RLM_BF16, bf16)
  RLM_NORM_CASE(RLM_F16, f16)
#undef RLM_NORM_CASE
  set_error("relation_norm_reduce: unsupported raw dtype %s", dtype_name(dtype));
  return hipErrorInvalidValue;
}

template <int RPW>
hipError_t launch_norm_query_rpw(const NormParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.Q));
  const int gi = (p.D / 4 + kWave - 1) / kWave;
#define RLM_NORMQ_NP(GI, NP)                                                                  \
  hipLaunchKernelGGL((norm_reduce_query_kernel<RPW, GI, NP>), grid, dim3(kQWaves * kWave), 0, \
                     stream, p)
#define RLM_NORMQ_CASE(GI)                                                                    \
  if (gi <= GI) {                                                                             \
    switch (p.nparts) {                                                                       \
      case 0: RLM_NORMQ_NP(GI, 0); break;                                                     \
      case 1: RLM_NORMQ_NP(GI, 1); break;                                                     \
      case 2: RLM_NORMQ_NP(GI, 2); break;                                                     \
      case 3: RLM_NORMQ_NP(GI, 3); break;                                                     \
      default: RLM_NORMQ_NP(GI, 4); break;                                                    \
    }                                                                                         \
    return launch_status("relation_norm_reduce");                                            \
  }
  RLM_NORMQ_CASE(1)
  RLM_NORMQ_CASE(2)
  RLM_NORMQ_CASE(3)
  RLM_NORMQ_CASE(4)
#undef RLM_NORMQ_CASE
#undef RLM_NORMQ_NP
  set_error("relation_norm_reduce: width %d too large for the per-query kernel", p.D);
  return hipErrorInvalidValue;
}

hipError_t launch_norm_query(const NormParams& p, hipStream_t stream) {
  switch ((p.K + kQWaves - 1) / kQWaves) {
    case 1: return launch_norm_query_rpw<1>(p, stream);
    case 2: return launch_norm_query_rpw<2>(p, stream);
    case 3: return launch_norm_query_rpw<3>(p, stream);
    default: return launch_norm_query_rpw<4>(p, stream);
  }
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

// Output-head preparation arguments of norm_impl (all null: context only).
struct OutputPrep {
  // Raw rows as split-K partial products [S, Q*K, D] fp32 plus the second
  // linear's bias (the raw tensor then only describes the shape).
  const rlm_tensor* parts = nullptr;
  const rlm_tensor* b2 = nullptr;
  const rlm_tensor* query = nullptr;
  const rlm_tensor* mix_logit = nullptr;
  const rlm_tensor* weight = nullptr;
  const rlm_tensor* bias = nullptr;
  double eps = 0.0;
  const rlm_tensor* final = nullptr;
};

// Checks the norm-reduce arguments and fills the kernel parameters; `raw`
// only describes the shape when the rows come as partial products (prep.parts).
hipError_t norm_setup(bool seq, const rlm_tensor* raw, const rlm_tensor* partner_scores,
                      const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
                      const rlm_tensor* position, double norm_eps, const rlm_tensor* out,
                      const OutputPrep& prep, NormParams& p) {
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
  p = NormParams{};
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
  p.prep = prep.query != nullptr;
  p.query = p.mix = p.ow = p.ob = p.w;
  p.query_dtype = p.mix_dtype = p.ow_dtype = p.ob_dtype = p.w_dtype;
  p.final = nullptr;
  if (p.prep) {
    const int qd = seq ? 2 : 1;
    RLM_TRY(check_tensor(prep.query, "query", qd + 1));
    RLM_TRY(check_dtype_float(prep.query, "query"));
    RLM_TRY(check_dim(prep.query, "query", 0, B));
    if (seq) RLM_TRY(check_dim(prep.query, "query", 1, Tq));
    RLM_TRY(check_dim(prep.query, "query", qd, D));
    RLM_TRY(check_tensor(prep.mix_logit, "mix_logit", 0));
    RLM_TRY(check_dtype_float(prep.mix_logit, "mix_logit"));
    RLM_TRY(check_tensor(prep.weight, "output_weight", 1));
    RLM_TRY(check_dtype_float(prep.weight, "output_weight"));
    RLM_TRY(check_dim(prep.weight, "output_weight", 0, D));
    RLM_TRY(check_tensor(prep.bias, "output_bias", 1));
    RLM_TRY(check_dtype_float(prep.bias, "output_bias"));
    RLM_TRY(check_dim(prep.bias, "output_bias", 0, D));
    RLM_TRY(check_tensor(prep.final, "out_final", qd + 1));
    RLM_TRY(check_same_dtype(prep.final, "out_final", prep.query, "query"));
    RLM_TRY(check_dim(prep.final, "out_final", 0, B));
    if (seq) RLM_TRY(check_dim(prep.final, "out_final", 1, Tq));
    RLM_TRY(check_dim(prep.final, "out_final", qd, D));
    for (const rlm_tensor* t : {prep.query, prep.weight, prep.bias, prep.final})
      RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                  "query, output_weight, output_bias and out_final must be 16-byte aligned");
    p.query = prep.query->data;
    p.query_dtype = prep.query->dtype;
    p.mix = prep.mix_logit->data;
    p.mix_dtype = prep.mix_logit->dtype;
    p.ow = prep.weight->data;
    p.ow_dtype = prep.weight->dtype;
    p.ob = prep.bias->data;
    p.ob_dtype = prep.bias->dtype;
    p.out_eps = static_cast<float>(prep.eps);
    p.final = prep.final->data;
  }
  if (prep.parts != nullptr) {
    RLM_TRY(check_tensor(prep.parts, "partials", 3));
    RLM_TRY(check_dtype_is(prep.parts, "partials", RLM_F32));
    RLM_TRY(check_dim(prep.parts, "partials", 1, p.Q * K));
    RLM_TRY(check_dim(prep.parts, "partials", 2, D));
    RLM_TRY(check_tensor(prep.b2, "second_bias", 1));
    RLM_TRY(check_dtype_float(prep.b2, "second_bias"));
    RLM_TRY(check_dim(prep.b2, "second_bias", 0, D));
    RLM_REQUIRE(prep.parts->shape[0] >= 1 && prep.parts->shape[0] <= kMaxParts,
                "relation_linear_norm_reduce: 1..%d hidden-dim splits", kMaxParts);
    RLM_REQUIRE(p.Q <= kQueryKernelMaxQ && D % 4 == 0 && D <= kQMaxD && K <= 16 &&
                    (reinterpret_cast<uintptr_t>(prep.parts->data) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(norm_weight->data) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(norm_bias->data) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(prep.b2->data) & 15u) == 0,
                "relation_linear_norm_reduce: decode shapes only (at most %lld queries, "
                "D %% 4 == 0, D <= %d, K <= 16, 16-byte aligned vectors)",
                (long long)kQueryKernelMaxQ, kQMaxD);
    p.parts = static_cast<const float*>(prep.parts->data);
    p.nparts = static_cast<int>(prep.parts->shape[0]);
    p.b2 = prep.b2->data;
    p.b2_dtype = prep.b2->dtype;
  }
  return hipSuccess;
}

hipError_t norm_impl(bool seq, const rlm_tensor* raw, const rlm_tensor* partner_scores,
                     const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
                     const rlm_tensor* position, double norm_eps, const rlm_tensor* out,
                     hipStream_t stream, const OutputPrep& prep = OutputPrep()) {
  clear_error();
  NormParams p;
  const hipError_t err = norm_setup(seq, raw, partner_scores, norm_weight, norm_bias, position,
                                    norm_eps, out, prep, p);
  if (err != hipSuccess) return err;
  if (p.Q == 0) return hipSuccess;
  if (prep.parts != nullptr) return launch_norm_query(p, stream);
  const int64_t K = p.K, D = p.D;
  const bool vec_ok = D % 4 == 0 && (reinterpret_cast<uintptr_t>(raw->data) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(norm_weight->data) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(norm_bias->data) & 15u) == 0;
  // A few queries (decode): one workgroup per query.
  if (vec_ok && p.Q <= kQueryKernelMaxQ && raw->dtype == RLM_F32 && D <= kQMaxD && K <= 16)
    return launch_norm_query(p, stream);
  if (vec_ok) {
    const int groups = static_cast<int>((D / 4 + kWave - 1) / kWave);
    if (groups <= 1) return launch_norm_vec<1, 8>(p, raw->dtype, stream);
    if (groups <= 2) return launch_norm_vec<2, 8>(p, raw->dtype, stream);
    if (groups <= 3) return launch_norm_vec<3, 8>(p, raw->dtype, stream);
    if (groups <= 4) return launch_norm_vec<4, 8>(p, raw->dtype, stream);
    return launch_norm_vec<8, 2>(p, raw->dtype, stream);
  }
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

namespace rlm {
namespace {

// Shapes relation_mlp_kernel takes: relation dim 64 or 128, a hidden dim that
// is a positive multiple of 128, d_model 256, 512 or 768 (32 columns per wave
// times 1..3).
bool mlp_fits_shape(int64_t R, int64_t H, int64_t D) {
  return (R == 64 || R == 128) && H > 0 && H % kMlpChunk == 0 && H <= (1 << 20) &&
         (D == 256 || D == 512 || D == 768);
}

template <int R, int TNB>
hipError_t launch_mlp_rt(const MlpParams& mp, hipStream_t stream) {
  constexpr size_t lds = mlp_lds_bytes<R, TNB>();
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&relation_mlp_kernel<R, TNB>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr != hipSuccess) {
    set_error("relation_hidden_linear_seq: cannot reserve %zu bytes of LDS: %s", lds,
              hipGetErrorString(attr));
    return attr;
  }
  const int64_t tiles = (mp.h.rows + kMlpRows - 1) / kMlpRows;
  hipLaunchKernelGGL((relation_mlp_kernel<R, TNB>), dim3(static_cast<unsigned>(tiles)),
                     dim3(kMlpThreads), lds, stream, mp);
  return launch_status("relation_hidden_linear_seq");
}

template <int R>
hipError_t launch_mlp_r(const MlpParams& mp, hipStream_t stream) {
  if (mp.D == 256) return launch_mlp_rt<R, 1>(mp, stream);
  if (mp.D == 512) return launch_mlp_rt<R, 2>(mp, stream);
  return launch_mlp_rt<R, 3>(mp, stream);
}

}  // namespace
}  // namespace rlm

// Element (n, k) of a [N, K] weight in MFMA fragment order: fragment
// (n / 32, k / 16), lane 32 * ((k % 16) / 8) + n % 32, element k % 8.
__global__ void mfma_fragments_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                      int64_t N, int64_t K) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // one 16-byte piece
  if (i >= N * K / 8) return;
  const int64_t lane = i & 63, frag = i >> 6;
  const int64_t kg = K / 16;
  const int64_t nb = frag / kg, g = frag - nb * kg;
  const int64_t n = 32 * nb + (lane & 31), k = 16 * g + 8 * (lane >> 5);
  *reinterpret_cast<uint4*>(out + 8 * i) = *reinterpret_cast<const uint4*>(w + n * K + k);
}

extern "C" hipError_t rlm_mfma_fragments(const rlm_tensor* weight, const rlm_tensor* out,
                                         hipStream_t stream) {
  using namespace rlm;
  clear_error();
  RLM_TRY(check_tensor(weight, "weight", 2));
  RLM_TRY(check_tensor(out, "out", 4));
  RLM_REQUIRE(weight->dtype == RLM_BF16 || weight->dtype == RLM_F16,
              "mfma_fragments: weight must be bfloat16 or float16");
  RLM_TRY(check_dtype_is(out, "out", weight->dtype));
  const int64_t N = weight->shape[0], K = weight->shape[1];
  RLM_REQUIRE(N % 32 == 0 && K % 16 == 0,
              "mfma_fragments: weight rows must be a multiple of 32 and columns of 16, got [%lld, %lld]",
              (long long)N, (long long)K);
  RLM_TRY(check_dim(out, "out", 0, N / 32));
  RLM_TRY(check_dim(out, "out", 1, K / 16));
  RLM_TRY(check_dim(out, "out", 2, 64));
  RLM_TRY(check_dim(out, "out", 3, 8));
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(weight->data) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(out->data) & 15u) == 0,
              "mfma_fragments: weight and out must be 16-byte aligned");
  const int64_t pieces = N * K / 8;
  if (pieces == 0) return hipSuccess;
  hipLaunchKernelGGL(mfma_fragments_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)),
                     dim3(256), 0, stream, static_cast<const uint16_t*>(weight->data),
                     static_cast<uint16_t*>(out->data), N, K);
  return launch_status("mfma_fragments");
}

namespace rlm {
namespace {
// A [N/32, K/16, 64, 8] weight in fragment order of an [N, K] weight: N and K.
bool frag_dims(const rlm_tensor* t, int64_t& N, int64_t& K) {
  if (t == nullptr || t->ndim != 4 || t->shape[2] != 64 || t->shape[3] != 8) return false;
  N = t->shape[0] * 32;
  K = t->shape[1] * 16;
  return true;
}
}  // namespace
}  // namespace rlm

extern "C" int rlm_relation_hidden_linear_seq_fits(const rlm_tensor* expanded_cache,
                                                   const rlm_tensor* operand_cache,
                                                   const rlm_tensor* product_weight,
                                                   const rlm_tensor* second_weight) {
  using namespace rlm;
  for (const rlm_tensor* t : {expanded_cache, operand_cache, product_weight, second_weight})
    if (t == nullptr || t->dtype != RLM_BF16) return 0;
  if (operand_cache->ndim != 3 || expanded_cache->ndim != 3) return 0;
  int64_t H, R, D, H2;
  if (!frag_dims(product_weight, H, R) || !frag_dims(second_weight, D, H2)) return 0;
  if (R != operand_cache->shape[2] || H2 != H || expanded_cache->shape[2] != 2 * H) return 0;
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight, expanded_cache})
    if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) return 0;
  return mlp_fits_shape(R, H, D) ? 1 : 0;
}

extern "C" hipError_t rlm_relation_hidden_linear_seq(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight, const rlm_tensor* out,
    hipStream_t stream) {
  using namespace rlm;
  clear_error();
  const char* what = "relation_hidden_linear_seq";
  RLM_TRY(check_tensor(operand_cache, "operand_cache", 3));
  RLM_TRY(check_tensor(expanded_cache, "expanded_cache", 3));
  RLM_TRY(check_tensor(product_weight, "product_weight", 4));
  RLM_TRY(check_tensor(second_weight, "second_weight", 4));
  for (const rlm_tensor* t : {operand_cache, expanded_cache, product_weight, second_weight})
    RLM_REQUIRE(t->dtype == RLM_BF16, "%s: caches and weights must be bfloat16", what);
  int64_t H, Rw, D, H2;
  RLM_REQUIRE(frag_dims(product_weight, H, Rw) && frag_dims(second_weight, D, H2),
              "%s: product_weight and second_weight must be in MFMA fragment order "
              "[N/32, K/16, 64, 8] (rlm_mfma_fragments)", what);
  const int64_t B = operand_cache->shape[0], T = operand_cache->shape[1];
  const int64_t R = operand_cache->shape[2];
  RLM_REQUIRE(Rw == R, "%s: product_weight is for relation dim %lld, the operand cache has %lld",
              what, (long long)Rw, (long long)R);
  RLM_REQUIRE(H2 == H, "%s: second_weight is for hidden dim %lld, product_weight has %lld", what,
              (long long)H2, (long long)H);
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 0, B));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 1, T));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 2, 2 * H));
  RLM_TRY(check_tensor(anchor_index, "anchor_index", 2));
  RLM_TRY(check_tensor(partner_index, "partner_index", 3));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype) && is_index_dtype(partner_index->dtype),
              "anchor_index/partner_index must be int32 or int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, B));
  RLM_TRY(check_dim(partner_index, "partner_index", 0, B));
  const int64_t Tq = anchor_index->shape[1];
  RLM_TRY(check_dim(partner_index, "partner_index", 1, Tq));
  const int64_t K = partner_index->shape[2];
  RLM_REQUIRE(mlp_fits_shape(R, H, D),
              "%s: needs relation dim 64 or 128, a hidden dim that is a multiple of %d and "
              "d_model 256, 512 or 768 (got R=%lld H=%lld D=%lld); other shapes run "
              "relation_hidden_cached_seq + relation_linear",
              what, kMlpChunk, (long long)R, (long long)H, (long long)D);
  constexpr int64_t kMaxBytes = int64_t(1) << 31;
  RLM_REQUIRE(B * T * 2 * H * 2 < kMaxBytes && B * T * R * 2 < kMaxBytes && H * R * 2 < kMaxBytes &&
                  D * H * 2 < kMaxBytes,
              "%s: caches and weights must each be smaller than 2 GiB", what);
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight, expanded_cache})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "%s: caches and weights must be 16-byte aligned", what);
  RLM_TRY(check_tensor(out, "out", 4));
  RLM_TRY(check_dtype_is(out, "out", RLM_F32));
  RLM_TRY(check_dim(out, "out", 0, B));
  RLM_TRY(check_dim(out, "out", 1, Tq));
  RLM_TRY(check_dim(out, "out", 2, K));
  RLM_TRY(check_dim(out, "out", 3, D));
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(out->data) & 15u) == 0, "%s: out must be 16-byte aligned",
              what);
  const int64_t rows = B * Tq * K;
  RLM_REQUIRE((rows + kMlpRows - 1) / kMlpRows <= 0x7fffffff, "%s: too many relation rows", what);
  if (rows == 0) return hipSuccess;
  MlpParams mp{};
  HiddenParams& p = mp.h;
  p.B = B;
  p.Tq = Tq;
  p.T = T;
  p.R = static_cast<int>(R);
  p.H = static_cast<int>(H);
  p.K = static_cast<int>(K);
  p.rows = rows;
  p.expanded = expanded_cache->data;
  p.expanded_out = expanded_cache->data;
  p.operand = operand_cache->data;
  p.anchor = anchor_index->data;
  p.partner = partner_index->data;
  p.index_dtype_a = anchor_index->dtype;
  p.index_dtype_p = partner_index->dtype;
  p.wm = product_weight->data;
  p.expanded_bytes = static_cast<uint32_t>(B * T * 2 * H * 2);
  p.operand_bytes = static_cast<uint32_t>(B * T * R * 2);
  p.wm_bytes = static_cast<uint32_t>(H * R * 2);
  mp.w2 = second_weight->data;
  mp.w2_bytes = static_cast<uint32_t>(D * H * 2);
  mp.out = static_cast<float*>(out->data);
  mp.D = static_cast<int>(D);
  return R == 128 ? launch_mlp_r<128>(mp, stream) : launch_mlp_r<64>(mp, stream);
}

namespace rlm {
namespace {

hipError_t require_ring(const HiddenParams& p) {
  RLM_REQUIRE(p.T > 0 && (p.T & (p.T - 1)) == 0,
              "ring-buffer caches need a power-of-two cache length, got %lld", (long long)p.T);
  return hipSuccess;
}

hipError_t hidden_update_impl(
    bool ring, const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias, const rlm_tensor* position,
    const rlm_tensor* out, hipStream_t stream) {
  clear_error();
  HiddenParams p{};
  hipError_t err = hidden_impl(false, expanded_cache, operand_cache, anchor_index, partner_index,
                               product_weight, out, p);
  if (err != hipSuccess) return err;
  if (ring) {
    err = require_ring(p);
    if (err != hipSuccess) return err;
    p.ring = 1;
  }
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

}  // namespace
}  // namespace rlm

extern "C" hipError_t rlm_relation_hidden_cache_update(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias, const rlm_tensor* position,
    const rlm_tensor* out, hipStream_t stream) {
  return hidden_update_impl(false, expanded_cache, operand_cache, anchor_index, partner_index,
                            anchor_weight, partner_weight, product_weight, first_bias, position,
                            out, stream);
}

extern "C" hipError_t rlm_relation_hidden_cache_update_ring(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* anchor_weight, const rlm_tensor* partner_weight,
    const rlm_tensor* product_weight, const rlm_tensor* first_bias, const rlm_tensor* position,
    const rlm_tensor* out, hipStream_t stream) {
  return hidden_update_impl(true, expanded_cache, operand_cache, anchor_index, partner_index,
                            anchor_weight, partner_weight, product_weight, first_bias, position,
                            out, stream);
}

extern "C" hipError_t rlm_relation_hidden_cached_ring(const rlm_tensor* expanded_cache,
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
  err = require_ring(p);
  if (err != hipSuccess) return err;
  p.ring = 1;
  return launch_hidden(p, operand_cache->dtype, false, stream);
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

extern "C" hipError_t rlm_relation_norm_reduce_output(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* position, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, const rlm_tensor* out_context,
    const rlm_tensor* out_final, hipStream_t stream) {
  RLM_REQUIRE(query != nullptr, "query: missing tensor");
  OutputPrep prep;
  prep.query = query;
  prep.mix_logit = mix_logit;
  prep.weight = output_weight;
  prep.bias = output_bias;
  prep.eps = output_eps;
  prep.final = out_final;
  return norm_impl(false, raw, partner_scores, norm_weight, norm_bias, position, norm_eps,
                   out_context, stream, prep);
}

extern "C" hipError_t rlm_relation_linear_norm_reduce_output(
    const rlm_tensor* hidden, const rlm_tensor* second_weight, const rlm_tensor* second_bias,
    const rlm_tensor* partner_scores, const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
    const rlm_tensor* position, double norm_eps, const rlm_tensor* query,
    const rlm_tensor* mix_logit, const rlm_tensor* output_weight, const rlm_tensor* output_bias,
    double output_eps, const rlm_tensor* partials, const rlm_tensor* out_context,
    const rlm_tensor* out_final, hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(hidden, "hidden", 3));
  RLM_REQUIRE(second_bias != nullptr, "second_bias: missing tensor");
  const int64_t B = hidden->shape[0], K = hidden->shape[1], H = hidden->shape[2];
  // The hidden rows as a [B*K, H] matrix (contiguous rows).
  rlm_tensor rows = *hidden;
  rows.ndim = 2;
  rows.shape[0] = B * K;
  rows.shape[1] = H;
  rows.stride[0] = hidden->stride[1];
  rows.stride[1] = hidden->stride[2];
  RLM_REQUIRE(B <= 1 || hidden->stride[0] == K * hidden->stride[1],
              "hidden: rows of consecutive batch entries must be contiguous");
  RLM_TRY(check_tensor(partials, "partials", 3));
  hipError_t err = linear_partials_impl(&rows, second_weight, partials, stream);
  if (err != hipSuccess) return err;
  // The raw shape [B, K, D] for norm_impl's checks; the values come from the partials.
  rlm_tensor raw = *partials;
  raw.ndim = 3;
  raw.shape[0] = B;
  raw.shape[1] = K;
  raw.shape[2] = partials->shape[2];
  raw.stride[2] = 1;
  raw.stride[1] = raw.shape[2];
  raw.stride[0] = K * raw.shape[2];
  OutputPrep prep;
  prep.parts = partials;
  prep.b2 = second_bias;
  if (query != nullptr) {
    prep.query = query;
    prep.mix_logit = mix_logit;
    prep.weight = output_weight;
    prep.bias = output_bias;
    prep.eps = output_eps;
    prep.final = out_final;
  }
  return norm_impl(false, &raw, partner_scores, norm_weight, norm_bias, position, norm_eps,
                   out_context, stream, prep);
}

extern "C" hipError_t rlm_relation_norm_reduce_output_seq(
    const rlm_tensor* raw, const rlm_tensor* partner_scores, const rlm_tensor* norm_weight,
    const rlm_tensor* norm_bias, const rlm_tensor* positions, double norm_eps,
    const rlm_tensor* query, const rlm_tensor* mix_logit, const rlm_tensor* output_weight,
    const rlm_tensor* output_bias, double output_eps, const rlm_tensor* out_context,
    const rlm_tensor* out_final, hipStream_t stream) {
  RLM_REQUIRE(query != nullptr, "query: missing tensor");
  OutputPrep prep;
  prep.query = query;
  prep.mix_logit = mix_logit;
  prep.weight = output_weight;
  prep.bias = output_bias;
  prep.eps = output_eps;
  prep.final = out_final;
  return norm_impl(true, raw, partner_scores, norm_weight, norm_bias, positions, norm_eps,
                   out_context, stream, prep);
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

extern "C" int rlm_relation_hidden_linear_norm_reduce_output_fits(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* partner_index, const rlm_tensor* product_weight,
    const rlm_tensor* second_weight) {
  for (const rlm_tensor* t : {expanded_cache, operand_cache, partner_index, product_weight,
                              second_weight})
    if (t == nullptr) return 0;
  if (operand_cache->ndim != 3 || expanded_cache->ndim != 3 || partner_index->ndim != 2 ||
      product_weight->ndim != 2 || second_weight->ndim != 2)
    return 0;
  for (const rlm_tensor* t : {expanded_cache, operand_cache, product_weight, second_weight})
    if (t->dtype != RLM_BF16) return 0;
  const int64_t B = operand_cache->shape[0], R = operand_cache->shape[2];
  const int64_t H = product_weight->shape[0], D = second_weight->shape[0];
  if (product_weight->shape[1] != R || second_weight->shape[1] != H ||
      partner_index->shape[0] != B)
    return 0;
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) return 0;
  if ((reinterpret_cast<uintptr_t>(expanded_cache->data) & 7u) != 0) return 0;
  return decode_fits_shape(B, partner_index->shape[1], R, H, D) ? 1 : 0;
}

extern "C" hipError_t rlm_relation_hidden_linear_norm_reduce_output_workspace(
    int64_t batch, int64_t partners, int64_t hidden_dim, int64_t d_model,
    int64_t* workspace_floats, int64_t* counters) {
  clear_error();
  RLM_REQUIRE(workspace_floats != nullptr && counters != nullptr, "null output pointer");
  RLM_REQUIRE(batch >= 0 && partners >= 0 && d_model >= 0 && hidden_dim > 0 &&
                  hidden_dim % kDecSlice == 0,
              "relation_hidden_linear_norm_reduce_output: hidden dim must be a positive "
              "multiple of %d, got %lld", kDecSlice, (long long)hidden_dim);
  const DecodeShape sh = decode_shape(hidden_dim);
  *workspace_floats = static_cast<int64_t>(sh.S + sh.G) * batch * partners * d_model;
  *counters = batch * (sh.G + 1);
  return hipSuccess;
}

extern "C" hipError_t rlm_relation_hidden_linear_norm_reduce_output(
    const rlm_tensor* expanded_cache, const rlm_tensor* operand_cache,
    const rlm_tensor* anchor_index, const rlm_tensor* partner_index,
    const rlm_tensor* product_weight, const rlm_tensor* second_weight,
    const rlm_tensor* second_bias, const rlm_tensor* partner_scores,
    const rlm_tensor* norm_weight, const rlm_tensor* norm_bias, const rlm_tensor* position,
    double norm_eps, const rlm_tensor* query, const rlm_tensor* mix_logit,
    const rlm_tensor* output_weight, const rlm_tensor* output_bias, double output_eps,
    int32_t ring, const rlm_tensor* workspace, const rlm_tensor* counters,
    const rlm_tensor* out_context, const rlm_tensor* out_final, hipStream_t stream) {
  clear_error();
  const char* what = "relation_hidden_linear_norm_reduce_output";
  RLM_TRY(check_tensor(operand_cache, "operand_cache", 3));
  RLM_TRY(check_tensor(expanded_cache, "expanded_cache", 3));
  RLM_TRY(check_tensor(product_weight, "product_weight", 2));
  RLM_TRY(check_tensor(second_weight, "second_weight", 2));
  for (const rlm_tensor* t : {operand_cache, expanded_cache, product_weight, second_weight})
    RLM_REQUIRE(t->dtype == RLM_BF16, "%s: caches and weights must be bfloat16", what);
  const int64_t B = operand_cache->shape[0], T = operand_cache->shape[1];
  const int64_t R = operand_cache->shape[2], H = product_weight->shape[0];
  const int64_t D = second_weight->shape[0];
  RLM_TRY(check_dim(product_weight, "product_weight", 1, R));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 0, B));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 1, T));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 2, 2 * H));
  RLM_TRY(check_dim(second_weight, "second_weight", 1, H));
  RLM_TRY(check_tensor(anchor_index, "anchor_index", 1));
  RLM_TRY(check_tensor(partner_index, "partner_index", 2));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype) && is_index_dtype(partner_index->dtype),
              "anchor_index/partner_index must be int32 or int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, B));
  RLM_TRY(check_dim(partner_index, "partner_index", 0, B));
  const int64_t K = partner_index->shape[1];
  RLM_REQUIRE(decode_fits_shape(B, K, R, H, D),
              "%s: needs relation dim 64 or 128, a hidden dim that is a multiple of %d up to "
              "%d, 1..%d partners, d_model a multiple of 4 up to %d and 1..65535 queries (got "
              "R=%lld H=%lld K=%lld D=%lld B=%lld); other shapes run "
              "relation_hidden_cached + relation_linear_norm_reduce_output",
              what, kDecSlice, kDecSlice * kDecGroups * kDecMaxSpg, kDecMaxK, kDecMaxD,
              (long long)R, (long long)H, (long long)K, (long long)D, (long long)B);
  RLM_REQUIRE(!ring || (T > 0 && (T & (T - 1)) == 0),
              "ring-buffer caches need a power-of-two cache length, got %lld", (long long)T);
  constexpr int64_t kMaxBytes = int64_t(1) << 31;
  RLM_REQUIRE(B * T * 2 * H * 2 < kMaxBytes && B * T * R * 2 < kMaxBytes && D * H * 2 < kMaxBytes,
              "%s: caches and weights must each be smaller than 2 GiB", what);
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "%s: operand_cache, product_weight and second_weight must be 16-byte aligned", what);
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(expanded_cache->data) & 7u) == 0,
              "%s: expanded_cache must be 8-byte aligned", what);
  const DecodeShape sh = decode_shape(H);
  const int64_t rows = B * K;
  RLM_TRY(check_tensor(workspace, "workspace", 1));
  RLM_TRY(check_dtype_is(workspace, "workspace", RLM_F32));
  RLM_REQUIRE(workspace->shape[0] >= (sh.S + sh.G) * rows * D,
              "%s: workspace needs %lld fp32 elements, got %lld", what,
              (long long)((sh.S + sh.G) * rows * D), (long long)workspace->shape[0]);
  RLM_REQUIRE((sh.S + sh.G) * rows * D * 4 < kMaxBytes, "%s: workspace over 2 GiB", what);
  RLM_REQUIRE((reinterpret_cast<uintptr_t>(workspace->data) & 15u) == 0,
              "%s: workspace must be 16-byte aligned", what);
  RLM_TRY(check_tensor(counters, "counters", 1));
  RLM_TRY(check_dtype_is(counters, "counters", RLM_I32));
  RLM_REQUIRE(counters->shape[0] >= B * (sh.G + 1), "%s: counters needs %lld int32 elements",
              what, (long long)(B * (sh.G + 1)));
  RLM_REQUIRE(query != nullptr, "query: missing tensor");
  RLM_REQUIRE(second_bias != nullptr, "second_bias: missing tensor");
  float* partials = static_cast<float*>(workspace->data);
  float* gsum = partials + static_cast<int64_t>(sh.S) * rows * D;
  // The raw shape [B, K, D] for the norm checks; the values come from the group sums.
  rlm_tensor raw{};
  raw.data = gsum;
  raw.dtype = RLM_F32;
  raw.ndim = 3;
  raw.shape[0] = B;
  raw.shape[1] = K;
  raw.shape[2] = D;
  raw.stride[0] = K * D;
  raw.stride[1] = D;
  raw.stride[2] = 1;
  rlm_tensor parts{};
  parts.data = gsum;
  parts.dtype = RLM_F32;
  parts.ndim = 3;
  parts.shape[0] = sh.G;
  parts.shape[1] = rows;
  parts.shape[2] = D;
  parts.stride[0] = rows * D;
  parts.stride[1] = D;
  parts.stride[2] = 1;
  OutputPrep prep;
  prep.parts = &parts;
  prep.b2 = second_bias;
  prep.query = query;
  prep.mix_logit = mix_logit;
  prep.weight = output_weight;
  prep.bias = output_bias;
  prep.eps = output_eps;
  prep.final = out_final;
  DecodeParams p{};
  const hipError_t err = norm_setup(false, &raw, partner_scores, norm_weight, norm_bias, position,
                                    norm_eps, out_context, prep, p.n);
  if (err != hipSuccess) return err;
  p.T = T;
  p.B = static_cast<int>(B);
  p.K = static_cast<int>(K);
  p.R = static_cast<int>(R);
  p.H = static_cast<int>(H);
  p.D = static_cast<int>(D);
  p.S = sh.S;
  p.G = sh.G;
  p.spg = sh.spg;
  p.ring = ring ? 1 : 0;
  p.expanded = expanded_cache->data;
  p.operand = operand_cache->data;
  p.anchor = anchor_index->data;
  p.partner = partner_index->data;
  p.index_dtype_a = anchor_index->dtype;
  p.index_dtype_p = partner_index->dtype;
  p.wm = product_weight->data;
  p.w2 = second_weight->data;
  p.partials = partials;
  p.gsum = gsum;
  p.counters = static_cast<uint32_t*>(counters->data);
  p.expanded_bytes = static_cast<uint32_t>(B * T * 2 * H * 2);
  p.operand_bytes = static_cast<uint32_t>(B * T * R * 2);
  p.wm_bytes = static_cast<uint32_t>(H * R * 2);
  p.w2_bytes = static_cast<uint32_t>(D * H * 2);
  p.partials_bytes = static_cast<uint32_t>(static_cast<int64_t>(sh.S) * rows * D * 4);
  p.gsum_bytes = static_cast<uint32_t>(static_cast<int64_t>(sh.G) * rows * D * 4);
  return launch_decode(p, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free form of rlm_relation_linear_norm_reduce_output.  The split-K
// partials live in `scratch`, a file-scope device array (one copy per GPU, held
// until the process ends) of at most 4 splits x 64 rows x 1024 columns fp32
// (1 MiB).  Host code never passes the array's name to a kernel: its device
// address is taken once per device with hipGetSymbolAddress and kept.  Every
// partial the norm kernel reads is written by the linear first, so nothing is
// cleared.  Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------

constexpr int64_t kScratchFloats = int64_t(4) * 64 * 1024;
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchMaxDevices] = {};

// The current device's copy of `scratch` (its address taken on first use).
hipError_t scratch_for_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    rlm::set_error("relation_linear_norm_reduce (no-alloc): hipGetDevice failed: %s",
                   hipGetErrorString(e));
    return e;
  }
  if (dev < 0 || dev >= kScratchMaxDevices) {
    rlm::set_error("relation_linear_norm_reduce (no-alloc): device %d beyond the %d supported",
                   dev, kScratchMaxDevices);
    return hipErrorInvalidDevice;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      rlm::set_error("relation_linear_norm_reduce (no-alloc): hipGetSymbolAddress failed: %s",
                     hipGetErrorString(e));
      return e != hipSuccess ? e : hipErrorInvalidSymbol;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}
}  // namespace

extern "C" hipError_t rlm_relation_linear_norm_reduce_output_noalloc(
    const rlm_tensor* hidden, const rlm_tensor* second_weight, const rlm_tensor* second_bias,
    const rlm_tensor* partner_scores, const rlm_tensor* norm_weight, const rlm_tensor* norm_bias,
    const rlm_tensor* position, double norm_eps, const rlm_tensor* query,
    const rlm_tensor* mix_logit, const rlm_tensor* output_weight, const rlm_tensor* output_bias,
    double output_eps, int32_t splits, const rlm_tensor* out_context, const rlm_tensor* out_final,
    hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(hidden, "hidden", 3));
  RLM_TRY(check_tensor(second_weight, "second_weight", 2));
  const int64_t rows = hidden->shape[0] * hidden->shape[1];
  const int64_t D = second_weight->shape[0];
  RLM_REQUIRE(splits >= 1 && splits <= 4, "relation_linear_norm_reduce (no-alloc): splits must "
              "be in [1, 4], got %d", splits);
  RLM_REQUIRE(static_cast<int64_t>(splits) * rows * D <= kScratchFloats,
              "relation_linear_norm_reduce (no-alloc): %d splits x %lld rows x %lld columns "
              "exceed the static workspace of %lld fp32 values",
              splits, (long long)rows, (long long)D, (long long)kScratchFloats);
  float* ws = nullptr;
  const hipError_t e = scratch_for_current_device(&ws);
  if (e != hipSuccess) return e;
  rlm_tensor part{};
  part.data = ws;
  part.dtype = RLM_F32;
  part.ndim = 3;
  part.shape[0] = splits;
  part.shape[1] = rows;
  part.shape[2] = D;
  part.stride[2] = 1;
  part.stride[1] = D;
  part.stride[0] = rows * D;
  return rlm_relation_linear_norm_reduce_output(
      hidden, second_weight, second_bias, partner_scores, norm_weight, norm_bias, position,
      norm_eps, query, mix_logit, output_weight, output_bias, output_eps, &part, out_context,
      out_final, stream);
}

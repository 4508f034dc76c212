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
//   set-up   wave w keeps the exact hi/lo bf16 split of the operand products
//            (op[anchor] * op[partner], exact in fp32) of rows 16w..16w+15 in
//            registers; the rows' active-K softmax weights and the b2 / gamma /
//            beta vectors go to LDS.
//   phase 1  per 128-column chunk of the hidden dimension, wave w forms
//            hidden^T[128 cols x its 16 rows] = W_m[chunk] . P^T on the matrix
//            cores, adds the rows' expanded-cache halves, applies GELU and
//            rounds to bf16 -- the operand the unfused path's bf16 second linear
//            sees -- into the LDS hidden chunk.  The W_m chunk and the gathered
//            expanded-cache halves of the 128 rows reach LDS by LDS-DMA
//            (buffer_load ... lds), issued while the previous chunk's phase 2
//            runs.  The transposed product leaves 4 consecutive hidden columns
//            of one row in a lane, so the LDS writes are ds_write_b64.
//   phase 2  raw[128 rows x D/8 cols of wave w] += hidden chunk . W2^T; the
//            hidden fragments come from LDS, W2 fragments from L2 one k-step
//            ahead, and the raw accumulators stay in registers for the whole
//            kernel.  Two waves per SIMD let one wave's GELU work overlap the
//            other's matrix-core work.
// Epilogue: + b2, LayerNorm per row (moments combined across the 8 waves in
// LDS), partner weights, sum over the query's rows (in-lane, then the
// neighbouring 16-lane groups), fp32 buffer stores.
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
constexpr int kMaxR = 128;
constexpr int kMaxD = 512;
constexpr int kLd = 136;                   // hidden row stride (bf16): conflict-free b128 reads
// LDS layout (bytes): the W_m chunk, the gathered expanded-cache halves of the
// chunk ([128 rows][anchor half 256 B | partner half 256 B]), the hidden chunk,
// fp32 vectors, the rows' expanded-cache byte offsets.
constexpr int kWmBytes = kHC * kMaxR * 2;
constexpr int kGatherRowBytes = 2 * kHC * 2;
constexpr int kOffGather = kWmBytes;
constexpr int kOffHid = kOffGather + kRows * kGatherRowBytes;
constexpr int kOffF32 = kOffHid + kRows * kLd * 2;
constexpr int kF32Words = kRows + 2 * kRows + 2 * kWaves * kRows + 3 * kMaxD;
constexpr int kOffRowOff = kOffF32 + kF32Words * 4;
constexpr size_t kLdsBytes = static_cast<size_t>(kOffRowOff) + kRows * 2 * 4;
constexpr int kWaitVm0 = 0x0F70;           // s_waitcnt vmcnt(0), other counters untouched

struct FusedParams {
  int64_t T;
  uint32_t Tq, K, k_log2, R, H, D;
  uint32_t rows;       // B*Tq*K
  uint32_t queries;    // B*Tq
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

__device__ __forceinline__ u16x8 lds_frag(const unsigned char* p) {
  return *reinterpret_cast<const u16x8*>(p);
}

__device__ __forceinline__ u16x8 as_frag(uint4 v) { return __builtin_bit_cast(u16x8, v); }

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land
// at lds_addr + 16*i.  Issued as inline assembly so that the compiler does not
// follow it with a full vmcnt(0) before the next LDS access; the caller waits
// (s_waitcnt vmcnt(0) + barrier) before the tile is read.  M0 (the LDS base of
// the transfer) is set inside the same asm statement.  M0 is a reserved
// register that a clobber list cannot name; nothing else in this kernel uses
// it (the compiler emits no M0 access of its own here), so the write cannot
// disturb compiler-generated code.
__device__ __forceinline__ void lds_dma16(rsrc_t r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(r)
               : "memory");
}

// Weight p_k of row `grow` (< rows) in its query's partner mixture: softmax
// over the active partners (rank < k_limit, score > -1e30; inactive scores
// -1e4), renormalised by max(sum, 1e-9) -- relation_reduce.py:399-411.
__device__ float row_weight(const FusedParams& p, uint32_t grow) {
  const uint32_t K = p.K;
  const uint32_t q = grow >> p.k_log2;
  const uint32_t k = grow & (K - 1);
  const uint32_t b = q / p.Tq;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + (q - b * p.Tq) * p.pos_sq);
  const int64_t n = t + 1;
  int k_limit = n > 0 ? 64 - __clzll(static_cast<unsigned long long>(n)) : 0;  // ceil(log2(t+2))
  k_limit = k_limit < 1 ? 1 : (k_limit > static_cast<int>(K) ? static_cast<int>(K) : k_limit);
  const float* sq = p.scores + static_cast<size_t>(q) * K;
  float sc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) sc[c] = c < static_cast<int>(K) ? sq[c] : -INFINITY;
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < 16; ++c)
    if (c < static_cast<int>(K)) m = fmaxf(m, (c < k_limit && sc[c] > -1.0e30f) ? sc[c] : -1.0e4f);
  float total = 0.0f, mine = 0.0f;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const float pc = (c < k_limit && sc[c] > -1.0e30f) ? expf(sc[c] - m) : 0.0f;
    total += pc;
    mine = c == static_cast<int>(k) ? pc : mine;
  }
  return mine / fmaxf(total, 1.0e-9f);
}

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Streams rows [chunk*128, chunk*128+128) of W_m into an LDS tile of 128 rows
// x R bf16.  16-byte piece q of row n is stored at piece q ^ (n % (R/8)) so
// that the 16 rows of an MFMA fragment read hit distinct banks.
// Instruction i of kHC*R/8/kThreads = KS1 per lane.
template <int KS1>
__device__ __forceinline__ void dma_wm_one(rsrc_t wmr, uint32_t tile, int chunk, int wave, int lane,
                                           int i) {
  constexpr int R = KS1 * 32;
  constexpr int QPR = R / 8;                               // pieces per row
  const int slot = (i * kWaves + wave) * kWave + lane;     // LDS piece written by this lane
  const int n = slot / QPR;
  const int src = (slot % QPR) ^ (n % QPR);
  const uint32_t voff = (static_cast<uint32_t>(chunk * kHC + n) * R + 8 * src) * 2u;
  lds_dma16(wmr, __builtin_amdgcn_readfirstlane(tile + (i * kWaves + wave) * kWave * 16), voff);
}
template <int KS1>
__device__ __forceinline__ void dma_wm_chunk(rsrc_t wmr, uint32_t tile, int chunk, int wave,
                                             int lane) {
  static_assert(kHC * KS1 * 4 % kThreads == 0 && kHC * KS1 * 4 / kThreads == KS1, "");
#pragma unroll
  for (int i = 0; i < KS1; ++i) dma_wm_one<KS1>(wmr, tile, chunk, wave, lane, i);
}

// Gathered expanded-cache halves of one chunk: LDS row m holds the anchor
// half's columns [chunk*128, +128) then the partner half's, 16 pieces of 16 B
// each, piece q stored at q ^ (m % 16).  Each wave gathers its own 16 rows
// (the rows its phase 1 reads): lane `lane` of DMA instruction i of wave w
// writes piece lane % 32 of row 16w + 2i + lane / 32; src[i] is that piece's
// byte offset for chunk 0 (kNoOffset for a missing row: zeros).
constexpr int kGatherInsts = kRows * kGatherRowBytes / 16 / kThreads;
static_assert(kGatherInsts * 2 * kWaves == kRows, "each wave gathers its own rows");
__device__ __forceinline__ void dma_gather_chunk(rsrc_t xr, uint32_t tile,
                                                 const uint32_t (&src)[kGatherInsts], int chunk,
                                                 int wave) {
#pragma unroll
  for (int i = 0; i < kGatherInsts; ++i)
    lds_dma16(xr, __builtin_amdgcn_readfirstlane(tile + (wave * kGatherInsts + i) * kWave * 16),
              src[i] == kNoOffset ? kNoOffset : src[i] + chunk * kHC * 2u);
}

template <int DT, int KS1>
__global__ void __launch_bounds__(kThreads) fused_reduce_kernel(const FusedParams p) {
  // DT = 16-column tiles of D per wave in phase 2 (D = 128*DT); KS1 = R/32.
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* hid = smem + kOffHid;                            // [kRows][kLd] bf16
  float* wts = reinterpret_cast<float*>(smem + kOffF32);           // [kRows]
  float* mom = wts + kRows;                                        // [2][kRows] mean, rstd
  float* part = mom + 2 * kRows;                                   // [2][kWaves][kRows]
  float* cst = part + 2 * kWaves * kRows;                          // [3][kMaxD] b2, gamma, beta
  uint32_t* rowoff = reinterpret_cast<uint32_t*>(smem + kOffRowOff);  // [kRows][2]
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  constexpr int R = KS1 * 32;
  constexpr int QPR = R / 8;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const uint32_t row0 = blockIdx.x * kRows;
  const uint32_t H = p.H;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wmr = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t w2r = make_rsrc(p.w2, p.w2_bytes);

  // ---- Set-up: two dependent round trips.  (1) this lane's row indices
  // (beside the W_m DMA of chunk 0); (2) the wave's gather DMA of chunk 0, the
  // operand rows, the row-weight inputs and b2 / gamma / beta, all in flight
  // together.
  dma_wm_chunk<KS1>(wmr, lds0, 0, wave, lane);
  // This lane's phase-1 row: 16*wave + r16.
  const int lrow = 16 * wave + r16;
  u16x8 ph[KS1], pl[KS1];
  // Gather DMA sources of this lane (piece lane%32 of row 16*wave + 2i + lane/32), chunk 0.
  auto gather_src = [&](int i) {
    const int m = 16 * wave + 2 * i + lane / 32;
    const int q = lane & 31;
    const uint32_t base = rowoff[2 * m + q / 16];
    return base == kNoOffset ? kNoOffset : base + 16u * ((q & 15) ^ (m & 15));
  };
  auto gather_chunk = [&](int chunk) {
    uint32_t src[kGatherInsts];
#pragma unroll
    for (int i = 0; i < kGatherInsts; ++i) src[i] = gather_src(i);
    dma_gather_chunk(xr, lds0 + kOffGather, src, chunk, wave);
  };
  {
    const uint32_t grow = row0 + lrow;
    int32_t a = -1, pp = -1;
    uint32_t base = 0;
    if (grow < p.rows) {
      const uint32_t q = grow >> p.k_log2;
      base = (q / p.Tq) * static_cast<uint32_t>(p.T);
      const int64_t ai = load_any_i(p.anchor, p.index_dtype_a, q);
      const int64_t pi = load_any_i(p.partner, p.index_dtype_p, grow);
      a = (ai >= 0 && ai < p.T) ? static_cast<int32_t>(ai) : -1;
      pp = (pi >= 0 && pi < p.T) ? static_cast<int32_t>(pi) : -1;
    }
    if (g == 0) {
      rowoff[2 * lrow] = a >= 0 ? (base + a) * (4u * H) : kNoOffset;               // anchor, first half
      rowoff[2 * lrow + 1] = pp >= 0 ? (base + pp) * (4u * H) + 2u * H : kNoOffset;  // partner, second half
    }
    wave_sync();  // the wave's row offsets are in LDS (it reads only its own rows)
    gather_chunk(0);
    const bool ok = a >= 0 && pp >= 0;
    const uint32_t oa = ok ? (base + a) * (2u * R) + 16u * g : kNoOffset;
    const uint32_t op = ok ? (base + pp) * (2u * R) + 16u * g : kNoOffset;
    uint4 va[KS1], vp[KS1];
#pragma unroll
    for (int s = 0; s < KS1; ++s) {
      va[s] = buf_load_b128(opr, ok ? oa + 64u * s : kNoOffset);
      vp[s] = buf_load_b128(opr, ok ? op + 64u * s : kNoOffset);
    }
    if (tid < kRows) wts[tid] = row0 + tid < p.rows ? row_weight(p, row0 + tid) : 0.0f;
    for (int i = tid; i < static_cast<int>(p.D); i += kThreads) {
      cst[i] = load_any_f(p.b2, p.b2_dtype, i);
      cst[kMaxD + i] = load_any_f(p.gamma, p.gamma_dtype, i);
      cst[2 * kMaxD + i] = load_any_f(p.beta, p.beta_dtype, i);
    }
#pragma unroll
    for (int s = 0; s < KS1; ++s) {
      const uint32_t wa[4] = {va[s].x, va[s].y, va[s].z, va[s].w};
      const uint32_t wp[4] = {vp[s].x, vp[s].y, vp[s].z, vp[s].w};
      uint32_t h[4], l[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = bf16_lo(wp[k]) * bf16_lo(wa[k]);  // exact: 8-bit x 8-bit significands
        const float x1 = bf16_hi(wp[k]) * bf16_hi(wa[k]);
        h[k] = pack_bf16x2(x0, x1);
        l[k] = pack_bf16x2(x0 - bf16_lo(h[k]), x1 - bf16_hi(h[k]));
      }
      ph[s] = as_frag(make_uint4(h[0], h[1], h[2], h[3]));
      pl[s] = as_frag(make_uint4(l[0], l[1], l[2], l[3]));
    }
  }

  // W2 fragments (B operand of phase 2) in groups of JC column tiles: rows
  // dcol0 + 16(JC*jg + j) + r16, k = chunk*128 + 32s + 8g.
  constexpr int JC = (DT % 2 == 0) ? DT / 2 : DT;
  constexpr int NG = DT / JC;
  const int dcol0 = wave * DT * 16;
  const uint32_t w2_lane = (static_cast<uint32_t>(dcol0 + r16) * H + 8 * g) * 2u;
  auto load_w2 = [&](u16x8 (&w)[JC], int chunk, int jg, int s) {
#pragma unroll
    for (int j = 0; j < JC; ++j)
      w[j] = as_frag(buf_load_b128(
          w2r, w2_lane + (16u * (JC * jg + j) * H + chunk * kHC + 32 * s) * 2u));
  };

  f32x4 raw[kRowTiles][DT];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int j = 0; j < DT; ++j) raw[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const unsigned char* my_gat = smem + kOffGather + lrow * kGatherRowBytes;
  // Constant A operand [I16 | I16]: lane (r16, g) holds row r16, k = 8g..8g+7,
  // 1.0 (bf16 0x3F80) where k % 16 == r16.
  u16x8 ident;
#pragma unroll
  for (int k = 0; k < 8; ++k) ident[k] = (8 * (g & 1) + k == r16) ? 0x3F80 : 0;
  unsigned char* my_hid = hid + lrow * (2 * kLd) + 8 * g;

  const int nchunks = H / kHC;
  __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this lane's W_m and gather pieces of chunk 0 are in LDS
  __syncthreads();

  for (int c = 0; c < nchunks; ++c) {
    // ---- Phase 1, two halves of 64 columns: hidden^T[cols x 16 rows of this wave].
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      f32x4 acc[4];
      // The row's expanded-cache values enter on the matrix cores: B operand
      // rows k < 16 are the anchor half's columns 16j + k, rows k >= 16 the
      // partner half's columns 16j + k - 16 (piece 2j + g%2 of half g/2, one
      // 16-byte read), against the constant A = [I | I].  The products by 1.0
      // are exact.
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * hh + jj;
        const u16x8 gv = lds_frag(my_gat + 256 * (g >> 1) + ((2 * j + (g & 1)) ^ r16) * 16);
        acc[jj] = mfma_bf16(ident, gv, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
      }
#pragma unroll
      for (int s = 0; s < KS1; ++s) {
        // A fragment: W_m tile row 16j + r16, k-piece (4s + g) stored swizzled.
        const uint32_t frag = r16 * (2u * R) + 16u * ((4 * s + g) ^ (r16 % QPR));
        u16x8 w[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) w[jj] = lds_frag(smem + (16 * (4 * hh + jj)) * (2 * R) + frag);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          acc[jj] = mfma_bf16(w[jj], ph[s], acc[jj]);
          acc[jj] = mfma_bf16(w[jj], pl[s], acc[jj]);
        }
      }
      // acc[jj][e] = hidden[row lrow][col 16(4hh+jj) + 4g + e].
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 h = acc[jj];
        *reinterpret_cast<uint2*>(my_hid + 32 * (4 * hh + jj)) =
            make_uint2(pack_bf16x2(gelu_erf(h[0]), gelu_erf(h[1])),
                       pack_bf16x2(gelu_erf(h[2]), gelu_erf(h[3])));
      }
    }
    u16x8 b[JC];
    load_w2(b, c, 0, 0);
    __syncthreads();  // hidden chunk complete; the W_m and gather tiles are free
    if (c + 1 < nchunks) {
      dma_wm_chunk<KS1>(wmr, lds0, c + 1, wave, lane);
      gather_chunk(c + 1);
    }
    // ---- Phase 2: raw[128 x 16*DT] += hidden chunk . W2[cols, chunk]^T, JC column
    // tiles at a time (W2 fragments of the next k-step in flight), row tile by
    // row tile (the next hidden fragment in flight).
#pragma unroll
    for (int jg = 0; jg < NG; ++jg) {
#pragma unroll
      for (int s = 0; s < kHC / 32; ++s) {
        u16x8 bn[JC];
        if (s + 1 < kHC / 32) load_w2(bn, c, jg, s + 1);
        else if (jg + 1 < NG) load_w2(bn, c, jg + 1, 0);
        const unsigned char* arow = hid + r16 * (2 * kLd) + 64 * s + 16 * g;
        u16x8 a = lds_frag(arow);
#pragma unroll
        for (int i = 0; i < kRowTiles; ++i) {
          u16x8 an;
          if (i + 1 < kRowTiles) an = lds_frag(arow + (i + 1) * 16 * (2 * kLd));
#pragma unroll
          for (int j = 0; j < JC; ++j) raw[i][JC * jg + j] = mfma_bf16(a, b[j], raw[i][JC * jg + j]);
          if (i + 1 < kRowTiles) a = an;
        }
        if (s + 1 < kHC / 32 || jg + 1 < NG) {
#pragma unroll
          for (int j = 0; j < JC; ++j) b[j] = bn[j];
        }
        __builtin_amdgcn_sched_barrier(0);  // keep each k-step's loads next to its products
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this lane's pieces of chunk c+1 are in LDS
    __syncthreads();  // ... and everyone's; the hidden chunk is free again
  }

  // ---- Epilogue.  raw[i][j][e] = row 16i+4g+e, column dcol0+16j+r16.
  const float inv_d = 1.0f / static_cast<float>(p.D);
#pragma unroll
  for (int j = 0; j < DT; ++j) {
    const float bias = cst[dcol0 + 16 * j + r16];
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) raw[i][j][e] += bias;
  }
  // Row moments.  Each wave takes the mean and centred sum of squares of its
  // 16*DT columns of every row (DPP sums over the 16 lanes of a column tile
  // row); threads 0..127 merge the 8 waves' pairs (Chan, Golub and LeVeque's
  // pairwise update, equal counts) -- one barrier round, no E[x^2]-mu^2.
  constexpr float kInvCols = 1.0f / (16.0f * DT);
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < DT; ++j) sum += raw[i][j][e];
      const float mu = row16_sum(sum) * kInvCols;
      float sq = 0.0f;
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        const float d = raw[i][j][e] - mu;
        sq = fmaf(d, d, sq);
      }
      sq = row16_sum(sq);
      if (r16 == 0) {
        part[wave * kRows + 16 * i + 4 * g + e] = mu;
        part[(kWaves + wave) * kRows + 16 * i + 4 * g + e] = sq;
      }
    }
  __syncthreads();
  if (tid < kRows) {
    float mw[kWaves], mu = 0.0f, m2 = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = part[w * kRows + tid];
      mu += mw[w];
      m2 += part[(kWaves + w) * kRows + tid];
    }
    mu *= 1.0f / kWaves;
    float spread = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) spread = fmaf(mw[w] - mu, mw[w] - mu, spread);
    mom[tid] = mu;
    mom[kRows + tid] = rsqrtf(fmaf(spread, 16.0f * DT, m2) * inv_d + p.eps);
  }
  __syncthreads();
  float4 mean[kRowTiles];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i) mean[i] = *reinterpret_cast<const float4*>(mom + 16 * i + 4 * g);
  // LayerNorm, weights, sum over each query's K consecutive rows, store:
  //   out[q] = sum_k w_k (gamma (x_k - mu_k) rs_k + beta)
  //          = gamma * sum_k (A_k x_k - B_k) + beta * sum_k w_k,
  // A_k = w_k rs_k, B_k = A_k mu_k, so each raw value costs one FMA.  Rows of
  // one query: K <= 4 -> inside a lane group, K = 8 -> groups {0,1} / {2,3}
  // (v_permlane16_swap), K = 16 -> all four (and v_permlane32_swap).  The
  // store descriptor covers this workgroup's queries only, so rows past the end
  // of the last workgroup are dropped by the buffer bounds check.
  const uint32_t K = p.K, D = p.D;
  const uint32_t q0 = row0 >> p.k_log2;
  const uint32_t nq = min(p.queries - q0, static_cast<uint32_t>(kRows) >> p.k_log2);
  const rsrc_t outr = make_rsrc(p.out + static_cast<size_t>(q0) * D, nq * D * 4u);
  float gm[DT], bt[DT];
#pragma unroll
  for (int j = 0; j < DT; ++j) {
    gm[j] = cst[kMaxD + dcol0 + 16 * j + r16];
    bt[j] = cst[2 * kMaxD + dcol0 + 16 * j + r16];
  }
  auto cross16 = [](float v) { return swap16_sum(v); };
  auto cross32 = [](float v) { return swap32_sum(v); };
  if (K >= 4) {
    float v[kRowTiles][DT], W[kRowTiles];
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i) {
      const float4 m4 = mean[i];
      const float4 r4 = *reinterpret_cast<const float4*>(mom + kRows + 16 * i + 4 * g);
      const float4 w4 = *reinterpret_cast<const float4*>(wts + 16 * i + 4 * g);
      const float A[4] = {w4.x * r4.x, w4.y * r4.y, w4.z * r4.z, w4.w * r4.w};
      const float nB[4] = {-A[0] * m4.x, -A[1] * m4.y, -A[2] * m4.z, -A[3] * m4.w};
      W[i] = (w4.x + w4.y) + (w4.z + w4.w);
#pragma unroll
      for (int j = 0; j < DT; ++j)
        v[i][j] = (fmaf(raw[i][j][0], A[0], nB[0]) + fmaf(raw[i][j][1], A[1], nB[1])) +
                  (fmaf(raw[i][j][2], A[2], nB[2]) + fmaf(raw[i][j][3], A[3], nB[3]));
    }
    if (K >= 8) {
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i) {
        W[i] = cross16(W[i]);
#pragma unroll
        for (int j = 0; j < DT; ++j) v[i][j] = cross16(v[i][j]);
      }
    }
    if (K >= 16) {
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i) {
        W[i] = cross32(W[i]);
#pragma unroll
        for (int j = 0; j < DT; ++j) v[i][j] = cross32(v[i][j]);
      }
    }
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i) {
      const uint32_t lrow = 16 * i + 4 * g;  // first local row of this lane group
      if ((lrow & (K - 1)) != 0) continue;
      const uint32_t obase = (lrow >> p.k_log2) * D + dcol0 + r16;
#pragma unroll
      for (int j = 0; j < DT; ++j)
        buf_store_f32(fmaf(gm[j], v[i][j], bt[j] * W[i]), outr, (obase + 16 * j) * 4u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i) {
      const float4 m4 = mean[i];
      const float4 r4 = *reinterpret_cast<const float4*>(mom + kRows + 16 * i + 4 * g);
      const float4 w4 = *reinterpret_cast<const float4*>(wts + 16 * i + 4 * g);
      const float A[4] = {w4.x * r4.x, w4.y * r4.y, w4.z * r4.z, w4.w * r4.w};
      const float nB[4] = {-A[0] * m4.x, -A[1] * m4.y, -A[2] * m4.z, -A[3] * m4.w};
      const uint32_t lrow = 16 * i + 4 * g;
      if (K == 2) {
        const float W0 = w4.x + w4.y, W1 = w4.z + w4.w;
        const uint32_t obase = (lrow >> 1) * D + dcol0 + r16;
#pragma unroll
        for (int j = 0; j < DT; ++j) {
          const float v0 = fmaf(raw[i][j][0], A[0], nB[0]) + fmaf(raw[i][j][1], A[1], nB[1]);
          const float v1 = fmaf(raw[i][j][2], A[2], nB[2]) + fmaf(raw[i][j][3], A[3], nB[3]);
          buf_store_f32(fmaf(gm[j], v0, bt[j] * W0), outr, (obase + 16 * j) * 4u);
          buf_store_f32(fmaf(gm[j], v1, bt[j] * W1), outr, (obase + D + 16 * j) * 4u);
        }
      } else {
        const float Wk[4] = {w4.x, w4.y, w4.z, w4.w};
        const uint32_t obase = lrow * D + dcol0 + r16;
#pragma unroll
        for (int j = 0; j < DT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            buf_store_f32(fmaf(gm[j], fmaf(raw[i][j][e], A[e], nB[e]), bt[j] * Wk[e]), outr,
                          (obase + e * D + 16 * j) * 4u);
      }
    }
  }
}

template <int DT, int KS1>
hipError_t launch_fused(const FusedParams& p, hipStream_t stream) {
  const dim3 grid((p.rows + kRows - 1) / kRows);
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
  RLM_REQUIRE(B * Tq * K < kMaxBytes && B * Tq * D * 4 < kMaxBytes,
              "fused relation reduce: B*Tq*K rows and the fp32 output must stay below 2^31");
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "operand_cache, product_weight and second_weight must be 16-byte aligned");
  p.Tq = static_cast<uint32_t>(Tq);
  p.T = T;
  p.R = static_cast<uint32_t>(R);
  p.H = static_cast<uint32_t>(H);
  p.D = static_cast<uint32_t>(D);
  p.K = static_cast<uint32_t>(K);
  p.k_log2 = static_cast<uint32_t>(__builtin_ctzll(static_cast<unsigned long long>(K)));
  p.rows = static_cast<uint32_t>(B * Tq * K);
  p.queries = static_cast<uint32_t>(B * Tq);
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

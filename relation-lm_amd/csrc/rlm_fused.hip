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
// (query, partner) rows, so it holds whole queries (K rounded up to a power
// of two, at most 16; the padding rows of a query carry weight 0).
// Inside the workgroup the rows are kept in "slot" order (slot_row below),
// chosen so that phase 2 leaves each query's partners in as few lanes as
// possible.
//   set-up   wave w keeps the exact hi/lo bf16 split of the operand products
//            (op[anchor] * op[partner], exact in fp32) of slots 16w..16w+15 in
//            registers; the rows' active-K softmax weights and the b2 / gamma /
//            beta vectors go to LDS.  All loads that do not depend on the row
//            indices are issued in one round, branch-free.
//   phase 1  per 128-column chunk of the hidden dimension, wave w forms
//            hidden^T[128 cols x its 16 slots] = W_m[chunk] . P^T on the matrix
//            cores (16x16x32), adds the rows' expanded-cache halves (one more
//            MFMA against a constant [I|I]), applies GELU and rounds to bf16 --
//            the operand the unfused path's bf16 second linear sees -- into the
//            LDS hidden chunk.  The W_m chunk and the gathered expanded-cache
//            halves reach LDS by LDS-DMA (buffer_load ... lds), issued while
//            the previous chunk's phase 2 runs.
//   phase 2  raw^T[D cols x 128 slots] += W2[:, chunk] . hidden chunk^T on
//            32x32x16 MFMAs: wave (dg, rg) owns DTW 32-column tiles of D and
//            RTW 32-slot tiles; W2 fragments come from L2 three k-steps ahead,
//            hidden fragments from LDS one fragment ahead, and the raw
//            accumulators stay in registers for the whole kernel.  The
//            transposed product leaves one slot's columns in a lane.
// Epilogue (the accumulators start at b2): LayerNorm moments per slot (in-lane
// sums, the two wave halves, then the D-direction waves merged in LDS); partner
// weights and the sum over a query's partners (in-lane over row tiles, then DPP
// / permlane across the lanes of the query); 16-byte buffer stores.
#include "rlm_common.hpp"

namespace rlm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kRows = 128;                 // (query, partner) rows per workgroup
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
#ifndef RLM_W2_AHEAD
#define RLM_W2_AHEAD 3
#endif
constexpr int kW2Ahead = RLM_W2_AHEAD;      // phase-2 W2 prefetch distance (k-steps)
constexpr int kWaitVm0 = 0x0F70;           // s_waitcnt vmcnt(0), other counters untouched

struct FusedParams {
  int64_t T;
  uint32_t Tq, K, k_log2, R, H, D;
  uint32_t Kr;         // partners per query in the inputs (K is Kr rounded up to a power of two)
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
  uint32_t pos_count;    // elements of the positions tensor
  float eps;
  float* out;             // [B*Tq, D]
  uint32_t expanded_bytes, operand_bytes, wm_bytes, w2_bytes;
};

__device__ __forceinline__ f32x4 mfma_bf16(const u16x8& a, const u16x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// D[32x32] += A[32x16] B[16x32]: lane l holds A row l%32, k = 8(l/32)..+7, and
// B column l%32, same k; D element 4i+j is row 8i + 4(l/32) + j, column l%32.
__device__ __forceinline__ f32x16 mfma32_bf16(const u16x8& a, const u16x8& b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Sum of lanes l and l +- N within each 16-lane row (DPP row_ror).
template <int N>
__device__ __forceinline__ float ror_sum(float v) {
  return v + __uint_as_float(dpp_u32<0x120 + N>(__float_as_uint(v)));
}

__device__ __forceinline__ void buf_store_f32x4(float4 v, rsrc_t r, uint32_t off) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, 0);
}

// Phase 2 and the epilogue see the workgroup's 128 (query, partner) rows in
// "slot" order: slot s = 32*rt + n is column n of 32-row tile rt, and a wave of
// row group rg covers tiles RTW*rg .. RTW*rg + RTW-1.  The map keeps each
// query inside one row group and puts its partners in as few lanes as
// possible: K <= RTW -> one lane holds RTW/K whole queries (tile rt' of the
// group = K*(query/32) + partner); K > RTW -> a query's partners sit in lanes
// n = q, q + QG, q + 2QG, ... (QG = 32*RTW/K queries per group), RTW each.
// Returns the local row (query*K + partner) of slot s.
template <int RTW>
__device__ __forceinline__ uint32_t slot_row(int s, uint32_t K, uint32_t k_log2) {
  const int rt = s >> 5, n = s & 31;
  const int rgs = rt / RTW, rtp = rt % RTW;
  const int qg = (32 * RTW) >> k_log2;
  int q_in, k;
  if (static_cast<int>(K) <= RTW) {
    q_in = 32 * (rtp >> k_log2) + n;
    k = rtp & static_cast<int>(K - 1);
  } else {
    k = rtp + RTW * (n / qg);
    q_in = n % qg;
  }
  return static_cast<uint32_t>((rgs * qg + q_in) * static_cast<int>(K) + k);
}

__device__ __forceinline__ u16x8 lds_frag(const unsigned char* p) {
  return *reinterpret_cast<const u16x8*>(p);
}

__device__ __forceinline__ u16x8 as_frag(uint4 v) { return __builtin_bit_cast(u16x8, v); }

// Weight p_k of partner k in its query's mixture, from the query's K scores
// and position t: softmax over the active partners (rank < k_limit, score >
// -1e30; inactive scores -1e4), renormalised by max(sum, 1e-9) --
// relation_reduce.py:399-411.
__device__ float row_weight(const float (&sc)[16], int64_t t, uint32_t K, uint32_t k) {
  const int64_t n = t + 1;
  int k_limit = n > 0 ? 64 - __clzll(static_cast<unsigned long long>(n)) : 0;  // ceil(log2(t+2))
  k_limit = k_limit < 1 ? 1 : (k_limit > static_cast<int>(K) ? static_cast<int>(K) : k_limit);
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

template <int DT, int KS1, bool FRAG>
__global__ void __launch_bounds__(kThreads) fused_reduce_kernel(const FusedParams p) {
  // DT = D / 128; KS1 = R / 32; FRAG: W2 in MFMA fragment order (rlm_mfma_fragments).
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
  // Phase 2 tiling: DG waves along D times RG along the rows; a wave owns DTW
  // 32-wide column tiles of D and RTW 32-row tiles.
  constexpr int DG = (DT % 2 == 0) ? 8 : 4;
  constexpr int RG = kWaves / DG;
  constexpr int DTW = 4 * DT / DG;
  constexpr int RTW = 4 / RG;
  static_assert(DG * DTW * 32 == 128 * DT && RG * RTW == 4, "phase-2 tiling");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  // Consecutive logical workgroups (the queries of one batch row) share an
  // XCD, so the expanded-cache rows they gather are fetched into one L2.
  const uint32_t row0 = static_cast<uint32_t>(xcd_tile(blockIdx.x, gridDim.x)) * kRows;
  const uint32_t H = p.H;
  const rsrc_t xr = make_rsrc(p.expanded, p.expanded_bytes);
  const rsrc_t opr = make_rsrc(p.operand, p.operand_bytes);
  const rsrc_t wmr = make_rsrc(p.wm, p.wm_bytes);
  const rsrc_t w2r = make_rsrc(p.w2, p.w2_bytes);

  // ---- Set-up: two dependent round trips.  (1) everything that does not
  // depend on the row indices is issued together, branch-free (dtype
  // dispatch by offset selection, so no load waits at a branch join): the
  // W_m DMA of chunk 0, this lane's row indices, the row-weight inputs of slot
  // tid and element tid of b2 / gamma / beta.  (2) the wave's gather DMA of
  // chunk 0 and the operand rows.  Everything is decoded after the second
  // round trip.
  dma_wm_chunk<KS1>(wmr, lds0, 0, wave, lane);
  // This lane's phase-1 slot: 16*wave + r16 (rows of the hidden chunk in LDS are slots).
  const int lslot = 16 * wave + r16;
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
  // Rows are numbered query*K + k with K a power of two; rows k >= Kr (padding
  // of a non-power-of-two partner count) read no index: zero operands, weight 0.
  const uint32_t grow = row0 + slot_row<RTW>(lslot, p.K, p.k_log2);
  const uint32_t q = grow >> p.k_log2;
  const uint32_t kr = grow & (p.K - 1);
  const bool live = grow < p.rows && kr < p.Kr;
  const IndexWords ai = issue_index(p.anchor, p.index_dtype_a, p.queries, q, live);
  const IndexWords pi = issue_index(p.partner, p.index_dtype_p, p.queries * p.Kr, q * p.Kr + kr,
                                    live);
  // Row-weight inputs of slot tid (threads 0..127): its query's position and K scores.
  const uint32_t wrow = row0 + slot_row<RTW>(tid & (kRows - 1), p.K, p.k_log2);
  const bool wlive = tid < kRows && wrow < p.rows;
  const uint32_t wq = wrow >> p.k_log2;
  const uint32_t wb = wq / p.Tq;
  const IndexWords wpos = issue_index(p.pos, p.pos_dtype, p.pos_count,
                                      static_cast<uint32_t>(wb * p.pos_sb + (wq - wb * p.Tq) * p.pos_sq),
                                      wlive);
  const rsrc_t scr = make_rsrc(p.scores, p.queries * p.Kr * 4u);
  uint32_t sc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c)
    sc[c] = buf_load_b32(scr, wlive && c < static_cast<int>(p.Kr) ? (wq * p.Kr + c) * 4u : kNoOffset);
  // Element tid of b2 / gamma / beta (D <= kThreads).
  const bool dlive = tid < static_cast<int>(p.D);
  const FloatWords cb2 = issue_float(p.b2, p.b2_dtype, p.D, tid, dlive);
  const FloatWords cgm = issue_float(p.gamma, p.gamma_dtype, p.D, tid, dlive);
  const FloatWords cbt = issue_float(p.beta, p.beta_dtype, p.D, tid, dlive);
  {
    const int64_t a64 = decode_index(ai, p.index_dtype_a);
    const int64_t p64 = decode_index(pi, p.index_dtype_p);
    const int32_t a = live && a64 >= 0 && a64 < p.T ? static_cast<int32_t>(a64) : -1;
    const int32_t pp = live && p64 >= 0 && p64 < p.T ? static_cast<int32_t>(p64) : -1;
    const uint32_t base = (q / p.Tq) * static_cast<uint32_t>(p.T);
    if (g == 0) {
      rowoff[2 * lslot] = a >= 0 ? (base + a) * (4u * H) : kNoOffset;               // anchor, first half
      rowoff[2 * lslot + 1] = pp >= 0 ? (base + pp) * (4u * H) + 2u * H : kNoOffset;  // partner, second half
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
    if (tid < kRows) {
      float scf[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) scf[c] = __uint_as_float(sc[c]);
      // Padding rows (k >= Kr) get weight 0: row_weight only weighs k < Kr.
      wts[tid] = wlive ? row_weight(scf, decode_index(wpos, p.pos_dtype), p.Kr, wrow & (p.K - 1))
                       : 0.0f;
    }
    if (dlive) {
      cst[tid] = decode_float(cb2, p.b2_dtype);
      cst[kMaxD + tid] = decode_float(cgm, p.gamma_dtype);
      cst[2 * kMaxD + tid] = decode_float(cbt, p.beta_dtype);
    }
  }

  // W2 fragments (A operand of phase 2): rows d0 + 32j + n32 of W2, k = chunk*128
  // + 16s + 8h (8 bf16 per lane).  In fragment order the wave reads each
  // fragment as one contiguous 1 KiB (fragment (n-block, k-group) at
  // ((nb * H/16 + g) * 64 + lane) * 16 bytes); row-major, 32 rows of 32 bytes.
  const int dg = wave % DG, rg = wave / DG;
  const int d0 = dg * DTW * 32;
  const int n32 = lane & 31, h = lane >> 5;
  const uint32_t w2_lane = FRAG ? ((static_cast<uint32_t>(d0 / 32) * (H / 16)) * kWave + lane) * 16u
                                : (static_cast<uint32_t>(d0 + n32) * H + 8 * h) * 2u;
  auto load_w2 = [&](u16x8 (&w)[DTW], int chunk, int s) {
    const uint32_t kg = FRAG ? static_cast<uint32_t>(chunk * (kHC / 16) + s) * 1024u
                             : static_cast<uint32_t>(chunk * kHC + 16 * s) * 2u;
#pragma unroll
    for (int j = 0; j < DTW; ++j) w[j] = as_frag(buf_load_b128(w2r, w2_lane + 64u * j * H + kg));
  };

  // raw[j][i][4ii + jj] = raw^T[d = d0 + 32j + 8ii + 4h + jj][slot 32(RTW rg + i) + n32],
  // started at b2[d] once the set-up has put b2 in LDS.
  f32x16 raw[DTW][RTW];

  const unsigned char* my_gat = smem + kOffGather + lslot * kGatherRowBytes;
  // Constant A operand [I16 | I16]: lane (r16, g) holds row r16, k = 8g..8g+7,
  // 1.0 (bf16 0x3F80) where k % 16 == r16.
  u16x8 ident;
#pragma unroll
  for (int k = 0; k < 8; ++k) ident[k] = (8 * (g & 1) + k == r16) ? 0x3F80 : 0;
  asm volatile("" : "+v"(ident));  // kept in four registers, not rebuilt in every chunk
  unsigned char* my_hid = hid + lslot * (2 * kLd) + 8 * g;
  // B operand of phase 2: hidden slot 32(RTW rg + i) + n32, k = 16s + 8h.
  const unsigned char* brow = hid + (32 * RTW * rg + n32) * (2 * kLd) + 16 * h;

  const int nchunks = H / kHC;
  __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this lane's W_m and gather pieces of chunk 0 are in LDS
  __syncthreads();
#pragma unroll
  for (int j = 0; j < DTW; ++j)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const float4 b4 = *reinterpret_cast<const float4*>(cst + d0 + 32 * j + 8 * ii + 4 * h);
#pragma unroll
      for (int i = 0; i < RTW; ++i) {
        raw[j][i][4 * ii + 0] = b4.x;
        raw[j][i][4 * ii + 1] = b4.y;
        raw[j][i][4 * ii + 2] = b4.z;
        raw[j][i][4 * ii + 3] = b4.w;
      }
    }

  for (int c = 0; c < nchunks; ++c) {
    // W2 fragments of this chunk's phase 2, k-step by k-step.  The first
    // kW2Ahead are loaded before the last GELU of phase 1, while no LDS-DMA is
    // in flight, and are complete before the next chunk's DMA is issued: loads
    // return in issue order, so a wait for a load issued after a DMA also waits
    // for the DMA.  The DMA is covered by the first kW2Ahead k-steps.
    u16x8 wq[kHC / 16][DTW];
    // ---- Phase 1, two halves of 64 columns: hidden^T[cols x 16 slots of this wave].
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
      if (hh == 1) {
#pragma unroll
        for (int s = 0; s < kW2Ahead; ++s) load_w2(wq[s], c, s);
      }
      // acc[jj][e] = hidden[slot lslot][col 16(4hh+jj) + 4g + e].
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const f32x4 hv = acc[jj];
        *reinterpret_cast<uint2*>(my_hid + 32 * (4 * hh + jj)) =
            make_uint2(pack_bf16x2(gelu_erf(hv[0]), gelu_erf(hv[1])),
                       pack_bf16x2(gelu_erf(hv[2]), gelu_erf(hv[3])));
      }
    }
    __syncthreads();  // hidden chunk complete; the W_m and gather tiles are free
    if (c + 1 < nchunks) {
#pragma unroll
      for (int s = 0; s < kW2Ahead; ++s)
#pragma unroll
        for (int j = 0; j < DTW; ++j) asm volatile("" ::"v"(wq[s][j]));  // landed before the DMA
      dma_wm_chunk<KS1>(wmr, lds0, c + 1, wave, lane);
      gather_chunk(c + 1);
    }
    // ---- Phase 2: raw^T[32 DTW x 32 RTW] += W2[cols, chunk] . hidden chunk^T,
    // k-step by k-step (W2 fragments kW2Ahead k-steps ahead), row tile by row
    // tile (the next hidden fragment in flight).
    u16x8 b = lds_frag(brow);
#pragma unroll
    for (int s = 0; s < kHC / 16; ++s) {
      if (s + kW2Ahead < kHC / 16) load_w2(wq[s + kW2Ahead], c, s + kW2Ahead);
#pragma unroll
      for (int i = 0; i < RTW; ++i) {
        // The next fragment in (k-step, row tile) order, across k-step boundaries.
        const bool more = i + 1 < RTW || s + 1 < kHC / 16;
        u16x8 bn;
        if (more)
          bn = lds_frag(i + 1 < RTW ? brow + (i + 1) * 32 * (2 * kLd) + 32 * s : brow + 32 * (s + 1));
#pragma unroll
        for (int j = 0; j < DTW; ++j) raw[j][i] = mfma32_bf16(wq[s][j], b, raw[j][i]);
        if (more) b = bn;
      }
      __builtin_amdgcn_sched_barrier(0);  // keep each k-step's loads next to its products
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this lane's pieces of chunk c+1 are in LDS
    __syncthreads();  // ... and everyone's; the hidden chunk is free again
  }

  // ---- Epilogue.  A lane holds, for each of its RTW slots, 16*DTW of the
  // wave's 32*DTW columns; the other 16*DTW are in lane ^ 32.  b2 is already in.
  // Row moments.  Each wave takes the mean and centred sum of squares of its
  // 32*DTW columns of each of its slots (in-lane sums, then the two halves of
  // the wave); threads 0..127 merge the DG waves of the slot's row group (Chan,
  // Golub and LeVeque's pairwise update, equal counts) -- one barrier round, no
  // E[x^2]-mu^2.
  constexpr float kCols = 32.0f * DTW;
#pragma unroll
  for (int i = 0; i < RTW; ++i) {
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < DTW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += raw[j][i][e];
    const float mu = swap32_sum(sum) * (1.0f / kCols);
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < DTW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float d = raw[j][i][e] - mu;
        sq = fmaf(d, d, sq);
      }
    sq = swap32_sum(sq);
    if (h == 0) {
      const int slot = 32 * (RTW * rg + i) + n32;
      part[dg * kRows + slot] = mu;
      part[(DG + dg) * kRows + slot] = sq;
    }
  }
  __syncthreads();
  if (tid < kRows) {
    float mw[DG], mu = 0.0f, m2 = 0.0f;
#pragma unroll
    for (int w = 0; w < DG; ++w) {
      mw[w] = part[w * kRows + tid];
      mu += mw[w];
      m2 += part[(DG + w) * kRows + tid];
    }
    mu *= 1.0f / DG;
    float spread = 0.0f;
#pragma unroll
    for (int w = 0; w < DG; ++w) spread = fmaf(mw[w] - mu, mw[w] - mu, spread);
    mom[tid] = mu;
    mom[kRows + tid] = rsqrtf(fmaf(spread, kCols, m2) * (1.0f / static_cast<float>(p.D)) + p.eps);
  }
  __syncthreads();
  // LayerNorm, weights, sum over each query's K rows, store:
  //   out[q] = sum_k w_k (gamma (x_k - mu_k) rs_k + beta)
  //          = gamma * sum_k (A_k x_k - B_k) + beta * sum_k w_k,
  // A_k = w_k rs_k, B_k = A_k mu_k, so each raw value costs one FMA.  The
  // store descriptor covers this workgroup's queries only, so queries past the
  // end of the last workgroup are dropped by the buffer bounds check.
  const uint32_t K = p.K, D = p.D;
  const uint32_t q0 = row0 >> p.k_log2;
  const uint32_t nq = min(p.queries - q0, static_cast<uint32_t>(kRows) >> p.k_log2);
  const rsrc_t outr = make_rsrc(p.out + static_cast<size_t>(q0) * D, nq * D * 4u);
  const int qg = (32 * RTW) >> p.k_log2;  // queries per row group
  float A[RTW], nB[RTW], wk[RTW];
#pragma unroll
  for (int i = 0; i < RTW; ++i) {
    const int slot = 32 * (RTW * rg + i) + n32;
    wk[i] = wts[slot];
    A[i] = wk[i] * mom[kRows + slot];
    nB[i] = -A[i] * mom[slot];
  }
  // Stores the 16*DTW columns of one query: v holds sum_k (A_k x_k - B_k), W = sum_k w_k.
  auto store_query = [&](const float (&v)[DTW][16], float W, uint32_t qloc) {
#pragma unroll
    for (int j = 0; j < DTW; ++j)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d = d0 + 32 * j + 8 * ii + 4 * h;
        const float4 g4 = *reinterpret_cast<const float4*>(cst + kMaxD + d);
        const float4 b4 = *reinterpret_cast<const float4*>(cst + 2 * kMaxD + d);
        const float4 o = make_float4(fmaf(g4.x, v[j][4 * ii + 0], b4.x * W),
                                     fmaf(g4.y, v[j][4 * ii + 1], b4.y * W),
                                     fmaf(g4.z, v[j][4 * ii + 2], b4.z * W),
                                     fmaf(g4.w, v[j][4 * ii + 3], b4.w * W));
        buf_store_f32x4(o, outr, (qloc * D + d) * 4u);
      }
  };
  if (static_cast<int>(K) >= RTW) {
    // One query per lane; its partners also sit in lanes n32 + QG, + 2QG, ...
    float v[DTW][16], W = 0.0f;
#pragma unroll
    for (int i = 0; i < RTW; ++i) W += wk[i];
#pragma unroll
    for (int j = 0; j < DTW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < RTW; ++i) acc += fmaf(raw[j][i][e], A[i], nB[i]);
        v[j][e] = acc;
      }
    const int lanes = static_cast<int>(K) / RTW;  // lanes per query, QG apart
    if (lanes >= 8) {
      W = ror_sum<4>(W);
#pragma unroll
      for (int j = 0; j < DTW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[j][e] = ror_sum<4>(v[j][e]);
    }
    if (lanes >= 4) {
      W = ror_sum<8>(W);
#pragma unroll
      for (int j = 0; j < DTW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[j][e] = ror_sum<8>(v[j][e]);
    }
    if (lanes >= 2) {
      W = swap16_sum(W);
#pragma unroll
      for (int j = 0; j < DTW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[j][e] = swap16_sum(v[j][e]);
    }
    if (n32 < qg) store_query(v, W, static_cast<uint32_t>(rg * qg + n32));
  } else {
    // K < RTW: this lane holds RTW/K whole queries, tiles K*qq .. K*qq + K-1.
#pragma unroll
    for (int qq = 0; qq < RTW; ++qq) {
      if (qq * static_cast<int>(K) >= RTW) break;
      float v[DTW][16], W = 0.0f;
#pragma unroll
      for (int j = 0; j < DTW; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[j][e] = 0.0f;
#pragma unroll
      for (int i = 0; i < RTW; ++i) {
        if (i / static_cast<int>(K) != qq) continue;
        W += wk[i];
#pragma unroll
        for (int j = 0; j < DTW; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) v[j][e] += fmaf(raw[j][i][e], A[i], nB[i]);
      }
      store_query(v, W, static_cast<uint32_t>(rg * qg + 32 * qq + n32));
    }
  }
}

template <int DT, int KS1, bool FRAG>
hipError_t launch_fused(const FusedParams& p, hipStream_t stream) {
  const dim3 grid((p.rows + kRows - 1) / kRows);
  static bool attr_set = false;  // the LDS opt-in is a per-process function attribute
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&fused_reduce_kernel<DT, KS1, FRAG>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
    if (e != hipSuccess) {
      set_error("relation_reduce_fused: cannot reserve %zu bytes of LDS: %s", kLdsBytes,
                hipGetErrorString(e));
      return e;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL((fused_reduce_kernel<DT, KS1, FRAG>), grid, dim3(kThreads), kLdsBytes, stream,
                     p);
  return launch_status("relation_reduce_fused");
}

}  // namespace
}  // namespace rlm

using namespace rlm;

namespace {
// second_weight as [D, H] (row-major) or in MFMA fragment order [D/32, H/16, 64, 8]:
// D and H; false for any other shape.
bool second_weight_dims(const rlm_tensor* w, int64_t& D, int64_t& H) {
  if (w->ndim == 2) {
    D = w->shape[0];
    H = w->shape[1];
    return true;
  }
  if (w->ndim == 4 && w->shape[2] == 64 && w->shape[3] == 8) {
    D = w->shape[0] * 32;
    H = w->shape[1] * 16;
    return true;
  }
  return false;
}
}  // namespace

extern "C" int rlm_relation_reduce_fused_seq_fits(const rlm_tensor* expanded_cache,
                                                  const rlm_tensor* operand_cache,
                                                  const rlm_tensor* partner_index,
                                                  const rlm_tensor* product_weight,
                                                  const rlm_tensor* second_weight) {
  for (const rlm_tensor* t : {expanded_cache, operand_cache, partner_index, product_weight,
                              second_weight})
    if (t == nullptr) return 0;
  if (operand_cache->ndim != 3 || expanded_cache->ndim != 3 || partner_index->ndim != 3 ||
      product_weight->ndim != 2)
    return 0;
  for (const rlm_tensor* t : {expanded_cache, operand_cache, product_weight, second_weight})
    if (t->dtype != RLM_BF16) return 0;
  const int64_t R = operand_cache->shape[2], H = product_weight->shape[0];
  int64_t D, H2;
  if (!second_weight_dims(second_weight, D, H2) || H2 != H) return 0;
  const int64_t K = partner_index->shape[2];
  if (K < 1 || K > 16 || !(R == 32 || R == 64 || R == 128) || H <= 0 || H % kHC != 0) return 0;
  if (!(D == 128 || D == 256 || D == 384 || D == 512)) return 0;
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) return 0;
  return 1;
}

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
  RLM_REQUIRE(second_weight != nullptr, "second_weight: missing tensor");
  const bool frag = second_weight->ndim == 4;
  RLM_TRY(check_tensor(second_weight, "second_weight", frag ? 4 : 2));
  RLM_TRY(check_dtype_is(operand_cache, "operand_cache", RLM_BF16));
  RLM_TRY(check_dtype_is(expanded_cache, "expanded_cache", RLM_BF16));
  RLM_TRY(check_dtype_is(product_weight, "product_weight", RLM_BF16));
  RLM_TRY(check_dtype_is(second_weight, "second_weight", RLM_BF16));
  const int64_t B = operand_cache->shape[0], T = operand_cache->shape[1];
  const int64_t R = operand_cache->shape[2], H = product_weight->shape[0];
  int64_t D, H2;
  RLM_REQUIRE(second_weight_dims(second_weight, D, H2),
              "second_weight must be [D, H] or in MFMA fragment order [D/32, H/16, 64, 8]");
  RLM_TRY(check_dim(product_weight, "product_weight", 1, R));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 0, B));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 1, T));
  RLM_TRY(check_dim(expanded_cache, "expanded_cache", 2, 2 * H));
  RLM_REQUIRE(H2 == H, "second_weight is for hidden dim %lld, product_weight has %lld",
              (long long)H2, (long long)H);
  RLM_TRY(check_tensor(anchor_index, "anchor_index", 2));
  RLM_TRY(check_tensor(partner_index, "partner_index", 3));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype) && is_index_dtype(partner_index->dtype),
              "anchor_index/partner_index must be int32 or int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, B));
  const int64_t Tq = anchor_index->shape[1];
  RLM_TRY(check_dim(partner_index, "partner_index", 0, B));
  RLM_TRY(check_dim(partner_index, "partner_index", 1, Tq));
  const int64_t K = partner_index->shape[2];
  RLM_REQUIRE(K >= 1 && K <= 16, "fused relation reduce supports 1 <= K <= 16, got %lld",
              (long long)K);
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
    p.pos_count = static_cast<uint32_t>(Tq);
  } else {
    RLM_TRY(check_tensor(positions, "positions", 2));
    RLM_TRY(check_dim(positions, "positions", 0, B));
    RLM_TRY(check_dim(positions, "positions", 1, Tq));
    p.pos_sb = Tq;
    p.pos_sq = 1;
    p.pos_count = static_cast<uint32_t>(B * Tq);
  }
  constexpr int64_t kMaxBytes = int64_t(1) << 31;
  RLM_REQUIRE(B * T * 2 * H * 2 < kMaxBytes && B * T * R * 2 < kMaxBytes && D * H * 2 < kMaxBytes,
              "caches and weights must each be smaller than 2 GiB");
  RLM_REQUIRE(B * Tq * K * 8 < kMaxBytes && B * Tq * D * 4 < kMaxBytes,
              "fused relation reduce: the index tensors and the fp32 output must stay below 2 GiB");
  for (const rlm_tensor* t : {operand_cache, product_weight, second_weight})
    RLM_REQUIRE((reinterpret_cast<uintptr_t>(t->data) & 15u) == 0,
                "operand_cache, product_weight and second_weight must be 16-byte aligned");
  p.Tq = static_cast<uint32_t>(Tq);
  p.T = T;
  p.R = static_cast<uint32_t>(R);
  p.H = static_cast<uint32_t>(H);
  p.D = static_cast<uint32_t>(D);
  // A non-power-of-two K runs as the next power of two with zero-weight padding rows.
  const int64_t Kp = K <= 1 ? 1 : int64_t(1) << (64 - __builtin_clzll(static_cast<unsigned long long>(K - 1)));
  p.Kr = static_cast<uint32_t>(K);
  p.K = static_cast<uint32_t>(Kp);
  p.k_log2 = static_cast<uint32_t>(__builtin_ctzll(static_cast<unsigned long long>(Kp)));
  p.rows = static_cast<uint32_t>(B * Tq * Kp);
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
#define RLM_FUSED_KS(DT, KS)                                                      \
  return frag ? launch_fused<DT, KS, true>(p, stream) : launch_fused<DT, KS, false>(p, stream);
#define RLM_FUSED_CASE(DT)           \
  if (D == 128 * DT) {               \
    if (ks1 == 1) RLM_FUSED_KS(DT, 1) \
    if (ks1 == 2) RLM_FUSED_KS(DT, 2) \
    RLM_FUSED_KS(DT, 4)              \
  }
  RLM_FUSED_CASE(1)
  RLM_FUSED_CASE(2)
  RLM_FUSED_CASE(3)
  RLM_FUSED_CASE(4)
#undef RLM_FUSED_CASE
#undef RLM_FUSED_KS
  set_error("fused relation reduce supports d_model in {128, 256, 384, 512} (a wave keeps "
            "[128, d_model/8] accumulators in registers), got %lld; use the unfused "
            "relation_hidden_cached_seq / relation_linear / relation_norm_reduce_seq chain",
            (long long)D);
  return hipErrorInvalidValue;
}

// Routed selection, sequence form, for gfx950: exact results from matrix-core
// candidate scores plus a float64 verification of the few candidates that can
// reach the top-k.
//
// Reference semantics: src/relation_lm/kernels/relation_select.py:9-308 (the
// packed selection), applied to one query per position.  The outputs are the
// same as select_kernel's (rlm_select.hip) under the same numerics contract:
// every exact score is the float64 dot of the bf16/fp32 inputs rounded once to
// float32, block scores are float64 rounded once, and every comparison and tie
// uses those float32 values.
//
// Mapping.  A workgroup of 16 waves owns 16 queries of one batch row, one
// wave per query (4 waves per SIMD, so that one query's dependent LDS and
// VALU latencies overlap the others').  The batch row's keys (every cache row)
// and both streams' block statistics are staged in LDS.  Per stream:
//   1. the matrix cores score every staged key against the 16 queries,
//      s~[row][query] = bf16 MFMA with fp32 accumulation (the partner query is
//      fp32 and enters as a bf16 hi + lo pair);
//   2. block scores (relation_select.py:53-106): the per-head dot products
//      with the block means and stds run on float64 MFMA (v_mfma_f64_16x16x4,
//      16 queries x 16 blocks per tile, one (head, block tile) per wave); each
//      query's wave then folds the heads with a float64 log-sum-exp (lane =
//      (block, head)) and ranks the blocks into the TOP picks;
//   3. lane l of the query's wave reads s~ of candidates l, l + 64, ...; with
//      theta a lower bound of the k-th largest s~ among the valid candidates
//      (the k-th largest of the lanes' maxima) and eps a bound on |s~ - s|
//      (below), every candidate with s~ >= theta - 2 eps is a member: at least
//      k candidates have s >= theta - eps, strictly above every non-member, so
//      the exact top-k lies among the members;
//   4. the members get their exact float64 scores (4 lanes per member, 16
//      dims each) and are ranked by (score, tie index); up to 16 members are
//      scored and ranked in one pass, more (near-ties) in windows of 64 merged
//      into a running top-k, so any number of near-ties (duplicate keys) is
//      handled.
// The partner keys replace the anchor keys in LDS once every wave has its
// anchor; their loads are issued with the anchor's cached partner row, so both
// round trips overlap.
//
// Error bound.  Products of bf16 values are exact in fp32; the MFMA sums 64
// (anchor) or 128 (partner hi + lo) of them in fp32, and the partner query's
// bf16 hi + lo split drops at most 2^-16 of each element.  With any summation
// order and unit roundoff up to 2^-22 (4x the fp32 value), |s~ - s| <= 4.6e-5
// * sum_d |k_d q_d|; sum_d |k_d q_d| <= ||q||_1 * max|k| over the staged keys.
// eps = 2^-13 * ||q||_1 * max|k| covers that with a 2.6x margin plus the
// rounding of float64 sums to float32 (2^-22 relative), and 2^-100 covers
// products that underflow fp32.
#include "rlm_common.hpp"
#include "rlm_select_tile.hpp"
#include "rlm_tile_util.hpp"

namespace rlm {
namespace {

constexpr int kQ = 16;          // queries (waves) per workgroup
constexpr int kThreads = 1024;
constexpr int kRowBytes = 128;  // one staged key row (64 bf16)
constexpr int kSQ = 16;         // floats per s~ row (one per query)
constexpr int kStatRow = 68;    // floats per staged statistics row (64 + 4: conflict-free MFMA operand reads)
constexpr int kQRow = 68;       // doubles per staged query row (64 + 4 zeros: dead k-steps of a head)
constexpr int kListCap = 64;    // members per query per window
constexpr int kMaxNCL = 4;      // candidates per lane (CAP <= 256)

// Per-query record in LDS: the position and the candidate table, entry 0 the
// local window, entry 1 + r the block of pick r, each (first position,
// position limit): a candidate at offset o of an entry is position x + o,
// valid when 0 <= x + o < limit (and inside the cache).
struct QRec {
  int t, pad0, pad1, pad2;
  int2 ent[1 + kTileMaxTop];
};

struct Lds {
  unsigned char* keys;  // [T][128 B], 16-byte chunks XOR-swizzled by row
  float* sc;            // [T][16]: s~ of every row for the 16 queries
  float* stats;         // [2 sides][mean, std][NB][kStatRow] fp32
  double* rq;           // [16][kQRow]: router query, float64
  double* eq;           // [16][kQRow]: exact query, float64
  double* sh;           // [H][16][NB]: per-head block scores (aliases `list`)
  uint64_t* blk;        // [16][NB]: block selection keys
  uint64_t* list;       // [16][kListCap]
  uint64_t* top;        // [2][16][kTileMaxK]
  uint16_t* frag;       // [hi, lo][16][64] bf16 partner query (aliases `top`)
  QRec* qr;             // [16]
  double* bias;         // [2 sides][H*RB]
  double* sp;           // [2 sides][16]
  uint32_t* kmax;       // [16] per-wave max |key| bits
};

__device__ __forceinline__ Lds carve(const TileParams& p, unsigned char* smem) {
  Lds s;
  s.keys = smem + p.off_keys;
  s.sc = reinterpret_cast<float*>(smem + p.off_sc);
  s.stats = reinterpret_cast<float*>(smem + p.off_stats);
  s.rq = reinterpret_cast<double*>(smem + p.off_rq);
  s.eq = reinterpret_cast<double*>(smem + p.off_pq);
  s.list = reinterpret_cast<uint64_t*>(smem + p.off_list);
  s.sh = reinterpret_cast<double*>(smem + p.off_list);
  s.blk = reinterpret_cast<uint64_t*>(smem + p.off_blk);
  s.top = reinterpret_cast<uint64_t*>(smem + p.off_top);
  s.frag = reinterpret_cast<uint16_t*>(smem + p.off_top);
  s.qr = reinterpret_cast<QRec*>(smem + p.off_qrec);
  s.bias = reinterpret_cast<double*>(smem + p.off_bias);
  s.sp = reinterpret_cast<double*>(smem + p.off_sp);
  s.kmax = reinterpret_cast<uint32_t*>(smem + p.off_kmax);
  return s;
}

__device__ __forceinline__ int key_chunk_offset(int row, int ch) {
  return row * kRowBytes + 16 * (ch ^ ((row >> 1) & 7));
}

// Element e of query row r in the partner fragment table (16-byte chunks
// XOR-swizzled by row, so that the fragment reads of 16 rows do not conflict).
// The table lives in the running top-k lists, which are dead from the anchor's
// last use of them until the partner side's block picks.
__device__ __forceinline__ int frag_offset(int r, int e) {
  return r * 64 + 8 * ((e >> 3) ^ (r & 7)) + (e & 7);
}
static_assert(2 * kQ * 64 * 2 <= 2 * kQ * kTileMaxK * 8, "fragment table exceeds the top-k lists");

// Both streams' block statistics (mean and std, NB*64 <= 4096 elements each),
// staged as fp32 rows of kStatRow by every wave alike: wave w reads tensor
// w & 3 (amean, astd, pmean, pstd), four elements per lane per round, rounds
// of 256 groups of four.  The loads are issued first (issue_stats) and stored
// once they are needed (put_stats), so no wave waits for them on its own.
template <typename TS>
struct StatGroup;
template <>
struct StatGroup<float> {
  uint4 v[4];
  __device__ __forceinline__ void issue(rsrc_t r, int u, uint32_t grp, bool live) {
    v[u] = buf_load_b128(r, live ? grp * 16u : kNoOffset);
  }
  __device__ __forceinline__ float4 at(int u) const {
    return make_float4(__uint_as_float(v[u].x), __uint_as_float(v[u].y), __uint_as_float(v[u].z),
                       __uint_as_float(v[u].w));
  }
};
template <>
struct StatGroup<bf16> {
  uint2 v[4];
  __device__ __forceinline__ void issue(rsrc_t r, int u, uint32_t grp, bool live) {
    v[u] = buf_load_b64(r, live ? grp * 8u : kNoOffset);
  }
  __device__ __forceinline__ float4 at(int u) const {
    return make_float4(__uint_as_float(v[u].x << 16), __uint_as_float(v[u].x & 0xffff0000u),
                       __uint_as_float(v[u].y << 16), __uint_as_float(v[u].y & 0xffff0000u));
  }
};

template <typename TS>
__device__ __forceinline__ void issue_stats(const TileParams& p, int64_t b, int wave, int lane,
                                            StatGroup<TS>& g) {
  const int w = wave & 3;
  const void* src = w == 0 ? p.amean : w == 1 ? p.astd : w == 2 ? p.pmean : p.pstd;
  const uint32_t groups = static_cast<uint32_t>(p.NB) * 16u;  // per batch row
  const rsrc_t r = make_rsrc(static_cast<const TS*>(src) + b * p.NB * 64,
                             groups * 4u * static_cast<uint32_t>(sizeof(TS)));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t grp = static_cast<uint32_t>((wave >> 2) * kWave + lane + 256 * u);
    if (256 * u < static_cast<int>(groups)) g.issue(r, u, grp, grp < groups);
  }
}

template <typename TS>
__device__ __forceinline__ void put_stats(const TileParams& p, const Lds& L, int wave, int lane,
                                          const StatGroup<TS>& g) {
  const int w = wave & 3;
  const int groups = p.NB * 16;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int grp = (wave >> 2) * kWave + lane + 256 * u;
    if (256 * u < groups && grp < groups)
      *reinterpret_cast<float4*>(L.stats + (w * p.NB + (grp >> 4)) * kStatRow + 4 * (grp & 15)) =
          g.at(u);
  }
}

// Router constants of both streams: thread i < 2 H*RB one relative-bias entry
// (anchor table, then partner), the next 2 H threads one gamma each.  Issued
// before any other load of the kernel (both dtype forms; out-of-range lanes
// read 0), so that the decode and the softplus wait for these loads only and
// run while the key rows are still in flight.
struct RouterWords {
  FloatWords ab, pb, ag, pg;
};

__device__ __forceinline__ void issue_router_consts(const TileParams& p, int tid, RouterWords& w) {
  const uint32_t n = static_cast<uint32_t>(p.H * p.RB);
  const uint32_t H = static_cast<uint32_t>(p.H);
  const uint32_t i = static_cast<uint32_t>(tid);
  if (i < 2 * n + 2 * H) {
    const uint32_t kb = i < n ? i : i - n;
    const uint32_t h = i - 2 * n < H ? i - 2 * n : i - 2 * n - H;
    w.ab = issue_float(p.abias, p.abias_dtype, n, kb, i < n);
    w.pb = issue_float(p.pbias, p.pbias_dtype, n, kb, i >= n && i < 2 * n);
    w.ag = issue_float(p.agamma, p.agamma_dtype, H, h, i >= 2 * n && i < 2 * n + H);
    w.pg = issue_float(p.pgamma, p.pgamma_dtype, H, h, i >= 2 * n + H);
  }
}

// Bias tables (float64) and softplus(gamma) (float64) of both streams into LDS.
__device__ __forceinline__ void put_router_consts(const TileParams& p, const Lds& L, int tid,
                                                  const RouterWords& w) {
  const uint32_t n = static_cast<uint32_t>(p.H * p.RB);
  const uint32_t H = static_cast<uint32_t>(p.H);
  const uint32_t i = static_cast<uint32_t>(tid);
  if (i < 2 * n) {
    L.bias[i] = static_cast<double>(i < n ? decode_float(w.ab, p.abias_dtype)
                                          : decode_float(w.pb, p.pbias_dtype));
  } else if (i < 2 * n + 2 * H) {
#pragma clang fp contract(off)
    const bool partner = i >= 2 * n + H;
    const uint32_t h = partner ? i - 2 * n - H : i - 2 * n;
    const double g = static_cast<double>(partner ? decode_float(w.pg, p.pgamma_dtype)
                                                 : decode_float(w.ag, p.agamma_dtype));
    L.sp[(partner ? 16 : 0) + h] = log(1.0 + exp(g));  // softplus without threshold, relation_select.py:87
  }
}

// Per-head block scores of the 16 queries (relation_select.py:70-96) on
// float64 MFMA, one (head, block tile) per wave of the first `hw` waves (the
// others score the keys meanwhile):
//   content[q][j] = sum_d mean[j][h,d] q[q][h,d],  unc[q][j] = sum_d std[j][h,d] |q[q][h,d]|
//   s_h = (content + softplus(gamma_h) unc) * HD^-0.5 + bias[h, bucket(t_q, j)]
// into sh[h][q][j].  v_mfma_f64_16x16x4f64 takes A[i = lane%16][k = lane/16],
// B[k = lane/16][j = lane%16] and leaves D[4r + lane/16][lane%16] in register r.
__device__ void head_scores(const TileParams& p, const Lds& L, int side, int wave, int hw,
                            int lane) {
  const float* mean = L.stats + (2 * side) * p.NB * kStatRow;
  const float* stdv = L.stats + (2 * side + 1) * p.NB * kStatRow;
  const double* sp = L.sp + 16 * side;
  const double* bias = L.bias + side * p.H * p.RB;
  const int kq = lane >> 4, c16 = lane & 15;
  const int nbt = (p.NB + 15) >> 4;
  for (int item = wave; item < p.H * nbt; item += hw) {
    const int h = item / nbt;
    const int jt = item - h * nbt;
    const int j = jt * 16 + c16;
    const bool jv = j < p.NB;
    const int jc = jv ? j : 0;
    // The epilogue's operands first (query positions, then the bucket biases),
    // so that their LDS round trips overlap the matrix-core chain.
    const int end = (j + 1) * p.BS - 1;
    double bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = L.qr[4 * r + kq].t;
      const int dist = (t > end ? t - end : 0) + 1;
      int bucket = 31 - __clz(dist);
      bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
      bv[r] = bias[h * p.RB + bucket];
    }
    const double sph = sp[h];
    f64x4_t content = {0.0, 0.0, 0.0, 0.0}, unc = {0.0, 0.0, 0.0, 0.0};
    for (int ks0 = 0; ks0 < p.HD; ks0 += 16) {
      // Four k-steps, every operand read before the first MFMA and no operand
      // masked: a k-step past the head's HD dims (HD = 8) takes its query
      // values from the zero pad of the query row, a block past NB reads
      // block 0 (its column is not stored).
      double a[4];
      float bm[4], bs[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool live = ks0 + 4 * u < p.HD;
        const int d = h * p.HD + (live ? ks0 + 4 * u : 0) + kq;
        a[u] = L.rq[c16 * kQRow + (live ? d : 64 + kq)];
        bm[u] = mean[jc * kStatRow + d];
        bs[u] = stdv[jc * kStatRow + d];
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the chain
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        content = __builtin_amdgcn_mfma_f64_16x16x4f64(a[u], static_cast<double>(bm[u]), content,
                                                       0, 0, 0);
        unc = __builtin_amdgcn_mfma_f64_16x16x4f64(fabs(a[u]), static_cast<double>(bs[u]), unc,
                                                   0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      double v;
      {
#pragma clang fp contract(off)
        const double c = content[r] + sph * unc[r];
        v = c * p.head_scale + bv[r];
      }
      if (jv) L.sh[(h * kQ + 4 * r + kq) * p.NB + j] = v;
    }
  }
}

// Block picks of all 16 queries, one lane per (query, block): pair g = 16 NB
// pairs in query order on waves [0, NB / 4) (NB % 4 == 0).
//   block_keys: the log-sum-exp over the H heads (relation_select.py:97-106)
//     of the per-head scores, summed as the pairwise tree ((e0 + e1) + (e2 +
//     e3)) + ..., and the 64-bit selection key (score, lower block first) of
//     an eligible block, -inf otherwise, into blk[q][j];
//   block_ranks: pick rank(j) = #{k : key_k > key_j} among the query's NB
//     keys -- the reference's sequential argmax with ties to the lowest block
//     (:229-242) -- into the query's candidate table.
// Each query's wave clears its table first (picks past the last block are
// block 0, invalid) and sets the local-window entry.
template <int HL>
__device__ __forceinline__ void block_keys(const TileParams& p, const Lds& L, int g) {
  constexpr int H = 1 << HL;
  const int q = g / p.NB;
  const int j = g - q * p.NB;
  double v[H];
#pragma unroll
  for (int h = 0; h < H; ++h) v[h] = L.sh[(h * kQ + q) * p.NB + j];
  const int t = L.qr[q].t;
  double m = v[0];
#pragma unroll
  for (int h = 1; h < H; ++h) m = fmax(m, v[h]);
  double e[H];
#pragma unroll
  for (int h = 0; h < H; ++h) e[h] = exp(v[h] - m);
#pragma unroll
  for (int w = 1; w < H; w *= 2)
#pragma unroll
    for (int h = 0; h < H; h += 2 * w) e[h] += e[h + w];
  const double lse = m + log(e[0]);
  const int ls = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
  const int end = (j + 1) * p.BS - 1;
  const bool eligible = end <= t && (!p.strict || end < ls);
  L.blk[g] = select_key(eligible ? static_cast<float>(lse) : -INFINITY, static_cast<uint32_t>(j));
}

__device__ __forceinline__ void block_ranks(const TileParams& p, const Lds& L, int g) {
  const int q = g / p.NB;
  const int j = g - q * p.NB;
  const uint64_t* row = L.blk + q * p.NB;
  const uint64_t kj = row[j];
  int rank = 0;
  for (int k = 0; k < p.NB; k += 2) {
    const uint4 o = *reinterpret_cast<const uint4*>(row + k);
    rank += ((static_cast<uint64_t>(o.y) << 32) | o.x) > kj;
    rank += ((static_cast<uint64_t>(o.w) << 32) | o.z) > kj;
  }
  if (rank < p.TOP) {
    const int t = L.qr[q].t;
    const int ls = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
    L.qr[q].ent[1 + rank] =
        make_int2(j << p.BS_log2, key_score(kj) > -1.0e30f ? min(t + 1, ls) : 0);
  }
}

// The picks phase of one stream, between two workgroup barriers: keys, then
// (once every key of a query is written) ranks.
__device__ __forceinline__ void block_picks(const TileParams& p, const Lds& L, int wave, int lane) {
  const int g = wave * kWave + lane;
  const bool mine = g < kQ * p.NB;  // whole waves: 16 NB is a multiple of 64
  if (mine) {
    switch (p.H_log2) {
      case 0: block_keys<0>(p, L, g); break;
      case 1: block_keys<1>(p, L, g); break;
      case 2: block_keys<2>(p, L, g); break;
      default: block_keys<3>(p, L, g); break;
    }
  }
  // A query's keys sit in one wave when NB divides 64, else they may span two.
  if (kWave % p.NB != 0) {
    __syncthreads();
  } else {
    wave_sync();
  }
  if (mine) block_ranks(p, L, g);
}

// Clears the wave's query's candidate table: the local window (positions
// t - L + 1 .. t) and TOP invalid picks.
__device__ __forceinline__ void clear_table(const TileParams& p, const Lds& L, int qi, int lane,
                                            int t) {
  QRec& R = L.qr[qi];
  if (lane < p.TOP) R.ent[1 + lane] = make_int2(0, 0);
  if (lane == kWave - 1) R.ent[0] = make_int2(t - p.L + 1, t + 1);
}

// Candidate-table entry and offset of candidate lane c (relation_select.py:
// 244-284): the local window first, then the picks' blocks in pick order.  The
// local window's positions t - L + 1 + c are valid up to t; a pick's up to
// min(t, ls - 1), none for an invalid pick.
__device__ __forceinline__ void cand_slot(const TileParams& p, int c, int& e, int& off) {
  const bool local = c < p.L;
  int r = (c - p.L) >> p.BS_log2;
  r = r < kTileMaxTop - 1 ? r : kTileMaxTop - 1;
  e = local ? 0 : 1 + r;
  off = local ? c : (c - p.L) & (p.BS - 1);
}

// Position and validity of candidate lane c.
__device__ __forceinline__ int cand_pos(const TileParams& p, const QRec& R, int c, bool& valid) {
  int e, off;
  cand_slot(p, c, e, off);
  const int2 en = R.ent[e];
  const int pos = en.x + off;
  valid = (pos >= 0) & (pos < en.y) & (pos < static_cast<int>(p.T));
  return pos;
}

// Exact float64 score of member c on 4 lanes: sub-lane s takes dims
// [16 s, 16 s + 16) of the staged key row and of the float64 query row `qrow`;
// the four partial sums are combined in float64.  Returns the 64-bit selection
// key (score, tie index), the same in the member's 4 lanes.
template <bool ANCHOR>
__device__ __forceinline__ uint64_t member_key(const TileParams& p, const Lds& L, const QRec& R,
                                               int c, int s, const double* qrow) {
  bool v;
  const int pos = cand_pos(p, R, c, v);
  const int row = v ? pos : 0;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) {
    const int chunk = 2 * s + ch;
    const uint4 kv = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, chunk));
    const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const double2 q2 = *reinterpret_cast<const double2*>(qrow + 8 * chunk + 2 * e);
      acc[e] = fma(static_cast<double>(__uint_as_float(w[e] << 16)), q2.x, acc[e]);
      acc[e] = fma(static_cast<double>(__uint_as_float(w[e] & 0xffff0000u)), q2.y, acc[e]);
    }
  }
  double d = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  d += dpp_f64<kDppXor1>(d);
  d += dpp_f64<kDppXor2>(d);
  const float score = static_cast<float>(d * p.exact_scale);
  return select_key(score, static_cast<uint32_t>(ANCHOR ? pos : c));
}

// Output slot `slot` of the wave's query from the 64-bit key `key` or, when
// !have, the exhausted-slot sentinel (position t - L + 1, score -inf;
// relation_select.py:298-308).  Returns the position.
template <bool ANCHOR>
__device__ __forceinline__ int emit(const TileParams& p, const QRec& R, int64_t qrow, int slot,
                                    bool have, uint64_t key, int t, int ls, bool active) {
  int pos = t - p.L + 1;
  float score = -INFINITY;
  if (have) {
    score = key_score(key);
    const int tie = static_cast<int>(key_index(key));
    if (ANCHOR) {
      pos = tie;
    } else {
      bool v;
      pos = cand_pos(p, R, tie, v);
    }
  }
  if (active) {
    if (ANCHOR) {
      p.out_anchor[qrow] = pos;
      p.out_anchor_score[qrow] = score;
    } else {
      p.out_partner[qrow * p.K + slot] = pos;
      p.out_partner_score[qrow * p.K + slot] = score;
    }
  }
  return pos;
}

// Exact top-k of the wave's query among its candidates, from the s~ column of
// query qi, written to the outputs.  ANCHOR: k = 1, ties to the lowest position
// (returns the anchor); else k = p.K, ties to the lowest candidate lane, and
// `exclude` is not a candidate.  `qrow` is the float64 query, `qn1` its L1 norm.
template <bool ANCHOR>
__device__ int exact_select(const TileParams& p, const Lds& L, int qi, int lane, int t, int ls,
                            int exclude, const double* qrow, float qn1, float kmax, bool active,
                            int64_t qrow_out) {
  QRec& R = L.qr[qi];
  const int K = ANCHOR ? 1 : p.K;
  // s~ of the lane's candidates (positions as cand_pos gives them), without
  // branches: every candidate's table entry is read, then every s~ entry
  // (row 0 for invalid candidates, masked after).
  const int T32 = static_cast<int>(p.T);
  int2 en[kMaxNCL];
  int off[kMaxNCL];
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i) {
    int e;
    cand_slot(p, lane + kWave * i, e, off[i]);
    en[i] = R.ent[e];
  }
  int row[kMaxNCL];
  bool ok[kMaxNCL];
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i) {
    const int pos = en[i].x + off[i];
    bool v = (pos >= 0) & (pos < en[i].y) & (pos < T32) & (lane + kWave * i < p.CAP) & active;
    if (!ANCHOR) v = v & (pos != exclude);
    ok[i] = v;
    row[i] = v ? pos : 0;
  }
  float st[kMaxNCL];
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i) st[i] = L.sc[row[i] * kSQ + qi];
  float lm = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i) {
    st[i] = ok[i] ? st[i] : -INFINITY;
    lm = fmaxf(lm, st[i]);
  }
  // theta: a lower bound of the k-th largest approximate score.
  float theta;
  if (ANCHOR) {
    theta = wave_max_f32(lm);
  } else {
    // The k-th largest lane maximum, bit by bit from the top of its
    // order-preserving key: the largest key with at least k lanes at or above it.
    // The top 20 bits suffice: a lower bound is all theta must be.  A prefix
    // in the -inf / NaN part of the key range means no k-th candidate: -inf.
    const uint32_t key = ordered_key(lm);
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 12; --bit) {
      const uint32_t cand = prefix | (1u << bit);
      if (__builtin_popcountll(__builtin_amdgcn_ballot_w64(key >= cand)) >= K) prefix = cand;
    }
    theta = prefix >= 0x00800000u ? key_to_float(prefix) : -INFINITY;  // key of -FLT_MAX
  }
  const float eps = kErrScale * qn1 * kmax;
  const float thr = theta - (2.0f * eps + kErrAbs);
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i)
    if (st[i] > -INFINITY && st[i] >= thr) mask |= 1u << i;
  int mi[kMaxNCL];
  const int members = number_members<kMaxNCL>(mask, mi);
  uint64_t* list = L.list + qi * kListCap;
  const int s = lane & 3;
  int anchor = t - p.L + 1;

  if (members <= 16) {
    // Every member scored in one pass (4 lanes each), ranked, emitted.
#pragma unroll
    for (int i = 0; i < kMaxNCL; ++i)
      if ((mask >> i) & 1u) list[mi[i]] = static_cast<uint64_t>(lane + kWave * i);
    wave_sync();
    {
      const int m = lane >> 2;
      const bool act = m < members;
      const int c = act ? static_cast<int>(list[m]) : 0;
      const uint64_t key = member_key<ANCHOR>(p, L, R, c, s, qrow);
      if (act && s == 0) list[m] = key;
    }
    wave_sync();
    int rank = kWave;
    uint64_t ke = 0;
    if (lane < members) {
      ke = list[lane];
      rank = 0;
#pragma unroll
      for (int f = 0; f < 16; f += 2) {
        const uint4 kk = *reinterpret_cast<const uint4*>(list + f);
        const uint64_t k0 = (static_cast<uint64_t>(kk.y) << 32) | kk.x;
        const uint64_t k1 = (static_cast<uint64_t>(kk.w) << 32) | kk.z;
        rank += (f < members && k0 > ke) + (f + 1 < members && k1 > ke);
      }
    }
    int mine = -(1 << 30) - 1;
    if (rank < K) mine = emit<ANCHOR>(p, R, qrow_out, rank, true, ke, t, ls, active);
    if (lane >= members && lane < K) emit<ANCHOR>(p, R, qrow_out, lane, false, 0, t, ls, active);
    if (ANCHOR && members > 0) anchor = wave_max_i(rank == 0 ? mine : -(1 << 30) - 1);
    wave_sync();
    return anchor;
  }

  // Many members (near-ties): windows of 64 merged into a running top-k.
  const int nwin = (members + kListCap - 1) / kListCap;
  int ntop = 0;
  int cur = 0;
  for (int w = 0; w < nwin; ++w) {
    const int lo = w * kListCap;
    const int nw = min(members - lo, kListCap);
#pragma unroll
    for (int i = 0; i < kMaxNCL; ++i)
      if (((mask >> i) & 1u) && mi[i] >= lo && mi[i] < lo + kListCap)
        list[mi[i] - lo] = static_cast<uint64_t>(lane + kWave * i);
    wave_sync();
    for (int m0 = 0; m0 < nw; m0 += 16) {
      const int m = m0 + (lane >> 2);
      const bool act = m < nw;
      const int c = act ? static_cast<int>(list[m]) : 0;
      const uint64_t key = member_key<ANCHOR>(p, L, R, c, s, qrow);
      if (act && s == 0) list[m] = key;
    }
    wave_sync();
    const uint64_t* topc = L.top + (cur * kQ + qi) * kTileMaxK;
    uint64_t* topn = L.top + ((cur ^ 1) * kQ + qi) * kTileMaxK;
    const int ntot = ntop + nw;
    for (int e = lane; e < ntot; e += kWave) {
      const uint64_t ke = e < ntop ? topc[e] : list[e - ntop];
      int rank = 0;
      for (int f = 0; f < ntot; ++f) {
        const uint64_t kf = f < ntop ? topc[f] : list[f - ntop];
        rank += kf > ke;
      }
      if (rank < K) topn[rank] = ke;
    }
    ntop = min(K, ntot);
    cur ^= 1;
    wave_sync();
  }
  const uint64_t* topf = L.top + (cur * kQ + qi) * kTileMaxK;
  if (lane < K) {
    const uint64_t key = lane < ntop ? topf[lane] : 0;
    emit<ANCHOR>(p, R, qrow_out, lane, lane < ntop, key, t, ls, active);
  }
  if (ANCHOR && ntop > 0) anchor = static_cast<int>(key_index(topf[0]));
  wave_sync();
  return anchor;
}

// Stages one stream's keys (already loaded, 4 chunks per thread) into LDS and
// records this wave's max |key| bits.
__device__ __forceinline__ void put_keys(const Lds& L, const uint4 (&kv)[4], int tid, int nchunks,
                                         int wave, int lane) {
  u16x2_t km = {0, 0};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = tid + kThreads * u;
    if (k < nchunks) {
      *reinterpret_cast<uint4*>(L.keys + key_chunk_offset(k >> 3, k & 7)) = kv[u];
      km = absmax8(kv[u], km);
    }
  }
  const uint32_t kbits = wave_max_u32(umax32(km.x, km.y));
  if (lane == 0) L.kmax[wave] = kbits;
}

__device__ __forceinline__ float staged_kmax(const Lds& L) {
  uint32_t kb = 0;
#pragma unroll
  for (int w = 0; w < kQ; ++w) kb = umax32(kb, L.kmax[w]);
  return __uint_as_float(kb << 16) * (1.0f + 1.0f / 1024.0f);
}

// The expanded-cache projection of this workgroup, when the launch carries it
// (no reference kernel: the reference projects the cache with its own linear
// call): tile i of the (x_rows / 128) x (x_N / 128) grid for i = wg, wg + G,
// ..., each a 128 x 128 output tile formed as the library's small-K GEMM forms
// it (W . A^T per 16x16x32 k-step, k-steps in order, fp32 sums, + bias,
// rounded to bf16), so the bits equal that GEMM's.  The tile's A and W rows go
// straight to LDS (`stage`, the key rows' LDS before the keys are put there) by
// LDS-DMA: 16 KS instructions of 64 pieces per tile, KS per wave, each lane's
// source chosen so that piece q of row r lands at q ^ (r % SW) (rows past the
// cache read zeros; their outputs are not stored).
// LDS byte address of a pointer into the dynamic LDS (wave-uniform).
__device__ __forceinline__ uint32_t lds_u32(const void* ptr) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ptr)));
}

template <int KS>
__device__ __forceinline__ void expand_issue(const TileParams& p, uint32_t stage, int64_t tile,
                                             int wave, int lane) {
  constexpr int K = 32 * KS;
  constexpr int QPR = K / 8;
  constexpr int SW = QPR % 16 == 0 ? 16 : (QPR % 8 == 0 ? 8 : 4);
  const rsrc_t ar = make_rsrc(p.x_op, p.x_op_bytes);
  const rsrc_t wr = make_rsrc(p.x_w, p.x_w_bytes);
  const int64_t tiles_n = p.x_N / 128;
  const int64_t mt = (tile / tiles_n) * 128, nt = (tile % tiles_n) * 128;
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // the resource choice stays scalar
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int ins = wv * KS + k;             // 0 .. 16 KS - 1: A's 2 QPR, then W's
    const bool is_w = ins >= 2 * QPR;
    const int J = is_w ? ins - 2 * QPR : ins;
    const int pd = 64 * J + lane;            // LDS piece of this lane
    const int row = pd / QPR, q = (pd % QPR) ^ (row % SW);
    const int64_t src_row = (is_w ? nt : mt) + row;
    const uint32_t off = is_w || src_row < p.x_rows
                             ? static_cast<uint32_t>((src_row * K + 8 * q) * 2)
                             : kNoOffset;
    lds_dma16(is_w ? wr : ar, stage + (is_w ? 128 * K * 2 : 0) + 1024u * J, off);
  }
}

// The products and stores of one staged tile; returns after every wave is done
// with the staged rows.  Wave w forms rows 32 (w / 4) .. +31 and columns
// 32 (w % 4) .. +31.
template <int KS>
__device__ void expand_compute(const TileParams& p, const unsigned char* stage, int64_t tile,
                               int lane, int wave) {
  constexpr int K = 32 * KS;
  constexpr int QPR = K / 8;
  constexpr int SW = QPR % 16 == 0 ? 16 : (QPR % 8 == 0 ? 8 : 4);
  const unsigned char* ta = stage;
  const unsigned char* tw = stage + 128 * K * 2;
  const int64_t tiles_n = p.x_N / 128;
  const int64_t mt = (tile / tiles_n) * 128, nt = (tile % tiles_n) * 128;
  const int r16 = lane & 15, g = lane >> 4;
  const int wm = (wave >> 2) * 32, wn = (wave & 3) * 32;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int q = 4 * s + g;
    uint4 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = *reinterpret_cast<const uint4*>(ta + (wm + 16 * i + r16) * (2 * K) + 16 * (q ^ (r16 % SW)));
      b[i] = *reinterpret_cast<const uint4*>(tw + (wn + 16 * i + r16) * (2 * K) + 16 * (q ^ (r16 % SW)));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(b[j], a[i], acc[i][j]);
  }
  // Lane (r16, g) holds row wm + 16 i + r16, columns wn + 16 j + 4 g .. + 3:
  // + bias, bf16, restaged over the A tile (every wave is done with it) as
  // [128 rows][128 + 8 columns], then stored as whole 256-byte row segments.
  float bv[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      bv[j][e] = p.x_bias != nullptr
                     ? load_any_f(p.x_bias, p.x_bias_dtype, nt + wn + 16 * j + 4 * g + e)
                     : 0.0f;
  constexpr int kOut = 128 + 8;  // staged row stride (bf16); 34 KiB, within the key rows' LDS
  bf16* st = reinterpret_cast<bf16*>(const_cast<unsigned char*>(stage));
  __syncthreads();  // every wave is done reading the A and W tiles
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<uint2*>(st + (wm + 16 * i + r16) * kOut + wn + 16 * j + 4 * g) =
          make_uint2(pack_bf16x2(acc[i][j][0] + bv[j][0], acc[i][j][1] + bv[j][1]),
                     pack_bf16x2(acc[i][j][2] + bv[j][2], acc[i][j][3] + bv[j][3]));
  __syncthreads();  // the tile's outputs staged
  // 128 rows x 16 pieces of 16 bytes: two per thread, 16 lanes per row.
  const int tid = wave * kWave + lane;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int piece = t * kThreads + tid;
    const int row = piece >> 4, col = 8 * (piece & 15);
    if (mt + row < p.x_rows)
      *reinterpret_cast<uint4*>(p.x_out + (mt + row) * p.x_N + nt + col) =
          *reinterpret_cast<const uint4*>(st + row * kOut + col);
  }
  __syncthreads();  // every wave is done with the staged rows
}

// The workgroup's projection tiles after the first (issued with the kernel's
// own loads and computed by the caller): each staged, waited for, computed.
template <int KS>
__device__ void expand_rest(const TileParams& p, unsigned char* stage, int64_t wg, int64_t G,
                            int lane, int wave) {
  const int64_t ntile = ((p.x_rows + 127) / 128) * (p.x_N / 128);
  for (int64_t tile = wg + G; tile < ntile; tile += G) {
    expand_issue<KS>(p, lds_u32(stage), tile, wave, lane);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();  // the tile's rows in LDS
    expand_compute<KS>(p, stage, tile, lane, wave);
  }
}

// XP: the launch also projects the expanded cache (TileParams::x_*).
template <typename TS, bool XP>
__global__ void __launch_bounds__(kThreads) select_tile_kernel(const TileParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Lds L = carve(p, smem);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;  // = the wave's query within the workgroup
  const int qi = wave;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int64_t wg = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t b = wg / p.tiles;
  const int64_t tq0 = (wg - b * p.tiles) * kQ;
  const int64_t tq = tq0 + qi;
  const bool active = tq < p.Tq;
  const int64_t qrow = b * p.Tq + (active ? tq : tq0);
  const int T = static_cast<int>(p.T);
  const int nchunks = T * 8;
  const uint32_t side_bytes = static_cast<uint32_t>(T) * kRowBytes;

  // ---- One round of loads: the router constants, the anchor keys (every
  //      row), the query-side rows, the position and the statistics of both
  //      streams. ----
  RouterWords rw;
  issue_router_consts(p, tid, rw);
  const rsrc_t akr = make_rsrc(p.akeys + b * p.T * 64, side_bytes);
  uint4 kv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = tid + kThreads * u;
    kv[u] = buf_load_b128(akr, k < nchunks ? static_cast<uint32_t>(k) * 16u : kNoOffset);
  }
  const IndexWords pw = issue_index(p.pos, p.pos_dtype, static_cast<uint32_t>(p.pos_count),
                                    static_cast<uint32_t>(b * p.pos_sb + (active ? tq : tq0) * p.pos_sq),
                                    true);
  // MFMA A fragments of the anchor query: row lane%16 of the workgroup.
  const int64_t arow = b * p.Tq + (tq0 + c16 < p.Tq ? tq0 + c16 : tq0);
  const uint4 a0 = *reinterpret_cast<const uint4*>(p.aq + arow * 64 + 8 * g4);
  const uint4 a1 = *reinterpret_cast<const uint4*>(p.aq + arow * 64 + 32 + 8 * g4);
  // Exact and router query element `lane` of this wave's query.
  const float aqe = to_f32(p.aq[qrow * 64 + lane]);
  const float arqe = to_f32(p.arq[qrow * 64 + lane]);
  StatGroup<TS> sg;
  issue_stats<TS>(p, b, wave, lane, sg);
  if constexpr (XP) {
    // The expanded-cache projection: the workgroup's first tile goes to the key
    // rows' LDS (free until the keys are put there) by LDS-DMA together with
    // the loads above, one wait covers both, and the tile is formed and stored
    // before the keys are staged; further tiles follow one by one.
    const int64_t ntile = ((p.x_rows + 127) / 128) * (p.x_N / 128);
    if (wg < ntile) {
      switch (p.x_KS) {
        case 1: expand_issue<1>(p, lds_u32(L.keys), wg, wave, lane); break;
        case 2: expand_issue<2>(p, lds_u32(L.keys), wg, wave, lane); break;
        case 3: expand_issue<3>(p, lds_u32(L.keys), wg, wave, lane); break;
        default: expand_issue<4>(p, lds_u32(L.keys), wg, wave, lane); break;
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      __syncthreads();  // the first tile's rows in LDS
      switch (p.x_KS) {
        case 1: expand_compute<1>(p, L.keys, wg, lane, wave); expand_rest<1>(p, L.keys, wg, gridDim.x, lane, wave); break;
        case 2: expand_compute<2>(p, L.keys, wg, lane, wave); expand_rest<2>(p, L.keys, wg, gridDim.x, lane, wave); break;
        case 3: expand_compute<3>(p, L.keys, wg, lane, wave); expand_rest<3>(p, L.keys, wg, gridDim.x, lane, wave); break;
        default: expand_compute<4>(p, L.keys, wg, lane, wave); expand_rest<4>(p, L.keys, wg, gridDim.x, lane, wave); break;
      }
    }
  }
  put_router_consts(p, L, tid, rw);
  put_stats<TS>(p, L, wave, lane, sg);

  put_keys(L, kv, tid, nchunks, wave, lane);
  L.eq[qi * kQRow + lane] = static_cast<double>(aqe);
  L.rq[qi * kQRow + lane] = static_cast<double>(arqe);
  if (lane < kQRow - 64) L.rq[qi * kQRow + 64 + lane] = 0.0;
  const int t = clamp_pos(decode_index(pw, p.pos_dtype));
  const int ls = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
  if (lane == 0) L.qr[qi].t = t;
  clear_table(p, L, qi, lane, t);
  float qn1 = wave_sum_f32(fabsf(aqe)) * (1.0f + 1.0f / 1024.0f);  // covers fp32 rounding
  __syncthreads();  // B0

  float kmax = staged_kmax(L);
  const int ntiles = T >> 4;
  // Waves [0, hw) compute the head scores (a chain of LDS round trips and
  // float64 MFMAs), the other waves score the key tiles meanwhile.
  const int hw = min(p.H * ((p.NB + 15) >> 4), 8);
  if (wave < hw) {
    head_scores(p, L, 0, wave, hw, lane);
  } else {
    for (int tt = wave - hw; tt < ntiles; tt += kQ - hw) {
      const int row = tt * 16 + c16;
      const uint4 b0 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, g4));
      const uint4 b1 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, 4 + g4));
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = mfma_bf16(a0, b0, acc);
      acc = mfma_bf16(a1, b1, acc);
      *reinterpret_cast<float4*>(L.sc + row * kSQ + 4 * g4) =
          make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
  }
  __syncthreads();  // B1: s~ and the head scores complete

  block_picks(p, L, wave, lane);
  __syncthreads();  // every query's picks are in its candidate table
  const int anchor = exact_select<true>(p, L, qi, lane, t, ls, -1, L.eq + qi * kQRow, qn1, kmax,
                                        active, qrow);
  clear_table(p, L, qi, lane, t);

  // ---- Partner side.  The anchor's cached row and the partner keys are
  //      loaded together; the keys replace the anchor's once every wave is
  //      done with them. ----
  const bool have = anchor >= 0 && anchor < T;
  const float pbe = to_f32(p.pbase[qrow * 128 + lane]);
  const float pbr = to_f32(p.pbase[qrow * 128 + 64 + lane]);
  // The anchor's cached partner row: branch-free buffer loads (no anchor reads
  // 0), issued together and ahead of the partner keys.
  const rsrc_t pcr_r = make_rsrc(p.pcache + b * p.T * 128, side_bytes * 2u);
  const uint32_t pco = have ? static_cast<uint32_t>(anchor * 128 + lane) * 2u : kNoOffset;
  const uint32_t pce_w = buf_load_b16(pcr_r, pco);
  const uint32_t pcr_w = buf_load_b16(pcr_r, have ? pco + 128u : kNoOffset);
  const float pce = __uint_as_float(pce_w << 16);
  const float pcr = __uint_as_float(pcr_w << 16);
  const rsrc_t pkr = make_rsrc(p.pkeys + b * p.T * 64, side_bytes);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = tid + kThreads * u;
    kv[u] = buf_load_b128(pkr, k < nchunks ? static_cast<uint32_t>(k) * 16u : kNoOffset);
  }
  __syncthreads();  // B2: every wave is done with the anchor side's LDS

  put_keys(L, kv, tid, nchunks, wave, lane);
  const float pqe = pbe + pce;  // fp32 adds, relation_select.py:165-193
  const float pqr = pbr + pcr;
  L.eq[qi * kQRow + lane] = static_cast<double>(pqe);
  L.rq[qi * kQRow + lane] = static_cast<double>(pqr);
  {
    // bf16 hi (round to nearest even) + lo = bf16(x - hi) of the wave's own
    // query element, for every wave's MFMA A fragments.
    const uint32_t hl = pack_bf16x2(pqe, 0.0f) & 0xffffu;
    const uint32_t ll = pack_bf16x2(pqe - __uint_as_float(hl << 16), 0.0f) & 0xffffu;
    const int o = frag_offset(qi, lane);
    L.frag[o] = static_cast<uint16_t>(hl);
    L.frag[kQ * 64 + o] = static_cast<uint16_t>(ll);
  }
  qn1 = wave_sum_f32(fabsf(pqe)) * (1.0f + 1.0f / 1024.0f);
  __syncthreads();  // B3

  kmax = staged_kmax(L);
  // Partner A fragments: bf16 hi + lo of the fp32 query, row lane%16.
  const uint4 ah0 = *reinterpret_cast<const uint4*>(L.frag + frag_offset(c16, 8 * g4));
  const uint4 al0 = *reinterpret_cast<const uint4*>(L.frag + kQ * 64 + frag_offset(c16, 8 * g4));
  const uint4 ah1 = *reinterpret_cast<const uint4*>(L.frag + frag_offset(c16, 32 + 8 * g4));
  const uint4 al1 = *reinterpret_cast<const uint4*>(L.frag + kQ * 64 + frag_offset(c16, 32 + 8 * g4));
  if (wave < hw) {
    head_scores(p, L, 1, wave, hw, lane);
  } else {
    for (int tt = wave - hw; tt < ntiles; tt += kQ - hw) {
      const int row = tt * 16 + c16;
      const uint4 b0 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, g4));
      const uint4 b1 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, 4 + g4));
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = mfma_bf16(ah0, b0, acc);
      acc = mfma_bf16(al0, b0, acc);
      acc = mfma_bf16(ah1, b1, acc);
      acc = mfma_bf16(al1, b1, acc);
      *reinterpret_cast<float4*>(L.sc + row * kSQ + 4 * g4) =
          make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
  }
  __syncthreads();  // B4: s~ and the head scores complete

  block_picks(p, L, wave, lane);
  __syncthreads();  // every query's picks are in its candidate table
  exact_select<false>(p, L, qi, lane, t, ls, anchor, L.eq + qi * kQRow, qn1, kmax, active, qrow);
}

}  // namespace

bool select_tile_layout(TileParams& p) {
  int off = 0;
  auto take = [&](int bytes) {
    const int o = off;
    off += (bytes + 15) & ~15;
    return o;
  };
  p.off_keys = take(static_cast<int>(p.T) * kRowBytes);
  p.off_sc = take(static_cast<int>(p.T) * kSQ * 4);
  p.off_stats = take(4 * p.NB * kStatRow * 4);
  p.off_rq = take(kQ * kQRow * 8);
  p.off_pq = take(kQ * kQRow * 8);
  const int list_bytes = kQ * kListCap * 8;
  const int sh_bytes = p.H * kQ * p.NB * 8;
  p.off_list = take(list_bytes > sh_bytes ? list_bytes : sh_bytes);  // per-head scores alias the lists
  p.off_blk = take(kQ * p.NB * 8);
  p.off_lmax = 0;
  p.off_top = take(2 * kQ * kTileMaxK * 8);
  p.off_qrec = take(kQ * static_cast<int>(sizeof(QRec)));
  p.off_bias = take(2 * p.H * p.RB * 8);
  p.off_sp = take(2 * 16 * 8);
  p.off_kmax = take(kQ * 4);
  p.lds_total = off;
  return off <= 160 * 1024;
}

hipError_t select_tile_launch(const TileParams& p, int stat_dtype, hipStream_t stream) {
  const dim3 block(kThreads);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles));
  const size_t lds = static_cast<size_t>(p.lds_total);
  // The LDS opt-in above 64 KiB is a per-process function attribute (set once
  // per instantiation, for the full 160 KiB).
#define RLM_TILE_CASE(TS_ID, TS, XP)                                                      \
  if (stat_dtype == TS_ID && (p.x_out != nullptr) == XP) {                                \
    static const hipError_t attr = hipFuncSetAttribute(                                   \
        reinterpret_cast<const void*>(&select_tile_kernel<TS, XP>),                       \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                          \
    if (attr != hipSuccess) {                                                             \
      set_error("relation_select (tile): cannot reserve LDS: %s", hipGetErrorString(attr)); \
      return attr;                                                                        \
    }                                                                                     \
    hipLaunchKernelGGL((select_tile_kernel<TS, XP>), grid, block, lds, stream, p);        \
    return launch_status("relation_select (tile)");                                       \
  }
  RLM_TILE_CASE(RLM_F32, float, false)
  RLM_TILE_CASE(RLM_BF16, bf16, false)
  RLM_TILE_CASE(RLM_F32, float, true)
  RLM_TILE_CASE(RLM_BF16, bf16, true)
#undef RLM_TILE_CASE
  set_error("relation_select (tile): unsupported statistics dtype %s", dtype_name(stat_dtype));
  return hipErrorInvalidValue;
}

}  // namespace rlm

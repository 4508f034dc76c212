// Routed multi-anchor selection, sequence form, for gfx950: matrix-core
// candidate scores shared by the 16 queries of a workgroup, then a float64
// verification of the few candidates that can reach each query's top-k.
//
// Reference semantics: src/relation_lm/models/multi_relation_blocks.py:69-147
// in its routed form, the same as multi_select_kernel (rlm_select.hip): S
// anchor slots per query; the anchor router picks one candidate set per query
// (local window + TOP blocks, relation_select.py:53-106, 229-284); slot s takes
// the argmax of its own exact score over the candidates not taken by slots
// < s (ties to the lowest position) and is active iff s <= t; each active
// slot's partner query is partner_base[s] + partner_anchor_cache[anchor_s, s]
// (fp32 adds), routed against the partner block statistics, and takes the
// top-k exact scores (ties to the lowest candidate lane) with every active
// anchor of the query excluded.  Numerics as multi_select_kernel's: every
// exact score is the float64 dot of the inputs rounded once to float32, block
// scores are float64 rounded once, and every comparison uses those values.
//
// Mapping.  A workgroup of 16 waves owns 16 consecutive queries of one batch
// row, one wave per query.  Keys are [B,T,S,64] (slot s's vector of position p
// at byte (p S + s) 128), too many rows to stage whole, so per routing
// (the anchor routing, then each slot's partner routing):
//   1. the statistics of the side are staged in LDS once; the per-head block
//      dots of the 16 queries run on float64 MFMA and each query's wave folds
//      the heads and ranks its TOP picks (as rlm_select_tile.hip);
//   2. the workgroup walks the 16-row key tiles that are a candidate of at
//      least one of its queries (the union of the local windows and of the
//      picked blocks), each tile read once from L2 straight into MFMA operand
//      registers and scored against the 16 queries (bf16 MFMA, fp32 sums; the
//      fp32 partner query as a bf16 hi + lo pair); each score goes to the
//      candidate lane it is for in each query's list, so a query sees exactly
//      its own candidates;
//   3. each query's wave takes theta, a lower bound of its k-th largest
//      approximate score among its valid, non-excluded candidates, and
//      verifies every candidate with s~ >= theta - 2 eps exactly in float64
//      (4 lanes per member, the key row from L2), ranking by the 64-bit
//      (score, tie) key; more than 16 members (near-ties) go in windows of 64
//      merged into a running top-k.
// eps = 2^-13 ||q||_1 max|k| bounds |s~ - s| for 64 (anchor) or 128 (partner
// hi + lo) bf16 products summed in fp32 (the bound of rlm_select_tile.hip),
// with max|k| taken over every key the workgroup scored for the routing.
#include "rlm_common.hpp"
#include "rlm_multi_tile.hpp"
#include "rlm_tile_util.hpp"

namespace rlm {
namespace {

constexpr int kMQ = 16;          // queries per workgroup
constexpr int kMWaves = 16;      // waves per workgroup: wave w owns query w
constexpr int kMThreads = kMWaves * kWave;
constexpr int kMStatRow = 68;    // floats per staged statistics row (64 + 4)
constexpr int kMQRow = 66;       // doubles per staged query row (64 + 2)
constexpr int kMListCap = 64;    // members per query per window
constexpr int kMListRow = kMListCap + 2;  // + a trash entry (branch-free stores), 16-byte rows
constexpr int kKeyRow = 128;     // bytes of one slot vector (64 bf16)

// Per-query record of the current routing.
struct MRec {
  uint64_t picks;  // bit j: block j is a valid pick
  int t, ls, on, nact;
  int pick[kMultiTileMaxTop];     // block of pick r, -1 when the pick is invalid
  int taken[kMultiTileMaxSlots];  // anchors of the active slots, in slot order
};

struct MLds {
  float* stats;       // [mean, std][NB][kMStatRow] fp32 of the current side
  // Region q (q_bytes from sc) belongs to query q: first its per-head block
  // scores sh [H][NB] (float64), then, from its block picks on, its candidate
  // list sc: s~ of each candidate lane, -inf for lanes that are not a candidate
  // or are excluded and for the padding up to a multiple of 256 lanes, then a
  // trash slot for branch-free stores (list_trash).
  float* sc;
  double* sh;
  signed char* rank;  // [16][NB]: pick rank of block j, -1 if not a valid pick
  double* rq;         // [16][kMQRow]: router query, float64
  double* eq;         // [16][kMQRow]: exact query, float64
  uint64_t* list;     // [16][kMListRow]
  uint64_t* top;      // [2][16][kMultiTileMaxK]
  MRec* qr;           // [16]
  double* bias;       // [2 sides][H*RB]
  double* sp;         // [2 sides][16]
  uint32_t* kmax;     // [kMWaves] per-wave max |key| bits
  bf16* aq;           // [16][S][64]: the queries' anchor query rows, staged once
};

// The s~ list of a query: CAP candidate lanes padded to a multiple of 256
// (read four lanes per thread, 256 at a time, with no bound checks), then the
// trash slot; 16-byte rows.
__host__ __device__ __forceinline__ int list_trash(int cap) { return (cap + 255) & ~255; }
__host__ __device__ __forceinline__ int list_floats(int cap) { return list_trash(cap) + 4; }

__device__ __forceinline__ MLds carve(const MultiTileParams& p, unsigned char* smem) {
  MLds s;
  s.stats = reinterpret_cast<float*>(smem + p.off_stats);
  s.sc = reinterpret_cast<float*>(smem + p.off_sc);
  s.sh = reinterpret_cast<double*>(smem + p.off_sc);
  s.rank = reinterpret_cast<signed char*>(smem + p.off_rank);
  s.rq = reinterpret_cast<double*>(smem + p.off_rq);
  s.eq = reinterpret_cast<double*>(smem + p.off_eq);
  s.list = reinterpret_cast<uint64_t*>(smem + p.off_list);
  s.top = reinterpret_cast<uint64_t*>(smem + p.off_top);
  s.qr = reinterpret_cast<MRec*>(smem + p.off_qrec);
  s.bias = reinterpret_cast<double*>(smem + p.off_bias);
  s.sp = reinterpret_cast<double*>(smem + p.off_sp);
  s.kmax = reinterpret_cast<uint32_t*>(smem + p.off_kmax);
  s.aq = reinterpret_cast<bf16*>(smem + p.off_aq);
  return s;
}

// One side's block statistics (mean and std, NB*64 <= 4096 elements each) into
// LDS as fp32 rows: thread tid < NB*8 (<= 512) moves 8 consecutive elements of each.
template <typename TS>
__device__ void stage_side_stats(const MultiTileParams& p, const MLds& L, int side, int64_t b,
                                 int tid) {
  const int per = p.NB * 64;
  const TS* mean = static_cast<const TS*>(side ? p.pmean : p.amean);
  const TS* stdv = static_cast<const TS*>(side ? p.pstd : p.astd);
  const bool mine = 8 * tid < per;
  const int e = mine ? 8 * tid : 0;
  float m[8], sd[8];
  load_stat8<TS>(mean + b * per + e, m);
  load_stat8<TS>(stdv + b * per + e, sd);
  if (!mine) return;
  float* dm = L.stats + (e >> 6) * kMStatRow + (e & 63);
  float* ds = L.stats + (p.NB + (e >> 6)) * kMStatRow + (e & 63);
  *reinterpret_cast<float4*>(dm) = make_float4(m[0], m[1], m[2], m[3]);
  *reinterpret_cast<float4*>(dm + 4) = make_float4(m[4], m[5], m[6], m[7]);
  *reinterpret_cast<float4*>(ds) = make_float4(sd[0], sd[1], sd[2], sd[3]);
  *reinterpret_cast<float4*>(ds + 4) = make_float4(sd[4], sd[5], sd[6], sd[7]);
}

// Bias tables and softplus(gamma) of both sides into LDS (float64).
__device__ void stage_router_consts(const MultiTileParams& p, const MLds& L, int tid) {
  const uint32_t n = static_cast<uint32_t>(p.H * p.RB);
  const uint32_t i = static_cast<uint32_t>(tid);
  const bool is_bias = i < 2 * n;
  const uint32_t kb = i < n ? i : i - n;
  const FloatWords ab = issue_float(p.abias, p.abias_dtype, n, kb, is_bias && i < n);
  const FloatWords pb = issue_float(p.pbias, p.pbias_dtype, n, kb, is_bias && i >= n);
  const uint32_t h = i < static_cast<uint32_t>(p.H) ? i : i - static_cast<uint32_t>(p.H);
  const bool is_gamma = i < 2u * static_cast<uint32_t>(p.H);
  const FloatWords ag = issue_float(p.agamma, p.agamma_dtype, static_cast<uint32_t>(p.H), h,
                                    is_gamma && i < static_cast<uint32_t>(p.H));
  const FloatWords pg = issue_float(p.pgamma, p.pgamma_dtype, static_cast<uint32_t>(p.H), h,
                                    is_gamma && i >= static_cast<uint32_t>(p.H));
  if (is_bias)
    L.bias[i] = static_cast<double>(i < n ? decode_float(ab, p.abias_dtype)
                                          : decode_float(pb, p.pbias_dtype));
  if (is_gamma) {
#pragma clang fp contract(off)
    const bool partner = i >= static_cast<uint32_t>(p.H);
    const double g = static_cast<double>(partner ? decode_float(pg, p.pgamma_dtype)
                                                 : decode_float(ag, p.agamma_dtype));
    L.sp[(partner ? 16 : 0) + h] = log(1.0 + exp(g));  // softplus without threshold, relation_select.py:87
  }
}

// Per-head block scores of the 16 queries' router queries (relation_select.py:70-96)
// on float64 MFMA, one (head, block tile) per wave, into sh[h][q][j]:
//   s_h = (sum_d mean q + softplus(gamma_h) sum_d std |q|) * HD^-0.5 + bias[h, bucket(t_q, j)].
// v_mfma_f64_16x16x4f64 takes A[i = lane%16][k = lane/16], B[k = lane/16][j = lane%16]
// and leaves D[4r + lane/16][lane%16] in register r.
__device__ void head_scores(const MultiTileParams& p, const MLds& L, int side, int wave, int lane) {
  const float* mean = L.stats;
  const float* stdv = L.stats + p.NB * kMStatRow;
  const double* sp = L.sp + 16 * side;
  const double* bias = L.bias + side * p.H * p.RB;
  const int kq = lane >> 4, c16 = lane & 15;
  const int nbt = (p.NB + 15) >> 4;
  for (int item = wave; item < p.H * nbt; item += kMWaves) {
    const int h = item / nbt;
    const int jt = item - h * nbt;
    const int j = jt * 16 + c16;
    const int jc = j < p.NB ? j : 0;
    f64x4_t content = {0.0, 0.0, 0.0, 0.0}, unc = {0.0, 0.0, 0.0, 0.0};
    for (int ks0 = 0; ks0 < p.HD; ks0 += 16) {
      double a[4];
      float bm[4], bs[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int d = h * p.HD + (ks0 + 4 * u < p.HD ? ks0 + 4 * u : 0) + kq;
        a[u] = L.rq[c16 * kMQRow + d];
        bm[u] = mean[jc * kMStatRow + d];
        bs[u] = stdv[jc * kMStatRow + d];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (ks0 + 4 * u >= p.HD) break;  // uniform
        const double m = j < p.NB ? static_cast<double>(bm[u]) : 0.0;
        const double sd = j < p.NB ? static_cast<double>(bs[u]) : 0.0;
        content = __builtin_amdgcn_mfma_f64_16x16x4f64(a[u], m, content, 0, 0, 0);
        unc = __builtin_amdgcn_mfma_f64_16x16x4f64(fabs(a[u]), sd, unc, 0, 0, 0);
      }
    }
    const int end = (j + 1) * p.BS - 1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = 4 * r + kq;
      const int t = L.qr[q].t;
      const int dist = (t > end ? t - end : 0) + 1;
      int bucket = 31 - __clz(dist);
      bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
      double v;
      {
#pragma clang fp contract(off)
        const double c = content[r] + sp[h] * unc[r];
        v = c * p.head_scale + bias[h * p.RB + bucket];
      }
      if (j < p.NB) L.sh[q * (p.q_bytes >> 3) + h * p.NB + j] = v;
    }
  }
}

// Log-sum-exp over heads (relation_select.py:97-106) of query qi's routing and
// its TOP picks by rank (block j is pick rank(j) = #{k : key_k > key_j}, key =
// (score, lower block first): the reference's sequential argmax, :229-242).
// Also the block -> pick rank map and the valid-pick mask the tile walk uses.
// Picks past the last block are block 0, invalid.  NB <= 64: one block per lane.
__device__ void block_picks(const MultiTileParams& p, const MLds& L, int qi, int lane) {
  MRec& R = L.qr[qi];
  const int t = R.t, ls = R.ls;
  const int j = lane;
  const bool live = j < p.NB;
  uint64_t kj = 0;  // lane j's block key; 0 (below every block's key) past the blocks
  {
    // Lane j: block j's heads, summed pairwise (((h0 + h1) + (h2 + h3)) + ...),
    // the order of a lane-group tree reduction over the heads (H a power of
    // two <= 8).  Four independent exps at a time.
    const double* shj = L.sh + qi * (p.q_bytes >> 3) + (live ? j : 0);
    double m = -INFINITY;
    for (int h = 0; h < p.H; ++h) m = fmax(m, shj[h * p.NB]);
    auto group4 = [&](int h0) {  // heads h0 .. h0 + 3 (those < H), tree-summed
      double x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = exp(shj[(h0 + e < p.H ? h0 + e : h0) * p.NB] - m);
      const double s01 = p.H >= 2 ? x[0] + x[1] : x[0];
      return p.H >= 4 ? s01 + (x[2] + x[3]) : s01;
    };
    double sum = group4(0);
    if (p.H == 8) sum = sum + group4(4);
    if (live) {
      const double lse = m + log(sum);
      const int end = (j + 1) * p.BS - 1;
      const bool eligible = end <= t && (!p.strict || end < ls);
      kj = select_key(eligible ? static_cast<float>(lse) : -INFINITY, static_cast<uint32_t>(j));
    }
  }
  if (lane < p.TOP) R.pick[lane] = -1;
  // The TOP largest keys.  T: the TOP-th largest score half over the blocks
  // (0 when there are fewer than TOP blocks), bit by bit from the top (a lane
  // past the blocks holds 0, below every threshold tried); then every block
  // scoring above T and the lowest blocks scoring T.
  const uint32_t sk = static_cast<uint32_t>(kj >> 32);
  uint32_t T = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    if (__builtin_popcountll(__builtin_amdgcn_ballot_w64(sk >= cand)) >= p.TOP) T = cand;
  }
  const uint64_t at_t = __builtin_amdgcn_ballot_w64(live && sk == T);
  const int above = __builtin_popcountll(__builtin_amdgcn_ballot_w64(live && sk > T));
  const int below_t = static_cast<int>(__builtin_amdgcn_mbcnt_hi(
      static_cast<uint32_t>(at_t >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(at_t), 0u)));
  const bool sel = live && (sk > T || (sk == T && below_t < p.TOP - above));
  // Pick rank of a selected block: #{k : key_k > key_j}; every such k is
  // selected, so it counts among the selected keys, gathered in the query's
  // (still unused) member list.
  const uint64_t selm = __builtin_amdgcn_ballot_w64(sel);
  const int nsel = __builtin_popcountll(selm);
  uint64_t* gathered = L.list + qi * kMListRow;
  if (sel)
    gathered[__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(selm >> 32),
                                       __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(selm), 0u))] = kj;
  wave_sync();
  int rank = 0;
#pragma unroll
  for (int f = 0; f < kMultiTileMaxTop; f += 2) {
    const uint4 kk = *reinterpret_cast<const uint4*>(gathered + f);
    rank += (f < nsel && ((static_cast<uint64_t>(kk.y) << 32) | kk.x) > kj) +
            (f + 1 < nsel && ((static_cast<uint64_t>(kk.w) << 32) | kk.z) > kj);
  }
  wave_sync();  // the pick slots are cleared
  const bool valid = sel && key_score(kj) > -1.0e30f && R.on != 0;
  if (sel) R.pick[rank] = key_score(kj) > -1.0e30f ? j : -1;
  if (live) L.rank[qi * p.NB + j] = static_cast<signed char>(valid ? rank : -1);
  const uint64_t picks = __builtin_amdgcn_ballot_w64(valid);
  if (lane == 0) R.picks = picks;
  wave_sync();
}

// Query qi's candidate list to -inf (the tile walk then files every candidate
// of the routing; a lane it does not file is not a candidate).  The list takes
// over the region of the query's per-head block scores, which only this wave's
// block_picks reads.
__device__ __forceinline__ void clear_list(const MultiTileParams& p, const MLds& L, int qi,
                                           int lane) {
  float4* row = reinterpret_cast<float4*>(L.sc + qi * (p.q_bytes >> 2));
  const float4 ninf = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  for (int i = lane; i < (p.q_bytes >> 4); i += kWave) row[i] = ninf;
}

// Position and validity of candidate lane c (relation_select.py:244-284):
// local window first, then the picks' blocks in pick order.
__device__ __forceinline__ int cand_pos(const MultiTileParams& p, const MRec& R, int c, int t,
                                        int ls, bool& valid) {
  if (c < p.L) {
    const int pos = t - p.L + 1 + c;
    valid = pos >= 0 && pos <= t && pos < p.T;
    return pos;
  }
  const int pk = R.pick[(c - p.L) >> p.BS_log2];
  const int pos = pk * p.BS + ((c - p.L) & (p.BS - 1));
  valid = pk >= 0 && pos <= t && pos < ls && pos < p.T;
  return pos;
}

// Byte offset of slot vector (b, pos, slot) in a [B,T,S,64] bf16 key cache.
__device__ __forceinline__ uint32_t key_off(const MultiTileParams& p, int64_t b, int pos, int s) {
  return static_cast<uint32_t>(((b * p.T + pos) * p.S + s) * kKeyRow);
}

// Exact float64 score of member c on 4 lanes: sub-lane sub takes dims
// [16 sub, 16 sub + 16) of the key row (from L2) and of the float64 query row
// `qrow`; the four partial sums are combined in float64.  Returns the 64-bit
// selection key (score, tie index) in the member's 4 lanes; when the score is
// not above -inf, c + 1 instead: below every selection key (whose high word is
// nonzero) and distinct per member, so such a member ranks last and counts as
// absent.
template <bool ANCHOR>
__device__ __forceinline__ uint64_t member_key(const MultiTileParams& p, const MRec& R, int c,
                                               int t, int ls, int sub, const double* qrow,
                                               rsrc_t keys, int64_t b, int s) {
  bool v;
  const int pos = cand_pos(p, R, c, t, ls, v);
  const uint32_t base = key_off(p, b, v ? pos : 0, s);
  uint4 kv[2];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch) kv[ch] = buf_load_b128(keys, base + 16u * (2 * sub + ch));
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 1
  for (int ch = 0; ch < 2; ++ch) {
    const int chunk = 2 * sub + ch;
    // A select, not kv[ch]: a runtime index would put the array in scratch memory.
    const uint4 kc = ch == 0 ? kv[0] : kv[1];
    const uint32_t w[4] = {kc.x, kc.y, kc.z, kc.w};
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
  return score > -INFINITY ? select_key(score, static_cast<uint32_t>(ANCHOR ? pos : c))
                           : static_cast<uint64_t>(c) + 1;
}

// Writes entry `slot` of output row `orow` from key `key` (high word 0: none).  Anchor:
// none is anchor 0 with score -inf (multi_relation_blocks.py:94); partner:
// none is the exhausted entry, position t - L + 1 with score -inf
// (relation_select.py:298-308).  Returns the position, -1 for none.
template <bool ANCHOR>
__device__ __forceinline__ int emit(const MultiTileParams& p, const MRec& R, int64_t orow,
                                    int slot, uint64_t key, int t, int ls) {
  int pos = ANCHOR ? 0 : t - p.L + 1;
  float score = -INFINITY;
  int found = -1;
  if ((key >> 32) != 0) {
    score = key_score(key);
    const int tie = static_cast<int>(key_index(key));
    if (ANCHOR) {
      pos = tie;
    } else {
      bool v;
      pos = cand_pos(p, R, tie, t, ls, v);
    }
    found = pos;
  }
  if (ANCHOR) {
    p.out_anchor[orow] = pos;
    p.out_anchor_score[orow] = score;
  } else {
    p.out_partner[orow * p.K + slot] = pos;
    p.out_partner_score[orow * p.K + slot] = score;
  }
  return found;
}

// Exact top-k of query qi's routing among its candidates from the s~ list,
// written to output row `orow`.  ANCHOR: k = 1, ties to the lowest position;
// else k = K, ties to the lowest candidate lane.  The record's anchors so far
// (taken[0..nact)) are not candidates.  `qrow` is the float64 query and `qn1` its L1 norm.  Returns the
// anchor position (ANCHOR; -1 for none).
template <bool ANCHOR>
__device__ int exact_select(const MultiTileParams& p, const MLds& L, int qi, int lane,
                            const double* qrow, float qn1, float kmax, rsrc_t keys, int64_t b,
                            int s, int64_t orow) {
  const MRec& R = L.qr[qi];
  const int t = R.t, ls = R.ls;
  const int K = ANCHOR ? 1 : p.K;
  float* sc = L.sc + qi * (p.q_bytes >> 2);
  // The query's anchors so far are not candidates: lane x < nact puts -inf in
  // the lane of anchor x, if it is a candidate of this routing (local window,
  // else its block's pick).  Anchors are at most t.
  if (lane < R.nact) {
    const int pos = R.taken[lane];
    int c = -1;
    if (pos >= ls) {
      c = pos - (t - p.L + 1);
    } else {
      const int r = L.rank[qi * p.NB + (pos >> p.BS_log2)];
      if (r >= 0) c = p.L + r * p.BS + (pos & (p.BS - 1));
    }
    if (c >= 0) sc[c] = -INFINITY;
  }
  wave_sync();
  // The list in quads: lane l reads candidates 256 j + 4 l + e (e < 4); the
  // padding past CAP reads -inf.
  const int nquad = list_trash(p.CAP) >> 8;
  auto quad = [&](int j, float (&x)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(sc + 256 * j + 4 * lane);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  };
  float lm = -INFINITY;
  for (int j = 0; j < nquad; ++j) {
    float x[4];
    quad(j, x);
    lm = fmaxf(fmaxf(lm, fmaxf(x[0], x[1])), fmaxf(x[2], x[3]));
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
  // Members (candidates with s~ >= thr) numbered in candidate order; those of
  // window [lo, lo + 64) go to the list (others to its trash entry).
  uint64_t* list = L.list + qi * kMListRow;
  auto list_members = [&](int lo) {
    int n = 0;
    for (int j = 0; j < nquad; ++j) {
      float x[4];
      quad(j, x);
      bool mem[4];
      uint64_t bal[4];
      int mi = n, tot = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        mem[e] = x[e] > -INFINITY && x[e] >= thr;
        bal[e] = __builtin_amdgcn_ballot_w64(mem[e]);
        mi += static_cast<int>(__builtin_amdgcn_mbcnt_hi(
            static_cast<uint32_t>(bal[e] >> 32),
            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[e]), 0u)));
        tot += __builtin_popcountll(bal[e]);
      }
      // mi: members in the lanes below; then this lane's, in e order.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (bal[e] != 0)  // uniform
          list[mem[e] && mi >= lo && mi < lo + kMListCap ? mi - lo : kMListCap] =
              static_cast<uint64_t>(256 * j + 4 * lane + e);
        mi += mem[e];
      }
      n += tot;
    }
    return n;
  };
  const int members = list_members(0);
  const int sub = lane & 3;
  int anchor = -1;

  if (members <= 16) {
    // Every member scored in one pass (4 lanes each), ranked, emitted.
    wave_sync();
    {
      const int m = lane >> 2;
      const bool act = m < members;
      const int c = act ? static_cast<int>(list[m]) : 0;
      const uint64_t key = member_key<ANCHOR>(p, R, c, t, ls, sub, qrow, keys, b, s);
      if (act && sub == 0) list[m] = key;
    }
    wave_sync();
    int rank = kWave;
    uint64_t ke = 0;
    if (lane < members) {
      ke = list[lane];
      rank = 0;
#pragma unroll 2
      for (int f = 0; f < 16; f += 2) {
        const uint4 kk = *reinterpret_cast<const uint4*>(list + f);
        const uint64_t k0 = (static_cast<uint64_t>(kk.y) << 32) | kk.x;
        const uint64_t k1 = (static_cast<uint64_t>(kk.w) << 32) | kk.z;
        rank += (f < members && k0 > ke) + (f + 1 < members && k1 > ke);
      }
    }
    int mine = -1;
    if (rank < K) mine = emit<ANCHOR>(p, R, orow, rank, ke, t, ls);
    if (lane >= members && lane < K) emit<ANCHOR>(p, R, orow, lane, 0, t, ls);
    if (ANCHOR) anchor = wave_max_i(rank == 0 ? mine : -1);
    wave_sync();
    return anchor;
  }

  // Many members (near-ties): windows of 64 merged into a running top-k.
  const int nwin = (members + kMListCap - 1) / kMListCap;
  int ntop = 0;
  int cur = 0;
  for (int w = 0; w < nwin; ++w) {
    const int lo = w * kMListCap;
    const int nw = min(members - lo, kMListCap);
    if (w > 0) list_members(lo);  // window 0 is in the list already
    wave_sync();
    for (int m0 = 0; m0 < nw; m0 += 16) {
      const int m = m0 + (lane >> 2);
      const bool act = m < nw;
      const int c = act ? static_cast<int>(list[m]) : 0;
      const uint64_t key = member_key<ANCHOR>(p, R, c, t, ls, sub, qrow, keys, b, s);
      if (act && sub == 0) list[m] = key;
    }
    wave_sync();
    const uint64_t* topc = L.top + (cur * kMQ + qi) * kMultiTileMaxK;
    uint64_t* topn = L.top + ((cur ^ 1) * kMQ + qi) * kMultiTileMaxK;
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
  const uint64_t* topf = L.top + (cur * kMQ + qi) * kMultiTileMaxK;
  if (lane < K) emit<ANCHOR>(p, R, orow, lane, lane < ntop ? topf[lane] : 0, t, ls);
  if (ANCHOR && ntop > 0 && (topf[0] >> 32) != 0) anchor = static_cast<int>(key_index(topf[0]));
  wave_sync();
  return anchor;
}

// The union of the workgroup's candidate rows for the current routing: the
// local windows [min ls, max t] and the valid picked blocks of every query
// whose routing is on.  Lane l reads query l % 16's record and DPP row steps
// combine the 16 (every row holds the same copies); wave-uniform result.
struct Union {
  int lo, hi;
  uint64_t picks;
};
template <int CTRL>
__device__ __forceinline__ void union_step(uint32_t& nlo, uint32_t& hi1, uint32_t& plo,
                                           uint32_t& phi) {
  nlo = umax32(nlo, dpp_u32<CTRL>(nlo));
  hi1 = umax32(hi1, dpp_u32<CTRL>(hi1));
  plo |= dpp_u32<CTRL>(plo);
  phi |= dpp_u32<CTRL>(phi);
}
__device__ __forceinline__ Union candidate_union(const MultiTileParams& p, const MLds& L,
                                                 int lane) {
  const MRec& R = L.qr[lane & 15];
  const bool on = R.on != 0;
  uint32_t nlo = ~static_cast<uint32_t>(on ? R.ls : 1 << 30);  // max of ~ls: min of ls
  uint32_t hi1 = on ? static_cast<uint32_t>(R.t + 1) : 0u;
  uint32_t plo = on ? static_cast<uint32_t>(R.picks) : 0u;
  uint32_t phi = on ? static_cast<uint32_t>(R.picks >> 32) : 0u;
  union_step<kDppXor1>(nlo, hi1, plo, phi);
  union_step<kDppXor2>(nlo, hi1, plo, phi);
  union_step<kDppHalfMirror>(nlo, hi1, plo, phi);
  union_step<kDppMirror>(nlo, hi1, plo, phi);
  Union u;
  u.lo = static_cast<int>(~__builtin_amdgcn_readfirstlane(nlo));
  u.hi = min(static_cast<int>(__builtin_amdgcn_readfirstlane(hi1)) - 1, static_cast<int>(p.T) - 1);
  u.picks = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(phi)) << 32) |
            __builtin_amdgcn_readfirstlane(plo);
  return u;
}

// Scores every candidate tile of the union `u` against the 16 queries and files
// each score under its candidate lane of each query.  The product is
// D[position][query] = keys (A, row lane%16) x queries (B, column lane%16):
// lane l holds positions 4 (l/16) .. +3 of the tile for query l%16, so it
// files scores for one query only.  The query fragments are given; PAIR: the
// hi/lo pair of an fp32 query.  Returns this wave's max |key| bits over the
// tiles it read.
template <bool PAIR>
__device__ uint32_t score_tiles(const MultiTileParams& p, const MLds& L, rsrc_t keys, int64_t b,
                                int s, const uint4& ah0, const uint4& al0, const uint4& ah1,
                                const uint4& al1, const Union& u, int wave, int lane) {
  const int c16 = lane & 15, g4 = lane >> 4;
  // The query this lane files scores for.
  const MRec& R = L.qr[c16];
  const int tq = R.on ? R.t : -1;  // no candidates when the routing is off
  const int lq = R.ls;
  const signed char* rank = L.rank + c16 * p.NB;
  float* sc = L.sc + c16 * (p.q_bytes >> 2);
  const int trash = list_trash(p.CAP);
  u16x2_t km = {0, 0};
  const int ntiles = (u.hi + 16) >> 4;
  // The union's tiles numbered in position order, 64 tiles per group; tile
  // number i goes to wave i % 16, so every wave walks its share of the union
  // only.  next_tile() returns this wave's next tile (wave-uniform), -1 at the end.
  const int ngroups = (ntiles + 63) >> 6;
  int grp = -1, base = 0;
  uint64_t mine = 0;
  auto next_tile = [&]() -> int {
    while (mine == 0) {
      if (grp + 1 >= ngroups) return -1;
      ++grp;
      const int tt = 64 * grp + lane;
      const int p0 = tt * 16;
      const bool rel = tt < ntiles && ((p0 + 15 >= u.lo && p0 <= u.hi) ||
                                       ((u.picks >> ((p0 >> p.BS_log2) & 63)) & 1u));
      const uint64_t in_union = __builtin_amdgcn_ballot_w64(rel);
      const int idx = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                 static_cast<uint32_t>(in_union >> 32),
                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(in_union), 0u)));
      mine = __builtin_amdgcn_ballot_w64(rel && (idx & (kMWaves - 1)) == wave);
      base += __builtin_popcountll(in_union);
    }
    const int k = static_cast<int>(__builtin_ctzll(mine));
    mine &= mine - 1;
    return 64 * grp + k;
  };
  // kTB tiles per round: every key load of the round is issued before the
  // first product.
  constexpr int kTB = 2;
  for (bool more = true; more;) {
    int tl[kTB];
    uint4 b0[kTB], b1[kTB];
#pragma unroll
    for (int v = 0; v < kTB; ++v) {
      tl[v] = (v == 0 || tl[v - 1] >= 0) ? next_tile() : -1;
      const uint32_t off = tl[v] >= 0 ? key_off(p, b, tl[v] * 16 + c16, s) + 16u * g4 : kNoOffset;
      b0[v] = buf_load_b128(keys, off);
      b1[v] = buf_load_b128(keys, tl[v] >= 0 ? off + 64u : kNoOffset);
    }
    more = tl[kTB - 1] >= 0;
#pragma unroll
    for (int v = 0; v < kTB; ++v) {
      if (tl[v] < 0) break;  // uniform
      const int p0 = tl[v] * 16;
      km = absmax8(b1[v], absmax8(b0[v], km));
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = mfma_bf16(b0[v], ah0, acc);
      if (PAIR) acc = mfma_bf16(b0[v], al0, acc);
      acc = mfma_bf16(b1[v], ah1, acc);
      if (PAIR) acc = mfma_bf16(b1[v], al1, acc);
      // Candidate lane of position pb + e: local window from e >= lq - pb on,
      // else the block's pick (an unpicked block: the trash slots after the
      // list); past tq, the trash slot.
      const int pb = p0 + 4 * g4;
      const int r = rank[p0 >> p.BS_log2];
      const int local0 = pb - (tq - p.L + 1);
      const int pick0 = r >= 0 ? p.L + r * p.BS + (pb & (p.BS - 1)) : trash;
      const int dl = lq - pb, dv = tq - pb;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sc[e <= dv ? (e >= dl ? local0 : pick0) + e : trash] = acc[e];
    }
  }
  return wave_max_u32(umax32(km.x, km.y));
}

__device__ __forceinline__ float routing_kmax(const MLds& L) {
  uint32_t kb = 0;
#pragma unroll
  for (int w = 0; w < kMWaves; ++w) kb = umax32(kb, L.kmax[w]);
  return __uint_as_float(kb << 16) * (1.0f + 1.0f / 1024.0f);
}

template <typename TS>
__global__ void __launch_bounds__(kMThreads) multi_tile_kernel(const MultiTileParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const MLds L = carve(p, smem);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  // Block i takes the i-th most expensive query tile (later positions route
  // more candidates): batch rows interleaved, positions descending.  Blocks go
  // to the 8 XCDs in turn, so every XCD gets the same mix of positions, the
  // costliest tiles start first, and with 4 or 8 batch rows each XCD reads one
  // row's keys.
  const int64_t b = static_cast<int64_t>(blockIdx.x) % p.B;
  const int64_t tq0 = (p.tiles - 1 - static_cast<int64_t>(blockIdx.x) / p.B) * kMQ;
  const rsrc_t akeys = make_rsrc(p.akeys, p.key_bytes);
  const rsrc_t pkeys = make_rsrc(p.pkeys, p.key_bytes);
  // Query qi = wave + kMWaves h of the workgroup: its row and whether it exists.
  auto query_row = [&](int qi, bool& active) {
    active = tq0 + qi < p.Tq;
    return b * p.Tq + (active ? tq0 + qi : tq0);
  };
  auto l1_norm = [&](int qi) {  // ||q||_1 of the staged exact query, covering fp32 rounding
    return wave_sum_f32(fabsf(static_cast<float>(L.eq[qi * kMQRow + lane]))) * (1.0f + 1.0f / 1024.0f);
  };

  // ---- Anchor routing: positions, router queries, statistics. ----
  stage_side_stats<TS>(p, L, 0, b, tid);
  stage_router_consts(p, L, tid);
  {
    // Every slot's anchor query row of the 16 queries (S 128-byte rows per
    // query, contiguous), 16 bytes per thread.
    const int per = p.S * 8;
    for (int i = tid; i < kMQ * per; i += kMThreads) {
      const int qi = i / per;
      bool active;
      const int64_t qrow = query_row(qi, active);
      reinterpret_cast<uint4*>(L.aq + qi * p.S * 64)[i - qi * per] =
          reinterpret_cast<const uint4*>(p.aq + qrow * p.S * 64)[i - qi * per];
    }
  }
#pragma unroll
  for (int h = 0; h < kMQ / kMWaves; ++h) {
    const int qi = wave + kMWaves * h;
    bool active;
    const int64_t qrow = query_row(qi, active);
    const IndexWords pw = issue_index(p.pos, p.pos_dtype, static_cast<uint32_t>(p.pos_count),
                                      static_cast<uint32_t>(b * p.pos_sb + (qrow - b * p.Tq) * p.pos_sq),
                                      true);
    L.rq[qi * kMQRow + lane] = static_cast<double>(to_f32(p.arq[qrow * 64 + lane]));
    const int t = clamp_pos(decode_index(pw, p.pos_dtype));
    if (lane == 0) {
      L.qr[qi].t = t;
      L.qr[qi].ls = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
      L.qr[qi].on = active ? 1 : 0;
      L.qr[qi].nact = 0;
    }
  }
  __syncthreads();
  head_scores(p, L, 0, wave, lane);
  __syncthreads();
  for (int h = 0; h < kMQ / kMWaves; ++h) {
    block_picks(p, L, wave + kMWaves * h, lane);
    clear_list(p, L, wave + kMWaves * h, lane);  // the anchor slots share one candidate set
  }
  __syncthreads();
  const Union anchor_union = candidate_union(p, L, lane);

  // ---- Anchor slots: distinct argmaxes over the one candidate set. ----
  for (int s = 0; s < p.S; ++s) {
    if (s > 0) __syncthreads();  // every wave is done with the previous slot's scores
    for (int h = 0; h < kMQ / kMWaves; ++h) {
      const int qi = wave + kMWaves * h;
      L.eq[qi * kMQRow + lane] = static_cast<double>(to_f32(L.aq[(qi * p.S + s) * 64 + lane]));
    }
    const bf16* arow = L.aq + (c16 * p.S + s) * 64;
    const uint4 a0 = *reinterpret_cast<const uint4*>(arow + 8 * g4);
    const uint4 a1 = *reinterpret_cast<const uint4*>(arow + 32 + 8 * g4);
    const uint32_t kb = score_tiles<false>(p, L, akeys, b, s, a0, a0, a1, a1, anchor_union, wave, lane);
    if (lane == 0) L.kmax[wave] = kb;
    __syncthreads();
    const float kmax = routing_kmax(L);
    for (int h = 0; h < kMQ / kMWaves; ++h) {
      const int qi = wave + kMWaves * h;
      bool active;
      const int64_t qrow = query_row(qi, active);
      const int64_t orow = qrow * p.S + s;
      if (!active) continue;
      if (s > L.qr[qi].t) {  // inactive slot: anchor 0, no partners (multi_relation_blocks.py:84, 94)
        if (lane == 0) {
          p.out_anchor[orow] = 0;
          p.out_anchor_score[orow] = -INFINITY;
        }
        continue;
      }
      const int anchor = exact_select<true>(p, L, qi, lane, L.eq + qi * kMQRow, l1_norm(qi), kmax,
                                            akeys, b, s, orow);
      if (anchor >= 0 && lane == 0) {
        MRec& R = L.qr[qi];
        R.taken[R.nact] = anchor;
        R.nact = R.nact + 1;
      }
      wave_sync();
    }
  }

  // ---- Partner routing of each active slot. ----
  // Partner query of slot s (wave w's query w): the fp32 sum of its query-side
  // row and the anchor's cached row.  Lane l holds elements l and 64 + l of
  // both rows; slot s + 1's are loaded while slot s runs.
  static_assert(kMQ == kMWaves, "one query per wave");
  bool pactive;
  const int64_t prow = query_row(wave, pactive);
  auto partner_rows = [&](int s, bf16 (&v)[4]) {
    const bool on = pactive && s < L.qr[wave].nact;
    const int anchor = on ? L.qr[wave].taken[s] : 0;
    const bf16* pb = p.pbase + (prow * p.S + s) * 128;
    const bf16* pc = p.pcache + ((b * p.T + anchor) * p.S + s) * 128;
    v[0] = pb[lane];
    v[1] = pc[lane];
    v[2] = pb[64 + lane];
    v[3] = pc[64 + lane];
  };
  __syncthreads();  // every wave is done with the anchor side's LDS
  bf16 next_rows[4];
  partner_rows(0, next_rows);
  stage_side_stats<TS>(p, L, 1, b, tid);
  for (int s = 0; s < p.S; ++s) {
    {
      const bf16 rows[4] = {next_rows[0], next_rows[1], next_rows[2], next_rows[3]};
      if (s + 1 < p.S) partner_rows(s + 1, next_rows);
      L.eq[wave * kMQRow + lane] = static_cast<double>(to_f32(rows[0]) + to_f32(rows[1]));
      L.rq[wave * kMQRow + lane] = static_cast<double>(to_f32(rows[2]) + to_f32(rows[3]));
      if (lane == 0) L.qr[wave].on = pactive && s < L.qr[wave].nact ? 1 : 0;
    }
    __syncthreads();  // query rows, statistics; previous slot's lists done
    head_scores(p, L, 1, wave, lane);
    __syncthreads();
    for (int h = 0; h < kMQ / kMWaves; ++h) {
      block_picks(p, L, wave + kMWaves * h, lane);
      clear_list(p, L, wave + kMWaves * h, lane);
    }
    __syncthreads();
    uint4 ah0, al0, ah1, al1;
    {
      const double* src = L.eq + c16 * kMQRow;
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = static_cast<float>(src[8 * g4 + e]);
      split_hi_lo(x, ah0, al0);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = static_cast<float>(src[32 + 8 * g4 + e]);
      split_hi_lo(x, ah1, al1);
    }
    const uint32_t kb = score_tiles<true>(p, L, pkeys, b, s, ah0, al0, ah1, al1, candidate_union(p, L, lane),
                                         wave, lane);
    if (lane == 0) L.kmax[wave] = kb;
    __syncthreads();
    const float kmax = routing_kmax(L);
    for (int h = 0; h < kMQ / kMWaves; ++h) {
      const int qi = wave + kMWaves * h;
      bool active;
      const int64_t qrow = query_row(qi, active);
      const int64_t orow = qrow * p.S + s;
      if (L.qr[qi].on) {
        exact_select<false>(p, L, qi, lane, L.eq + qi * kMQRow, l1_norm(qi), kmax, pkeys, b, s,
                            orow);
      } else if (active) {  // inactive (or anchorless) slot: every entry exhausted
        for (int k = lane; k < p.K; k += kWave) {
          p.out_partner[orow * p.K + k] = L.qr[qi].t - p.L + 1;
          p.out_partner_score[orow * p.K + k] = -INFINITY;
        }
      }
    }
  }
}

}  // namespace

bool multi_tile_layout(MultiTileParams& p) {
  int off = 0;
  auto take = [&](int bytes) {
    const int o = off;
    off += (bytes + 15) & ~15;
    return o;
  };
  p.off_stats = take(2 * p.NB * kMStatRow * 4);
  // Per query: its per-head block scores, then its candidate list.
  const int sc_bytes = list_floats(p.CAP) * 4;
  const int sh_bytes = p.H * p.NB * 8;
  p.q_bytes = ((sc_bytes > sh_bytes ? sc_bytes : sh_bytes) + 15) & ~15;
  p.off_sc = take(kMQ * p.q_bytes);
  p.off_rank = take(kMQ * p.NB);
  p.off_rq = take(kMQ * kMQRow * 8);
  p.off_eq = take(kMQ * kMQRow * 8);
  p.off_list = take(kMQ * kMListRow * 8);
  p.off_top = take(2 * kMQ * kMultiTileMaxK * 8);
  p.off_qrec = take(kMQ * static_cast<int>(sizeof(MRec)));
  p.off_bias = take(2 * p.H * p.RB * 8);
  p.off_sp = take(2 * 16 * 8);
  p.off_kmax = take(kMWaves * 4);
  p.off_aq = take(kMQ * p.S * 64 * 2);
  p.lds_total = off;
  return off <= 160 * 1024;
}

hipError_t multi_tile_launch(const MultiTileParams& p, int stat_dtype, hipStream_t stream) {
  const dim3 block(kMThreads);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles));
  const size_t lds = static_cast<size_t>(p.lds_total);
#define RLM_MTILE_CASE(TS_ID, TS)                                                          \
  if (stat_dtype == TS_ID) {                                                               \
    static const hipError_t attr = hipFuncSetAttribute(                                    \
        reinterpret_cast<const void*>(&multi_tile_kernel<TS>),                             \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                           \
    if (attr != hipSuccess) {                                                              \
      set_error("multi_relation_select (tile): cannot reserve LDS: %s",                    \
                hipGetErrorString(attr));                                                  \
      return attr;                                                                         \
    }                                                                                      \
    hipLaunchKernelGGL((multi_tile_kernel<TS>), grid, block, lds, stream, p);              \
    return launch_status("multi_relation_select (tile)");                                  \
  }
  RLM_MTILE_CASE(RLM_F32, float)
  RLM_MTILE_CASE(RLM_BF16, bf16)
#undef RLM_MTILE_CASE
  set_error("multi_relation_select (tile): unsupported statistics dtype %s",
            dtype_name(stat_dtype));
  return hipErrorInvalidValue;
}

}  // namespace rlm

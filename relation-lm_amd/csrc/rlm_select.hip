// Routed selection for gfx950: block scoring, exact top-1 anchor, factorized
// partner query, partner block routing and exact top-k partners.
//
// Reference semantics: src/relation_lm/kernels/relation_select.py:9-308 (packed)
// and src/relation_lm/kernels/triton_select.py:9-252 (two-op form).
//
// Mapping.  A workgroup holds up to W queries of one batch row, one wavefront
// per query (W = 8 consecutive positions for the sequence form, 1 for the
// decode form).  The workgroup first stages, in one round of loads, what its
// queries share: the block statistics of both streams and the union of their
// local key windows (rows [t0-L+1, t0+W-1]).  Each wave then runs the
// reference's chain for its query -- block scores, TOP block picks, exact
// candidate scores, argmax -- with every reduction inside the wave.
//
// Exact scores: one lane per candidate (3 candidates per lane per pass at
// CAP = 192): the lane streams its candidate's key row in 16-byte chunks --
// local-window rows from the staged LDS window, picked remote blocks from L2
// through a buffer descriptor (out-of-range rows read as zero) -- and
// accumulates the dot with the query, held in float64 registers, in float64.
//
// Numerics: every dot product is accumulated in float64 from exact products
// and rounded once to float32; block scores (softplus, per-head terms, the
// log-sum-exp over heads, m + log(sum_h exp(s_h - m))) are evaluated in
// float64 and rounded once.  The reference combines heads pairwise in float32
// (relation_select.py:97-103); in float64 the one-shot and pairwise forms
// agree far below a float32 ulp.  All comparisons use those float32 values.
// Ties: anchor -> lowest position, blocks -> lowest block, partners -> lowest
// candidate lane (local window first, then picked blocks in pick order).
// Each rule is one 64-bit key (order-preserving score bits above the
// complemented tie index), so one wave max-reduction yields the winner.
#include <cstdlib>

#include "rlm_common.hpp"
#include "rlm_multi_tile.hpp"
#include "rlm_select_decode.hpp"
#include "rlm_select_tile.hpp"

namespace rlm {
namespace {

enum SelectMode { kPacked = 0, kAnchorOnly = 1, kPartnerOnly = 2 };

struct Stream {
  const void* keys;   // [B,T,E] activation dtype
  const void* mean;   // [B,NB,H,HD] stat dtype
  const void* stdev;  // [B,NB,H,HD] stat dtype
  const void* gamma;  // [H]
  const void* bias;   // [H,RB]
  int gamma_dtype;
  int bias_dtype;
};

struct SelectParams {
  int64_t B, Tq, T;
  int NB, BS, E, H, HD, RB, L, TOP, K, CAP;
  int strict;
  double exact_scale, head_scale;
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  // anchor side
  const void* aq;   // [B*Tq, E]
  const void* arq;  // [B*Tq, RD]
  Stream as;
  // partner side: exact / router query rows (row strides in elements), plus
  // the cached anchor-side contribution [B,T,2E] for the packed form.
  const void* pq;
  int64_t pq_row;
  const void* prq;
  int64_t prq_row;
  const void* pcache;
  Stream ps;
  const void* anchor_in;
  int anchor_dtype;
  // outputs
  int32_t* out_anchor;
  float* out_anchor_score;
  int32_t* out_partner;
  float* out_partner_score;
  // launch geometry and LDS layout (bytes)
  int W;            // queries per workgroup
  int split;        // waves per query (W == 1 only): candidate scoring split over them
  int tiles;        // workgroups per batch row
  int G;            // lanes per key row (E * sizeof / 16)
  int H_log2;       // heads is a power of two
  int BS_log2;      // block size is a power of two
  int G_log2;
  int WR;           // rows of each staged local-key window
  int row_bytes;    // LDS bytes per staged key row (padded by 16)
  int stage;        // statistics, bias tables and windows staged in LDS (W > 1)
  int off_stats_a, off_stats_p, off_bias_a, off_bias_p, off_win_a, off_win_p;
  int off_wave, wave_bytes, lds_total;
  uint32_t key_bytes;  // byte size of each key cache (range of the buffer descriptors)
};

// Per-wave LDS region: f64 exact query [E] and router query [RD], then f32
// block scores [NB], picks [TOP] and their validity [TOP], candidate scores [CAP].
inline int wave_region_bytes(int E, int NB, int RD, int TOP, int CAP) {
  const int bytes = 8 * (E + RD) + 4 * (NB + 2 * TOP + CAP);
  return (bytes + 15) & ~15;
}

template <typename TA>
__device__ __forceinline__ void chunk_to_f64(const uint4& v, double* out);
template <>
__device__ __forceinline__ void chunk_to_f64<bf16>(const uint4& v, double* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = static_cast<double>(__uint_as_float(w[i] << 16));
    out[2 * i + 1] = static_cast<double>(__uint_as_float(w[i] & 0xffff0000u));
  }
}
template <>
__device__ __forceinline__ void chunk_to_f64<f16>(const uint4& v, double* out) {
  const f16* h = reinterpret_cast<const f16*>(&v);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<double>(static_cast<float>(h[i]));
}
template <>
__device__ __forceinline__ void chunk_to_f64<float>(const uint4& v, double* out) {
  out[0] = static_cast<double>(__uint_as_float(v.x));
  out[1] = static_cast<double>(__uint_as_float(v.y));
  out[2] = static_cast<double>(__uint_as_float(v.z));
  out[3] = static_cast<double>(__uint_as_float(v.w));
}

// Elements of TA per 16-byte chunk.
template <typename TA>
constexpr int kEpc = 16 / static_cast<int>(sizeof(TA));

// Group max over aligned groups of G lanes (G a power of two <= 64).
__device__ __forceinline__ double group_max_f64(double v, int G) {
  if (G >= 2) v = fmax(v, dpp_f64<kDppXor1>(v));
  if (G >= 4) v = fmax(v, dpp_f64<kDppXor2>(v));
  if (G >= 8) v = fmax(v, dpp_f64<kDppHalfMirror>(v));
  if (G >= 16) v = fmax(v, dpp_f64<kDppMirror>(v));
  if (G >= 32) v = fmax(v, __shfl_xor(v, 16, kWave));
  if (G >= 64) v = fmax(v, __shfl_xor(v, 32, kWave));
  return v;
}

struct WaveScratch {
  double* qx;    // [E]
  double* qr;    // [RD]
  float* blk;    // [NB]
  int* sel;      // [TOP]
  int* selv;     // [TOP]
  float* sc;     // [CAP]
};

struct Query {
  int64_t b, q, t, local_start;
  int64_t wbase;  // first position of the staged windows
};

// Ring-buffer caches of T rows: position p lives in row p mod T, and
// statistics slot j holds the newest absolute block jb <= t/BS with
// jb = j (mod NB) -- negative when no such block has been written.  Every
// block from t/BS - NB + 1 on is wholly resident, so eligibility and distance
// follow the linear rules on jb.
__device__ __forceinline__ int ring_block(const SelectParams& p, const Query& qy, int j) {
  const int cur = static_cast<int>(qy.t >> p.BS_log2);
  return cur - ((cur - j) & (p.NB - 1));
}

// Block scores of one stream (relation_select.py:53-106) into ws.blk[NB]
// (float32, -inf where not eligible).  Lane = (block j, head h) pair, heads of
// a block in consecutive lanes:
//   s_h = (sum_d mean*q_h + softplus(gamma_h) * sum_d std*|q_h|) * HD^-0.5 + bias[h, bucket]
// then log-sum-exp over the block's H lanes, m + log(sum_h exp(s_h - m)), with
// DPP group reductions.  All in float64, rounded once.  Statistics and bias
// come from LDS when the workgroup staged them, else from L2.  `sp` is
// softplus(gamma_h) for this lane's head h = lane mod H.
template <typename TS, bool RING = false, bool PRELOAD = false>
__device__ void block_scores(const SelectParams& p, const Stream& s, const float* stats,
                             const float* bias_tab, double sp, const Query& qy, WaveScratch& ws,
                             int lane) {
  const int pairs = p.NB * p.H;
  const int RD = p.H * p.HD;
  for (int base = 0; base < pairs; base += kWave) {
    const int pr = base + lane;
    const bool live = pr < pairs;
    const int prc = live ? pr : 0;
    const int j = prc >> p.H_log2;
    const int h = prc & (p.H - 1);
    const double* qh = ws.qr + h * p.HD;
    double c = 0.0, u = 0.0;
    if (stats != nullptr) {
      const float* mr = stats + prc * p.HD;
      const float* sr = stats + p.NB * RD + prc * p.HD;
      for (int d = 0; d < p.HD; d += 4) {
        const float4 m = *reinterpret_cast<const float4*>(mr + d);
        const float4 sd = *reinterpret_cast<const float4*>(sr + d);
        c += static_cast<double>(m.x) * qh[d] + static_cast<double>(m.y) * qh[d + 1] +
             static_cast<double>(m.z) * qh[d + 2] + static_cast<double>(m.w) * qh[d + 3];
        u += static_cast<double>(sd.x) * fabs(qh[d]) + static_cast<double>(sd.y) * fabs(qh[d + 1]) +
             static_cast<double>(sd.z) * fabs(qh[d + 2]) + static_cast<double>(sd.w) * fabs(qh[d + 3]);
      }
    } else {
      const TS* mr = static_cast<const TS*>(s.mean) + (qy.b * pairs + prc) * p.HD;
      const TS* sr = static_cast<const TS*>(s.stdev) + (qy.b * pairs + prc) * p.HD;
      // PRELOAD (decode) and head dims up to 16: every statistics load of the
      // lane is issued before the first is used (chunks past HD re-read chunk
      // 0 and are not summed); otherwise the loop below.
      constexpr int kQ = 4;
      const int hd_pre = PRELOAD && p.HD <= 4 * kQ ? p.HD : 0;  // wave-uniform
      float4 mq[kQ], sq[kQ];
#pragma unroll
      for (int q = 0; q < (PRELOAD ? kQ : 0); ++q) {
        const int d = 4 * q < hd_pre ? 4 * q : 0;
        mq[q] = load4(mr + d);
        sq[q] = load4(sr + d);
      }
      // Every chunk is used (a select drops those past HD): a load used only
      // under a condition would be sunk into that branch and waited for there.
#pragma unroll
      for (int q = 0; q < (PRELOAD ? kQ : 0); ++q) {
        const bool use = 4 * q < hd_pre;
        const int d = use ? 4 * q : 0;
        const float4 m = mq[q], sd = sq[q];
        const double cq = static_cast<double>(m.x) * qh[d] + static_cast<double>(m.y) * qh[d + 1] +
                          static_cast<double>(m.z) * qh[d + 2] + static_cast<double>(m.w) * qh[d + 3];
        const double uq = static_cast<double>(sd.x) * fabs(qh[d]) + static_cast<double>(sd.y) * fabs(qh[d + 1]) +
                          static_cast<double>(sd.z) * fabs(qh[d + 2]) + static_cast<double>(sd.w) * fabs(qh[d + 3]);
        c += use ? cq : 0.0;
        u += use ? uq : 0.0;
      }
      for (int d = hd_pre == 0 ? 0 : p.HD; d < p.HD; d += 4) {
        const float4 m = load4(mr + d);
        const float4 sd = load4(sr + d);
        c += static_cast<double>(m.x) * qh[d] + static_cast<double>(m.y) * qh[d + 1] +
             static_cast<double>(m.z) * qh[d + 2] + static_cast<double>(m.w) * qh[d + 3];
        u += static_cast<double>(sd.x) * fabs(qh[d]) + static_cast<double>(sd.y) * fabs(qh[d + 1]) +
             static_cast<double>(sd.z) * fabs(qh[d + 2]) + static_cast<double>(sd.w) * fabs(qh[d + 3]);
      }
    }
    const int jb = RING ? ring_block(p, qy, j) : j;  // absolute block held by slot j
    const int end = (jb + 1) * p.BS - 1;
    const int dist = (qy.t > end ? static_cast<int>(qy.t - end) : 0) + 1;
    int bucket = 31 - __clz(dist);
    bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
    // Unstaged: both dtype forms are loaded and one is kept (no branch, so the
    // load is not waited for on its own).
    double bias;
    if constexpr (PRELOAD)
      bias = bias_tab != nullptr
                 ? bias_tab[h * p.RB + bucket]
                 : decode_float(issue_float(s.bias, s.bias_dtype, static_cast<uint32_t>(p.H * p.RB),
                                            static_cast<uint32_t>(h * p.RB + bucket), true),
                                s.bias_dtype);
    else
      bias = bias_tab != nullptr ? bias_tab[h * p.RB + bucket]
                                 : load_any_f(s.bias, s.bias_dtype, h * p.RB + bucket);
    double sv;
    {
#pragma clang fp contract(off)
      const double content = c + sp * u;
      sv = live ? content * p.head_scale + bias : 0.0;
    }
    const double m = group_max_f64(sv, p.H);
    const double sum = group_sum_f64(exp(sv - m), p.H);
    if (live && h == 0) {
      const double lse = m + log(sum);
      const bool eligible = jb >= 0 && end <= qy.t && (!p.strict || end < qy.local_start);
      ws.blk[j] = eligible ? static_cast<float>(lse) : -INFINITY;
    }
  }
  wave_sync();
}

// The TOP picks of the reference's sequential argmax loop (ties to the lowest
// block; a pick is valid iff its value is > -1e30, relation_select.py:229-242),
// found by ranking: block j is pick number rank(j) = #{k : key_k > key_j}.
// Picks past the last block repeat block 0 as invalid, as the reference's
// argmax over an all -inf vector does.  NB <= 64: block scores are held one
// per lane and broadcast with readlane; larger NB reads them from LDS.
template <bool RING = false>
__device__ void pick_blocks(const SelectParams& p, const Query& qy, WaveScratch& ws, int lane) {
  for (int r = lane; r < p.TOP; r += kWave) {
    ws.sel[r] = 0;
    ws.selv[r] = 0;
  }
  wave_sync();
  if (p.NB <= kWave) {
    // Ties rank by block id: the slot, or for ring caches the absolute block.
    const float mine = lane < p.NB ? ws.blk[lane] : -INFINITY;
    const int id = RING ? ring_block(p, qy, lane) : lane;
    const uint64_t kj = select_key(mine, static_cast<uint32_t>(id));
    int rank = 0;
    for (int k = 0; k < p.NB; ++k) {
      const float other = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), k));
      const int other_id = RING ? ring_block(p, qy, k) : k;
      rank += select_key(other, static_cast<uint32_t>(other_id)) > kj;
    }
    if (lane < p.NB && rank < p.TOP) {
      ws.sel[rank] = id;
      ws.selv[rank] = mine > -1.0e30f ? 1 : 0;
    }
  } else {
    for (int j = lane; j < p.NB; j += kWave) {
      const int id = RING ? ring_block(p, qy, j) : j;
      const uint64_t kj = select_key(ws.blk[j], static_cast<uint32_t>(id));
      int rank = 0;
      for (int k = 0; k < p.NB; ++k)
        rank += select_key(ws.blk[k], static_cast<uint32_t>(RING ? ring_block(p, qy, k) : k)) > kj;
      if (rank < p.TOP) {
        ws.sel[rank] = id;
        ws.selv[rank] = ws.blk[j] > -1.0e30f ? 1 : 0;
      }
    }
  }
  wave_sync();
}

// Candidate lane c: local window first, then TOP*BS remote lanes in pick order
// (relation_select.py:244-283).
// Ring caches hold every position of [t-T+1, t], so the cache-end test drops
// (a valid pick is an eligible, hence non-negative, absolute block).
template <bool RING = false>
__device__ __forceinline__ void candidate(const SelectParams& p, int c, const Query& qy,
                                          const WaveScratch& ws, int64_t& pos, bool& valid) {
  if (c < p.L) {
    pos = qy.t - p.L + 1 + c;
    valid = pos >= 0 && pos <= qy.t && (RING || pos < p.T);
  } else {
    const int r = (c - p.L) >> p.BS_log2;
    const int o = (c - p.L) & (p.BS - 1);
    pos = static_cast<int64_t>(ws.sel[r]) * p.BS + o;
    valid = ws.selv[r] != 0 && pos <= qy.t && pos < qy.local_start && (RING || pos < p.T);
  }
}

// Exact scores of every candidate lane into ws.sc (float32; -inf when invalid
// or equal to `exclude`).  One lane per candidate, NCL candidates per lane per
// pass: each lane gathers its rows whole (16-byte loads, all in flight before
// any is used) and accumulates the 64-element dot alone in float64 against
// the query, which the wave reads from LDS by broadcast -- no cross-lane
// reduction at all.  Local rows come from the staged LDS window when the
// query's whole window lies inside it (a per-wave decision); other rows come
// through range-checked buffer loads whose offset is pushed past the end for
// invalid rows (they read zero and are masked to -inf).
// `part` of `parts` waves sharing one query scores candidate passes part,
// part + parts, ... into the shared ws.sc.
// STAGED = false (decode: no staged windows) reads every row from L2 with no
// per-lane branch, so the compiler waits once per group of loads rather than
// once per load.
template <typename TA, int NCL, bool RING = false, bool STAGED = true>
__device__ void candidate_scores(const SelectParams& p, const Stream& s, const unsigned char* win,
                                 const Query& qy, int exclude, WaveScratch& ws, int lane,
                                 int part = 0, int parts = 1) {
  constexpr int EPC = kEpc<TA>;
  const rsrc_t keys = make_rsrc(s.keys, p.key_bytes);
  const uint32_t row0 = static_cast<uint32_t>(qy.b * p.T);
  const uint32_t row_bytes = static_cast<uint32_t>(p.E) * sizeof(TA);
  const int t = static_cast<int>(qy.t);
  const int ls = static_cast<int>(qy.local_start);
  const int T = static_cast<int>(p.T);
  const bool lds = win != nullptr && t - p.L + 1 >= qy.wbase && t < qy.wbase + p.WR;
  const int wb = static_cast<int>(qy.wbase);
  const int chunks = p.G;  // 16-byte chunks per row
  for (int c0 = part * kWave * NCL; c0 < p.CAP; c0 += parts * kWave * NCL) {
    int pos[NCL];
    bool ok[NCL], from_lds[NCL];
#pragma unroll
    for (int u = 0; u < NCL; ++u) {
      const int c = c0 + lane + kWave * u;
      bool v = c < p.CAP;
      int ps;
      if (c < p.L) {
        ps = t - p.L + 1 + c;
        v = v && ps >= 0 && ps <= t && (RING || ps < T);
        from_lds[u] = lds;
      } else {
        const int r = v ? (c - p.L) >> p.BS_log2 : 0;
        ps = ws.sel[r] * p.BS + ((c - p.L) & (p.BS - 1));
        v = v && ws.selv[r] != 0 && ps <= t && ps < ls && (RING || ps < T);
        from_lds[u] = false;
      }
      ok[u] = v && ps != exclude;
      pos[u] = RING ? (ps & (T - 1)) : ps;  // ring: the cache row (staged windows are linear only)
    }
    double acc[NCL];
#pragma unroll
    for (int u = 0; u < NCL; ++u) acc[u] = 0.0;
    // Rows in groups of CG chunks: all loads of a group in flight.  With
    // staged windows both sources are read for every row (the L2 read of a
    // window row goes out of range and returns zeros, the LDS read of a remote
    // row reads window row 0) and a select keeps the right one: a per-lane
    // branch between them would make the compiler wait for each L2 load before
    // the next.  Two chunks per group keep the registers of four.
    constexpr int CG = STAGED ? 2 : 4;
    for (int ch0 = 0; ch0 < chunks; ch0 += CG) {
      uint4 kc[NCL][CG];
#pragma unroll
      for (int u = 0; u < NCL; ++u)
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
          const int ch = ch0 + cc;
          const bool in = ch < chunks;  // wave-uniform
          const bool l2 = !STAGED || !from_lds[u];
          const uint4 g = buf_load_b128(
              keys, in && ok[u] && l2 ? (row0 + static_cast<uint32_t>(pos[u])) * row_bytes + 16u * ch
                                      : kNoOffset);
          if constexpr (STAGED) {
            uint4 l = make_uint4(0, 0, 0, 0);
            if (win != nullptr && in) {  // wave-uniform
              const int wr = ok[u] && from_lds[u] ? pos[u] - wb : 0;
              l = *reinterpret_cast<const uint4*>(win + wr * p.row_bytes + 16 * ch);
            }
            kc[u][cc] = from_lds[u] ? l : g;
          } else {
            kc[u][cc] = g;
          }
        }
      // Chunks past the row end were loaded as zeros and add exact zeros, so
      // every chunk is used unconditionally (a load used only under a
      // condition would be sunk into that branch and waited for there).
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const int ch = ch0 + cc < chunks ? ch0 + cc : 0;
        double q[EPC];
#pragma unroll
        for (int e = 0; e < EPC; e += 2) {
          const double2 q2 = *reinterpret_cast<const double2*>(ws.qx + EPC * ch + e);
          q[e] = q2.x;
          q[e + 1] = q2.y;
        }
#pragma unroll
        for (int u = 0; u < NCL; ++u) {
          double k[EPC];
          chunk_to_f64<TA>(kc[u][cc], k);
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[u] += k[e] * q[e];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NCL; ++u) {
      const int c = c0 + lane + kWave * u;
      if (c < p.CAP) ws.sc[c] = ok[u] ? static_cast<float>(acc[u] * p.exact_scale) : -INFINITY;
    }
  }
  wave_sync();
}

// Workgroup staging (W > 1): block statistics (f32), bias tables (f32) and
// the union of the local key windows of both streams, in one burst of loads
// (eight 16-byte chunks per thread in flight before any LDS store).
template <typename TA, typename TS, int MODE>
__device__ void stage_workgroup(const SelectParams& p, int64_t b, int64_t wbase,
                                unsigned char* smem) {
  constexpr int EPC = kEpc<TA>;
  constexpr bool kUseA = MODE != kPartnerOnly;
  constexpr bool kUseP = MODE != kAnchorOnly;
  const int tid = threadIdx.x;
  const int nt = blockDim.x;
  const int RD = p.H * p.HD;
  const int n_stat = p.NB * RD / 4;            // float4 per statistic tensor
  const int n_stats = 4 * n_stat;              // mean+std of both streams
  const int n_win = p.WR * p.G;                // 16-byte chunks per window
  const int total = n_stats + 2 * n_win;
  // bias tables (tiny): one element per thread
  for (int i = tid; i < 2 * p.H * p.RB; i += nt) {
    const int side = i / (p.H * p.RB);
    const int k = i - side * p.H * p.RB;
    if ((side == 0 && !kUseA) || (side == 1 && !kUseP)) continue;
    const Stream& s = side == 0 ? p.as : p.ps;
    float* dst = reinterpret_cast<float*>(smem + (side == 0 ? p.off_bias_a : p.off_bias_p));
    dst[k] = load_any_f(s.bias, s.bias_dtype, k);
  }
  // Item i < n_stats: statistic float4 (side, mean/std, index) with n_stat a
  // power of two; else window chunk: row-major over 2*WR rows (side 0 then 1)
  // of G chunks, G a power of two.  No divisions.
  const int stat_log2 = 31 - __clz(n_stat);
  constexpr int UB = 8;
  for (int i0 = tid; i0 < total; i0 += UB * nt) {
    uint4 v[UB];
    int dst[UB];  // LDS byte offset, -1: nothing to store
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int i = i0 + u * nt;
      v[u] = make_uint4(0, 0, 0, 0);
      dst[u] = -1;
      if (i >= total) continue;
      if (i < n_stats) {
        const int side = i >> (stat_log2 + 1);
        const int k = i & (2 * n_stat - 1);
        if ((side == 0 && !kUseA) || (side == 1 && !kUseP)) continue;
        const Stream& s = side == 0 ? p.as : p.ps;
        const bool is_std = k >= n_stat;
        const TS* src = static_cast<const TS*>(is_std ? s.stdev : s.mean) + b * p.NB * RD;
        const float4 f = load4(src + 4 * (k & (n_stat - 1)));
        v[u] = make_uint4(__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z),
                          __float_as_uint(f.w));
        dst[u] = (side == 0 ? p.off_stats_a : p.off_stats_p) + 16 * k;
      } else {
        const int w = i - n_stats;
        int row = w >> p.G_log2;
        const int ch = w & (p.G - 1);
        const int side = row >= p.WR ? 1 : 0;
        row -= side * p.WR;
        if ((side == 0 && !kUseA) || (side == 1 && !kUseP)) continue;
        const int64_t pos = wbase + row;
        const TA* keys = static_cast<const TA*>(side == 0 ? p.as.keys : p.ps.keys) + b * p.T * p.E;
        if (pos >= 0 && pos < p.T)
          v[u] = *reinterpret_cast<const uint4*>(keys + pos * p.E + EPC * ch);
        dst[u] = (side == 0 ? p.off_win_a : p.off_win_p) + row * p.row_bytes + 16 * ch;
      }
    }
#pragma unroll
    for (int u = 0; u < UB; ++u)
      if (dst[u] >= 0) *reinterpret_cast<uint4*>(smem + dst[u]) = v[u];
  }
}

// RING: ring-buffer caches (decode form only, no staged windows).
// SPLIT: one query per workgroup (decode), its candidate scoring shared by
// p.split waves.
template <typename TA, typename TS, int MODE, bool RING = false, bool SPLIT = false>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) select_kernel(const SelectParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int EPC = kEpc<TA>;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  // split > 1 (one query per workgroup): waves wq*split .. +split-1 share
  // query wq; sub-wave sw scores every split-th pass of 64 candidates.
  const int split = SPLIT ? p.split : 1;
  const int wq = wave / split;
  const int sw = wave - wq * split;
  // Consecutive logical workgroups (one batch row's query tiles) share an XCD,
  // so a batch row's keys and caches are fetched into one L2.
  const int64_t wg = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t b = wg / p.tiles;
  const int64_t tq0 = (wg - b * p.tiles) * static_cast<int64_t>(p.W);
  const int64_t tq = tq0 + wq;
  const int RD = p.H * p.HD;
  constexpr bool kUseA = MODE != kPartnerOnly;
  constexpr bool kUseP = MODE != kAnchorOnly;

  // ---- Query-side loads first (independent of everything staged below). ----
  // Waves past the last query read row tq0's vectors and leave after staging.
  const int64_t tq_ld = tq < p.Tq ? tq : tq0;
  const int64_t q_ld = b * p.Tq + tq_ld;
  const int64_t t_own = SPLIT ? index_at(p.pos, p.pos_dtype, b * p.pos_sb + tq_ld * p.pos_sq)
                              : load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq_ld * p.pos_sq);
  const int jg = lane & (p.G - 1);
  const TA* q_exact = static_cast<const TA*>(kUseA ? p.aq : p.pq) +
                      q_ld * (kUseA ? static_cast<int64_t>(p.E) : p.pq_row);
  const uint4 q_chunk = *reinterpret_cast<const uint4*>(q_exact + EPC * jg);
  uint4 pb_chunk = make_uint4(0, 0, 0, 0);
  if (MODE == kPacked)
    pb_chunk = *reinterpret_cast<const uint4*>(static_cast<const TA*>(p.pq) + q_ld * p.pq_row +
                                               EPC * jg);
  // softplus(gamma_h) = log(1 + exp(gamma_h)) in float64 (relation_select.py:87)
  // for this lane's head h = lane mod H, both streams, while the loads fly.
  double sp_a = 0.0, sp_p = 0.0;
  {
#pragma clang fp contract(off)
    const int h = lane & (p.H - 1);
    if constexpr (SPLIT) {
      // Decode: both dtype forms loaded, one kept -- no branch for the loads to
      // wait at (a lone wave's chain has nothing else to hide that latency).
      const FloatWords ga = issue_float(p.as.gamma, p.as.gamma_dtype, static_cast<uint32_t>(p.H),
                                        static_cast<uint32_t>(h), kUseA);
      const FloatWords gp = issue_float(p.ps.gamma, p.ps.gamma_dtype, static_cast<uint32_t>(p.H),
                                        static_cast<uint32_t>(h), kUseP);
      if (kUseA) sp_a = log(1.0 + exp(static_cast<double>(decode_float(ga, p.as.gamma_dtype))));
      if (kUseP) sp_p = log(1.0 + exp(static_cast<double>(decode_float(gp, p.ps.gamma_dtype))));
    } else {
      if (kUseA) sp_a = log(1.0 + exp(static_cast<double>(load_any_f(p.as.gamma, p.as.gamma_dtype, h))));
      if (kUseP) sp_p = log(1.0 + exp(static_cast<double>(load_any_f(p.ps.gamma, p.ps.gamma_dtype, h))));
    }
  }
  constexpr int kRq = 4;  // router-query elements held per lane (RD <= 256)
  float rq_a[kRq], rq_p[kRq];
  {
    const TA* ra = static_cast<const TA*>(kUseA ? p.arq : p.prq) +
                   q_ld * (kUseA ? static_cast<int64_t>(RD) : p.prq_row);
    const TA* rp = static_cast<const TA*>(p.prq) + q_ld * p.prq_row;
#pragma unroll
    for (int i = 0; i < kRq; ++i) {
      const int d = lane + kWave * i;
      if constexpr (SPLIT) {
        // Decode: unconditional loads (index clamped) and selects.
        const int dc = d < RD ? d : 0;
        const float va = to_f32(ra[dc]);
        rq_a[i] = d < RD ? va : 0.0f;
        const float vp = MODE == kPacked ? to_f32(rp[dc]) : 0.0f;
        rq_p[i] = (MODE == kPacked && d < RD) ? vp : 0.0f;
      } else {
        rq_a[i] = d < RD ? to_f32(ra[d]) : 0.0f;
        rq_p[i] = (MODE == kPacked && d < RD) ? to_f32(rp[d]) : 0.0f;
      }
    }
  }

  // ---- Workgroup staging (several queries share statistics and windows). ----
  const int64_t t_first = p.W > 1 ? load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq0 * p.pos_sq)
                                  : t_own;
  const int64_t wbase = t_first - p.L + 1;
  const bool staged = p.stage != 0;
  if (staged) {
    stage_workgroup<TA, TS, MODE>(p, b, wbase, smem);
    __syncthreads();
  }
  if (tq >= p.Tq) return;  // no workgroup barriers below
  const float* stats_a = staged && kUseA ? reinterpret_cast<const float*>(smem + p.off_stats_a) : nullptr;
  const float* stats_p = staged && kUseP ? reinterpret_cast<const float*>(smem + p.off_stats_p) : nullptr;
  const float* bias_a = staged && kUseA ? reinterpret_cast<const float*>(smem + p.off_bias_a) : nullptr;
  const float* bias_p = staged && kUseP ? reinterpret_cast<const float*>(smem + p.off_bias_p) : nullptr;
  const unsigned char* win_a = staged && kUseA ? smem + p.off_win_a : nullptr;
  const unsigned char* win_p = staged && kUseP ? smem + p.off_win_p : nullptr;

  unsigned char* base = smem + p.off_wave + wave * p.wave_bytes;
  WaveScratch ws;
  ws.qx = reinterpret_cast<double*>(base);
  ws.qr = ws.qx + p.E;
  ws.blk = reinterpret_cast<float*>(ws.qr + RD);
  ws.sel = reinterpret_cast<int*>(ws.blk + p.NB);
  ws.selv = ws.sel + p.TOP;
  ws.sc = reinterpret_cast<float*>(ws.selv + p.TOP);
  // Candidate scores live in the region of the query's first wave.
  ws.sc = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws.sc) - sw * p.wave_bytes);

  Query qy;
  qy.b = b;
  qy.q = b * p.Tq + tq;
  qy.t = t_own;
  qy.local_start = qy.t - p.L + 1 > 0 ? qy.t - p.L + 1 : 0;
  qy.wbase = wbase;
  const int j = jg;
  double qx[EPC];
  // The exact query chunk of this lane (lanes of one chunk group hold the
  // same values) into the wave's scratch.
  auto put_exact = [&]() {
    if (lane < p.G) {
#pragma unroll
      for (int e = 0; e < EPC; ++e) ws.qx[EPC * lane + e] = qx[e];
    }
  };
  // Router query into the wave's scratch (f64); RD > 4*64 reloads the rest.
  auto put_router = [&](const float* held, const TA* src, int64_t row_stride) {
#pragma unroll
    for (int i = 0; i < kRq; ++i) {
      const int d = lane + kWave * i;
      if (d < RD) ws.qr[d] = static_cast<double>(held[i]);
    }
    for (int d = lane + kWave * kRq; d < RD; d += kWave)
      ws.qr[d] = static_cast<double>(to_f32(src[qy.q * row_stride + d]));
  };

  int64_t anchor;
  if (kUseA) {
    chunk_to_f64<TA>(q_chunk, qx);
    put_exact();
    put_router(rq_a, static_cast<const TA*>(p.arq), RD);
    wave_sync();
    block_scores<TS, RING, SPLIT>(p, p.as, stats_a, bias_a, sp_a, qy, ws, lane);
    pick_blocks<RING>(p, qy, ws, lane);
    if constexpr (SPLIT) {
      candidate_scores<TA, 1, RING, false>(p, p.as, win_a, qy, -1, ws, lane, sw, split);
      __syncthreads();  // every wave of the query sees all candidate scores
    } else {
      candidate_scores<TA, 3, RING>(p, p.as, win_a, qy, -1, ws, lane);
    }
    uint64_t best = 0;
    float best_score = -INFINITY;
    for (int c = lane; c < p.CAP; c += kWave) {
      int64_t pos;
      bool valid;
      candidate<RING>(p, c, qy, ws, pos, valid);
      if (valid) {
        const float sc = ws.sc[c];
        const uint64_t k = select_key(sc, static_cast<uint32_t>(pos));
        if (k > best) {
          best = k;
          best_score = sc;
        }
      }
    }
    const uint64_t win = wave_max_u64(best);
    if (win == 0) {
      anchor = qy.t - p.L + 1;
      if (lane == 0 && sw == 0) {
        p.out_anchor[qy.q] = static_cast<int32_t>(anchor);
        p.out_anchor_score[qy.q] = -INFINITY;
      }
    } else {
      anchor = key_index(win);
      if (best == win && sw == 0) {
        p.out_anchor[qy.q] = static_cast<int32_t>(anchor);
        p.out_anchor_score[qy.q] = best_score;
      }
    }
    if (MODE == kAnchorOnly) return;
    wave_sync();
  } else {
    anchor = load_any_i(p.anchor_in, p.anchor_dtype, qy.q);
  }

  // Partner queries (relation_select.py:165-193): fp32 sum of the query-side
  // projection and the anchor row of the cached anchor-side projection.
  {
    const TA* prq = static_cast<const TA*>(p.prq) + qy.q * p.prq_row;
    if (MODE == kPacked) {
      const bool have = anchor >= 0 && (RING || anchor < p.T);
      const int64_t arow = RING ? (anchor & (p.T - 1)) : anchor;
      const TA* pc = static_cast<const TA*>(p.pcache) + (b * p.T + (have ? arow : 0)) * (2 * p.E);
      double base_q[EPC], cache_q[EPC];
      chunk_to_f64<TA>(pb_chunk, base_q);
      const uint4 cc = *reinterpret_cast<const uint4*>(pc + EPC * j);
      float cr[kRq];
#pragma unroll
      for (int i = 0; i < kRq; ++i) {
        const int d = lane + kWave * i;
        if constexpr (SPLIT) {
          const float v = to_f32(pc[p.E + (d < RD ? d : 0)]);
          cr[i] = d < RD ? v : 0.0f;
        } else {
          cr[i] = d < RD ? to_f32(pc[p.E + d]) : 0.0f;
        }
      }
      chunk_to_f64<TA>(cc, cache_q);
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        qx[e] = static_cast<double>(static_cast<float>(base_q[e]) +
                                    (have ? static_cast<float>(cache_q[e]) : 0.0f));
#pragma unroll
      for (int i = 0; i < kRq; ++i) {
        const int d = lane + kWave * i;
        if (d < RD) ws.qr[d] = static_cast<double>(rq_p[i] + (have ? cr[i] : 0.0f));
      }
      for (int d = lane + kWave * kRq; d < RD; d += kWave)
        ws.qr[d] = static_cast<double>(to_f32(prq[d]) + (have ? to_f32(pc[p.E + d]) : 0.0f));
    } else {
      chunk_to_f64<TA>(q_chunk, qx);
      put_router(rq_a, static_cast<const TA*>(p.prq), p.prq_row);
    }
    put_exact();
  }
  wave_sync();
  block_scores<TS, RING, SPLIT>(p, p.ps, stats_p, bias_p, sp_p, qy, ws, lane);
  pick_blocks<RING>(p, qy, ws, lane);
  if constexpr (SPLIT) __syncthreads();  // every wave has read the anchor scores
  if constexpr (SPLIT) {
    candidate_scores<TA, 1, RING, false>(p, p.ps, win_p, qy, static_cast<int>(anchor), ws, lane, sw,
                                         split);
    __syncthreads();
  } else {
    candidate_scores<TA, 3, RING>(p, p.ps, win_p, qy, static_cast<int>(anchor), ws, lane);
  }
  if (sw != 0) return;  // the query's first wave ranks the partners

  // K argmax passes (relation_select.py:298-308), ties to the lowest lane.
  // While finite scores remain, this is a stable descending order of the
  // lanes; once they are exhausted the reference's argmax over an all -inf
  // vector returns lane 0 for every remaining slot: position t-L+1, -inf.
  const int nc = (p.CAP + kWave - 1) / kWave;
  if (nc <= 4 && p.K <= kWave) {
    // Each lane keeps its (at most four) candidate keys sorted in registers
    // and pops its head when it wins a pass; lane k collects the k-th winner
    // and all K slots are written together at the end.
    uint64_t k4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + kWave * i;
      k4[i] = c < p.CAP ? select_key(ws.sc[c], static_cast<uint32_t>(c)) : 0;
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int bb = 0; bb < 3 - a; ++bb)
        if (k4[bb] < k4[bb + 1]) {
          const uint64_t tmp = k4[bb];
          k4[bb] = k4[bb + 1];
          k4[bb + 1] = tmp;
        }
    int my_c = -1;  // winning candidate lane of slot `lane` (-1: exhausted)
    for (int k = 0; k < p.K; ++k) {
      const uint64_t win = wave_max_u64(k4[0]);
      if (!(key_score(win) > -INFINITY)) break;  // wave-uniform
      if (lane == k) my_c = static_cast<int>(key_index(win));
      if (k4[0] == win) {
        k4[0] = k4[1];
        k4[1] = k4[2];
        k4[2] = k4[3];
        k4[3] = 0;
      }
    }
    if (lane < p.K) {
      int64_t pos = qy.t - p.L + 1;
      float score = -INFINITY;
      if (my_c >= 0) {
        bool valid;
        candidate<RING>(p, my_c, qy, ws, pos, valid);
        score = ws.sc[my_c];
      }
      p.out_partner[qy.q * p.K + lane] = static_cast<int32_t>(pos);
      p.out_partner_score[qy.q * p.K + lane] = score;
    }
    return;
  }
  uint64_t best = 0;
  for (int c = lane; c < p.CAP; c += kWave) {
    const uint64_t k = select_key(ws.sc[c], static_cast<uint32_t>(c));
    best = k > best ? k : best;
  }
  for (int k = 0; k < p.K; ++k) {
    const uint64_t win = wave_max_u64(best);
    const int c = static_cast<int>(key_index(win));
    if ((c & (kWave - 1)) == lane) {
      int64_t pos;
      bool valid;
      candidate<RING>(p, c, qy, ws, pos, valid);
      const bool exhausted = !(key_score(win) > -INFINITY);
      p.out_partner[qy.q * p.K + k] = static_cast<int32_t>(pos);
      p.out_partner_score[qy.q * p.K + k] = exhausted ? -INFINITY : ws.sc[c];
      ws.sc[c] = -INFINITY;
      best = 0;
      for (int cc = lane; cc < p.CAP; cc += kWave) {
        const uint64_t kk = select_key(ws.sc[cc], static_cast<uint32_t>(cc));
        best = kk > best ? kk : best;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Routed multi-anchor selection (semantics: multi_relation_blocks.py:69-147)
// ---------------------------------------------------------------------------
//
// S anchor slots per query.  The anchor router picks one candidate set per
// query (local window + TOP blocks); slot s takes the argmax of its own exact
// score over the candidates not taken by slots < s (distinct anchors,
// :86-95), and is active only when s <= t (:84).  Each active slot then forms
// its partner query (partner_base[s] + partner_anchor_cache[anchor_s, s], the
// split form of partner_query[s](cat(query, anchor)), :116-124), routes its
// own partner candidate set against the shared partner block statistics and
// takes the top-k exact scores with every active anchor of the query excluded
// (:133-139).  One wave per query, slots in order; keys are [B,T,S,E] rows, so
// slot s's vector of position p sits at byte (p*S + s)*E*elem.

constexpr int kMaxSlots = 8;

struct MultiParams {
  int S;                   // anchor slots per query
  uint32_t key_pos_bytes;  // bytes between positions of a key cache (S*E*elem)
  uint32_t slot_bytes;     // bytes of one slot's exact vector (E*elem)
  int64_t qrow;            // elements per (query, slot) row of partner_base and of the cache (E+RD)
};

// Exact scores of every candidate lane of one slot into ws.sc (float32; -inf
// when invalid or taken by an excluded position).  As candidate_scores, with
// strided key rows and no staged windows: rows come through range-checked
// buffer loads from L2.
template <typename TA, int NCL>
__device__ void slot_candidate_scores(const SelectParams& p, const void* keys_ptr,
                                      uint32_t pos_bytes, uint32_t col_bytes, const Query& qy,
                                      const int (&excl)[kMaxSlots], int nex, WaveScratch& ws,
                                      int lane) {
  constexpr int EPC = kEpc<TA>;
  const rsrc_t keys = make_rsrc(keys_ptr, p.key_bytes);
  const uint32_t row0 = static_cast<uint32_t>(qy.b * p.T);
  const int t = static_cast<int>(qy.t);
  const int ls = static_cast<int>(qy.local_start);
  const int T = static_cast<int>(p.T);
  const int chunks = p.G;
  for (int c0 = 0; c0 < p.CAP; c0 += kWave * NCL) {
    uint32_t off[NCL];
    bool ok[NCL];
#pragma unroll
    for (int u = 0; u < NCL; ++u) {
      const int c = c0 + lane + kWave * u;
      bool v = c < p.CAP;
      int ps;
      if (c < p.L) {
        ps = t - p.L + 1 + c;
        v = v && ps >= 0 && ps <= t && ps < T;
      } else {
        const int r = v ? (c - p.L) >> p.BS_log2 : 0;
        ps = ws.sel[r] * p.BS + ((c - p.L) & (p.BS - 1));
        v = v && ws.selv[r] != 0 && ps <= t && ps < ls && ps < T;
      }
      bool taken = false;
#pragma unroll
      for (int x = 0; x < kMaxSlots; ++x) taken = taken || (x < nex && ps == excl[x]);
      ok[u] = v && !taken;
      off[u] = ok[u] ? (row0 + static_cast<uint32_t>(ps)) * pos_bytes + col_bytes : 0u;
    }
    double acc[NCL];
#pragma unroll
    for (int u = 0; u < NCL; ++u) acc[u] = 0.0;
    constexpr int CG = 4;
    for (int ch0 = 0; ch0 < chunks; ch0 += CG) {
      uint4 kc[NCL][CG];
#pragma unroll
      for (int u = 0; u < NCL; ++u)
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
          const int ch = ch0 + cc;
          kc[u][cc] = ch < chunks ? buf_load_b128(keys, ok[u] ? off[u] + 16u * ch : kNoOffset)
                                  : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const int ch = ch0 + cc;
        if (ch >= chunks) break;
        double q[EPC];
#pragma unroll
        for (int e = 0; e < EPC; e += 2) {
          const double2 q2 = *reinterpret_cast<const double2*>(ws.qx + EPC * ch + e);
          q[e] = q2.x;
          q[e + 1] = q2.y;
        }
#pragma unroll
        for (int u = 0; u < NCL; ++u) {
          double k[EPC];
          chunk_to_f64<TA>(kc[u][cc], k);
#pragma unroll
          for (int e = 0; e < EPC; ++e) acc[u] += k[e] * q[e];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NCL; ++u) {
      const int c = c0 + lane + kWave * u;
      if (c < p.CAP) ws.sc[c] = ok[u] ? static_cast<float>(acc[u] * p.exact_scale) : -INFINITY;
    }
  }
  wave_sync();
}

// K argmax passes over ws.sc (ties to the lowest lane); exhausted slots repeat
// lane 0 with -inf, as the single-anchor partner pass.  Writes K entries.
__device__ void topk_lanes_out(const SelectParams& p, const Query& qy, WaveScratch& ws, int lane,
                               int32_t* out_idx, float* out_score) {
  uint64_t best = 0;
  for (int c = lane; c < p.CAP; c += kWave) {
    const uint64_t k = select_key(ws.sc[c], static_cast<uint32_t>(c));
    best = k > best ? k : best;
  }
  for (int k = 0; k < p.K; ++k) {
    const uint64_t win = wave_max_u64(best);
    const int c = static_cast<int>(key_index(win));
    if ((c & (kWave - 1)) == lane) {
      int64_t pos;
      bool valid;
      candidate(p, c, qy, ws, pos, valid);
      const bool exhausted = !(key_score(win) > -INFINITY);
      out_idx[k] = static_cast<int32_t>(exhausted ? qy.t - p.L + 1 : pos);
      out_score[k] = exhausted ? -INFINITY : ws.sc[c];
      ws.sc[c] = -INFINITY;
      best = 0;
      for (int cc = lane; cc < p.CAP; cc += kWave) {
        const uint64_t kk = select_key(ws.sc[cc], static_cast<uint32_t>(cc));
        best = kk > best ? kk : best;
      }
    }
  }
  wave_sync();
}

template <typename TA, typename TS>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
multi_select_kernel(const SelectParams p, const MultiParams m) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int EPC = kEpc<TA>;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  // Consecutive logical workgroups (one batch row's query tiles) share an XCD,
  // so a batch row's keys and caches are fetched into one L2.
  const int64_t wg = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t b = wg / p.tiles;
  const int64_t tq0 = (wg - b * p.tiles) * static_cast<int64_t>(p.W);
  const int64_t tq = tq0 + wave;
  const int RD = p.H * p.HD;

  // Partner statistics and bias tables are read by every slot of every query
  // of the workgroup: staged once.  Anchor statistics are read once per query,
  // from L2.
  if (p.stage) {
    stage_workgroup<TA, TS, kPartnerOnly>(p, b, 0, smem);
    __syncthreads();
  }
  if (tq >= p.Tq) return;  // no workgroup barriers below
  const float* stats_p = p.stage ? reinterpret_cast<const float*>(smem + p.off_stats_p) : nullptr;
  const float* bias_p = p.stage ? reinterpret_cast<const float*>(smem + p.off_bias_p) : nullptr;

  unsigned char* base = smem + p.off_wave + wave * p.wave_bytes;
  WaveScratch ws;
  ws.qx = reinterpret_cast<double*>(base);
  ws.qr = ws.qx + p.E;
  ws.blk = reinterpret_cast<float*>(ws.qr + RD);
  ws.sel = reinterpret_cast<int*>(ws.blk + p.NB);
  ws.selv = ws.sel + p.TOP;
  ws.sc = reinterpret_cast<float*>(ws.selv + p.TOP);

  Query qy;
  qy.b = b;
  qy.q = b * p.Tq + tq;
  qy.t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  qy.local_start = qy.t - p.L + 1 > 0 ? qy.t - p.L + 1 : 0;
  qy.wbase = 0;
  double sp_a, sp_p;
  {
#pragma clang fp contract(off)
    const int h = lane & (p.H - 1);
    sp_a = log(1.0 + exp(static_cast<double>(load_any_f(p.as.gamma, p.as.gamma_dtype, h))));
    sp_p = log(1.0 + exp(static_cast<double>(load_any_f(p.ps.gamma, p.ps.gamma_dtype, h))));
  }

  // ---- Anchors: one routed candidate set, S distinct argmaxes.
  {
    const TA* arq = static_cast<const TA*>(p.arq) + qy.q * RD;
    for (int d = lane; d < RD; d += kWave) ws.qr[d] = static_cast<double>(to_f32(arq[d]));
    wave_sync();
    block_scores<TS>(p, p.as, nullptr, nullptr, sp_a, qy, ws, lane);
    pick_blocks(p, qy, ws, lane);
  }
  int taken[kMaxSlots];
#pragma unroll
  for (int x = 0; x < kMaxSlots; ++x) taken[x] = -1;
  int active = 0;
  for (int s = 0; s < m.S; ++s) {
    const int64_t o = qy.q * m.S + s;
    if (s > qy.t) {  // inactive slot: anchor 0, no partners
      if (lane == 0) {
        p.out_anchor[o] = 0;
        p.out_anchor_score[o] = -INFINITY;
      }
      continue;
    }
    if (lane < p.G) {
      const TA* aq = static_cast<const TA*>(p.aq) + o * p.E;
      double qx[EPC];
      chunk_to_f64<TA>(*reinterpret_cast<const uint4*>(aq + EPC * lane), qx);
#pragma unroll
      for (int e = 0; e < EPC; ++e) ws.qx[EPC * lane + e] = qx[e];
    }
    wave_sync();
    slot_candidate_scores<TA, 3>(p, p.as.keys, m.key_pos_bytes, m.slot_bytes * s, qy, taken,
                                 active, ws, lane);
    uint64_t best = 0;
    float best_score = -INFINITY;
    for (int c = lane; c < p.CAP; c += kWave) {
      int64_t pos;
      bool valid;
      candidate(p, c, qy, ws, pos, valid);
      const float sc = ws.sc[c];
      if (valid && sc > -INFINITY) {
        const uint64_t k = select_key(sc, static_cast<uint32_t>(pos));
        if (k > best) {
          best = k;
          best_score = sc;
        }
      }
    }
    const uint64_t win = wave_max_u64(best);
    // With local_window >= S an active slot always has an untaken candidate
    // (the window holds min(t+1, L) >= s+1 positions); the host checks that.
    const int anchor = win == 0 ? 0 : static_cast<int>(key_index(win));
    if (win == 0) {
      if (lane == 0) {
        p.out_anchor[o] = 0;
        p.out_anchor_score[o] = -INFINITY;
      }
    } else if (best == win) {
      p.out_anchor[o] = anchor;
      p.out_anchor_score[o] = best_score;
    }
    if (win != 0) {
#pragma unroll
      for (int x = 0; x < kMaxSlots; ++x)
        if (x == active) taken[x] = anchor;
      ++active;
    }
    wave_sync();
  }

  // ---- Partners of each active slot.
  for (int s = 0; s < m.S; ++s) {
    const int64_t o = qy.q * m.S + s;
    int32_t* out_idx = p.out_partner + o * p.K;
    float* out_score = p.out_partner_score + o * p.K;
    if (s >= active) {  // inactive (or anchorless) slot: every entry exhausted
      for (int k = lane; k < p.K; k += kWave) {
        out_idx[k] = static_cast<int32_t>(qy.t - p.L + 1);
        out_score[k] = -INFINITY;
      }
      continue;
    }
    int anchor = taken[0];
#pragma unroll
    for (int x = 1; x < kMaxSlots; ++x)
      if (x == s) anchor = taken[x];
    // Partner query: float32 sum of the query-side row and the anchor's cached
    // row, exact half then router half.
    const TA* pb = static_cast<const TA*>(p.pq) + o * m.qrow;
    const TA* pc = static_cast<const TA*>(p.pcache) + ((b * p.T + anchor) * m.S + s) * m.qrow;
    if (lane < p.G) {
      double bq[EPC], cq[EPC];
      chunk_to_f64<TA>(*reinterpret_cast<const uint4*>(pb + EPC * lane), bq);
      chunk_to_f64<TA>(*reinterpret_cast<const uint4*>(pc + EPC * lane), cq);
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        ws.qx[EPC * lane + e] = static_cast<double>(static_cast<float>(bq[e]) +
                                                    static_cast<float>(cq[e]));
    }
    for (int d = lane; d < RD; d += kWave)
      ws.qr[d] = static_cast<double>(to_f32(pb[p.E + d]) + to_f32(pc[p.E + d]));
    wave_sync();
    block_scores<TS>(p, p.ps, stats_p, bias_p, sp_p, qy, ws, lane);
    pick_blocks(p, qy, ws, lane);
    slot_candidate_scores<TA, 3>(p, p.ps.keys, m.key_pos_bytes, m.slot_bytes * s, qy, taken,
                                 active, ws, lane);
    topk_lanes_out(p, qy, ws, lane, out_idx, out_score);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

struct Geometry {
  int64_t B, Tq, T;
  int NB, BS, E, H, HD, RB;
};

bool check_router_side(const rlm_tensor* mean, const rlm_tensor* stdv, const rlm_tensor* gamma,
                       const rlm_tensor* bias, const char* side, const Geometry& g,
                       int stat_dtype) {
  char name[96];
  snprintf(name, sizeof(name), "%s_block_mean", side);
  if (!check_tensor(mean, name, 4) || !check_dim(mean, name, 0, g.B) ||
      !check_dim(mean, name, 1, g.NB) || !check_dim(mean, name, 2, g.H) ||
      !check_dim(mean, name, 3, g.HD) || !check_dtype_is(mean, name, stat_dtype))
    return false;
  snprintf(name, sizeof(name), "%s_block_std", side);
  if (!check_tensor(stdv, name, 4) || !check_dim(stdv, name, 0, g.B) ||
      !check_dim(stdv, name, 1, g.NB) || !check_dim(stdv, name, 2, g.H) ||
      !check_dim(stdv, name, 3, g.HD) || !check_dtype_is(stdv, name, stat_dtype))
    return false;
  snprintf(name, sizeof(name), "%s_gamma", side);
  if (!check_tensor(gamma, name, 1) || !check_dim(gamma, name, 0, g.H) ||
      !check_dtype_float(gamma, name))
    return false;
  snprintf(name, sizeof(name), "%s_bias", side);
  if (!check_tensor(bias, name, 2) || !check_dim(bias, name, 0, g.H) ||
      !check_dim(bias, name, 1, g.RB) || !check_dtype_float(bias, name))
    return false;
  return true;
}

bool check_stream(const rlm_tensor* keys, const rlm_tensor* mean, const rlm_tensor* stdv,
                  const rlm_tensor* gamma, const rlm_tensor* bias, const char* side,
                  const Geometry& g, int act_dtype, int stat_dtype) {
  char name[96];
  snprintf(name, sizeof(name), "%s_keys", side);
  if (!check_tensor(keys, name, 3) || !check_dim(keys, name, 0, g.B) ||
      !check_dim(keys, name, 1, g.T) || !check_dim(keys, name, 2, g.E) ||
      !check_dtype_is(keys, name, act_dtype))
    return false;
  return check_router_side(mean, stdv, gamma, bias, side, g, stat_dtype);
}

bool aligned16(const rlm_tensor* t, const char* name) {
  if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) {
    set_error("%s: data pointer must be 16-byte aligned", name);
    return false;
  }
  return true;
}

Stream make_stream(const rlm_tensor* keys, const rlm_tensor* mean, const rlm_tensor* stdv,
                   const rlm_tensor* gamma, const rlm_tensor* bias) {
  Stream s;
  s.keys = keys->data;
  s.mean = mean->data;
  s.stdev = stdv->data;
  s.gamma = gamma->data;
  s.bias = bias->data;
  s.gamma_dtype = gamma->dtype;
  s.bias_dtype = bias->dtype;
  return s;
}

// Validates the routing hyper-parameters and fills the derived fields.
hipError_t finish_params(SelectParams& p, const Geometry& g, int64_t local_window,
                         int64_t top_blocks, int64_t k_out, int32_t strict_valid,
                         int act_size) {
  RLM_REQUIRE(local_window >= 1 && local_window <= 4096,
              "local_window must be in [1, 4096], got %lld", (long long)local_window);
  RLM_REQUIRE(top_blocks >= 0 && top_blocks <= 64, "top_blocks must be in [0, 64], got %lld",
              (long long)top_blocks);
  RLM_REQUIRE(k_out >= 0 && k_out <= 1024, "k_out must be in [0, 1024], got %lld",
              (long long)k_out);
  RLM_REQUIRE(g.NB >= 1 && g.BS >= 1, "need at least one block of at least one row");
  RLM_REQUIRE(g.H >= 1 && g.H * g.HD <= 1024, "heads*head_dim must be <= 1024");
  RLM_REQUIRE(g.RB >= 1, "relative buckets must be >= 1");
  const int64_t cap = local_window + top_blocks * static_cast<int64_t>(g.BS);
  RLM_REQUIRE(cap <= 8192, "local_window + top_blocks * block_size must be <= 8192");
  p.B = g.B;
  p.Tq = g.Tq;
  p.T = g.T;
  p.NB = g.NB;
  p.BS = g.BS;
  p.E = g.E;
  p.H = g.H;
  p.HD = g.HD;
  p.RB = g.RB;
  p.L = static_cast<int>(local_window);
  p.TOP = static_cast<int>(top_blocks);
  p.K = static_cast<int>(k_out);
  p.CAP = static_cast<int>(cap);
  p.strict = strict_valid ? 1 : 0;
  p.exact_scale = 1.0 / std::sqrt(static_cast<double>(g.E));
  p.head_scale = 1.0 / std::sqrt(static_cast<double>(g.HD));
  const int elem = act_size;
  RLM_REQUIRE((g.E * elem) % 16 == 0, "exact dim times element size must be a multiple of 16 bytes");
  const int G = g.E * elem / 16;
  RLM_REQUIRE(G <= kWave && (G & (G - 1)) == 0,
              "exact dim must be a power of two of at most %d elements for this dtype",
              kWave * 16 / elem);
  RLM_REQUIRE(g.HD % 4 == 0, "router head dim must be a multiple of 4");
  RLM_REQUIRE(g.H <= kWave && (g.H & (g.H - 1)) == 0, "router heads must be a power of two <= 64");
  RLM_REQUIRE((g.BS & (g.BS - 1)) == 0,
              "block size (cache length / blocks) must be a power of two, got %d", g.BS);
  p.G = G;
  p.G_log2 = 31 - __builtin_clz(static_cast<unsigned>(G));
  p.H_log2 = 31 - __builtin_clz(static_cast<unsigned>(g.H));
  p.BS_log2 = 31 - __builtin_clz(static_cast<unsigned>(g.BS));
  p.W = g.Tq > 1 ? 8 : 1;
  // One query per workgroup (decode): its candidate passes of 64 are shared
  // by up to 4 waves.
  p.split = p.W == 1 ? std::min(4, (p.CAP + kWave - 1) / kWave) : 1;
  p.tiles = static_cast<int>((g.Tq + p.W - 1) / p.W);
  p.WR = p.L + p.W - 1;
  p.row_bytes = g.E * elem + 16;
  const int RD = g.H * g.HD;
  const int stats_bytes = 2 * g.NB * RD * 4;  // mean + std, one stream
  const bool stats_pow2 = ((g.NB * RD / 4) & (g.NB * RD / 4 - 1)) == 0;
  const int bias_bytes = ((g.H * g.RB * 4) + 15) & ~15;
  int off = 0;
  p.stage = p.W > 1 && stats_pow2 ? 1 : 0;
  p.off_stats_a = p.off_stats_p = p.off_bias_a = p.off_bias_p = p.off_win_a = p.off_win_p = 0;
  if (p.stage) {
    p.off_stats_a = off;
    off += stats_bytes;
    p.off_stats_p = off;
    off += stats_bytes;
    p.off_bias_a = off;
    off += bias_bytes;
    p.off_bias_p = off;
    off += bias_bytes;
    p.off_win_a = off;
    off += p.WR * p.row_bytes;
    p.off_win_p = off;
    off += p.WR * p.row_bytes;
  }
  const int64_t key_bytes = g.B * g.T * g.E * elem;
  RLM_REQUIRE(key_bytes < (int64_t(1) << 31), "key caches must be smaller than 2 GiB");
  p.key_bytes = static_cast<uint32_t>(key_bytes);
  p.off_wave = off;
  p.wave_bytes = wave_region_bytes(g.E, g.NB, RD, p.TOP, p.CAP);
  off += p.W * p.split * p.wave_bytes;
  if (p.stage && off > 96 * 1024) {
    // Too large to share: every wave reads statistics and keys from L2.
    p.stage = 0;
    off = 0;
    p.off_wave = 0;
    off += p.W * p.split * p.wave_bytes;
  }
  RLM_REQUIRE(off <= 160 * 1024,
              "selection working set (%d bytes of LDS) exceeds the 160 KiB of one CU", off);
  p.lds_total = off;
  return hipSuccess;
}

template <int MODE, bool RING = false>
hipError_t launch_select(const SelectParams& p, int act_dtype, int stat_dtype,
                         hipStream_t stream) {
  const int64_t queries = p.B * p.Tq;
  if (queries == 0) return hipSuccess;
  const dim3 block(p.W * p.split * kWave);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles));
  const size_t lds = static_cast<size_t>(p.lds_total);
#define RLM_SELECT_CASE(TA_ID, TA, TS_ID, TS)                                             \
  if (act_dtype == TA_ID && stat_dtype == TS_ID) {                                        \
    /* ring caches are decode only (one query per workgroup): always the split */        \
    /* form, which also serves split == 1 */                                              \
    if (RING || p.split > 1)                                                              \
      hipLaunchKernelGGL((select_kernel<TA, TS, MODE, RING, true>), grid, block, lds, stream, p); \
    else if constexpr (!RING)                                                             \
      hipLaunchKernelGGL((select_kernel<TA, TS, MODE, RING, false>), grid, block, lds, stream, p); \
    return launch_status("relation_select");                                              \
  }
  RLM_SELECT_CASE(RLM_F32, float, RLM_F32, float)
  RLM_SELECT_CASE(RLM_F32, float, RLM_BF16, bf16)
  RLM_SELECT_CASE(RLM_BF16, bf16, RLM_F32, float)
  RLM_SELECT_CASE(RLM_BF16, bf16, RLM_BF16, bf16)
  RLM_SELECT_CASE(RLM_F16, f16, RLM_F32, float)
  RLM_SELECT_CASE(RLM_F16, f16, RLM_F16, f16)
#undef RLM_SELECT_CASE
  set_error("relation_select: unsupported dtype combination (activations %s, stats %s)",
            dtype_name(act_dtype), dtype_name(stat_dtype));
  return hipErrorInvalidValue;
}

bool check_position(const rlm_tensor* pos, const char* name, const Geometry& g, bool seq,
                    SelectParams& p) {
  if (pos == nullptr) {
    set_error("%s: missing tensor", name);
    return false;
  }
  if (!is_index_dtype(pos->dtype)) {
    set_error("%s: expected int32/int64, got %s", name, dtype_name(pos->dtype));
    return false;
  }
  p.pos = pos->data;
  p.pos_dtype = pos->dtype;
  if (!seq) {
    if (!check_tensor(pos, name, 0)) return false;
    p.pos_sb = 0;
    p.pos_sq = 0;
    return true;
  }
  if (pos->ndim == 1) {
    if (!check_tensor(pos, name, 1) || !check_dim(pos, name, 0, g.Tq)) return false;
    p.pos_sb = 0;
    p.pos_sq = 1;
    return true;
  }
  if (!check_tensor(pos, name, 2) || !check_dim(pos, name, 0, g.B) ||
      !check_dim(pos, name, 1, g.Tq))
    return false;
  p.pos_sb = g.Tq;
  p.pos_sq = 1;
  return true;
}

bool check_outputs(const rlm_tensor* idx, const rlm_tensor* score, const char* what,
                   const Geometry& g, bool seq, int64_t k) {
  char iname[64], sname[64];
  snprintf(iname, sizeof(iname), "out_%s", what);
  snprintf(sname, sizeof(sname), "out_%s_score", what);
  const int base = seq ? 2 : 1;
  const int nd = base + (k >= 0 ? 1 : 0);
  if (!check_tensor(idx, iname, nd) || !check_dtype_is(idx, iname, RLM_I32)) return false;
  if (!check_tensor(score, sname, nd) || !check_dtype_is(score, sname, RLM_F32)) return false;
  if (!check_dim(idx, iname, 0, g.B) || !check_dim(score, sname, 0, g.B)) return false;
  if (seq && (!check_dim(idx, iname, 1, g.Tq) || !check_dim(score, sname, 1, g.Tq))) return false;
  if (k >= 0 && (!check_dim(idx, iname, base, k) || !check_dim(score, sname, base, k)))
    return false;
  return true;
}

// The sequence form takes the matrix-core-filtered kernel where it applies
// unless RLM_SELECT_TILE=0 (both kernels give identical results; the switch
// exists to compare them).
bool tile_path_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("RLM_SELECT_TILE");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

// Fills the tile kernel's parameters when the shapes fit it.
bool tile_params(const SelectParams& p, const Geometry& g, int act, int stat,
                 const rlm_tensor* position, const rlm_tensor* aq, const rlm_tensor* arq,
                 const rlm_tensor* pbase, const rlm_tensor* pcache, const rlm_tensor* akeys,
                 const rlm_tensor* pkeys, const rlm_tensor* amean, const rlm_tensor* astd,
                 const rlm_tensor* agamma, const rlm_tensor* abias, const rlm_tensor* pmean,
                 const rlm_tensor* pstd, const rlm_tensor* pgamma, const rlm_tensor* pbias,
                 TileParams& tp) {
  if (act != RLM_BF16 || (stat != RLM_F32 && stat != RLM_BF16)) return false;
  if (g.E != 64 || g.H * g.HD != 64 || g.H > kTileMaxHeads || g.HD % 4 != 0 ||
      (g.H & (g.H - 1)) != 0)
    return false;
  if (g.T % 16 != 0 || g.T > kTileMaxRows || static_cast<int64_t>(g.NB) * g.BS != g.T) return false;
  if (g.NB > 64 || g.NB % 4 != 0 || p.CAP > 256 || p.TOP > kTileMaxTop || p.K < 1 || p.K > kTileMaxK) return false;
  if (g.H * g.RB > 512) return false;  // both sides' bias tables staged by one thread each
  tp.B = g.B;
  tp.Tq = g.Tq;
  tp.T = g.T;
  tp.NB = g.NB;
  tp.BS = g.BS;
  tp.BS_log2 = p.BS_log2;
  tp.L = p.L;
  tp.TOP = p.TOP;
  tp.K = p.K;
  tp.CAP = p.CAP;
  tp.NCL = (p.CAP + 15) / 16;
  tp.H = g.H;
  tp.H_log2 = p.H_log2;
  tp.HD = g.HD;
  tp.RB = g.RB;
  tp.strict = p.strict;
  tp.exact_scale = p.exact_scale;
  tp.head_scale = p.head_scale;
  tp.pos = position->data;
  tp.pos_dtype = position->dtype;
  tp.pos_sb = p.pos_sb;
  tp.pos_sq = p.pos_sq;
  tp.pos_count = p.pos_sb == 0 ? g.Tq : g.B * g.Tq;
  tp.aq = static_cast<const bf16*>(aq->data);
  tp.arq = static_cast<const bf16*>(arq->data);
  tp.pbase = static_cast<const bf16*>(pbase->data);
  tp.pcache = static_cast<const bf16*>(pcache->data);
  tp.akeys = static_cast<const bf16*>(akeys->data);
  tp.pkeys = static_cast<const bf16*>(pkeys->data);
  tp.amean = amean->data;
  tp.astd = astd->data;
  tp.pmean = pmean->data;
  tp.pstd = pstd->data;
  tp.agamma = agamma->data;
  tp.pgamma = pgamma->data;
  tp.abias = abias->data;
  tp.pbias = pbias->data;
  tp.agamma_dtype = agamma->dtype;
  tp.pgamma_dtype = pgamma->dtype;
  tp.abias_dtype = abias->dtype;
  tp.pbias_dtype = pbias->dtype;
  tp.out_anchor = p.out_anchor;
  tp.out_anchor_score = p.out_anchor_score;
  tp.out_partner = p.out_partner;
  tp.out_partner_score = p.out_partner_score;
  tp.tiles = static_cast<int>((g.Tq + 15) / 16);
  return select_tile_layout(tp);
}

// The decode form takes the latency-oriented kernel where it applies unless
// RLM_SELECT_DECODE=0 (both kernels give identical results; the switch exists
// to compare them).
bool decode_path_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("RLM_SELECT_DECODE");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

// Fills the decode kernel's parameters when the shapes fit it.
bool decode_params(const SelectParams& p, const Geometry& g, int act, int stat,
                   const rlm_tensor* position, const rlm_tensor* aq, const rlm_tensor* arq,
                   const rlm_tensor* pbase, const rlm_tensor* pcache, const rlm_tensor* akeys,
                   const rlm_tensor* pkeys, const rlm_tensor* amean, const rlm_tensor* astd,
                   const rlm_tensor* agamma, const rlm_tensor* abias, const rlm_tensor* pmean,
                   const rlm_tensor* pstd, const rlm_tensor* pgamma, const rlm_tensor* pbias,
                   DecodeParams& dp) {
  const bool dtypes = (act == RLM_BF16 && (stat == RLM_F32 || stat == RLM_BF16)) ||
                      (act == RLM_F16 && (stat == RLM_F32 || stat == RLM_F16));
  if (!dtypes || g.E != 64 || g.H != 4 || g.HD != 16) return false;
  dp.B = g.B;
  dp.T = g.T;
  dp.NB = g.NB;
  dp.BS = g.BS;
  dp.BS_log2 = p.BS_log2;
  dp.L = p.L;
  dp.TOP = p.TOP;
  dp.K = p.K;
  dp.CAP = p.CAP;
  dp.RB = g.RB;
  dp.strict = p.strict;
  dp.exact_scale = p.exact_scale;
  dp.head_scale = p.head_scale;
  dp.pos = position->data;
  dp.pos_dtype = position->dtype;
  dp.aq = aq->data;
  dp.arq = arq->data;
  dp.pbase = pbase->data;
  dp.pcache = pcache->data;
  dp.akeys = akeys->data;
  dp.pkeys = pkeys->data;
  dp.amean = amean->data;
  dp.astd = astd->data;
  dp.pmean = pmean->data;
  dp.pstd = pstd->data;
  dp.agamma = agamma->data;
  dp.pgamma = pgamma->data;
  dp.abias = abias->data;
  dp.pbias = pbias->data;
  dp.agamma_dtype = agamma->dtype;
  dp.pgamma_dtype = pgamma->dtype;
  dp.abias_dtype = abias->dtype;
  dp.pbias_dtype = pbias->dtype;
  dp.out_anchor = p.out_anchor;
  dp.out_anchor_score = p.out_anchor_score;
  dp.out_partner = p.out_partner;
  dp.out_partner_score = p.out_partner_score;
  return select_decode_layout(dp);
}

// The decode step's expanded-cache row, requested with the selection: for
// every batch row b, expanded_cache[b, row] = expanded_weight . operand_cache[b,
// row] + expanded_bias, row = position (linear caches) or position mod T (ring).
struct RowArgs {
  const rlm_tensor* operand;  // [B, T, R] bf16
  const rlm_tensor* weight;   // [N, R] bf16
  const rlm_tensor* bias;     // [N] or null
  const rlm_tensor* cache;    // [B, T, N] bf16, row written
};

hipError_t fill_expand_row(const RowArgs& a, const Geometry& g, const rlm_tensor* position,
                           bool ring, ExpandRowParams& x) {
  RLM_TRY(check_tensor(a.operand, "operand_cache", 3));
  RLM_TRY(check_dtype_is(a.operand, "operand_cache", RLM_BF16));
  RLM_TRY(check_dim(a.operand, "operand_cache", 0, g.B));
  RLM_TRY(check_dim(a.operand, "operand_cache", 1, g.T));
  const int64_t R = a.operand->shape[2];
  RLM_REQUIRE(R >= 32 && R <= 128 && R % 32 == 0,
              "operand_cache: the expanded row needs a relation dim of 32, 64, 96 or 128, got %lld",
              (long long)R);
  RLM_TRY(check_tensor(a.weight, "expanded_weight", 2));
  RLM_TRY(check_dtype_is(a.weight, "expanded_weight", RLM_BF16));
  RLM_TRY(check_dim(a.weight, "expanded_weight", 1, R));
  const int64_t N = a.weight->shape[0];
  RLM_REQUIRE(N >= 16 && N % 16 == 0,
              "expanded_weight: output width must be a positive multiple of 16, got %lld",
              (long long)N);
  if (a.bias != nullptr) {
    RLM_TRY(check_tensor(a.bias, "expanded_bias", 1));
    RLM_TRY(check_dtype_float(a.bias, "expanded_bias"));
    RLM_TRY(check_dim(a.bias, "expanded_bias", 0, N));
  }
  RLM_TRY(check_tensor(a.cache, "expanded_cache", 3));
  RLM_TRY(check_dtype_is(a.cache, "expanded_cache", RLM_BF16));
  RLM_TRY(check_dim(a.cache, "expanded_cache", 0, g.B));
  RLM_TRY(check_dim(a.cache, "expanded_cache", 1, g.T));
  RLM_TRY(check_dim(a.cache, "expanded_cache", 2, N));
  for (const rlm_tensor* t : {a.operand, a.weight, a.cache})
    RLM_TRY(aligned16(t, "expanded-row tensors"));
  const int64_t op_bytes = g.B * g.T * R * 2, w_bytes = N * R * 2;
  RLM_REQUIRE(op_bytes < (int64_t(1) << 31) && w_bytes < (int64_t(1) << 31),
              "operand_cache / expanded_weight: at most 2 GiB each");
  x.op = static_cast<const bf16*>(a.operand->data);
  x.w = static_cast<const bf16*>(a.weight->data);
  x.bias = a.bias != nullptr ? a.bias->data : nullptr;
  x.bias_dtype = a.bias != nullptr ? a.bias->dtype : RLM_F32;
  x.cache = static_cast<bf16*>(a.cache->data);
  x.pos = position->data;
  x.pos_dtype = position->dtype;
  x.B = g.B;
  x.T = g.T;
  x.KS = static_cast<int>(R / 32);
  x.N = static_cast<int>(N);
  x.ring = ring ? 1 : 0;
  x.op_bytes = static_cast<uint32_t>(op_bytes);
  x.w_bytes = static_cast<uint32_t>(w_bytes);
  return hipSuccess;
}

// The whole expanded cache as one launch of the library GEMM (rlm_linear):
// [B*T, R] . [N, R]^T + bias -> [B*T, N] bf16.
hipError_t expand_seq_linear(const RowArgs& a, const Geometry& g, hipStream_t stream) {
  const int64_t R = a.operand->shape[2], N = a.weight->shape[0];
  rlm_tensor in = *a.operand, out = *a.cache;
  in.ndim = 2;
  in.shape[0] = g.B * g.T;
  in.shape[1] = R;
  in.stride[0] = R;
  in.stride[1] = 1;
  out.ndim = 2;
  out.shape[0] = g.B * g.T;
  out.shape[1] = N;
  out.stride[0] = N;
  out.stride[1] = 1;
  return rlm_linear(&in, a.weight, a.bias, &out, stream);
}

hipError_t select_packed_impl(
    bool seq, bool ring, const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream,
    const RowArgs* xrow = nullptr, const RowArgs* xseq = nullptr) {
  clear_error();
  const int qd = seq ? 3 : 2;  // rank of query-side tensors
  RLM_TRY(check_tensor(anchor_query, "anchor_query", qd));
  RLM_TRY(check_dtype_float(anchor_query, "anchor_query"));
  RLM_TRY(check_tensor(anchor_keys, "anchor_keys", 3));
  RLM_TRY(check_tensor(anchor_block_mean, "anchor_block_mean", 4));
  RLM_TRY(check_tensor(anchor_bias, "anchor_bias", 2));
  Geometry g;
  g.B = anchor_query->shape[0];
  g.Tq = seq ? anchor_query->shape[1] : 1;
  g.E = static_cast<int>(anchor_query->shape[qd - 1]);
  g.T = anchor_keys->shape[1];
  g.NB = static_cast<int>(anchor_block_mean->shape[1]);
  g.H = static_cast<int>(anchor_block_mean->shape[2]);
  g.HD = static_cast<int>(anchor_block_mean->shape[3]);
  g.RB = static_cast<int>(anchor_bias->shape[1]);
  RLM_REQUIRE(g.NB >= 1 && g.T >= g.NB, "need 1 <= blocks <= cache length");
  g.BS = static_cast<int>(g.T / g.NB);
  const int act = anchor_query->dtype;
  const int stat = anchor_block_mean->dtype;
  RLM_REQUIRE(g.H * g.HD == g.E,
              "packed selection needs heads*head_dim == exact dim (router and exact partner "
              "queries share the 2*E packed rows); got %d*%d vs %d",
              g.H, g.HD, g.E);
  RLM_TRY(check_stream(anchor_keys, anchor_block_mean, anchor_block_std, anchor_gamma,
                       anchor_bias, "anchor", g, act, stat));
  RLM_TRY(check_stream(partner_keys, partner_block_mean, partner_block_std, partner_gamma,
                       partner_bias, "partner", g, act, stat));
  RLM_TRY(check_tensor(anchor_router_query, "anchor_router_query", qd));
  RLM_TRY(check_dtype_is(anchor_router_query, "anchor_router_query", act));
  RLM_TRY(check_tensor(partner_base, "partner_base", qd));
  RLM_TRY(check_dtype_is(partner_base, "partner_base", act));
  RLM_TRY(check_tensor(partner_anchor_cache, "partner_anchor_cache", 3));
  RLM_TRY(check_dtype_is(partner_anchor_cache, "partner_anchor_cache", act));
  RLM_TRY(check_dim(anchor_query, "anchor_query", 0, g.B));
  RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", 0, g.B));
  RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", qd - 1, g.H * g.HD));
  RLM_TRY(check_dim(partner_base, "partner_base", 0, g.B));
  RLM_TRY(check_dim(partner_base, "partner_base", qd - 1, 2 * g.E));
  if (seq) {
    RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", 1, g.Tq));
    RLM_TRY(check_dim(partner_base, "partner_base", 1, g.Tq));
  }
  RLM_TRY(check_dim(partner_anchor_cache, "partner_anchor_cache", 0, g.B));
  RLM_TRY(check_dim(partner_anchor_cache, "partner_anchor_cache", 1, g.T));
  RLM_TRY(check_dim(partner_anchor_cache, "partner_anchor_cache", 2, 2 * g.E));
  for (const rlm_tensor* t : {anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                              anchor_block_std, partner_base, partner_anchor_cache, partner_keys,
                              partner_block_mean, partner_block_std})
    RLM_TRY(aligned16(t, "selection inputs"));
  SelectParams p{};
  RLM_TRY(check_position(position, "position", g, seq, p));
  RLM_TRY(check_outputs(out_anchor, out_anchor_score, "anchor", g, seq, -1));
  RLM_TRY(check_outputs(out_partner, out_partner_score, "partner", g, seq, k_out));
  ExpandRowParams xr{};
  if (xrow != nullptr) {
    RLM_REQUIRE(!seq, "the expanded-cache row is computed with the decode form only");
    const hipError_t xe = fill_expand_row(*xrow, g, position, ring, xr);
    if (xe != hipSuccess) return xe;
  }
  ExpandRowParams xs{};
  if (xseq != nullptr) {
    RLM_REQUIRE(seq, "the whole expanded cache is computed with the sequence form only");
    // The row-wise checks of the decode form's expanded row (position unused).
    const hipError_t xe = fill_expand_row(*xseq, g, position, false, xs);
    if (xe != hipSuccess) return xe;
  }
  hipError_t err = finish_params(p, g, local_window, top_blocks, k_out, strict_valid,
                                 act == RLM_F32 ? 4 : 2);
  if (err != hipSuccess) return err;
  p.aq = anchor_query->data;
  p.arq = anchor_router_query->data;
  p.as = make_stream(anchor_keys, anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias);
  p.pq = partner_base->data;
  p.pq_row = 2 * g.E;
  p.prq = static_cast<const char*>(partner_base->data) +
          static_cast<size_t>(g.E) * (act == RLM_F32 ? 4 : 2);
  p.prq_row = 2 * g.E;
  p.pcache = partner_anchor_cache->data;
  p.ps = make_stream(partner_keys, partner_block_mean, partner_block_std, partner_gamma,
                     partner_bias);
  p.out_anchor = static_cast<int32_t*>(out_anchor->data);
  p.out_anchor_score = static_cast<float*>(out_anchor_score->data);
  p.out_partner = static_cast<int32_t*>(out_partner->data);
  p.out_partner_score = static_cast<float*>(out_partner_score->data);
  if (seq && !ring && tile_path_enabled()) {
    // bf16 activations, 64-wide exact and router vectors, caches of at most 512
    // rows: the matrix-core-filtered kernel (rlm_select_tile.hip).
    TileParams tp{};
    if (tile_params(p, g, act, stat, position, anchor_query, anchor_router_query,
                    partner_base, partner_anchor_cache, anchor_keys, partner_keys,
                    anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                    partner_block_mean, partner_block_std, partner_gamma, partner_bias, tp)) {
      // The whole expanded cache by the same launch when its 128 x 128 tiles
      // fit the key rows' LDS (two tiles of 128 rows x R bf16, then the tile's
      // bf16 outputs at a row stride of 136) and N is whole tiles; otherwise a
      // GEMM launch after the selection.
      const int64_t stage_bytes = std::max<int64_t>(2 * 128 * 32 * xs.KS * 2, 128 * 136 * 2);
      const bool fused = xseq != nullptr && xs.N % 128 == 0 && stage_bytes <= g.T * 128;
      if (fused) {
        tp.x_op = xs.op;
        tp.x_w = xs.w;
        tp.x_bias = xs.bias;
        tp.x_bias_dtype = xs.bias_dtype;
        tp.x_out = xs.cache;
        tp.x_rows = g.B * g.T;
        tp.x_KS = xs.KS;
        tp.x_N = xs.N;
        tp.x_op_bytes = xs.op_bytes;
        tp.x_w_bytes = xs.w_bytes;
      }
      const hipError_t te = select_tile_launch(tp, stat, stream);
      if (te != hipSuccess || xseq == nullptr || fused) return te;
      return expand_seq_linear(*xseq, g, stream);
    }
  }
  if (ring) {
    RLM_REQUIRE(!seq, "ring-buffer caches are supported by the decode form only");
    RLM_REQUIRE((g.T & (g.T - 1)) == 0 && static_cast<int64_t>(g.NB) * g.BS == g.T,
                "ring-buffer caches need a power-of-two cache length split into whole blocks "
                "(cache length %lld, %d blocks)",
                (long long)g.T, g.NB);
  }
  if (!seq && decode_path_enabled()) {
    // 16-bit activations, 4 router heads of 16, caches of at most 512 rows:
    // the latency-oriented decode kernel (rlm_select_decode.hip).
    DecodeParams dp{};
    if (decode_params(p, g, act, stat, position, anchor_query, anchor_router_query, partner_base,
                      partner_anchor_cache, anchor_keys, partner_keys, anchor_block_mean,
                      anchor_block_std, anchor_gamma, anchor_bias, partner_block_mean,
                      partner_block_std, partner_gamma, partner_bias, dp)) {
      if (xrow != nullptr) {
        // The expanded row on workgroups beside the B selection workgroups.
        dp.x = xr;
        dp.xgroups = (xr.N + kExpandCols - 1) / kExpandCols;
      }
      return select_decode_launch(dp, act, stat, ring, stream);
    }
  }
  const hipError_t se = ring ? launch_select<kPacked, true>(p, act, stat, stream)
                             : launch_select<kPacked>(p, act, stat, stream);
  if (se != hipSuccess) return se;
  if (xseq != nullptr) return expand_seq_linear(*xseq, g, stream);
  if (xrow == nullptr) return se;
  return expand_row_launch(xr, stream);
}

bool check_slot_rows(const rlm_tensor* t, const char* name, int64_t d0, int64_t d1, int64_t S,
                     int64_t width, int act) {
  return check_tensor(t, name, 4) && check_dim(t, name, 0, d0) && check_dim(t, name, 1, d1) &&
         check_dim(t, name, 2, S) && check_dim(t, name, 3, width) && check_dtype_is(t, name, act);
}

// The multi-anchor selection takes the matrix-core-filtered kernel where it
// applies unless RLM_MULTI_TILE=0 (both kernels give identical results; the
// switch exists for comparisons).
bool multi_tile_path_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("RLM_MULTI_TILE");
    return v == nullptr || v[0] != '0';
  }();
  return on;
}

// Fills the multi-anchor tile kernel's parameters when the shapes fit it:
// bf16 activations, 64-wide exact and router vectors, whole blocks of at least
// 16 rows, at most 64 blocks and 1024 candidates.
bool multi_tile_params(const SelectParams& p, const MultiParams& m, const Geometry& g, int act,
                       int stat, const rlm_tensor* positions, MultiTileParams& tp) {
  if (act != RLM_BF16 || (stat != RLM_F32 && stat != RLM_BF16)) return false;
  if (g.E != 64 || g.H * g.HD != 64 || g.H > kMultiTileMaxHeads || g.HD % 4 != 0 ||
      (g.H & (g.H - 1)) != 0)
    return false;
  if (static_cast<int64_t>(g.NB) * g.BS != g.T || g.BS < 16 || g.BS % 16 != 0) return false;
  if (g.NB > kMultiTileMaxBlocks || g.NB % 4 != 0) return false;
  if (p.CAP > kMultiTileMaxCap || p.TOP > kMultiTileMaxTop || p.K < 1 || p.K > kMultiTileMaxK)
    return false;
  if (m.S > kMultiTileMaxSlots || g.H * g.RB > 512) return false;
  tp.B = g.B;
  tp.Tq = g.Tq;
  tp.T = g.T;
  tp.S = m.S;
  tp.NB = g.NB;
  tp.BS = g.BS;
  tp.BS_log2 = p.BS_log2;
  tp.L = p.L;
  tp.TOP = p.TOP;
  tp.K = p.K;
  tp.CAP = p.CAP;
  tp.H = g.H;
  tp.H_log2 = p.H_log2;
  tp.HD = g.HD;
  tp.RB = g.RB;
  tp.strict = p.strict;
  tp.exact_scale = p.exact_scale;
  tp.head_scale = p.head_scale;
  tp.pos = positions->data;
  tp.pos_dtype = positions->dtype;
  tp.pos_sb = p.pos_sb;
  tp.pos_sq = p.pos_sq;
  tp.pos_count = p.pos_sb == 0 ? g.Tq : g.B * g.Tq;
  tp.aq = static_cast<const bf16*>(p.aq);
  tp.arq = static_cast<const bf16*>(p.arq);
  tp.pbase = static_cast<const bf16*>(p.pq);
  tp.pcache = static_cast<const bf16*>(p.pcache);
  tp.akeys = static_cast<const bf16*>(p.as.keys);
  tp.pkeys = static_cast<const bf16*>(p.ps.keys);
  tp.key_bytes = p.key_bytes;
  tp.amean = p.as.mean;
  tp.astd = p.as.stdev;
  tp.pmean = p.ps.mean;
  tp.pstd = p.ps.stdev;
  tp.agamma = p.as.gamma;
  tp.pgamma = p.ps.gamma;
  tp.abias = p.as.bias;
  tp.pbias = p.ps.bias;
  tp.agamma_dtype = p.as.gamma_dtype;
  tp.pgamma_dtype = p.ps.gamma_dtype;
  tp.abias_dtype = p.as.bias_dtype;
  tp.pbias_dtype = p.ps.bias_dtype;
  tp.out_anchor = p.out_anchor;
  tp.out_anchor_score = p.out_anchor_score;
  tp.out_partner = p.out_partner;
  tp.out_partner_score = p.out_partner_score;
  tp.tiles = static_cast<int>((g.Tq + 15) / 16);
  return multi_tile_layout(tp);
}

hipError_t multi_select_impl(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(anchor_query, "anchor_query", 4));
  RLM_TRY(check_dtype_float(anchor_query, "anchor_query"));
  RLM_TRY(check_tensor(anchor_keys, "anchor_keys", 4));
  RLM_TRY(check_tensor(anchor_block_mean, "anchor_block_mean", 4));
  RLM_TRY(check_tensor(anchor_bias, "anchor_bias", 2));
  Geometry g;
  g.B = anchor_query->shape[0];
  g.Tq = anchor_query->shape[1];
  const int64_t S = anchor_query->shape[2];
  g.E = static_cast<int>(anchor_query->shape[3]);
  g.T = anchor_keys->shape[1];
  g.NB = static_cast<int>(anchor_block_mean->shape[1]);
  g.H = static_cast<int>(anchor_block_mean->shape[2]);
  g.HD = static_cast<int>(anchor_block_mean->shape[3]);
  g.RB = static_cast<int>(anchor_bias->shape[1]);
  RLM_REQUIRE(S >= 1 && S <= kMaxSlots, "anchor slots must be in [1, %d], got %lld", kMaxSlots,
              (long long)S);
  RLM_REQUIRE(local_window >= S,
              "local_window (%lld) must be >= anchor slots (%lld): every active slot needs a "
              "distinct local candidate",
              (long long)local_window, (long long)S);
  RLM_REQUIRE(g.NB >= 1 && g.T >= g.NB, "need 1 <= blocks <= cache length");
  g.BS = static_cast<int>(g.T / g.NB);
  const int act = anchor_query->dtype;
  const int stat = anchor_block_mean->dtype;
  const int elem = act == RLM_F32 ? 4 : 2;
  const int RD = g.H * g.HD;
  RLM_TRY(check_slot_rows(anchor_keys, "anchor_keys", g.B, g.T, S, g.E, act));
  RLM_TRY(check_slot_rows(partner_keys, "partner_keys", g.B, g.T, S, g.E, act));
  RLM_TRY(check_slot_rows(partner_base, "partner_base", g.B, g.Tq, S, g.E + RD, act));
  RLM_TRY(check_slot_rows(partner_anchor_cache, "partner_anchor_cache", g.B, g.T, S, g.E + RD,
                          act));
  RLM_TRY(check_router_side(anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            "anchor", g, stat));
  RLM_TRY(check_router_side(partner_block_mean, partner_block_std, partner_gamma, partner_bias,
                            "partner", g, stat));
  RLM_TRY(check_tensor(anchor_router_query, "anchor_router_query", 3));
  RLM_TRY(check_dtype_is(anchor_router_query, "anchor_router_query", act));
  RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", 0, g.B));
  RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", 1, g.Tq));
  RLM_TRY(check_dim(anchor_router_query, "anchor_router_query", 2, RD));
  RLM_REQUIRE(((g.E + RD) * elem) % 16 == 0,
              "partner_base rows (exact dim + router dim) must be a multiple of 16 bytes");
  for (const rlm_tensor* t : {anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                              anchor_block_std, partner_base, partner_anchor_cache, partner_keys,
                              partner_block_mean, partner_block_std})
    RLM_TRY(aligned16(t, "multi-anchor selection inputs"));
  SelectParams p{};
  RLM_TRY(check_position(positions, "positions", g, true, p));
  {
    const rlm_tensor* outs[2] = {out_anchor, out_anchor_score};
    const int types[2] = {RLM_I32, RLM_F32};
    const char* names[2] = {"out_anchor", "out_anchor_score"};
    for (int i = 0; i < 2; ++i) {
      RLM_TRY(check_tensor(outs[i], names[i], 3));
      RLM_TRY(check_dtype_is(outs[i], names[i], types[i]));
      RLM_TRY(check_dim(outs[i], names[i], 0, g.B));
      RLM_TRY(check_dim(outs[i], names[i], 1, g.Tq));
      RLM_TRY(check_dim(outs[i], names[i], 2, S));
    }
  }
  RLM_TRY(check_slot_rows(out_partner, "out_partner", g.B, g.Tq, S, k_out, RLM_I32));
  RLM_TRY(check_slot_rows(out_partner_score, "out_partner_score", g.B, g.Tq, S, k_out, RLM_F32));
  hipError_t err = finish_params(p, g, local_window, top_blocks, k_out, strict_valid, elem);
  if (err != hipSuccess) return err;
  // LDS: partner statistics and bias table (when the statistic count is a
  // power of two), then the per-wave regions.  No key windows.
  p.WR = 0;
  const int stats_bytes = 2 * g.NB * RD * 4;
  const bool stats_pow2 = ((g.NB * RD / 4) & (g.NB * RD / 4 - 1)) == 0 && g.NB * RD >= 4;
  const int bias_bytes = ((g.H * g.RB * 4) + 15) & ~15;
  p.off_stats_a = p.off_bias_a = p.off_win_a = p.off_win_p = 0;
  p.off_stats_p = p.off_bias_p = 0;
  int off = 0;
  p.stage = p.W > 1 && stats_pow2 && stats_bytes + bias_bytes + p.W * p.wave_bytes <= 80 * 1024;
  if (p.stage) {
    p.off_stats_p = 0;
    p.off_bias_p = stats_bytes;
    off = stats_bytes + bias_bytes;
  }
  p.off_wave = off;
  off += p.W * p.wave_bytes;
  RLM_REQUIRE(off <= 160 * 1024,
              "selection working set (%d bytes of LDS) exceeds the 160 KiB of one CU", off);
  p.lds_total = off;
  const int64_t key_bytes = g.B * g.T * S * g.E * elem;
  RLM_REQUIRE(key_bytes < (int64_t(1) << 31), "key caches must be smaller than 2 GiB");
  p.key_bytes = static_cast<uint32_t>(key_bytes);
  p.aq = anchor_query->data;
  p.arq = anchor_router_query->data;
  p.as = make_stream(anchor_keys, anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias);
  p.pq = partner_base->data;
  p.pcache = partner_anchor_cache->data;
  p.ps = make_stream(partner_keys, partner_block_mean, partner_block_std, partner_gamma,
                     partner_bias);
  p.out_anchor = static_cast<int32_t*>(out_anchor->data);
  p.out_anchor_score = static_cast<float*>(out_anchor_score->data);
  p.out_partner = static_cast<int32_t*>(out_partner->data);
  p.out_partner_score = static_cast<float*>(out_partner_score->data);
  MultiParams m;
  m.S = static_cast<int>(S);
  m.slot_bytes = static_cast<uint32_t>(g.E * elem);
  m.key_pos_bytes = static_cast<uint32_t>(S * g.E * elem);
  m.qrow = g.E + RD;
  const int64_t queries = g.B * g.Tq;
  if (queries == 0) return hipSuccess;
  if (multi_tile_path_enabled()) {
    MultiTileParams tp{};
    if (multi_tile_params(p, m, g, act, stat, positions, tp))
      return multi_tile_launch(tp, stat, stream);
  }
  const dim3 block(p.W * kWave);
  const dim3 grid(static_cast<unsigned>(g.B * p.tiles));
  const size_t lds = static_cast<size_t>(p.lds_total);
#define RLM_MULTI_CASE(TA_ID, TA, TS_ID, TS)                                           \
  if (act == TA_ID && stat == TS_ID) {                                                 \
    hipLaunchKernelGGL((multi_select_kernel<TA, TS>), grid, block, lds, stream, p, m); \
    return launch_status("multi_relation_select");                                     \
  }
  RLM_MULTI_CASE(RLM_F32, float, RLM_F32, float)
  RLM_MULTI_CASE(RLM_BF16, bf16, RLM_F32, float)
  RLM_MULTI_CASE(RLM_BF16, bf16, RLM_BF16, bf16)
#undef RLM_MULTI_CASE
  set_error("multi_relation_select: unsupported dtype combination (activations %s, stats %s)",
            dtype_name(act), dtype_name(stat));
  return hipErrorInvalidValue;
}

}  // namespace
}  // namespace rlm

using namespace rlm;

extern "C" hipError_t rlm_relation_select_packed(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  return select_packed_impl(false, false, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, position,
                            local_window, top_blocks, k_out, strict_valid, out_anchor,
                            out_anchor_score, out_partner, out_partner_score, stream);
}

extern "C" hipError_t rlm_relation_select_packed_seq(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  return select_packed_impl(true, false, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, positions,
                            local_window, top_blocks, k_out, strict_valid, out_anchor,
                            out_anchor_score, out_partner, out_partner_score, stream);
}

extern "C" hipError_t rlm_relation_select_packed_seq_expand(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* operand_cache, const rlm_tensor* expanded_weight,
    const rlm_tensor* expanded_bias, const rlm_tensor* expanded_cache,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  const RowArgs x{operand_cache, expanded_weight, expanded_bias, expanded_cache};
  return select_packed_impl(true, false, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, positions,
                            local_window, top_blocks, k_out, strict_valid, out_anchor,
                            out_anchor_score, out_partner, out_partner_score, stream, nullptr,
                            &x);
}
extern "C" hipError_t rlm_relation_select_packed_expand_row(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* operand_cache, const rlm_tensor* expanded_weight,
    const rlm_tensor* expanded_bias, const rlm_tensor* expanded_cache, int32_t ring,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  const RowArgs x{operand_cache, expanded_weight, expanded_bias, expanded_cache};
  return select_packed_impl(false, ring != 0, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, position,
                            local_window, top_blocks, k_out, strict_valid, out_anchor,
                            out_anchor_score, out_partner, out_partner_score, stream, &x);
}

extern "C" hipError_t rlm_relation_select_packed_ring(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  return select_packed_impl(false, true, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, position,
                            local_window, top_blocks, k_out, strict_valid, out_anchor,
                            out_anchor_score, out_partner, out_partner_score, stream);
}

extern "C" hipError_t rlm_anchor_select(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* router_query, const rlm_tensor* block_mean, const rlm_tensor* block_std,
    const rlm_tensor* gamma, const rlm_tensor* bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int32_t strict_valid, const rlm_tensor* out_index,
    const rlm_tensor* out_score, hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(anchor_query, "anchor_query", 2));
  RLM_TRY(check_dtype_float(anchor_query, "anchor_query"));
  RLM_TRY(check_tensor(anchor_keys, "anchor_keys", 3));
  RLM_TRY(check_tensor(block_mean, "block_mean", 4));
  RLM_TRY(check_tensor(bias, "bias", 2));
  Geometry g;
  g.B = anchor_query->shape[0];
  g.Tq = 1;
  g.E = static_cast<int>(anchor_query->shape[1]);
  g.T = anchor_keys->shape[1];
  g.NB = static_cast<int>(block_mean->shape[1]);
  g.H = static_cast<int>(block_mean->shape[2]);
  g.HD = static_cast<int>(block_mean->shape[3]);
  g.RB = static_cast<int>(bias->shape[1]);
  RLM_REQUIRE(g.NB >= 1 && g.T >= g.NB, "need 1 <= blocks <= cache length");
  g.BS = static_cast<int>(g.T / g.NB);
  const int act = anchor_query->dtype;
  const int stat = block_mean->dtype;
  RLM_TRY(check_stream(anchor_keys, block_mean, block_std, gamma, bias, "anchor", g, act, stat));
  RLM_TRY(check_tensor(router_query, "router_query", 2));
  RLM_TRY(check_dtype_is(router_query, "router_query", act));
  RLM_TRY(check_dim(router_query, "router_query", 0, g.B));
  RLM_TRY(check_dim(router_query, "router_query", 1, g.H * g.HD));
  for (const rlm_tensor* t : {anchor_query, anchor_keys, router_query, block_mean, block_std})
    RLM_TRY(aligned16(t, "anchor_select inputs"));
  SelectParams p{};
  RLM_TRY(check_position(position, "position", g, false, p));
  RLM_TRY(check_outputs(out_index, out_score, "index", g, false, -1));
  hipError_t err = finish_params(p, g, local_window, top_blocks, 0, strict_valid,
                                 act == RLM_F32 ? 4 : 2);
  if (err != hipSuccess) return err;
  p.aq = anchor_query->data;
  p.arq = router_query->data;
  p.as = make_stream(anchor_keys, block_mean, block_std, gamma, bias);
  p.out_anchor = static_cast<int32_t*>(out_index->data);
  p.out_anchor_score = static_cast<float*>(out_score->data);
  return launch_select<kAnchorOnly>(p, act, stat, stream);
}

extern "C" hipError_t rlm_partner_topk(
    const rlm_tensor* partner_query, const rlm_tensor* partner_keys,
    const rlm_tensor* router_query, const rlm_tensor* block_mean, const rlm_tensor* block_std,
    const rlm_tensor* gamma, const rlm_tensor* bias, const rlm_tensor* position,
    const rlm_tensor* anchor_index, int64_t local_window, int64_t top_blocks, int64_t k_out,
    int32_t strict_valid, const rlm_tensor* out_index, const rlm_tensor* out_score,
    hipStream_t stream) {
  clear_error();
  RLM_TRY(check_tensor(partner_query, "partner_query", 2));
  RLM_TRY(check_dtype_float(partner_query, "partner_query"));
  RLM_TRY(check_tensor(partner_keys, "partner_keys", 3));
  RLM_TRY(check_tensor(block_mean, "block_mean", 4));
  RLM_TRY(check_tensor(bias, "bias", 2));
  Geometry g;
  g.B = partner_query->shape[0];
  g.Tq = 1;
  g.E = static_cast<int>(partner_query->shape[1]);
  g.T = partner_keys->shape[1];
  g.NB = static_cast<int>(block_mean->shape[1]);
  g.H = static_cast<int>(block_mean->shape[2]);
  g.HD = static_cast<int>(block_mean->shape[3]);
  g.RB = static_cast<int>(bias->shape[1]);
  RLM_REQUIRE(g.NB >= 1 && g.T >= g.NB, "need 1 <= blocks <= cache length");
  g.BS = static_cast<int>(g.T / g.NB);
  const int act = partner_query->dtype;
  const int stat = block_mean->dtype;
  RLM_TRY(check_stream(partner_keys, block_mean, block_std, gamma, bias, "partner", g, act, stat));
  RLM_TRY(check_tensor(router_query, "router_query", 2));
  RLM_TRY(check_dtype_is(router_query, "router_query", act));
  RLM_TRY(check_dim(router_query, "router_query", 0, g.B));
  RLM_TRY(check_dim(router_query, "router_query", 1, g.H * g.HD));
  RLM_TRY(check_tensor(anchor_index, "anchor_index", 1));
  RLM_REQUIRE(is_index_dtype(anchor_index->dtype), "anchor_index: expected int32/int64");
  RLM_TRY(check_dim(anchor_index, "anchor_index", 0, g.B));
  for (const rlm_tensor* t : {partner_query, partner_keys, router_query, block_mean, block_std})
    RLM_TRY(aligned16(t, "partner_topk inputs"));
  SelectParams p{};
  RLM_TRY(check_position(position, "position", g, false, p));
  RLM_TRY(check_outputs(out_index, out_score, "index", g, false, k_out));
  hipError_t err = finish_params(p, g, local_window, top_blocks, k_out, strict_valid,
                                 act == RLM_F32 ? 4 : 2);
  if (err != hipSuccess) return err;
  p.pq = partner_query->data;
  p.pq_row = g.E;
  p.prq = router_query->data;
  p.prq_row = static_cast<int64_t>(g.H) * g.HD;
  p.pcache = nullptr;
  p.ps = make_stream(partner_keys, block_mean, block_std, gamma, bias);
  p.anchor_in = anchor_index->data;
  p.anchor_dtype = anchor_index->dtype;
  p.out_partner = static_cast<int32_t*>(out_index->data);
  p.out_partner_score = static_cast<float*>(out_score->data);
  return launch_select<kPartnerOnly>(p, act, stat, stream);
}

extern "C" hipError_t rlm_multi_relation_select_seq(
    const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* positions,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
  return multi_select_impl(anchor_query, anchor_keys, anchor_router_query, anchor_block_mean,
                           anchor_block_std, anchor_gamma, anchor_bias, partner_base,
                           partner_anchor_cache, partner_keys, partner_block_mean,
                           partner_block_std, partner_gamma, partner_bias, positions,
                           local_window, top_blocks, k_out, strict_valid, out_anchor,
                           out_anchor_score, out_partner, out_partner_score, stream);
}

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
// Mapping.  A workgroup of 4 waves owns 16 queries of one batch row; each
// query has a group of 16 lanes (4 queries per wave).  Per stream:
//   1. the batch row's keys [0, nrows) are staged in LDS (nrows = one past the
//      largest position of the workgroup's queries, rounded up to 16);
//   2. the matrix cores score every staged key against the 16 queries,
//      s~[row][query] = bf16 MFMA (fp32 accumulation) -- the partner query is
//      fp32 and enters as a bf16 hi + lo pair;
//   3. each query's 16 lanes compute its block scores (lane = block, float64),
//      rank them into the TOP picks, and read s~ of their candidates (lane l
//      holds candidates l, l + 16, ...);
//   4. with theta a lower bound of the k-th largest s~ among the valid
//      candidates (the k-th largest of the lanes' maxima) and eps a bound on
//      |s~ - s| (below), every candidate with s~ >= theta - 2 eps is a member;
//      at least k candidates have s >= theta - eps, strictly above every
//      non-member, so the exact top-k lies among the members;
//   5. the members get their exact float64 scores (4 lanes per member, 16
//      dims each) and are ranked by (score, tie index) into the top-k.
// Members are processed in windows of 64 per query, each merged into a running
// top-k, so any number of near-ties (duplicate keys) is handled.
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

namespace rlm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int kQ = 16;          // queries per workgroup
constexpr int kThreads = 256;   // 4 waves
constexpr int kRowBytes = 128;  // one staged key row (64 bf16)
constexpr int kSQ = 18;         // floats per s~ row (16 queries + 2 pad: conflict-free column reads)
constexpr int kStatRow = 66;    // doubles per staged statistics row (64 + 2 pad)
constexpr int kRqRow = 66;      // doubles per router-query row
constexpr int kPqRow = 68;      // floats per partner-query row
constexpr int kListCap = 64;    // members per query per window
constexpr int kMaxNCL = 16;     // candidates per lane (CAP <= 256)
constexpr float kErrScale = 1.220703125e-4f;          // 2^-13
constexpr float kErrAbs = 7.888609052210118e-31f;     // 2^-100

// Per-query record in LDS.
struct QRec {
  int t, ls, anchor, members;
  int ntop, nwin, cur, pad;
  float theta, pad1, pad2, pad3;
  int sel[kTileMaxTop];
  int selv[kTileMaxTop];
};

struct Lds {
  unsigned char* keys;  // [nrows][128 B], 16-byte chunks XOR-swizzled by row
  float* sc;            // [T][kSQ]
  double* stats;        // [2][NB][kStatRow] (mean rows, then std rows)
  double* rq;           // [16][kRqRow]
  float* pq;            // [16][kPqRow]
  float* blk;           // [16][NB + 4]
  float* lmax;          // [16][16]
  uint64_t* list;       // [16][kListCap]
  uint64_t* top;        // [2][16][kTileMaxK]
  QRec* qr;             // [16]
  double* bias;         // [H*RB]
  double* sp;           // [16]
  uint32_t* kmax;       // [4] per-wave max |key| bits
};

__device__ __forceinline__ Lds carve(const TileParams& p, unsigned char* smem) {
  Lds s;
  s.keys = smem + p.off_keys;
  s.sc = reinterpret_cast<float*>(smem + p.off_sc);
  s.stats = reinterpret_cast<double*>(smem + p.off_stats);
  s.rq = reinterpret_cast<double*>(smem + p.off_rq);
  s.pq = reinterpret_cast<float*>(smem + p.off_pq);
  s.blk = reinterpret_cast<float*>(smem + p.off_blk);
  s.lmax = reinterpret_cast<float*>(smem + p.off_lmax);
  s.list = reinterpret_cast<uint64_t*>(smem + p.off_list);
  s.top = reinterpret_cast<uint64_t*>(smem + p.off_top);
  s.qr = reinterpret_cast<QRec*>(smem + p.off_qrec);
  s.bias = reinterpret_cast<double*>(smem + p.off_bias);
  s.sp = reinterpret_cast<double*>(smem + p.off_sp);
  s.kmax = reinterpret_cast<uint32_t*>(smem + p.off_kmax);
  return s;
}

__device__ __forceinline__ int key_chunk_offset(int row, int ch) {
  return row * kRowBytes + 16 * (ch ^ ((row >> 1) & 7));
}

__device__ __forceinline__ int clamp_pos(int64_t v) {
  constexpr int64_t kLim = int64_t(1) << 30;
  return static_cast<int>(v < -kLim ? -kLim : (v > kLim ? kLim : v));
}

__device__ __forceinline__ int load_pos(const TileParams& p, int64_t b, int64_t tq) {
  return clamp_pos(load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq));
}

// Max |x| bits of eight bf16 values (two per 32-bit word), packed 16-bit max.
__device__ __forceinline__ u16x2_t absmax8(const uint4& v, u16x2_t m) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, w[i] & 0x7fff7fffu));
  return m;
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = umax32(v, dpp_u32<kDppXor1>(v));
  v = umax32(v, dpp_u32<kDppXor2>(v));
  v = umax32(v, dpp_u32<kDppHalfMirror>(v));
  v = umax32(v, dpp_u32<kDppMirror>(v));
  uint32_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    best = umax32(best, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16 * r)));
  return best;
}

// Values over the 16 lanes of a DPP row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v))));
  return v;
}
__device__ __forceinline__ int row16_sum_i(int v) {
  v += static_cast<int>(dpp_u32<kDppXor1>(static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp_u32<kDppXor2>(static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp_u32<kDppHalfMirror>(static_cast<uint32_t>(v)));
  v += static_cast<int>(dpp_u32<kDppMirror>(static_cast<uint32_t>(v)));
  return v;
}
// Inclusive prefix sum over the 16 lanes of a row (row_shr steps; lanes that
// shift in from outside the row add 0).
__device__ __forceinline__ int row16_scan_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  return v;
}
// Wave-uniform maximum of a value that is uniform within each 16-lane row.
__device__ __forceinline__ int rows_max_i(int v) {
  int m = __builtin_amdgcn_readlane(v, 0);
  m = max(m, __builtin_amdgcn_readlane(v, 16));
  m = max(m, __builtin_amdgcn_readlane(v, 32));
  m = max(m, __builtin_amdgcn_readlane(v, 48));
  return m;
}

__device__ __forceinline__ f32x4_t mfma_bf16(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Eight fp32 -> bf16 hi (round to nearest even) and bf16 lo = bf16(x - hi).
__device__ __forceinline__ void split_hi_lo(const float (&x)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    const float h0 = __uint_as_float(h[i] << 16);
    const float h1 = __uint_as_float(h[i] & 0xffff0000u);
    l[i] = pack_bf16x2(x[2 * i] - h0, x[2 * i + 1] - h1);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

template <typename TS>
__device__ __forceinline__ void load_stat8(const TS* src, float (&out)[8]);
template <>
__device__ __forceinline__ void load_stat8<float>(const float* src, float (&out)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(src);
  const float4 c = *reinterpret_cast<const float4*>(src + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
}
template <>
__device__ __forceinline__ void load_stat8<bf16>(const bf16* src, float (&out)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(src);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// One stream's constant inputs.
struct Side {
  const bf16* keys;  // [B,T,64]
  const void* mean;  // [B,NB,64]
  const void* stdv;
  const void* gamma;
  const void* bias;
  int gamma_dtype, bias_dtype;
};

template <int NBL>
struct StatRegs {
  float v[NBL][8];
};

// Statistics elements owned by thread tid: 8 consecutive elements of the
// concatenation [mean (NB*64) | std (NB*64)] per unit u < NBL.
template <typename TS, int NBL>
__device__ __forceinline__ void fetch_stats(const TileParams& p, const Side& s, int64_t b, int tid,
                                            StatRegs<NBL>& r) {
  const int half = p.NB * 64;
#pragma unroll
  for (int u = 0; u < NBL; ++u) {
    int e = 8 * (tid + kThreads * u);
    e = e < 2 * half ? e : 0;  // threads past the statistics re-read element 0 (not stored)
    const bool is_std = e >= half;
    const int k = is_std ? e - half : e;
    const TS* src = static_cast<const TS*>(is_std ? s.stdv : s.mean) + b * half + k;
    load_stat8<TS>(src, r.v[u]);
  }
}
template <int NBL>
__device__ __forceinline__ void put_stats(const TileParams& p, const Lds& L, int tid,
                                          const StatRegs<NBL>& r) {
  const int half = p.NB * 64;
#pragma unroll
  for (int u = 0; u < NBL; ++u) {
    const int e = 8 * (tid + kThreads * u);
    if (e >= 2 * half) continue;
    const int which = e >= half ? 1 : 0;
    const int k = e - which * half;
    const int j = k >> 6, d = k & 63;
    double* dst = L.stats + (which * p.NB + j) * kStatRow + d;
#pragma unroll
    for (int i = 0; i < 8; i += 2)
      *reinterpret_cast<double2*>(dst + i) =
          make_double2(static_cast<double>(r.v[u][i]), static_cast<double>(r.v[u][i + 1]));
  }
}

// Bias table and softplus(gamma) of one stream into LDS (float64).
__device__ __forceinline__ void put_router_consts(const TileParams& p, const Side& s, const Lds& L,
                                                  int tid) {
  for (int i = tid; i < p.H * p.RB; i += kThreads)
    L.bias[i] = static_cast<double>(load_any_f(s.bias, s.bias_dtype, i));
  if (tid < p.H) {
#pragma clang fp contract(off)
    const double g = static_cast<double>(load_any_f(s.gamma, s.gamma_dtype, tid));
    L.sp[tid] = log(1.0 + exp(g));  // softplus without threshold, relation_select.py:87
  }
}

// Block scores of the group's query (relation_select.py:53-106): lane gl owns
// blocks gl + 16 i.  Writes L.blk[qi][j] (float32, -inf where not eligible).
template <int NBL>
__device__ void block_scores(const TileParams& p, const Lds& L, int qi, int gl, int t, int ls) {
  const double* Q = L.rq + qi * kRqRow;
  const int HD = p.HD;
#pragma unroll
  for (int u = 0; u < NBL; ++u) {
    const int j = gl + 16 * u;
    const int jc = j < p.NB ? j : 0;
    const double* M = L.stats + jc * kStatRow;
    const double* S = L.stats + (p.NB + jc) * kStatRow;
    const int end = (j + 1) * p.BS - 1;
    const int dist = (t > end ? t - end : 0) + 1;
    int bucket = 31 - __clz(dist);
    bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
    double sh[kTileMaxHeads];
    double m = -INFINITY;
    for (int h = 0; h < p.H; ++h) {
      double c = 0.0, uu = 0.0;
      for (int d = h * HD; d < (h + 1) * HD; d += 4) {
        const double2 m0 = *reinterpret_cast<const double2*>(M + d);
        const double2 m1 = *reinterpret_cast<const double2*>(M + d + 2);
        const double2 s0 = *reinterpret_cast<const double2*>(S + d);
        const double2 s1 = *reinterpret_cast<const double2*>(S + d + 2);
        const double2 q0 = *reinterpret_cast<const double2*>(Q + d);
        const double2 q1 = *reinterpret_cast<const double2*>(Q + d + 2);
        c = fma(m0.x, q0.x, c);
        c = fma(m0.y, q0.y, c);
        c = fma(m1.x, q1.x, c);
        c = fma(m1.y, q1.y, c);
        uu = fma(s0.x, fabs(q0.x), uu);
        uu = fma(s0.y, fabs(q0.y), uu);
        uu = fma(s1.x, fabs(q1.x), uu);
        uu = fma(s1.y, fabs(q1.y), uu);
      }
      double v;
      {
#pragma clang fp contract(off)
        const double content = c + L.sp[h] * uu;
        v = content * p.head_scale + L.bias[h * p.RB + bucket];
      }
#pragma unroll
      for (int hh = 0; hh < kTileMaxHeads; ++hh)
        if (hh == h) sh[hh] = v;
      m = fmax(m, v);
    }
    double sum = 0.0;
    for (int h = 0; h < p.H; ++h) {
      double v = 0.0;
#pragma unroll
      for (int hh = 0; hh < kTileMaxHeads; ++hh)
        if (hh == h) v = sh[hh];
      sum += exp(v - m);
    }
    const double lse = m + log(sum);
    const bool eligible = end <= t && (!p.strict || end < ls);
    if (j < p.NB) L.blk[qi * (p.NB + 4) + j] = eligible ? static_cast<float>(lse) : -INFINITY;
  }
}

// TOP picks by rank: block j is pick rank(j) = #{k : key_k > key_j} with key
// (score, lower block first) -- the reference's sequential argmax with ties to
// the lowest block (relation_select.py:229-242).  Picks past the last block
// are block 0, invalid.
template <int NBL>
__device__ void pick_blocks(const TileParams& p, const Lds& L, int qi, int gl) {
  QRec& R = L.qr[qi];
  if (gl < p.TOP) {
    R.sel[gl] = 0;
    R.selv[gl] = 0;
  }
  wave_sync();
  const float* row = L.blk + qi * (p.NB + 4);
#pragma unroll
  for (int u = 0; u < NBL; ++u) {
    const int j = gl + 16 * u;
    if (j < p.NB) {
      const float mine = row[j];
      const uint64_t kj = select_key(mine, static_cast<uint32_t>(j));
      int rank = 0;
      for (int k = 0; k < p.NB; k += 4) {
        const float4 o = *reinterpret_cast<const float4*>(row + k);
        rank += select_key(o.x, k) > kj;
        rank += (k + 1 < p.NB) && select_key(o.y, k + 1) > kj;
        rank += (k + 2 < p.NB) && select_key(o.z, k + 2) > kj;
        rank += (k + 3 < p.NB) && select_key(o.w, k + 3) > kj;
      }
      if (rank < p.TOP) {
        R.sel[rank] = j;
        R.selv[rank] = mine > -1.0e30f ? 1 : 0;
      }
    }
  }
  wave_sync();
}

// Position and validity of candidate lane c (relation_select.py:244-284):
// local window first, then the picks' blocks in pick order.
__device__ __forceinline__ int cand_pos(const TileParams& p, const QRec& R, int c, int t, int ls,
                                        bool& valid) {
  if (c < p.L) {
    const int pos = t - p.L + 1 + c;
    valid = pos >= 0 && pos <= t && pos < p.T;
    return pos;
  }
  const int r = (c - p.L) >> p.BS_log2;
  const int o = (c - p.L) & (p.BS - 1);
  const int pos = R.sel[r] * p.BS + o;
  valid = R.selv[r] != 0 && pos <= t && pos < ls && pos < p.T;
  return pos;
}

// Exact top-k of the group's query among its candidates, from the s~ column
// of query qi.  ANCHOR: k = 1, ties to the lowest position; else ties to the
// lowest candidate lane and `exclude` is not a candidate.  `qf` holds this
// lane's 16 query dims [16 (gl & 3), +16) in float64, `qn1` the query's
// L1 norm.  Leaves the top entries in L.top[R.cur][qi][0..ntop).
template <bool ANCHOR>
__device__ void exact_topk(const TileParams& p, const Lds& L, int qi, int gl, int t, int ls,
                           int exclude, int K, const double (&qf)[16], float qn1, float kmax,
                           bool active) {
  QRec& R = L.qr[qi];
  // Candidates' approximate scores.
  float st[kMaxNCL];
  float lm = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i) {
    st[i] = -INFINITY;
    const int c = gl + 16 * i;
    if (i < p.NCL && c < p.CAP && active) {
      bool v;
      const int pos = cand_pos(p, R, c, t, ls, v);
      if (!ANCHOR) v = v && pos != exclude;
      if (v) st[i] = L.sc[pos * kSQ + qi];
      lm = fmaxf(lm, st[i]);
    }
  }
  // theta: a lower bound of the k-th largest approximate score.
  float theta;
  if (ANCHOR) {
    theta = row16_max(lm);
  } else {
    float* lmr = L.lmax + qi * 16;
    lmr[gl] = lm;
    wave_sync();
    int rank = 0;
#pragma unroll
    for (int k = 0; k < 16; k += 4) {
      const float4 o = *reinterpret_cast<const float4*>(lmr + k);
      rank += (o.x > lm) || (o.x == lm && k < gl);
      rank += (o.y > lm) || (o.y == lm && k + 1 < gl);
      rank += (o.z > lm) || (o.z == lm && k + 2 < gl);
      rank += (o.w > lm) || (o.w == lm && k + 3 < gl);
    }
    if (rank == K - 1) R.theta = lm;
    wave_sync();
    theta = R.theta;
  }
  const float eps = kErrScale * qn1 * kmax;
  const float thr = theta - (2.0f * eps + kErrAbs);
  uint32_t mask = 0;
#pragma unroll
  for (int i = 0; i < kMaxNCL; ++i)
    if (st[i] > -INFINITY && st[i] >= thr) mask |= 1u << i;
  const int own = __builtin_popcount(mask);
  const int off = row16_scan_i(own) - own;
  const int members = row16_sum_i(own);
  const int maxown = static_cast<int>(wave_max_u32(static_cast<uint32_t>(own)));  // lanes differ
  const int nwin = rows_max_i((members + kListCap - 1) / kListCap);

  uint64_t* list = L.list + qi * kListCap;
  int ntop = 0;
  int cur = 0;
  for (int w = 0; w < nwin; ++w) {
    const int lo = w * kListCap;
    const int nw = min(max(members - lo, 0), kListCap);
    uint32_t mm = mask;
    for (int it = 0; it < maxown; ++it) {
      if (mm != 0u) {
        const int i = __builtin_ctz(mm);
        mm &= mm - 1u;
        const int mi = off + it - lo;
        if (mi >= 0 && mi < kListCap) list[mi] = static_cast<uint64_t>(gl + 16 * i);
      }
    }
    wave_sync();
    // Exact scores: member mi = 4 pass + gl/4 on lanes 4(gl/4) .. +3, each lane
    // 16 dims, the four partial sums combined in float64.
    const int s4 = gl & 3;
    const int passes = rows_max_i((nw + 3) >> 2);
    for (int ps = 0; ps < passes; ++ps) {
      const int mi = 4 * ps + (gl >> 2);
      const bool act = mi < nw;
      const int c = act ? static_cast<int>(list[mi]) : 0;
      bool v;
      int pos = cand_pos(p, R, c, t, ls, v);
      pos = act ? pos : 0;
      const unsigned char* krow = L.keys;
      const uint4 k0 = *reinterpret_cast<const uint4*>(krow + key_chunk_offset(pos, 2 * s4));
      const uint4 k1 = *reinterpret_cast<const uint4*>(krow + key_chunk_offset(pos, 2 * s4 + 1));
      const uint32_t w8[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      double d = 0.0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d = fma(static_cast<double>(__uint_as_float(w8[e] << 16)), qf[2 * e], d);
        d = fma(static_cast<double>(__uint_as_float(w8[e] & 0xffff0000u)), qf[2 * e + 1], d);
      }
      d += dpp_f64<kDppXor1>(d);
      d += dpp_f64<kDppXor2>(d);
      const float score = static_cast<float>(d * p.exact_scale);
      if (act && s4 == 0)
        list[mi] = select_key(score, static_cast<uint32_t>(ANCHOR ? pos : c));
    }
    wave_sync();
    // Merge into the running top-k: rank every entry of top[cur] + list.
    const uint64_t* topc = L.top + (cur * kQ + qi) * kTileMaxK;
    uint64_t* topn = L.top + ((cur ^ 1) * kQ + qi) * kTileMaxK;
    const int ntot = ntop + nw;
    const int ntot_max = rows_max_i(ntot);
    for (int e = gl; e < ntot_max; e += 16) {
      if (e < ntot) {
        const uint64_t ke = e < ntop ? topc[e] : list[e - ntop];
        int rank = 0;
        for (int f = 0; f < ntot; ++f) {
          const uint64_t kf = f < ntop ? topc[f] : list[f - ntop];
          rank += kf > ke;
        }
        if (rank < K) topn[rank] = ke;
      }
    }
    ntop = min(K, ntot);
    cur ^= 1;
    wave_sync();
  }
  if (gl == 0) {
    R.ntop = ntop;
    R.cur = cur;
  }
  wave_sync();
}

template <typename TS, int NBL>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1)))
select_tile_kernel(const TileParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Lds L = carve(p, smem);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int gl = lane & 15;
  const int qi = wave * 4 + (lane >> 4);
  const int64_t wg = xcd_tile(blockIdx.x, gridDim.x);
  const int64_t b = wg / p.tiles;
  const int64_t tq0 = (wg - b * p.tiles) * kQ;
  const int64_t tq = tq0 + qi;
  const bool active = tq < p.Tq;
  const int64_t qrow = b * p.Tq + (active ? tq : tq0);

  const Side as{p.akeys, p.amean, p.astd, p.agamma, p.abias, p.agamma_dtype, p.abias_dtype};
  const Side ps{p.pkeys, p.pmean, p.pstd, p.pgamma, p.pbias, p.pgamma_dtype, p.pbias_dtype};

  // ---- Positions: the group's own, and the workgroup's largest. ----
  const int t = load_pos(p, b, active ? tq : tq0);
  const int ls = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
  int tmax = -1;
  for (int i = 0; i < kQ; ++i) {
    const int64_t ti = tq0 + i < p.Tq ? tq0 + i : tq0;
    tmax = max(tmax, load_pos(p, b, ti));
  }
  int nrows = tmax + 1 < p.T ? tmax + 1 : static_cast<int>(p.T);
  nrows = nrows < 0 ? 0 : ((nrows + 15) & ~15);
  const int nchunks = nrows * 8;

  // ---- One round of loads: both streams' keys and statistics, the anchor
  //      query pieces. ----
  const uint32_t row_bytes_b = static_cast<uint32_t>(p.T) * kRowBytes;
  const rsrc_t akr = make_rsrc(p.akeys + b * p.T * 64, row_bytes_b);
  const rsrc_t pkr = make_rsrc(p.pkeys + b * p.T * 64, row_bytes_b);
  uint4 akv[16], pkv[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int k = tid + kThreads * u;
    const uint32_t off = k < nchunks ? static_cast<uint32_t>(k) * 16u : kNoOffset;
    akv[u] = buf_load_b128(akr, off);
    pkv[u] = buf_load_b128(pkr, off);
  }
  StatRegs<NBL> ast, pst;
  fetch_stats<TS, NBL>(p, as, b, tid, ast);
  // MFMA A fragments of the anchor query: row lane%16 of the workgroup.
  const int64_t arow = b * p.Tq + (tq0 + gl < p.Tq ? tq0 + gl : tq0);
  const int g4 = lane >> 4;
  const uint4 a0 = *reinterpret_cast<const uint4*>(p.aq + arow * 64 + 8 * g4);
  const uint4 a1 = *reinterpret_cast<const uint4*>(p.aq + arow * 64 + 32 + 8 * g4);
  // This lane's 16 exact-query dims, [16 (gl & 3), +16).
  const int s4 = gl & 3;
  const uint4 q0 = *reinterpret_cast<const uint4*>(p.aq + qrow * 64 + 16 * s4);
  const uint4 q1 = *reinterpret_cast<const uint4*>(p.aq + qrow * 64 + 16 * s4 + 8);
  // Router query: thread -> query tid/16, dims 4 (tid % 16) .. +3.
  const int rq_q = tid >> 4, rq_d = 4 * (tid & 15);
  const int64_t rq_row = b * p.Tq + (tq0 + rq_q < p.Tq ? tq0 + rq_q : tq0);
  const uint2 arq_v = *reinterpret_cast<const uint2*>(p.arq + rq_row * 64 + rq_d);

  // ---- Anchor side: stage keys, statistics, router query, bias. ----
  u16x2_t km = {0, 0};
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int k = tid + kThreads * u;
    if (k < nchunks) {
      *reinterpret_cast<uint4*>(L.keys + key_chunk_offset(k >> 3, k & 7)) = akv[u];
      km = absmax8(akv[u], km);
    }
  }
  uint32_t kbits = umax32(km.x, km.y);
  kbits = wave_max_u32(kbits);
  if (lane == 0) L.kmax[wave] = kbits;
  put_stats<NBL>(p, L, tid, ast);
  {
    double* dst = L.rq + rq_q * kRqRow + rq_d;
    *reinterpret_cast<double2*>(dst) = make_double2(static_cast<double>(__uint_as_float(arq_v.x << 16)),
                                                    static_cast<double>(__uint_as_float(arq_v.x & 0xffff0000u)));
    *reinterpret_cast<double2*>(dst + 2) = make_double2(static_cast<double>(__uint_as_float(arq_v.y << 16)),
                                                        static_cast<double>(__uint_as_float(arq_v.y & 0xffff0000u)));
  }
  put_router_consts(p, as, L, tid);
  double qf[16];
  float qn1 = 0.0f;
  {
    const uint32_t w8[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float lo = __uint_as_float(w8[e] << 16), hi = __uint_as_float(w8[e] & 0xffff0000u);
      qf[2 * e] = lo;
      qf[2 * e + 1] = hi;
      qn1 += fabsf(lo) + fabsf(hi);
    }
    qn1 += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(qn1)));
    qn1 += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(qn1)));
    qn1 *= 1.0f + 1.0f / 1024.0f;  // covers the fp32 rounding of the sum
  }
  __syncthreads();  // B0

  const uint32_t kb = umax32(umax32(L.kmax[0], L.kmax[1]), umax32(L.kmax[2], L.kmax[3]));
  float kmax = __uint_as_float(kb << 16) * (1.0f + 1.0f / 1024.0f);

  // ---- Anchor: matrix-core scores of every staged key. ----
  const int ntiles = nrows >> 4;
  for (int tt = wave; tt < ntiles; tt += 4) {
    const int row = tt * 16 + gl;
    const uint4 b0 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, g4));
    const uint4 b1 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, 4 + g4));
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = mfma_bf16(a0, b0, acc);
    acc = mfma_bf16(a1, b1, acc);
    float* dst = L.sc + row * kSQ + 4 * g4;
    *reinterpret_cast<float2*>(dst) = make_float2(acc[0], acc[1]);
    *reinterpret_cast<float2*>(dst + 2) = make_float2(acc[2], acc[3]);
  }
  block_scores<NBL>(p, L, qi, gl, t, ls);
  wave_sync();
  pick_blocks<NBL>(p, L, qi, gl);
  __syncthreads();  // B1: s~ complete

  exact_topk<true>(p, L, qi, gl, t, ls, -1, 1, qf, qn1, kmax, active);
  int anchor;
  {
    const QRec& R = L.qr[qi];
    if (R.ntop > 0) {
      const uint64_t key = L.top[(R.cur * kQ + qi) * kTileMaxK];
      anchor = static_cast<int>(key_index(key));
      if (active && gl == 0) {
        p.out_anchor[qrow] = anchor;
        p.out_anchor_score[qrow] = key_score(key);
      }
    } else {
      anchor = t - p.L + 1;
      if (active && gl == 0) {
        p.out_anchor[qrow] = anchor;
        p.out_anchor_score[qrow] = -INFINITY;
      }
    }
  }

  // ---- Partner query (relation_select.py:165-193): fp32 sum of the
  //      query-side projection and the anchor's cached row. ----
  fetch_stats<TS, NBL>(p, ps, b, tid, pst);
  const bool have = anchor >= 0 && anchor < p.T;
  const uint4 pb = *reinterpret_cast<const uint4*>(p.pbase + qrow * 128 + 8 * gl);
  const uint4 pc = *reinterpret_cast<const uint4*>(p.pcache + (b * p.T + (have ? anchor : 0)) * 128 + 8 * gl);
  __syncthreads();  // B2: every wave is done with the anchor side's LDS

  // ---- Partner side: stage keys, statistics, router query, bias. ----
  km = u16x2_t{0, 0};
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int k = tid + kThreads * u;
    if (k < nchunks) {
      *reinterpret_cast<uint4*>(L.keys + key_chunk_offset(k >> 3, k & 7)) = pkv[u];
      km = absmax8(pkv[u], km);
    }
  }
  kbits = umax32(km.x, km.y);
  kbits = wave_max_u32(kbits);
  if (lane == 0) L.kmax[wave] = kbits;
  put_stats<NBL>(p, L, tid, pst);
  put_router_consts(p, ps, L, tid);
  {
    const uint32_t wb[4] = {pb.x, pb.y, pb.z, pb.w};
    const uint32_t wc[4] = {pc.x, pc.y, pc.z, pc.w};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c0 = have ? __uint_as_float(wc[i] << 16) : 0.0f;
      const float c1 = have ? __uint_as_float(wc[i] & 0xffff0000u) : 0.0f;
      v[2 * i] = __uint_as_float(wb[i] << 16) + c0;
      v[2 * i + 1] = __uint_as_float(wb[i] & 0xffff0000u) + c1;
    }
    if (gl < 8) {
      float* dst = L.pq + qi * kPqRow + 8 * gl;
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      double* dst = L.rq + qi * kRqRow + 8 * (gl - 8);
#pragma unroll
      for (int i = 0; i < 8; i += 2)
        *reinterpret_cast<double2*>(dst + i) =
            make_double2(static_cast<double>(v[i]), static_cast<double>(v[i + 1]));
    }
  }
  __syncthreads();  // B3

  kmax = __uint_as_float(umax32(umax32(L.kmax[0], L.kmax[1]), umax32(L.kmax[2], L.kmax[3])) << 16) *
         (1.0f + 1.0f / 1024.0f);
  // Partner A fragments: bf16 hi + lo of the fp32 query, row lane%16.
  uint4 ah0, al0, ah1, al1;
  {
    const float* src = L.pq + gl * kPqRow;
    float x[8];
    const float4 u0 = *reinterpret_cast<const float4*>(src + 8 * g4);
    const float4 u1 = *reinterpret_cast<const float4*>(src + 8 * g4 + 4);
    x[0] = u0.x; x[1] = u0.y; x[2] = u0.z; x[3] = u0.w;
    x[4] = u1.x; x[5] = u1.y; x[6] = u1.z; x[7] = u1.w;
    split_hi_lo(x, ah0, al0);
    const float4 u2 = *reinterpret_cast<const float4*>(src + 32 + 8 * g4);
    const float4 u3 = *reinterpret_cast<const float4*>(src + 32 + 8 * g4 + 4);
    x[0] = u2.x; x[1] = u2.y; x[2] = u2.z; x[3] = u2.w;
    x[4] = u3.x; x[5] = u3.y; x[6] = u3.z; x[7] = u3.w;
    split_hi_lo(x, ah1, al1);
  }
  {
    const float* src = L.pq + qi * kPqRow + 16 * s4;
    qn1 = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
      const float4 u = *reinterpret_cast<const float4*>(src + e);
      qf[e] = u.x;
      qf[e + 1] = u.y;
      qf[e + 2] = u.z;
      qf[e + 3] = u.w;
      qn1 += fabsf(u.x) + fabsf(u.y) + fabsf(u.z) + fabsf(u.w);
    }
    qn1 += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(qn1)));
    qn1 += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(qn1)));
    qn1 *= 1.0f + 1.0f / 1024.0f;
  }
  for (int tt = wave; tt < ntiles; tt += 4) {
    const int row = tt * 16 + gl;
    const uint4 b0 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, g4));
    const uint4 b1 = *reinterpret_cast<const uint4*>(L.keys + key_chunk_offset(row, 4 + g4));
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = mfma_bf16(ah0, b0, acc);
    acc = mfma_bf16(al0, b0, acc);
    acc = mfma_bf16(ah1, b1, acc);
    acc = mfma_bf16(al1, b1, acc);
    float* dst = L.sc + row * kSQ + 4 * g4;
    *reinterpret_cast<float2*>(dst) = make_float2(acc[0], acc[1]);
    *reinterpret_cast<float2*>(dst + 2) = make_float2(acc[2], acc[3]);
  }
  block_scores<NBL>(p, L, qi, gl, t, ls);
  wave_sync();
  pick_blocks<NBL>(p, L, qi, gl);
  __syncthreads();  // B4: s~ complete

  const int K = p.K;
  exact_topk<false>(p, L, qi, gl, t, ls, anchor, K, qf, qn1, kmax, active);
  if (active && gl < K) {
    const QRec& R = L.qr[qi];
    int pos = t - p.L + 1;
    float score = -INFINITY;
    if (gl < R.ntop) {
      const uint64_t key = L.top[(R.cur * kQ + qi) * kTileMaxK + gl];
      bool v;
      pos = cand_pos(p, R, static_cast<int>(key_index(key)), t, ls, v);
      score = key_score(key);
    }
    p.out_partner[qrow * K + gl] = pos;
    p.out_partner_score[qrow * K + gl] = score;
  }
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
  p.off_stats = take(2 * p.NB * kStatRow * 8);
  p.off_rq = take(kQ * kRqRow * 8);
  p.off_pq = take(kQ * kPqRow * 4);
  p.off_blk = take(kQ * (p.NB + 4) * 4);
  p.off_lmax = take(kQ * 16 * 4);
  p.off_list = take(kQ * kListCap * 8);
  p.off_top = take(2 * kQ * kTileMaxK * 8);
  p.off_qrec = take(kQ * static_cast<int>(sizeof(QRec)));
  p.off_bias = take(p.H * p.RB * 8);
  p.off_sp = take(16 * 8);
  p.off_kmax = take(16);
  p.lds_total = off;
  return off <= 160 * 1024;
}

hipError_t select_tile_launch(const TileParams& p, int stat_dtype, hipStream_t stream) {
  const dim3 block(kThreads);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles));
  const size_t lds = static_cast<size_t>(p.lds_total);
  const int nbl = (p.NB + 15) / 16;
  // The LDS opt-in above 64 KiB is a per-process function attribute (set once
  // per instantiation, for the full 160 KiB).
#define RLM_TILE_CASE(TS_ID, TS, NBL_)                                                    \
  if (stat_dtype == TS_ID && nbl == NBL_) {                                               \
    static const hipError_t attr = hipFuncSetAttribute(                                   \
        reinterpret_cast<const void*>(&select_tile_kernel<TS, NBL_>),                     \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                          \
    if (attr != hipSuccess) {                                                             \
      set_error("relation_select (tile): cannot reserve LDS: %s", hipGetErrorString(attr)); \
      return attr;                                                                        \
    }                                                                                     \
    hipLaunchKernelGGL((select_tile_kernel<TS, NBL_>), grid, block, lds, stream, p);      \
    return launch_status("relation_select (tile)");                                       \
  }
  RLM_TILE_CASE(RLM_F32, float, 1)
  RLM_TILE_CASE(RLM_F32, float, 2)
  RLM_TILE_CASE(RLM_F32, float, 4)
  RLM_TILE_CASE(RLM_BF16, bf16, 1)
  RLM_TILE_CASE(RLM_BF16, bf16, 2)
  RLM_TILE_CASE(RLM_BF16, bf16, 4)
#undef RLM_TILE_CASE
  set_error("relation_select (tile): unsupported statistics dtype %s or %d blocks",
            dtype_name(stat_dtype), p.NB);
  return hipErrorInvalidValue;
}

}  // namespace rlm

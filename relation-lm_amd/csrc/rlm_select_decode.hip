// Routed selection, decode form (one query per batch row), for gfx950.
//
// Reference semantics: src/relation_lm/kernels/relation_select.py:9-308 (the
// packed selection) for one query at position t.  Same outputs and numerics
// contract as select_kernel (rlm_select.hip): exact scores are float64 dots of
// the 16-bit inputs rounded once to float32, block scores (softplus, per-head
// terms, the log-sum-exp over heads) are float64 rounded once, and every
// comparison and tie uses those float32 values with the same tie rules
// (anchor -> lowest position, blocks -> lowest block, partners -> lowest
// candidate lane: local window first, then picked blocks in pick order).
//
// The decode step is latency bound: a single query's chain of dependent
// steps is the whole kernel.  One workgroup of eight waves per batch row (two
// candidate passes of 128 instead of four of 64), and
// the chain is shortened three ways:
//   * one burst of loads at the start -- position, bias tables, gammas, both
//     streams' query vectors and block statistics -- then, as soon as t is
//     known, both streams' local-window key rows; the picked blocks' rows are
//     loaded right after each stream's picks (from L2, while the local rows'
//     dots run), and the anchor's cached partner row right after the anchor;
//   * every step is spread over the 512 lanes: lane (block, head) pairs for
//     the block scores, four lanes per candidate (16 dims each, four partial
//     sums) for the exact dots, one lane per block for the pick ranks (read
//     from LDS);
//   * the anchor's argmax is taken by each wave from LDS (no extra barrier),
//     and the partners' top-k by one wave from four sorted keys per lane;
//     both use wave maxima that stay in VALU (DPP and row swaps).
#include "rlm_common.hpp"
#include "rlm_select_decode.hpp"
#include "rlm_tile_util.hpp"

namespace rlm {
namespace {

constexpr int kThreads = 512;
constexpr int kRowBytes = 128;  // one key row: 64 16-bit values
constexpr int kHeads = 4;
constexpr int kHeadDim = 16;
constexpr int kPasses = kDecodeMaxCap / (kThreads / 4);  // candidate passes of 64 (4 lanes each)

template <typename T>
__device__ __forceinline__ void chunk_f64(const uint4& v, double* out);
template <>
__device__ __forceinline__ void chunk_f64<bf16>(const uint4& v, double* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = static_cast<double>(__uint_as_float(w[i] << 16));
    out[2 * i + 1] = static_cast<double>(__uint_as_float(w[i] & 0xffff0000u));
  }
}
template <>
__device__ __forceinline__ void chunk_f64<f16>(const uint4& v, double* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = static_cast<double>(
        static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(w[i] & 0xffffu))));
    out[2 * i + 1] = static_cast<double>(
        static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(w[i] >> 16))));
  }
}

// Eight 16-bit values as float32.
template <typename T>
__device__ __forceinline__ void chunk_f32(const uint4& v, float* out) {
  double d[8];
  chunk_f64<T>(v, d);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(d[i]);
}

// Statistics of one (block, head) pair: 16 values of TS in kStatChunks chunks.
template <typename TS>
struct StatRow {
  static constexpr int kChunks = sizeof(TS) == 4 ? 4 : 2;
  uint4 m[kChunks], s[kChunks];
  __device__ __forceinline__ void issue(rsrc_t mr, rsrc_t sr, uint32_t off, bool live) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      m[i] = buf_load_b128(mr, live ? off + 16u * i : kNoOffset);
      s[i] = buf_load_b128(sr, live ? off + 16u * i : kNoOffset);
    }
  }
  __device__ __forceinline__ void values(float* mean, float* stdv) const {
    if constexpr (sizeof(TS) == 4) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const uint32_t a[4] = {m[i].x, m[i].y, m[i].z, m[i].w};
        const uint32_t c[4] = {s[i].x, s[i].y, s[i].z, s[i].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          mean[4 * i + e] = __uint_as_float(a[e]);
          stdv[4 * i + e] = __uint_as_float(c[e]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        chunk_f32<TS>(m[i], mean + 8 * i);
        chunk_f32<TS>(s[i], stdv + 8 * i);
      }
    }
  }
};

struct Shared {
  float* sc;               // [2][kDecodeMaxCap] exact candidate scores
  uint64_t* key;           // [2][kDecodeMaxCap] selection keys of the candidates
  uint64_t* blk;           // [NB rounded up to 16] block selection keys
  int* sel;                // [TOP] picked blocks, then [TOP] validity flags
};

// Columns [kExpandCols * grp, + kExpandCols) of the token's expanded-cache row
// for every batch row: wave w takes two 16-column tiles, lane (r16, g) batch
// row b0 + r16 and k-pieces 8g .. 8g + 7 of each 32-wide k-step.  The sums are
// v_mfma_f32_16x16x32_bf16 with the weight rows as A, k-steps in order from
// zero, the bias added in fp32 and one bf16 rounding (relation_linear's
// smallk_kernel order for the same tile).  Every load of a row tile is issued
// before the first product.
__device__ void expand_row_group(const ExpandRowParams& x, int grp, int tid) {
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  if (wave >= kExpandCols / 32) return;  // four waves of two 16-column tiles each; the rest idle
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t t = index_at(x.pos, x.pos_dtype, 0);
  if (t < 0 || (!x.ring && t >= x.T)) return;  // no row to write (uniform)
  const int64_t row = x.ring ? (t & (x.T - 1)) : t;
  const uint32_t R = 32u * static_cast<uint32_t>(x.KS);
  const uint32_t N = static_cast<uint32_t>(x.N);
  const rsrc_t opr = make_rsrc(x.op, x.op_bytes);
  const rsrc_t wr = make_rsrc(x.w, x.w_bytes);
  const bool is32 = x.bias_dtype == RLM_F32;
  const bool has_bias = x.bias != nullptr;
  const rsrc_t br = make_rsrc(x.bias, N * (is32 ? 4u : 2u));
  for (int64_t b0 = 0; b0 < x.B; b0 += 16) {
    const int64_t b = b0 + r16;
    const bool bv = b < x.B;
    const uint32_t orow = static_cast<uint32_t>((bv ? b : 0) * x.T + row);
    uint4 af[4], wf[2][4], bq[2];
    uint2 bh[2];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      af[s] = buf_load_b128(opr, bv && s < x.KS ? (orow * R + 32u * s + 8u * g) * 2u : kNoOffset);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t n0 = static_cast<uint32_t>(grp * kExpandCols + wave * 32 + j * 16);
      const bool live = n0 < N;
      const uint32_t n = n0 + r16;  // weight row of the A operand
#pragma unroll
      for (int s = 0; s < 4; ++s)
        wf[j][s] = buf_load_b128(wr, live && s < x.KS ? (n * R + 32u * s + 8u * g) * 2u : kNoOffset);
      const uint32_t nc = n0 + 4u * g;  // this lane's output columns
      bq[j] = buf_load_b128(br, live && has_bias && is32 ? 4u * nc : kNoOffset);
      bh[j] = buf_load_b64(br, live && has_bias && !is32 ? 2u * nc : kNoOffset);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t n0 = static_cast<uint32_t>(grp * kExpandCols + wave * 32 + j * 16);
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (s < x.KS) acc = mfma_bf16(wf[j][s], af[s], acc);
      const uint32_t w16[4] = {bh[j].x & 0xffffu, bh[j].x >> 16, bh[j].y & 0xffffu, bh[j].y >> 16};
      const uint32_t w32[4] = {bq[j].x, bq[j].y, bq[j].z, bq[j].w};
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = acc[e] + decode_float(FloatWords{w32[e], w16[e]}, x.bias_dtype);
      // Lane (r16, g) holds batch row b, columns n0 + 4g .. + 3.
      if (bv && n0 < N)
        *reinterpret_cast<uint2*>(x.cache + (static_cast<size_t>(b) * x.T + row) * N + n0 + 4 * g) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
}

__global__ void __launch_bounds__(kThreads) expand_row_kernel(const ExpandRowParams x) {
  expand_row_group(x, static_cast<int>(blockIdx.x), static_cast<int>(threadIdx.x));
}

template <typename TA, typename TS, bool RING>
__global__ void __launch_bounds__(kThreads) select_decode_kernel(const DecodeParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (blockIdx.x >= p.B) {  // workgroup-uniform: the expanded-row workgroups
    expand_row_group(p.x, static_cast<int>(blockIdx.x - p.B), static_cast<int>(threadIdx.x));
    return;
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int64_t b = blockIdx.x;
  const int T = static_cast<int>(p.T);
  Shared sh;
  sh.sc = reinterpret_cast<float*>(smem + p.off_sc);
  sh.key = reinterpret_cast<uint64_t*>(smem + p.off_key);
  sh.blk = reinterpret_cast<uint64_t*>(smem + p.off_blk);
  sh.sel = reinterpret_cast<int*>(smem + p.off_sel);

  // ---- One burst of loads: everything that does not depend on a result. ----
  const IndexWords tw = issue_index(p.pos, p.pos_dtype, 1, 0, true);
  // Lane (block j, head h) of the block scores; bias table entry `lane` of
  // each stream (broadcast by ds_bpermute), the gammas of head h.
  const int npairs = p.NB * kHeads;
  const bool pair_live = tid < npairs;
  const int j = tid >> 2;
  const int h = tid & 3;
  const int tab = kHeads * p.RB;
  const FloatWords bias_a = issue_float(p.abias, p.abias_dtype, tab, lane, lane < tab);
  const FloatWords bias_p = issue_float(p.pbias, p.pbias_dtype, tab, lane, lane < tab);
  const FloatWords gam_a = issue_float(p.agamma, p.agamma_dtype, kHeads, h, true);
  const FloatWords gam_p = issue_float(p.pgamma, p.pgamma_dtype, kHeads, h, true);
  // Query vectors: the lane's quarter (16 dims) of the exact vectors, head h
  // of the router vectors.
  const int qd = tid & 3;
  const uint32_t qbytes = static_cast<uint32_t>(p.B) * 64u * 2u;
  const rsrc_t aqr = make_rsrc(p.aq, qbytes);
  const rsrc_t arqr = make_rsrc(p.arq, qbytes);
  const rsrc_t pbr = make_rsrc(p.pbase, 2u * qbytes);
  const uint32_t qrow = static_cast<uint32_t>(b) * 128u;
  uint4 aq[2], arq[2], pq[2], prq[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    aq[i] = buf_load_b128(aqr, qrow + 32u * qd + 16u * i);
    pq[i] = buf_load_b128(pbr, 2u * qrow + 32u * qd + 16u * i);
    arq[i] = buf_load_b128(arqr, qrow + 32u * h + 16u * i);
    prq[i] = buf_load_b128(pbr, 2u * qrow + 128u + 32u * h + 16u * i);
  }
  // Block statistics of the lane's pair, both streams.
  StatRow<TS> sta, stp;
  {
    const uint32_t sbytes = static_cast<uint32_t>(p.B * npairs * kHeadDim * sizeof(TS));
    const uint32_t off = static_cast<uint32_t>((b * npairs + (pair_live ? tid : 0)) * kHeadDim *
                                               sizeof(TS));
    sta.issue(make_rsrc(p.amean, sbytes), make_rsrc(p.astd, sbytes), off, pair_live);
    stp.issue(make_rsrc(p.pmean, sbytes), make_rsrc(p.pstd, sbytes), off, pair_live);
  }
  for (int r = tid; r < p.TOP; r += kThreads) {
    sh.sel[r] = 0;
    sh.sel[p.TOP + r] = 0;
  }

  // ---- Scalars of the query. ----
  const int64_t t64 = decode_index(tw, p.pos_dtype);
  const int t = static_cast<int>(t64);
  const int local_start = t - p.L + 1 > 0 ? t - p.L + 1 : 0;
  const int cur_block = t >> p.BS_log2;
  double sp_a, sp_p;  // softplus(gamma_h), float64 (relation_select.py:87)
  {
#pragma clang fp contract(off)
    sp_a = log(1.0 + exp(static_cast<double>(decode_float(gam_a, p.agamma_dtype))));
    sp_p = log(1.0 + exp(static_cast<double>(decode_float(gam_p, p.pgamma_dtype))));
  }
  const float btab_a = decode_float(bias_a, p.abias_dtype);
  const float btab_p = decode_float(bias_p, p.pbias_dtype);
  // Absolute block held by slot j (ring caches: the newest block jb <= t/BS
  // with jb = j mod NB, negative when never written).
  const int jb = RING ? cur_block - ((cur_block - j) & (p.NB - 1)) : j;
  const int bend = (jb + 1) * p.BS - 1;
  int bucket;
  {
    const int dist = (t > bend ? t - bend : 0) + 1;
    bucket = 31 - __clz(dist);
    bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
  }
  const bool eligible = jb >= 0 && bend <= t && (!p.strict || bend < local_start);

  // Block scores of one stream (relation_select.py:53-106):
  //   s_h = (sum_d mean*q_h + softplus(gamma_h) * sum_d std*|q_h|) * HD^-0.5 + bias[h, bucket]
  // and the log-sum-exp over the block's four head lanes, into sh.blk[j].
  auto block_scores = [&](const StatRow<TS>& st, const double* q, double sp, float btab) {
    float mean[kHeadDim], stdv[kHeadDim];
    st.values(mean, stdv);
    double c4[4] = {0.0, 0.0, 0.0, 0.0}, u4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int d = 0; d < kHeadDim; ++d) {
      c4[d & 3] += static_cast<double>(mean[d]) * q[d];
      u4[d & 3] += static_cast<double>(stdv[d]) * fabs(q[d]);
    }
    const double c = (c4[0] + c4[1]) + (c4[2] + c4[3]);
    const double u = (u4[0] + u4[1]) + (u4[2] + u4[3]);
    const float bias = __int_as_float(
        __builtin_amdgcn_ds_bpermute(4 * (h * p.RB + bucket), __float_as_int(btab)));
    double sv;
    {
#pragma clang fp contract(off)
      const double content = c + sp * u;
      sv = pair_live ? content * p.head_scale + static_cast<double>(bias) : 0.0;
    }
    double m = fmax(sv, dpp_f64<kDppXor1>(sv));
    m = fmax(m, dpp_f64<kDppXor2>(m));
    double e = exp(sv - m);
    e += dpp_f64<kDppXor1>(e);
    e += dpp_f64<kDppXor2>(e);
    if (pair_live && h == 0) {
      const float lse = static_cast<float>(m + log(e));
      sh.blk[j] = select_key(eligible ? lse : -INFINITY, static_cast<uint32_t>(jb));
    }
  };
  // The TOP picks of the reference's sequential argmax (ties to the lowest
  // block; valid iff > -1e30, relation_select.py:229-242) by rank:
  // block j is pick rank(j) = #{k : key_k > key_j}.
  auto pick_blocks = [&]() {
    if (tid < p.NB) {
      const uint64_t kj = sh.blk[tid];
      int rank = 0;
      for (int k0 = 0; k0 < p.NB; k0 += 16) {  // 16 keys read at once
        uint64_t kk[16];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const ulonglong2 v = *reinterpret_cast<const ulonglong2*>(sh.blk + k0 + i);
          kk[i] = v.x;
          kk[i + 1] = v.y;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) rank += (k0 + i < p.NB && kk[i] > kj) ? 1 : 0;
      }
      if (rank < p.TOP) {
        sh.sel[rank] = RING ? cur_block - ((cur_block - tid) & (p.NB - 1)) : tid;
        sh.sel[p.TOP + rank] = key_score(kj) > -1.0e30f ? 1 : 0;
      }
    }
  };
  // Candidate c (local window first, then TOP*BS rows of the picks in pick
  // order, relation_select.py:244-283): position and validity.  Local
  // candidates need only t; remote ones read the picks from LDS.
  auto local_candidate = [&](int c, int& pos, bool& valid) {
    pos = t - p.L + 1 + c;
    valid = pos >= 0 && pos <= t && (RING || pos < T);
  };
  auto remote_candidate = [&](int c, int& pos, bool& valid) {
    const int r = (c - p.L) >> p.BS_log2;
    pos = sh.sel[r] * p.BS + ((c - p.L) & (p.BS - 1));
    valid = sh.sel[p.TOP + r] != 0 && pos <= t && pos < local_start && (RING || pos < T);
  };
  // The lane's quarter (two 16-byte chunks) of candidate c = 64 i + tid/4 for
  // each pass i, loaded straight from the key cache (L2); invalid rows read
  // zeros through an out-of-range offset.
  struct Rows {
    uint4 k[kPasses][2];
    int pos[kPasses];
    bool valid[kPasses];
  };
  const uint32_t kbytes = static_cast<uint32_t>(T) * kRowBytes;
  const rsrc_t akr = make_rsrc(static_cast<const unsigned char*>(p.akeys) + b * kbytes, kbytes);
  const rsrc_t pkr = make_rsrc(static_cast<const unsigned char*>(p.pkeys) + b * kbytes, kbytes);
  auto load_rows = [&](Rows& rw, rsrc_t kr, bool remote) {
#pragma unroll
    for (int i = 0; i < kPasses; ++i) {
      const int c = i * (kThreads / 4) + (tid >> 2);
      if (c < p.CAP && (c >= p.L) == remote) {
        if (remote)
          remote_candidate(c, rw.pos[i], rw.valid[i]);
        else
          local_candidate(c, rw.pos[i], rw.valid[i]);
        const int row = RING ? (rw.pos[i] & (T - 1)) : rw.pos[i];
        const uint32_t off = rw.valid[i] ? static_cast<uint32_t>(row) * kRowBytes + 32u * qd : kNoOffset;
        rw.k[i][0] = buf_load_b128(kr, off);
        rw.k[i][1] = buf_load_b128(kr, rw.valid[i] ? off + 16u : kNoOffset);
      }
    }
  };
  // Exact scores of stream s's candidates of one kind (local or remote):
  // float64 dot of the lane's 16 dims in four partial sums, the four lanes of
  // a candidate summed with DPP.
  auto exact_scores = [&](int s, const Rows& rw, const double* q, int exclude, bool remote) {
#pragma unroll
    for (int i = 0; i < kPasses; ++i) {
      const int c = i * (kThreads / 4) + (tid >> 2);
      // Uniform per quad; the DPP sums below need all four lanes of a quad.
      const bool mine = c < p.CAP && (c >= p.L) == remote;
      if (!__builtin_amdgcn_ballot_w64(mine)) continue;
      double kv[16];
      chunk_f64<TA>(rw.k[i][0], kv);
      chunk_f64<TA>(rw.k[i][1], kv + 8);
      double a4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int e = 0; e < 16; ++e) a4[e & 3] += kv[e] * q[e];
      double acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
      acc += dpp_f64<kDppXor1>(acc);
      acc += dpp_f64<kDppXor2>(acc);
      if (mine && qd == 0) {
        const int pos = rw.pos[i];
        const bool valid = rw.valid[i];
        const bool ok = valid && pos != exclude;
        const float sc = ok ? static_cast<float>(acc * p.exact_scale) : -INFINITY;
        sh.sc[s * kDecodeMaxCap + c] = sc;
        // Anchor: valid candidates by (score, lower position); partners: all
        // lanes by (score, lower lane).
        sh.key[s * kDecodeMaxCap + c] =
            s == 0 ? (valid ? select_key(sc, static_cast<uint32_t>(pos)) : 0)
                   : select_key(sc, static_cast<uint32_t>(c));
      }
    }
  };

  // Local-window rows of both streams: they depend on t only.
  Rows ra, rp;
  load_rows(ra, akr, false);
  load_rows(rp, pkr, false);

  // ---- Anchor stream. ----
  double qh[kHeadDim];
  chunk_f64<TA>(arq[0], qh);
  chunk_f64<TA>(arq[1], qh + 8);
  block_scores(sta, qh, sp_a, btab_a);
  __syncthreads();
  pick_blocks();
  __syncthreads();
  load_rows(ra, akr, true);
  double qx[16];
  chunk_f64<TA>(aq[0], qx);
  chunk_f64<TA>(aq[1], qx + 8);
  exact_scores(0, ra, qx, -1, false);  // while the picked rows arrive
  exact_scores(0, ra, qx, -1, true);
  __syncthreads();
  // Every wave takes the argmax itself (no barrier): valid candidates by
  // (score, lower position); none valid -> position t-L+1, score -inf.
  int anchor;
  {
    uint64_t best = 0;
    float best_sc = -INFINITY;
#pragma unroll
    for (int i = 0; i < kDecodeMaxCap / kWave; ++i) {
      const int c = lane + kWave * i;
      const uint64_t k = c < p.CAP ? sh.key[c] : 0;
      if (k > best) {
        best = k;
        best_sc = sh.sc[c];
      }
    }
    const uint64_t win = wave_max_key(best);
    anchor = win == 0 ? t - p.L + 1 : static_cast<int>(key_index(win));
    anchor = __builtin_amdgcn_readfirstlane(anchor);
    if (tid < kWave && (win == 0 ? lane == 0 : best == win)) {
      p.out_anchor[b] = anchor;
      p.out_anchor_score[b] = win == 0 ? -INFINITY : best_sc;
    }
  }
  // Picks past the last block repeat block 0 as invalid (the anchor stream's
  // picks were last read before the barrier above).
  for (int r = tid; r < p.TOP; r += kThreads) {
    sh.sel[r] = 0;
    sh.sel[p.TOP + r] = 0;
  }

  // ---- Partner queries (relation_select.py:165-193): fp32 sums of the base
  // and the anchor's cached row (nothing added when the anchor is outside
  // the cache). ----
  {
    const bool have = anchor >= 0 && (RING || anchor < T);
    const int arow = RING ? (anchor & (T - 1)) : anchor;
    const uint32_t cbytes = static_cast<uint32_t>(T) * 256u;
    const rsrc_t pcr = make_rsrc(static_cast<const unsigned char*>(p.pcache) + b * cbytes, cbytes);
    const uint32_t roff = static_cast<uint32_t>(arow) * 256u;
    uint4 cx[2], cr[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      cx[i] = buf_load_b128(pcr, have ? roff + 32u * qd + 16u * i : kNoOffset);
      cr[i] = buf_load_b128(pcr, have ? roff + 128u + 32u * h + 16u * i : kNoOffset);
    }
    float bx[16], cxf[16], br[16], crf[16];
    chunk_f32<TA>(pq[0], bx);
    chunk_f32<TA>(pq[1], bx + 8);
    chunk_f32<TA>(prq[0], br);
    chunk_f32<TA>(prq[1], br + 8);
    chunk_f32<TA>(cx[0], cxf);
    chunk_f32<TA>(cx[1], cxf + 8);
    chunk_f32<TA>(cr[0], crf);
    chunk_f32<TA>(cr[1], crf + 8);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      qx[e] = static_cast<double>(bx[e] + cxf[e]);
      qh[e] = static_cast<double>(br[e] + crf[e]);
    }
  }

  // ---- Partner stream. ----
  exact_scores(1, rp, qx, anchor, false);  // local rows: no picks needed
  block_scores(stp, qh, sp_p, btab_p);
  __syncthreads();
  pick_blocks();
  __syncthreads();
  load_rows(rp, pkr, true);
  exact_scores(1, rp, qx, anchor, true);
  __syncthreads();
  if (tid >= kWave) return;
  // K argmax passes (relation_select.py:298-308), ties to the lowest lane.
  // While finite scores remain, a stable descending order of the lanes; once
  // they are exhausted the reference's argmax over an all -inf vector returns
  // lane 0: position t-L+1, score -inf.  Each lane keeps its four candidate
  // keys sorted and pops its head when it wins; lane k takes the k-th winner.
  uint64_t k4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + kWave * i;
    k4[i] = c < p.CAP ? sh.key[kDecodeMaxCap + c] : 0;
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
  int my_c = -1;
  for (int k = 0; k < p.K; ++k) {
    const uint64_t win = wave_max_key(k4[0]);
    // After the last finite winner every remaining key scores -inf.
    if (lane == k && key_score(win) > -INFINITY) my_c = static_cast<int>(key_index(win));
    if (k4[0] == win) {
      k4[0] = k4[1];
      k4[1] = k4[2];
      k4[2] = k4[3];
      k4[3] = 0;
    }
  }
  if (lane < p.K) {
    int pos = t - p.L + 1;
    float score = -INFINITY;
    if (my_c >= 0) {
      bool valid;
      if (my_c < p.L)
        local_candidate(my_c, pos, valid);
      else
        remote_candidate(my_c, pos, valid);
      score = sh.sc[kDecodeMaxCap + my_c];
    }
    p.out_partner[b * p.K + lane] = pos;
    p.out_partner_score[b * p.K + lane] = score;
  }
}

}  // namespace

bool select_decode_layout(DecodeParams& p) {
  if (p.T < 1 || p.T > kDecodeMaxRows || p.T % 32 != 0) return false;
  if (p.NB < 1 || p.NB * kHeads > kThreads || static_cast<int64_t>(p.NB) * p.BS != p.T) return false;
  if (p.CAP < 1 || p.CAP > kDecodeMaxCap || p.K < 1 || p.K > kWave) return false;
  if (p.TOP > kWave || p.RB < 1 || kHeads * p.RB > kWave) return false;
  int off = 0;
  p.off_sc = off;
  off += 2 * kDecodeMaxCap * 4;
  p.off_key = off;
  off += 2 * kDecodeMaxCap * 8;
  p.off_blk = off;
  off += 8 * kWave;
  p.off_sel = off;
  off += 2 * 4 * kWave;
  p.lds_total = off;
  return off <= 160 * 1024;
}

hipError_t select_decode_launch(const DecodeParams& p, int act_dtype, int stat_dtype, bool ring,
                                hipStream_t stream) {
  if (p.B == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(p.B + p.xgroups));
  const size_t lds = static_cast<size_t>(p.lds_total);
#define RLM_DECODE_CASE(TA_ID, TA, TS_ID, TS, RING)                                           \
  if (act_dtype == TA_ID && stat_dtype == TS_ID && ring == RING) {                          \
    /* LDS above 64 KiB is a per-function opt-in. */                                        \
    static const hipError_t attr = hipFuncSetAttribute(                                     \
        reinterpret_cast<const void*>(&select_decode_kernel<TA, TS, RING>),                 \
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);                            \
    if (attr != hipSuccess) {                                                               \
      set_error("relation_select: LDS opt-in failed (%s)", hipGetErrorString(attr));        \
      return attr;                                                                          \
    }                                                                                       \
    hipLaunchKernelGGL((select_decode_kernel<TA, TS, RING>), grid, dim3(kThreads), lds,     \
                       stream, p);                                                          \
    return launch_status("relation_select");                                                \
  }
  RLM_DECODE_CASE(RLM_BF16, bf16, RLM_F32, float, false)
  RLM_DECODE_CASE(RLM_BF16, bf16, RLM_BF16, bf16, false)
  RLM_DECODE_CASE(RLM_F16, f16, RLM_F32, float, false)
  RLM_DECODE_CASE(RLM_F16, f16, RLM_F16, f16, false)
  RLM_DECODE_CASE(RLM_BF16, bf16, RLM_F32, float, true)
  RLM_DECODE_CASE(RLM_BF16, bf16, RLM_BF16, bf16, true)
  RLM_DECODE_CASE(RLM_F16, f16, RLM_F32, float, true)
  RLM_DECODE_CASE(RLM_F16, f16, RLM_F16, f16, true)
#undef RLM_DECODE_CASE
  set_error("relation_select: unsupported dtype combination for the decode kernel");
  return hipErrorInvalidValue;
}

hipError_t expand_row_launch(const ExpandRowParams& x, hipStream_t stream) {
  const int groups = (x.N + kExpandCols - 1) / kExpandCols;
  if (x.B == 0 || groups == 0) return hipSuccess;
  hipLaunchKernelGGL(expand_row_kernel, dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0,
                     stream, x);
  return launch_status("relation_select (expanded row)");
}

}  // namespace rlm

// Routed selection for gfx950: block scoring, exact top-1 anchor, factorized
// partner query, partner block routing and exact top-k partners.
//
// Reference semantics: src/relation_lm/kernels/relation_select.py:9-308 (packed)
// and src/relation_lm/kernels/triton_select.py:9-252 (two-op form).
//
// Mapping: one wavefront per query (batch row b, position t).  The serial
// chain of the reference (block scoring -> picks -> exact scores -> argmax
// passes) stays inside one wave, so every reduction is a 6-step wave64
// shuffle and the only memory traffic is the query's own gathers.
//
// Numerics: every dot product is accumulated in float64 from exact products
// and rounded once to float32; block scores (softplus, per-head terms,
// pairwise log-sum-exp) are evaluated in float64 and rounded once.  All
// comparisons use those float32 values.  Ties: anchor -> lowest position,
// blocks -> lowest block, partners -> lowest candidate lane (local window
// first, then picked blocks in pick order).  Both are encoded in one 64-bit
// key so a single wave max-reduction yields the winner.
#include "rlm_common.hpp"

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
  int lds_per_wave;  // bytes
};

// LDS bytes one wave needs (layout mirrored in select_kernel).
// The float64 head-score region is padded to an even count so the float4
// query rows that follow it stay 16-byte aligned.
inline int select_lds_bytes(int NB, int H, int E, int RD, int TOP, int CAP) {
  const int bytes = 8 * ((NB * H + 1) & ~1) + 4 * (E + RD + NB + 2 * TOP + CAP);
  return (bytes + 15) & ~15;
}

template <typename TA>
__device__ __forceinline__ float exact_score(const TA* row, const float* q, int E, double scale) {
  double acc0 = 0.0, acc1 = 0.0;
  for (int d = 0; d < E; d += 4) {
    const float4 k = load4(row + d);
    const float4 v = *reinterpret_cast<const float4*>(q + d);
    acc0 += static_cast<double>(k.x) * static_cast<double>(v.x);
    acc1 += static_cast<double>(k.y) * static_cast<double>(v.y);
    acc0 += static_cast<double>(k.z) * static_cast<double>(v.z);
    acc1 += static_cast<double>(k.w) * static_cast<double>(v.w);
  }
  return static_cast<float>((acc0 + acc1) * scale);
}

// Per-head terms then pairwise log-sum-exp in head order, masked by
// eligibility (relation_select.py:53-106).  Writes blk[NB] (float32).
template <typename TS>
__device__ void block_scores(const SelectParams& p, const Stream& s, int64_t b, int64_t t,
                             int64_t local_start, const float* qr, double* sh, float* blk,
                             int lane) {
  const int pairs = p.NB * p.H;
  const TS* mean = static_cast<const TS*>(s.mean) + b * static_cast<int64_t>(pairs) * p.HD;
  const TS* stdv = static_cast<const TS*>(s.stdev) + b * static_cast<int64_t>(pairs) * p.HD;
  for (int pr = lane; pr < pairs; pr += kWave) {
    const int j = pr / p.H;
    const int h = pr - j * p.H;
    const TS* mr = mean + static_cast<int64_t>(pr) * p.HD;
    const TS* sr = stdv + static_cast<int64_t>(pr) * p.HD;
    const float* qh = qr + h * p.HD;
    double c = 0.0, u = 0.0;
    for (int d = 0; d < p.HD; d += 4) {
      const float4 m = load4(mr + d);
      const float4 sd = load4(sr + d);
      const float4 v = *reinterpret_cast<const float4*>(qh + d);
      c += static_cast<double>(m.x) * v.x;
      c += static_cast<double>(m.y) * v.y;
      c += static_cast<double>(m.z) * v.z;
      c += static_cast<double>(m.w) * v.w;
      u += static_cast<double>(sd.x) * fabsf(v.x);
      u += static_cast<double>(sd.y) * fabsf(v.y);
      u += static_cast<double>(sd.z) * fabsf(v.z);
      u += static_cast<double>(sd.w) * fabsf(v.w);
    }
    const double g = load_any_f(s.gamma, s.gamma_dtype, h);
    const int64_t end = static_cast<int64_t>(j + 1) * p.BS - 1;
    const int64_t dist = (t > end ? t - end : 0) + 1;
    int bucket = 63 - __clzll(static_cast<unsigned long long>(dist));
    bucket = bucket < p.RB - 1 ? bucket : p.RB - 1;
    const double bias = load_any_f(s.bias, s.bias_dtype, static_cast<int64_t>(h) * p.RB + bucket);
    {
#pragma clang fp contract(off)
      const double sp = log(1.0 + exp(g));
      const double uncertainty = sp * u;
      const double content = c + uncertainty;
      sh[pr] = content * p.head_scale + bias;
    }
  }
  wave_sync();
  for (int j = lane; j < p.NB; j += kWave) {
    double acc = sh[j * p.H];
    for (int h = 1; h < p.H; ++h) {
#pragma clang fp contract(off)
      const double v = sh[j * p.H + h];
      const double m = fmax(acc, v);
      acc = m + log(exp(acc - m) + exp(v - m));
    }
    const int64_t end = static_cast<int64_t>(j + 1) * p.BS - 1;
    const bool eligible = end <= t && (!p.strict || end < local_start);
    blk[j] = eligible ? static_cast<float>(acc) : -INFINITY;
  }
  wave_sync();
}

// TOP sequential argmax picks, ties to the lowest block; a pick is valid iff
// its value is > -1e30 (relation_select.py:229-242).
__device__ void pick_blocks(const SelectParams& p, float* blk, int* sel, int* selv, int lane) {
  for (int r = 0; r < p.TOP; ++r) {
    uint64_t best = 0;
    for (int j = lane; j < p.NB; j += kWave) {
      const uint64_t k = select_key(blk[j], static_cast<uint32_t>(j));
      best = k > best ? k : best;
    }
    const uint64_t win = wave_max_u64(best);
    const int j = static_cast<int>(key_index(win));
    if (lane == 0) {
      sel[r] = j;
      selv[r] = key_score(win) > -1.0e30f ? 1 : 0;
    }
    if ((j & (kWave - 1)) == lane) blk[j] = -INFINITY;
    wave_sync();
  }
}

// Candidate lane c: local window first, then TOP*BS remote lanes in pick order
// (relation_select.py:244-283).
__device__ __forceinline__ void candidate(const SelectParams& p, int c, int64_t t,
                                          int64_t local_start, const int* sel, const int* selv,
                                          int64_t& pos, bool& valid) {
  if (c < p.L) {
    pos = t - p.L + 1 + c;
    valid = pos >= 0 && pos <= t && pos < p.T;
  } else {
    const int r = (c - p.L) / p.BS;
    const int o = c - p.L - r * p.BS;
    pos = static_cast<int64_t>(sel[r]) * p.BS + o;
    valid = selv[r] != 0 && pos <= t && pos < local_start && pos < p.T;
  }
}

template <typename TA, typename TS, int MODE>
__global__ void __launch_bounds__(256) select_kernel(const SelectParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * waves + wave;
  if (q >= p.B * p.Tq) return;  // whole wave leaves; no workgroup barriers below

  unsigned char* base = smem + wave * p.lds_per_wave;
  double* sh = reinterpret_cast<double*>(base);
  float* qx = reinterpret_cast<float*>(sh + ((p.NB * p.H + 1) & ~1));
  float* qr = qx + p.E;
  float* blk = qr + p.H * p.HD;
  int* sel = reinterpret_cast<int*>(blk + p.NB);
  int* selv = sel + p.TOP;
  float* sc = reinterpret_cast<float*>(selv + p.TOP);

  const int RD = p.H * p.HD;
  const int64_t b = q / p.Tq;
  const int64_t tq = q - b * p.Tq;
  const int64_t t = load_any_i(p.pos, p.pos_dtype, b * p.pos_sb + tq * p.pos_sq);
  const int64_t local_start = t - p.L + 1 > 0 ? t - p.L + 1 : 0;

  int64_t anchor;
  if (MODE != kPartnerOnly) {
    const TA* aq = static_cast<const TA*>(p.aq) + q * p.E;
    const TA* arq = static_cast<const TA*>(p.arq) + q * RD;
    for (int d = lane; d < p.E; d += kWave) qx[d] = to_f32(aq[d]);
    for (int d = lane; d < RD; d += kWave) qr[d] = to_f32(arq[d]);
    wave_sync();
    block_scores<TS>(p, p.as, b, t, local_start, qr, sh, blk, lane);
    pick_blocks(p, blk, sel, selv, lane);
    const TA* keys = static_cast<const TA*>(p.as.keys) + b * p.T * p.E;
    uint64_t best = 0;
    float best_score = -INFINITY;
    for (int c = lane; c < p.CAP; c += kWave) {
      int64_t pos;
      bool valid;
      candidate(p, c, t, local_start, sel, selv, pos, valid);
      if (valid) {
        const float s = exact_score(keys + pos * p.E, qx, p.E, p.exact_scale);
        const uint64_t k = select_key(s, static_cast<uint32_t>(pos));
        if (k > best) {
          best = k;
          best_score = s;
        }
      }
    }
    const uint64_t win = wave_max_u64(best);
    if (win == 0) {
      anchor = t - p.L + 1;
      if (lane == 0) {
        p.out_anchor[q] = static_cast<int32_t>(anchor);
        p.out_anchor_score[q] = -INFINITY;
      }
    } else {
      anchor = key_index(win);
      if (best == win) {
        p.out_anchor[q] = static_cast<int32_t>(anchor);
        p.out_anchor_score[q] = best_score;
      }
    }
    if (MODE == kAnchorOnly) return;
    wave_sync();
  } else {
    anchor = load_any_i(p.anchor_in, p.anchor_dtype, q);
  }

  // Partner queries (relation_select.py:165-193): fp32 sum of the query-side
  // projection and the anchor row of the cached anchor-side projection.
  {
    const TA* pq = static_cast<const TA*>(p.pq) + q * p.pq_row;
    const TA* prq = static_cast<const TA*>(p.prq) + q * p.prq_row;
    if (MODE == kPacked) {
      const bool have = anchor >= 0 && anchor < p.T;
      const TA* pc = static_cast<const TA*>(p.pcache) + (b * p.T + (have ? anchor : 0)) * (2 * p.E);
      for (int d = lane; d < p.E; d += kWave)
        qx[d] = to_f32(pq[d]) + (have ? to_f32(pc[d]) : 0.0f);
      for (int d = lane; d < RD; d += kWave)
        qr[d] = to_f32(prq[d]) + (have ? to_f32(pc[p.E + d]) : 0.0f);
    } else {
      for (int d = lane; d < p.E; d += kWave) qx[d] = to_f32(pq[d]);
      for (int d = lane; d < RD; d += kWave) qr[d] = to_f32(prq[d]);
    }
  }
  wave_sync();
  block_scores<TS>(p, p.ps, b, t, local_start, qr, sh, blk, lane);
  pick_blocks(p, blk, sel, selv, lane);

  const TA* keys = static_cast<const TA*>(p.ps.keys) + b * p.T * p.E;
  uint64_t best = 0;
  for (int c = lane; c < p.CAP; c += kWave) {
    int64_t pos;
    bool valid;
    candidate(p, c, t, local_start, sel, selv, pos, valid);
    valid = valid && pos != anchor;
    const float s = valid ? exact_score(keys + pos * p.E, qx, p.E, p.exact_scale) : -INFINITY;
    sc[c] = s;
    const uint64_t k = select_key(s, static_cast<uint32_t>(c));
    best = k > best ? k : best;
  }
  // K argmax passes; picked lanes drop to -inf but stay in the pool, so once
  // the finite lanes are exhausted every pass lands on lane 0 with -inf
  // (relation_select.py:298-308).
  for (int k = 0; k < p.K; ++k) {
    const uint64_t win = wave_max_u64(best);
    const int c = static_cast<int>(key_index(win));
    if ((c & (kWave - 1)) == lane) {
      int64_t pos;
      bool valid;
      candidate(p, c, t, local_start, sel, selv, pos, valid);
      const bool exhausted = !(key_score(win) > -INFINITY);
      p.out_partner[q * p.K + k] = static_cast<int32_t>(pos);
      p.out_partner_score[q * p.K + k] = exhausted ? -INFINITY : sc[c];
      sc[c] = -INFINITY;
      best = 0;
      for (int cc = lane; cc < p.CAP; cc += kWave) {
        const uint64_t kk = select_key(sc[cc], static_cast<uint32_t>(cc));
        best = kk > best ? kk : best;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

struct Geometry {
  int64_t B, Tq, T;
  int NB, BS, E, H, HD, RB;
};

bool check_stream(const rlm_tensor* keys, const rlm_tensor* mean, const rlm_tensor* stdv,
                  const rlm_tensor* gamma, const rlm_tensor* bias, const char* side,
                  const Geometry& g, int act_dtype, int stat_dtype) {
  char name[96];
  snprintf(name, sizeof(name), "%s_keys", side);
  if (!check_tensor(keys, name, 3) || !check_dim(keys, name, 0, g.B) ||
      !check_dim(keys, name, 1, g.T) || !check_dim(keys, name, 2, g.E) ||
      !check_dtype_is(keys, name, act_dtype))
    return false;
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
                         int64_t top_blocks, int64_t k_out, int32_t strict_valid) {
  RLM_REQUIRE(local_window >= 1 && local_window <= 4096,
              "local_window must be in [1, 4096], got %lld", (long long)local_window);
  RLM_REQUIRE(top_blocks >= 0 && top_blocks <= 64, "top_blocks must be in [0, 64], got %lld",
              (long long)top_blocks);
  RLM_REQUIRE(k_out >= 0 && k_out <= 1024, "k_out must be in [0, 1024], got %lld",
              (long long)k_out);
  RLM_REQUIRE(g.NB >= 1 && g.BS >= 1, "need at least one block of at least one row");
  RLM_REQUIRE(g.E % 4 == 0 && g.E <= 1024, "exact dim must be a multiple of 4 and <= 1024");
  RLM_REQUIRE(g.HD % 4 == 0 && g.H >= 1 && g.H * g.HD <= 1024,
              "router head dim must be a multiple of 4 and heads*head_dim <= 1024");
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
  p.lds_per_wave = select_lds_bytes(p.NB, p.H, p.E, p.H * p.HD, p.TOP, p.CAP);
  RLM_REQUIRE(p.lds_per_wave <= 65536, "selection working set exceeds 64 KiB of LDS per query");
  return hipSuccess;
}

template <int MODE>
hipError_t launch_select(const SelectParams& p, int act_dtype, int stat_dtype,
                         hipStream_t stream) {
  const int64_t queries = p.B * p.Tq;
  if (queries == 0) return hipSuccess;
  int waves = p.Tq > 1 ? 4 : 1;
  while (waves > 1 && waves * p.lds_per_wave > 65536) waves >>= 1;
  const dim3 block(waves * kWave);
  const dim3 grid(static_cast<unsigned>((queries + waves - 1) / waves));
  const size_t lds = static_cast<size_t>(waves) * p.lds_per_wave;
#define RLM_SELECT_CASE(TA_ID, TA, TS_ID, TS)                                          \
  if (act_dtype == TA_ID && stat_dtype == TS_ID) {                                     \
    hipLaunchKernelGGL((select_kernel<TA, TS, MODE>), grid, block, lds, stream, p);    \
    return launch_status("relation_select");                                           \
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

hipError_t select_packed_impl(
    bool seq, const rlm_tensor* anchor_query, const rlm_tensor* anchor_keys,
    const rlm_tensor* anchor_router_query, const rlm_tensor* anchor_block_mean,
    const rlm_tensor* anchor_block_std, const rlm_tensor* anchor_gamma,
    const rlm_tensor* anchor_bias, const rlm_tensor* partner_base,
    const rlm_tensor* partner_anchor_cache, const rlm_tensor* partner_keys,
    const rlm_tensor* partner_block_mean, const rlm_tensor* partner_block_std,
    const rlm_tensor* partner_gamma, const rlm_tensor* partner_bias, const rlm_tensor* position,
    int64_t local_window, int64_t top_blocks, int64_t k_out, int32_t strict_valid,
    const rlm_tensor* out_anchor, const rlm_tensor* out_anchor_score,
    const rlm_tensor* out_partner, const rlm_tensor* out_partner_score, hipStream_t stream) {
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
  hipError_t err = finish_params(p, g, local_window, top_blocks, k_out, strict_valid);
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
  return launch_select<kPacked>(p, act, stat, stream);
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
  return select_packed_impl(false, anchor_query, anchor_keys, anchor_router_query,
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
  return select_packed_impl(true, anchor_query, anchor_keys, anchor_router_query,
                            anchor_block_mean, anchor_block_std, anchor_gamma, anchor_bias,
                            partner_base, partner_anchor_cache, partner_keys, partner_block_mean,
                            partner_block_std, partner_gamma, partner_bias, positions,
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
  hipError_t err = finish_params(p, g, local_window, top_blocks, 0, strict_valid);
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
  hipError_t err = finish_params(p, g, local_window, top_blocks, k_out, strict_valid);
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

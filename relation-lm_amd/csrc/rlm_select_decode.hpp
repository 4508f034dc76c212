// Parameters of the decode-form selection kernel (rlm_select_decode.hip): one
// query per batch row, 16-bit activations, 64-wide exact and router vectors
// (4 heads of 16), caches of at most 512 rows.
#pragma once

#include "rlm_common.hpp"

namespace rlm {

constexpr int kDecodeMaxRows = 512;  // cache rows staged in LDS per stream
constexpr int kDecodeMaxCap = 256;   // candidates per stream (4 per lane of one wave)

// The token's expanded-cache row (decode): for every batch row b,
// cache[b, row, :] = W . op[b, row, :] + bias in bf16, row = t (linear caches)
// or t mod T (ring caches) for the step's position t, read on the device.
// Each workgroup projects kExpandCols columns on its first four waves.
constexpr int kExpandCols = 128;
struct ExpandRowParams {
  const bf16* op;     // [B, T, R] operand cache, R = 32 * KS
  const bf16* w;      // [N, R] expanded weight
  const void* bias;   // [N] or nullptr
  int bias_dtype;
  bf16* cache;        // [B, T, N] expanded cache (row `row` written)
  const void* pos;    // 0-d position
  int pos_dtype;
  int64_t B, T;
  int KS, N;
  int ring;           // 1: T is a power of two and row = t mod T
  uint32_t op_bytes, w_bytes;
};

struct DecodeParams {
  int64_t B, T;
  int NB, BS, BS_log2, L, TOP, K, CAP, RB;
  int strict;
  double exact_scale, head_scale;
  const void* pos;
  int pos_dtype;
  const void* aq;      // [B, 64] exact anchor query
  const void* arq;     // [B, 64] anchor router query
  const void* pbase;   // [B, 128]: partner exact base | partner router base
  const void* pcache;  // [B, T, 128]: cached anchor-side partner contribution
  const void* akeys;   // [B, T, 64]
  const void* pkeys;   // [B, T, 64]
  const void* amean;   // [B, NB, 4, 16] statistics dtype
  const void* astd;
  const void* pmean;
  const void* pstd;
  const void* agamma;  // [4]
  const void* pgamma;
  const void* abias;   // [4, RB]
  const void* pbias;
  int agamma_dtype, pgamma_dtype, abias_dtype, pbias_dtype;
  int32_t* out_anchor;
  float* out_anchor_score;
  int32_t* out_partner;
  float* out_partner_score;
  int off_sc, off_key, off_blk, off_sel, lds_total;
  // Workgroups B .. B + xgroups - 1 of the launch project the expanded-cache
  // row instead (0: none).
  ExpandRowParams x;
  int xgroups;
};

// Fills the LDS layout; false when the shapes do not fit the kernel.
bool select_decode_layout(DecodeParams& p);
hipError_t select_decode_launch(const DecodeParams& p, int act_dtype, int stat_dtype, bool ring,
                                hipStream_t stream);
// The expanded-cache row as its own launch (shapes the decode kernel does not take).
hipError_t expand_row_launch(const ExpandRowParams& x, hipStream_t stream);

}  // namespace rlm

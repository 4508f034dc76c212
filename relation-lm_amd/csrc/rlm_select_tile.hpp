// Parameters of the matrix-core-filtered selection kernel (rlm_select_tile.hip),
// the sequence-form path of relation_select_packed_seq for bf16 activations,
// exact and router dims of 64 and caches of at most 512 rows.
#pragma once

#include "rlm_common.hpp"

namespace rlm {

constexpr int kTileMaxK = 16;      // partners per query
constexpr int kTileMaxTop = 16;    // picked blocks per stream
constexpr int kTileMaxHeads = 8;   // router heads
constexpr int kTileMaxRows = 512;  // cache rows staged in LDS

struct TileParams {
  int64_t B, Tq, T;
  int NB, BS, BS_log2, L, TOP, K, CAP, NCL, H, H_log2, HD, RB;
  int strict;
  double exact_scale, head_scale;
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  int64_t pos_count;  // elements of the position tensor
  const bf16* aq;      // [B*Tq, 64]
  const bf16* arq;     // [B*Tq, 64]
  const bf16* pbase;   // [B*Tq, 128]: exact half, router half
  const bf16* pcache;  // [B, T, 128]
  const bf16* akeys;   // [B, T, 64]
  const bf16* pkeys;
  const void* amean;   // [B, NB, 64] statistics dtype
  const void* astd;
  const void* pmean;
  const void* pstd;
  const void* agamma;
  const void* pgamma;
  const void* abias;
  const void* pbias;
  int agamma_dtype, pgamma_dtype, abias_dtype, pbias_dtype;
  int32_t* out_anchor;
  float* out_anchor_score;
  int32_t* out_partner;
  float* out_partner_score;
  int tiles;  // workgroups per batch row
  // Optional expanded-cache projection in the same launch (x_out != nullptr):
  // x_out[r, :] = x_w . x_op[r, :] + x_bias for every cache row r < x_rows,
  // bf16 with fp32 sums, x_N % 128 == 0, 2 x 128 x 32 x_KS x 2 bytes <= T x 128.
  const bf16* x_op;   // [x_rows, 32 x_KS]
  const bf16* x_w;    // [x_N, 32 x_KS]
  const void* x_bias; // [x_N] or nullptr
  int x_bias_dtype;
  bf16* x_out;        // [x_rows, x_N]
  int64_t x_rows;
  int x_KS, x_N;
  uint32_t x_op_bytes, x_w_bytes;
  int off_keys, off_sc, off_stats, off_rq, off_pq, off_blk, off_lmax, off_list, off_top,
      off_qrec, off_bias, off_sp, off_kmax, lds_total;
};

// Fills the LDS layout; false when it exceeds one CU's 160 KiB.
bool select_tile_layout(TileParams& p);
hipError_t select_tile_launch(const TileParams& p, int stat_dtype, hipStream_t stream);

}  // namespace rlm

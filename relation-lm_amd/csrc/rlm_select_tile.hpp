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
  int off_keys, off_sc, off_stats, off_rq, off_pq, off_blk, off_lmax, off_list, off_top,
      off_qrec, off_bias, off_sp, off_kmax, lds_total;
};

// Fills the LDS layout; false when it exceeds one CU's 160 KiB.
bool select_tile_layout(TileParams& p);
hipError_t select_tile_launch(const TileParams& p, int stat_dtype, hipStream_t stream);

}  // namespace rlm

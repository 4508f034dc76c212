// Parameters of the matrix-core-filtered routed multi-anchor selection
// (rlm_multi_tile.hip), the path of multi_relation_select_seq for bf16
// activations, 64-wide exact and router vectors and any cache length.
#pragma once

#include "rlm_common.hpp"

namespace rlm {

constexpr int kMultiTileMaxSlots = 8;   // anchor slots per query
constexpr int kMultiTileMaxK = 16;      // partners per slot
constexpr int kMultiTileMaxTop = 16;    // picked blocks per routing
constexpr int kMultiTileMaxHeads = 8;   // router heads
constexpr int kMultiTileMaxBlocks = 64; // cache blocks
constexpr int kMultiTileMaxCap = 1024;  // candidates per routing

struct MultiTileParams {
  int64_t B, Tq, T;
  int S, NB, BS, BS_log2, L, TOP, K, CAP, H, H_log2, HD, RB;
  int strict;
  double exact_scale, head_scale;
  const void* pos;
  int pos_dtype;
  int64_t pos_sb, pos_sq;
  int64_t pos_count;   // elements of the position tensor
  const bf16* aq;      // [B*Tq, S, 64]
  const bf16* arq;     // [B*Tq, 64]
  const bf16* pbase;   // [B*Tq, S, 128]: exact half, router half
  const bf16* pcache;  // [B, T, S, 128]
  const bf16* akeys;   // [B, T, S, 64]
  const bf16* pkeys;
  uint32_t key_bytes;  // byte size of each key cache
  const void* amean;   // [B, NB, 64] statistics dtype
  const void* astd;
  const void* pmean;
  const void* pstd;
  const void* agamma;
  const void* pgamma;
  const void* abias;
  const void* pbias;
  int agamma_dtype, pgamma_dtype, abias_dtype, pbias_dtype;
  int32_t* out_anchor;        // [B*Tq, S]
  float* out_anchor_score;
  int32_t* out_partner;       // [B*Tq, S, K]
  float* out_partner_score;
  int tiles;  // workgroups per batch row
  int off_stats, off_sc, off_rank, off_rq, off_eq, off_list, off_top, off_qrec,
      off_bias, off_sp, off_kmax, off_aq, lds_total;
  int q_bytes;  // LDS bytes per query of the region that holds its per-head block
                // scores, then its candidate score list
};

// Fills the LDS layout; false when it exceeds one CU's 160 KiB.
bool multi_tile_layout(MultiTileParams& p);
hipError_t multi_tile_launch(const MultiTileParams& p, int stat_dtype, hipStream_t stream);

}  // namespace rlm

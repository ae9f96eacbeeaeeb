// Kernel argument structs and launchers shared by the fmkv translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmkv_layout.h"

namespace fmkv {

// Where the head-blocks of one cache / pool live.
struct Store {
  uint8_t* base;
  int64_t head_stride;   // bytes between heads of one logical block
  int64_t block_stride;  // bytes between physical blocks
  const int32_t* block_table;  // paged: [n_seqs][table_stride]; null otherwise
  int32_t table_stride;
  int64_t n_blocks;            // physical blocks (bounds for table entries)
  int32_t n_kv_heads;
  BlockLayout layout;
};

// Decode split-K plan shared by the host and the kernels: wave pairs per
// work-group (each pair streams whole head-blocks, one half of head_dim per
// wave) and work-groups per CU the split count aims at (one: a work-group's
// LDS staging fills the CU).
constexpr int kAttnPairs = 4;
constexpr int kAttnWaves = 2 * kAttnPairs;

#ifndef FMKV_ATTN_WG_PER_CU
#define FMKV_ATTN_WG_PER_CU 1
#endif
constexpr int kAttnWgPerCu = FMKV_ATTN_WG_PER_CU;
// The XCD-aware single-sequence plan needs at least one block per stream in
// every split.
constexpr int kAttnPlanMinSkewBlocks = kAttnPairs;

struct AppendArgs {
  Store st;
  const uint16_t* k;  // bf16 [n_seqs][n_new][n_kv_heads][D]
  const uint16_t* v;
  const int32_t* start_pos;  // per sequence, or null -> start_scalar
  int64_t start_scalar;
  int32_t n_new;
  int32_t window;   // ring slots, 0 = linear
  uint32_t sign_bits[16];  // RHT signs of dims 0..D-1, bit d set = -1
  float c;             // 1/sqrt(D) (f32)
  float sqrt_d;        // sqrt(D) (f32), codebook mode
  int32_t cb_bits;     // codebook bits
  // The layer's prologue before the append (k_norm, v_norm, RoPE at each
  // token's position); k_norm_w null: the rows are stored as given.
  const uint16_t* k_norm_w = nullptr;  // bf16 [D]
  float eps = 0.0f;
  int32_t rope_dims = 0;
  float rope_theta = 0.0f;
  int32_t v_from_k = 0;  // V rows are v_norm of the raw K rows (K==V layers)
};

struct AttnArgs {
  Store st;
  const int32_t* seq_lens;  // per sequence, or null -> seq_len (visible positions,
                            // the new token of a decode step included)
  int64_t seq_len;
  int64_t window;
  int64_t vis_begin;
  int32_t group;      // q heads per kv head (<= 8)
  int32_t n_q_heads;
  const uint16_t* q;  // bf16 [n_seqs][n_q_heads][D]
  float qscale;       // softmax scale * log2(e)
  uint32_t sign_bits[16];  // RHT signs of dims 0..D-1, bit d set = -1
  float c;            // 1/sqrt(D)
  float sqrt_d;       // sqrt(D) (f32): binning scale of a codebook decode step's new token
  int32_t bps0;       // blocks of split 0 (>= bps)
  int32_t skew_p = 0;      // XCD-aware plan (split_range): period of the larger splits, 0 = off
  int32_t skew_extra = 0;  // number of splits with bps + 1 blocks
  int32_t bps;        // blocks of every later split
  int32_t max_splits; // split columns of the grid
  int32_t part_stride;  // partial slots per sequence: max_splits + new_col
  float* part_o;      // [n_seqs][part_stride][n_q_heads][D]
  float* part_ml;     // [n_seqs][part_stride][n_q_heads][2]
  void* out;          // [n_seqs][n_q_heads][D]
  int32_t out_f32;
  int32_t direct;     // 1: one split and no new-token column; no combine, write out
  // Decode step (new_col = 1): one more grid column appends the new token
  // (position seq_len - 1) of every (sequence, KV head) and contributes its
  // attention as partial slot n_splits; the split columns leave its slot out.
  int32_t new_col;
  const uint16_t* k_new;  // bf16 [n_seqs][n_kv_heads][D]
  const uint16_t* v_new;
  // The layer's prologue on the new token first (k_norm and RoPE at
  // position seq_len - 1 on K, v_norm on V, as AppendArgs); null: the rows
  // are stored as given.
  const uint16_t* k_norm_w = nullptr;  // bf16 [D]
  float eps = 0.0f;
  int32_t rope_dims = 0;
  float rope_theta = 0.0f;
  // Sparse-V threshold (0: dense). With tau > 0 the gated pass writes, per
  // (sequence, q head), the base-2 score threshold theta = M + log2(tau * L)
  // and the full softmax max M and sum L of the stats pass: tau_stats =
  // [theta | M | L], each [n_seqs][n_q_heads], for the combine.
  float tau;
  float* tau_stats;
  // Sparse-V: the stats pass's largest base-2 score per (sequence, KV head,
  // block) and q head of the group, [n_seqs][n_kv_heads][blk_stride][8]
  // block-major for the gated pass, which reads a block's 8 together and
  // skips the blocks in which no head has a score at or above its theta,
  // and [n_seqs][n_kv_heads][8][blk_stride] head-major for the gather
  // (blk_scores set), whose work-groups each read one head's row (-inf for
  // heads beyond the group; block index relative to the first visible
  // block).
  float* blk_max = nullptr;
  int32_t blk_stride = 0;
  int32_t stats_new_col = 0;  // gated pass, gather: the stats pass had a new-token column
  // Sparse-V: the stats pass's split (m, l), [n_seqs][part_stride][n_q_heads][2],
  // a region of its own: the stats launch writes it in place of part_ml and
  // the gated pass only reads it (the gated work-groups write their own
  // partials to part_ml while others may still be deriving thresholds).
  float* stat_ml = nullptr;
  // Sparse-V gather (launch_sparse_gather in place of the gated pass and the
  // combine): the stats pass also stores the base-2 scores of every block
  // that may hold a kept token, [n_seqs][n_kv_heads][blk_stride][8][16]
  // (q head of the group, token of the block), and zeroes the gather's
  // arrival counters, [n_seqs][n_q_heads]. Null: the gated pass.
  float* blk_scores = nullptr;
  int32_t* sv_count = nullptr;
  int32_t gather_parts = 0;  // work-groups per (sequence, q head) of the gather
  int32_t gather_rows = 0;   // the most visible head-blocks of a sequence (<= kGatherMaxRows)
};

// Prefill (chunked) attention: n_q queries at positions p0 .. p0 + n_q - 1,
// query p attending to key positions [lo(p), p], lo(p) = max(vis_begin,
// p - window + 1) (window 0: vis_begin). Keys below p_split come from
// old_st (a ring of ring_slots slots when window > 0, else linear), keys from
// p_split on from new_st, whose block 0 holds absolute block new_blk0 (a
// staging copy of the chunk for rings; the cache itself, p_split 0, for
// linear caches, which append before attending).
struct PrefillArgs {
  Store old_st;
  Store new_st;  // a paged pool: its block_table maps each sequence's blocks
  int64_t p0;
  const int32_t* start_pos;  // paged: per sequence p0 (device), else null -> p0
  int32_t n_seqs;            // grid z; q and out gain a leading [n_seqs]
  int32_t n_q;
  int64_t window;      // the sliding window of the masks (0: causal only)
  int64_t ring_slots;  // old_st's ring slots (the window rounded up to 16), 0: linear
  int64_t vis_begin;
  int64_t p_split;
  int64_t new_blk0;
  int32_t group;      // q heads per kv head (<= 8)
  int32_t n_q_heads;
  const uint16_t* q;  // bf16 [n_q][n_q_heads][D]
  float qscale;       // softmax scale * log2(e)
  uint32_t sign_bits[16];
  float c;            // 1/sqrt(D)
  void* out;          // [n_q][n_q_heads][D]
  int32_t out_f32;
};

struct ReadArgs {
  Store st;
  int64_t n_slots;    // slots to convert (ring: W; linear: capacity; pool: n_blocks*16)
  uint32_t* codes;    // [n_slots][2][H][words]
  uint16_t* meta;     // [n_slots][2][H][n_meta]
};

struct FetchArgs {
  Store st;
  int64_t offset;
  int64_t window;
  int64_t first_pos;  // first visible position
  int64_t n_pos;      // visible positions
  const float* signs;
  float c;
  void* k_out;        // [n_pos][H][D]
  void* v_out;
  int32_t out_f32;
};

// The leading scalar arguments of the affine decode split kernel, 14 dwords that
// the dispatch preloads into SGPRs (the argument struct follows them): the
// block range (geo_len: the visible length, at most the window on a ring;
// geo_vis_begin: the first visible position, 0 on a ring), the split plan
// (skew = skew_p | skew_extra << 8), the cache and q pointers and flags (bit
// 2 new-token column, bits 4-7 q heads per KV head, bits 8-31 q heads).
struct SplitPre {
  const uint8_t* base;
  const uint16_t* q;
  int32_t geo_len, geo_vis_begin, window, bps0, bps, max_splits;
  uint32_t skew;
  int32_t block_stride, head_stride;
  uint32_t flags;
};

// false when a value does not fit its 32-bit field
inline bool split_pre(const AttnArgs& a, SplitPre* p) {
  const bool ring = a.window > 0;
  const int64_t geo_len = ring ? (a.seq_len < a.window ? a.seq_len : a.window) : a.seq_len;
  if (geo_len > INT32_MAX || (!ring && a.vis_begin > INT32_MAX) || a.window > INT32_MAX ||
      a.st.block_stride > INT32_MAX || a.st.head_stride > INT32_MAX || a.n_q_heads >= (1 << 24) ||
      a.skew_extra >= (1 << 24) || a.skew_p > 255 || a.group > 15)
    return false;
  p->base = a.st.base;
  p->q = a.q;
  p->geo_len = (int32_t)geo_len;
  p->geo_vis_begin = ring ? 0 : (int32_t)a.vis_begin;
  p->window = (int32_t)a.window;
  p->bps0 = a.bps0;
  p->bps = a.bps;
  p->max_splits = a.max_splits;
  p->skew = (uint32_t)a.skew_p | ((uint32_t)a.skew_extra << 8);
  p->block_stride = (int32_t)a.st.block_stride;
  p->head_stride = (int32_t)a.st.head_stride;
  p->flags = (a.new_col ? 4u : 0u) | ((uint32_t)a.group << 4) | ((uint32_t)a.n_q_heads << 8);
  return true;
}

hipError_t launch_append(const AppendArgs& a, int n_seqs, int max_tasks, hipStream_t s);
// ev_begin / ev_end (optional, both or neither) are recorded by the split-K
// kernel's dispatch: the start and end of its execution.
hipError_t launch_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                                   hipEvent_t ev_begin = nullptr, hipEvent_t ev_end = nullptr);
// Decode attention over a codebook (TurboQuant) cache, planned as
// launch_decode_attention plans it: a decode step's new-token column, and
// sparse-V as a statistics pass and the gather (or the gated pass and the
// combine).
hipError_t launch_cb_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                                      hipEvent_t ev_begin = nullptr, hipEvent_t ev_end = nullptr);
// Decode attention over a plain (bf16) cache, planned as the codebook kernel.
hipError_t launch_plain_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads,
                                         hipStream_t s, hipEvent_t ev_begin = nullptr,
                                         hipEvent_t ev_end = nullptr);
// Sparse-V after the statistics pass: the kept weights of every q head and
// the V rows they weigh, straight to out (fmkv_readback.hip).
// At most kGatherMaxRows visible head-blocks per sequence.
constexpr int kGatherMaxRows = 16384;
hipError_t launch_sparse_gather(const AttnArgs& a, int n_seqs, hipStream_t s);
// The split merge of every decode kernel: out = LSE merge of the partials.
hipError_t launch_combine(const AttnArgs& a, int n_seqs, hipStream_t s);
hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t s);
hipError_t launch_read_codes(const ReadArgs& a, hipStream_t s);
hipError_t launch_fetch(const FetchArgs& a, hipStream_t s);

}  // namespace fmkv

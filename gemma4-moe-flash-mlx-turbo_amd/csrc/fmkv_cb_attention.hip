// Decode attention over codebook (TurboQuant) caches.
//
// Replaces mlx_rs::fast::scaled_dot_product_attention at decode
// (src/model/gemma4_attention.rs:94-103) when the cache holds the reference's
// own quantizer output (turbo_round_trip_kv, src/cache.rs:94-129): per token
// row, Lloyd-Max indices idx_d of the rotated, normalised row plus its f16 L2
// norm. In the rotated domain a row is y_d = centroid[idx_d] * norm / sqrt(D),
// so with q_rot = q . R (src/cache.rs:47-62)
//   score_t = (norm_t / sqrt D) * sum_d q_rot[d] * centroid[idx_{t,d}]
//   out     = (sum_t w_t (norm_t / sqrt D) centroid[idx_t]) . R^T.
// The cache is read as stored, with no bf16 round trip.
//
// One work-group = one (split of consecutive 16-token blocks, KV head,
// sequence) with four wave pairs, as in the affine kernel: pair p streams the
// head-blocks b_begin + p, b_begin + p + 4, ...; wave h of a pair owns half h
// of head_dim, which the layout keeps contiguous for K and V alike
// (fmkv_layout.h), copies that half of each block HBM -> LDS with
// buffer_load_dwordx4 ... lds several stages ahead, exchanges its partial
// scores with its partner through LDS and runs the same online softmax.
//
// Dequantization happens in registers on the way to the matrix cores. The 2-
// and 3-bit centroids times 1000 are integers f16 holds exactly, so an LDS
// table holds, for every pair of indices (two dims of a K row, or two tokens
// of a V dim), the two f16 integers as one word: one 4-byte lookup gives the
// operand word of two elements straight into the operand registers, and the
// 1/1000 joins the value scale norm / sqrt(D). 4-bit centroids need 12
// significant bits: their table holds {f16 high part, f16 residual} per
// index, paired by v_perm into a high and a residual operand word. Each table
// is replicated 32 times, entry e of copy l at (e * 32 + l) * 4, so the lanes
// of a half-wave never hit one bank twice. Per block, per 32-dim slice and per
// 16-dim tile of the wave's half:
//   QK   S^T[16 tok x 16 col] += K[16 x 32] . Q^T[32 x 16]
//        (v_mfma_f32_16x16x32_f16; 4 bits: once with the high and once with
//        the residual centroid parts, a product then keeping ~22 bits of the
//        centroid where one f16 alone is off by up to 2^-12 of the value).
//        Column c = q head c & 7, c < 8 the f16 high part of q_rot and
//        c >= 8 its residual; the columns fold with DPP row_ror:8.
//   PV   O^T[16 dim x 16 col] += V^T[16 dim x 16 tok] . P'^T[16 tok x 16 col]
//        (v_mfma_f32_16x16x16f16; 4 bits: high and residual centroid parts),
//        with P' = p * norm_t / sqrt D split hi/lo in the same columns.
// Epilogue: the pairs' (m, l, O) merge in LDS, the inverse rotation
// o . R^T = c * FWHT(o o s) follows, and the result is the final output (one
// split) or a split partial for the shared combine kernel.
//
// Decode step (a.new_col): one more grid column appends the step's new token
// (the append kernel's codebook arithmetic) and contributes its attention as
// one more partial; the split columns leave its slot out. A decode step is
// then this launch and the combine.
#include <hip/hip_ext.h>

#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_prologue.h"
#include "fmkv_quant.h"
#include "fmkv_attn_common.h"
#include "fmkv_cb_common.h"

namespace fmkv {
namespace {

constexpr int kCbWaves = 8;  // four wave pairs, two waves per SIMD
constexpr int kCbStreams = kCbWaves / 2;

template <int D, int BITS>
struct CbPlan {
  static constexpr BlockLayout L = make_layout(D, BITS, kCodebook);
  static constexpr int kHalfBytes = D * BITS;  // one half of K (or V) codes: 16 x D/2 x BITS bits
  static constexpr int kHalfPieces = kHalfBytes / 16;
  static constexpr int kHalfCopies = (kHalfPieces + 63) / 64;  // copy instructions per half
  static constexpr int kNSW = D / 64;                        // 32-dim QK slices per wave
  static constexpr int kNTW = D / 32;                        // 16-dim PV tiles per wave
  // a stage: [K half 0][K half 1][V half 0][V half 1][wave 0 norms][wave 1 norms],
  // codes at their head-block offsets; a wave's norms are K then V (32 B each)
  static constexpr int kNormOff = 4 * kHalfBytes;
  static constexpr int kStageBytes = kNormOff + 2 * 64;
  static constexpr int kCopies = 2 * kHalfCopies + 1;  // per wave per block
  // the centroid lookup table (fmkv_cb_common.h)
  static constexpr int kLutBytes = CbLut<BITS>::kBytes;
  // q table (the QK B operands, one KiB per slice), then the score exchange
  static constexpr int kTabBytes = (D / 32) * 1024;
  static constexpr int kXBytes = kCbWaves * 2 * 64 * 16;
  static constexpr int kScratch = cmax(cmax(kTabBytes, kXBytes), 8 * D * 2);
  static constexpr int kQS = D + 4;  // merge-row stride (floats)
  static constexpr int kFit =
      (160 * 1024 - 2048 - kLutBytes - kScratch) / (kCbStreams * kStageBytes);
  static constexpr int kStagesA = kFit > 8 ? 8 : kFit;
  static constexpr int kStages = kStagesA * kCopies <= 63 ? kStagesA : 63 / kCopies;
  static constexpr int kStageRegion = kCbStreams * kStages * kStageBytes;
  static_assert(kHalfBytes % 16 == 0, "halves are whole copy pieces");
  static_assert(kStages >= 2, "two stages per stream fit");
  static_assert(8 * kQS * 4 <= kStages * kStageBytes, "merge rows fit in a stream's stages");
};

// The raw bf16 q row of GQA head `wave` to LDS at dst + wave * D * 2, copied
// by that wave (lanes < D / 8).
template <int D>
__device__ inline void cb_copy_q_row(const AttnArgs& a, uint8_t* dst, int seq, int kvh, int wave,
                                     int lane) {
  if (wave < a.group && lane < D / 8) {
    const uint16_t* qh =
        a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * a.group + wave) * D;
    dma16(lds_addr(dst + wave * D * 2), lane * 16, buffer_rsrc(qh, (uint32_t)(D * 2)));
  }
}

// q_rot = (FWHT(q * qscale) * c) o s of head `wave` (every wave whose raw
// row has landed), written over the raw rows as the QK B operands: slice k
// (dims 32k .. 32k + 31) at k KiB, lane (jj, c) = (lane / 16, lane % 16):
// 8 f16 of head c & 7, dims 32k + 8jj .. + 7 -- the f16 high part of q_rot
// for c < 8, the residual for c >= 8, zero past the group. Every thread of
// the work-group calls it (it holds two barriers).
template <int D>
__device__ void cb_build_q_table(const AttnArgs& a, uint8_t* tab, int wave, int lane,
                                 uint32_t sbits) {
  constexpr int E = D / 64;
  float x[E];
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = 0.0f;
  if (wave < a.group) {
    const uint32_t* raw = reinterpret_cast<const uint32_t*>(tab + (wave * D + lane * E) * 2);
#pragma unroll
    for (int k = 0; k < E / 2; k++) {
      const uint32_t w = raw[k];
      x[2 * k] = __uint_as_float(w << 16) * a.qscale;
      x[2 * k + 1] = __uint_as_float(w & 0xffff0000u) * a.qscale;
    }
    wave_fwht_signed<E>(x, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = apply_sign(x[i] * cs, sbits, i);
  }
  _Float16 hv[E], lv[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    hv[i] = (_Float16)x[i];
    lv[i] = (_Float16)(x[i] - (float)hv[i]);
  }
  __syncthreads();  // every raw row is read before the table replaces them
  if (wave < 8) {
    const int d0 = lane * E, k = d0 >> 5, jj = (d0 & 31) >> 3, i0 = d0 & 7;
    uint8_t* ent = tab + k * 1024 + i0 * 2;
    store_halves<E>(ent + (jj * 16 + wave) * 16, hv);
    store_halves<E>(ent + (jj * 16 + wave + 8) * 16, lv);
  }
  __syncthreads();
}

// The new-token column of a decode step, one work-group per (seq, kvh): the
// token at position T - 1 is normalised, rotated and binned exactly as the
// append kernel does it (src/cache.rs:94-129), its indices and f16 norm go to
// its slot (ring: (T - 1) mod W; paged: through the block table) -- cleared
// and set bit by bit with atomics, since other tokens' indices share the
// words and the split columns may be reading them -- and, as the reference's
// current token attends to its own round-tripped K/V (src/cache.rs:295-298),
// it contributes partial slot n_splits: m = q_rot . k_deq (base 2), l = 1,
// o = v_deq . R^T, the same row for every head of the group. Wave 0 handles
// K, wave 1 V. With a.k_norm_w the layer's prologue runs on the raw
// projections first, exactly as the append kernel runs it (K = RoPE(k_norm(k))
// in bf16, V = v_norm(v) in f32); the RoPE (cos, sin) table of position T - 1
// is built by every thread into `rope` (LDS, rope_dims / 2 float2) before the
// q table's barriers.
template <int D, int BITS>
__device__ void cb_new_token_column(const AttnArgs& a, uint8_t* tab, float2* rope, int64_t T,
                                    int n_splits, int kvh, int seq, int wave, int lane) {
#pragma clang fp contract(off)
  constexpr BlockLayout L = make_layout(D, BITS, kCodebook);
  constexpr int E = D / 64;
  const int G = a.group;
  const bool pro = a.k_norm_w != nullptr;
  cb_copy_q_row<D>(a, tab, seq, kvh, wave, lane);
  if (pro && T >= 1) {
    for (int j = wave * 64 + lane; j < (a.rope_dims >> 1); j += kCbWaves * 64)
      rope[j] = rope_cos_sin(T - 1, rope_inv_freq(j, a.rope_dims, a.rope_theta));
  }
  wait_vmcnt<0>();
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  cb_build_q_table<D>(a, tab, wave, lane, sbits);
  if (wave >= 2) return;  // no barrier follows

  const bool isv = wave == 1;
  const int d0 = lane * E;
  const int64_t pbase = ((int64_t)seq * a.part_stride + n_splits) * a.n_q_heads + (int64_t)kvh * G;
  if (T < 1) {  // no token: an empty partial
    for (int h = 0; h < G; h++) {
      if (isv) {
#pragma unroll
        for (int i = 0; i < E; i++) a.part_o[(pbase + h) * D + d0 + i] = 0.0f;
      } else if (lane == 0) {
        a.part_ml[(pbase + h) * 2 + 0] = -1e30f;
        a.part_ml[(pbase + h) * 2 + 1] = 0.0f;
      }
    }
    return;
  }

  float x[E];
  load_row<E>((isv ? a.v_new : a.k_new) + ((int64_t)seq * a.st.n_kv_heads + kvh) * D + d0, x);
  if (pro) {  // the rope table is complete: cb_build_q_table's barriers passed
    if (!isv) {
      float w[E];
      load_row<E>(a.k_norm_w + d0, w);
      k_norm_row<E>(x, w, a.eps, lane);
      rope_row<E>(x, a.rope_dims, lane, [&](int j) { return rope[j]; });
    } else {
      v_norm_row<E>(x, a.eps, lane);
    }
  }
  const float norm = sqrtf(canonical_sumsq<E>(x, lane));
  const float den = norm + 1e-8f;
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = x[i] / den;
  wave_fwht_signed<E>(x, lane);
  const float cl = fwht_lane_sign(lane) * a.c;
  uint32_t code[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const float sc = ((sbits >> i) & 1u) ? -cl : cl;
    code[i] = (uint32_t)cb_index((x[i] * sc) * a.sqrt_d, BITS);
  }
  const uint16_t n16 = f32_to_f16_bits(norm);

  // slot write (a bad block-table entry skips it; the token still attends)
  const int64_t pos = T - 1;
  const int64_t slot = a.window > 0 ? pos % a.window : pos;
  const int64_t lb = slot / kBlockTokens;
  const int t = (int)(slot % kBlockTokens);
  int64_t phys = lb;
  bool ok = true;
  if (a.st.block_table) {
    ok = lb < a.st.table_stride;
    phys = ok ? (int64_t)a.st.block_table[(int64_t)seq * a.st.table_stride + lb] : -1;
  }
  ok = ok && phys >= 0 && phys < a.st.n_blocks;
  if (ok) {
    uint8_t* blk = a.st.base + phys * a.st.block_stride + (int64_t)kvh * a.st.head_stride;
    uint32_t* w = reinterpret_cast<uint32_t*>(blk + (isv ? L.v_codes : L.k_codes));
    // bits [bit, bit + n) of the region := v
    auto put = [&](int64_t bit, uint64_t v, int n) {
      const int wi = (int)(bit >> 5), off = (int)(bit & 31);
      const uint64_t m = (((uint64_t)1 << n) - 1) << off;
      v <<= off;
      atomicAnd(&w[wi], ~(uint32_t)m);
      atomicOr(&w[wi], (uint32_t)v);
      if (off + n > 32) {
        atomicAnd(&w[wi + 1], ~(uint32_t)(m >> 32));
        atomicOr(&w[wi + 1], (uint32_t)(v >> 32));
      }
    };
    if (!isv) {
      // the lane's E dims are E * BITS consecutive bits of the half row
      uint64_t v = 0;
#pragma unroll
      for (int i = 0; i < E; i++) v |= (uint64_t)code[i] << (i * BITS);
      put(cb_k_bit(D, BITS, t, d0), v, E * BITS);
    } else {
#pragma unroll
      for (int i = 0; i < E; i++) put(cb_v_bit(BITS, t, d0 + i), code[i], BITS);
    }
    if (lane == 0) *reinterpret_cast<uint16_t*>(blk + (isv ? L.v_meta : L.k_meta) + t * 2) = n16;
  }

  // the stored row in the rotated domain, as the split columns read it:
  // centroid * norm / sqrt(D), the norm as stored
  const float vs = f16_bits_to_f32(n16) * a.c;
  float y[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const uint32_t ci = code[i];
    y[i] = BITS == 2 ? kCbCent2[ci] : BITS == 3 ? kCbCent3[ci] : kCbCent4[ci];
  }
  if (!isv) {
    const int k = d0 >> 5, jj = (d0 & 31) >> 3, i0 = d0 & 7;
    const uint8_t* ent = tab + k * 1024 + i0 * 2;
    for (int h = 0; h < G; h++) {
      const _Float16* qh = reinterpret_cast<const _Float16*>(ent + (jj * 16 + h) * 16);
      const _Float16* ql = reinterpret_cast<const _Float16*>(ent + (jj * 16 + h + 8) * 16);
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < E; i++) p += ((float)qh[i] + (float)ql[i]) * y[i];
      p = group_sum<64>(p, lane);
      if (lane == 0) {
        a.part_ml[(pbase + h) * 2 + 0] = p * vs;
        a.part_ml[(pbase + h) * 2 + 1] = 1.0f;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; i++) y[i] = apply_sign(y[i] * vs, sbits, i);
    wave_fwht_signed<E>(y, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int i = 0; i < E; i++) a.part_o[(pbase + h) * D + d0 + i] = y[i] * cs;
  }
}

// MODE: kDense, or the statistics (kStats: keys only, split (m, l) and block
// maxima) and gated (kGated) passes of sparse-V, as the affine kernel runs
// them.
template <int D, int BITS, int MODE>
__global__ __launch_bounds__(kCbWaves * 64)
__attribute__((amdgpu_waves_per_eu(2, 2)))
void cb_decode_kernel(AttnArgs a) {
  using P = CbPlan<D, BITS>;
  constexpr BlockLayout L = P::L;
  constexpr int E = D / 64;
  constexpr int NSW = P::kNSW, NTW = P::kNTW;
  // copy instructions per wave per block (the stats pass copies no V codes)
  constexpr int NST = P::kStages, SB = P::kStageBytes;
  constexpr int CP = MODE == kStats ? P::kHalfCopies + 1 : P::kCopies;
  constexpr int HB = P::kHalfBytes;
  constexpr int QS = P::kQS;
  constexpr int NS = kCbStreams;

  __shared__ __align__(16) uint8_t stage[P::kStageRegion];
  __shared__ __align__(16) uint8_t scratch[P::kScratch];  // q rows, q table, then score exchange
  __shared__ __align__(16) uint8_t lut[P::kLutBytes];
  __shared__ float ml_s[NS][8][2];
  __shared__ int xflag[kCbWaves];
  __shared__ float th_s[8];  // sparse-V gated pass: the group's thresholds

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int stream = wave >> 1, half = wave & 1;
  const int j = lane >> 4, c = lane & 15;
  const int head = c & 7;
  const bool hi = c < 8;
  const int G = a.group;
  const bool col_valid = head < G;
  // this lane's copy of the tables
  const uint32_t lut_l = lds_addr(lut) + (lane & (kLutCopies - 1)) * 4;
  // grid (KV head, sequence, split column), as the affine kernel
  const int kvh = blockIdx.x, seq = blockIdx.y, split = blockIdx.z;

  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps0, a.bps, a.max_splits, a.skew_p);
  if constexpr (MODE != kGated) {
    if (a.new_col && split == (int)gridDim.z - 1) {
      static_assert(P::kStageRegion >= D / 2 * (int)sizeof(float2), "rope table fits the staging");
      cb_new_token_column<D, BITS>(a, scratch, reinterpret_cast<float2*>(stage), T, n_splits, kvh,
                                   seq, wave, lane);
      return;
    }
  }
  if (split >= n_splits) return;
  int64_t b_begin, b_end;
  split_range(geo, split, a.bps0, a.bps, a.skew_p, a.skew_extra, &b_begin, &b_end);

  // table entries through the constant address space: a uniform index then
  // becomes a scalar load, which never waits for the copies in flight
  typedef const int32_t __attribute__((address_space(4)))* table_ptr;
  const table_ptr table =
      a.st.block_table
          ? (table_ptr)(uintptr_t)(a.st.block_table + (int64_t)seq * a.st.table_stride)
          : nullptr;
  const uint8_t* hbase = a.st.base + (int64_t)kvh * a.st.head_stride;
  auto blk_ptr = [&](int64_t lb) -> const uint8_t* {
    int64_t phys = table ? (int64_t)table[lb] : lb;
    // a bad table entry reads a valid block rather than faulting
    phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
    return hbase + phys * a.st.block_stride;
  };

  const int64_t pb0 = b_begin + stream;
  const int nb = pb0 < b_end ? (int)((b_end - pb0 + NS - 1) / NS) : 0;
  // sparse-V: this (sequence, KV head)'s row of block maxima; the gated pass
  // visits only the blocks holding a score at or above a head's threshold
  const int64_t blk_row =
      MODE == kDense ? 0 : ((int64_t)seq * a.st.n_kv_heads + kvh) * a.blk_stride;
  BlockList blist{0ull, 0, nb};
  int nbx = nb;  // blocks visited
  if constexpr (MODE == kGated) {
    gated_thresholds(a, n_splits, seq, kvh, G, split, wave, lane, th_s);
    float thk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) thk[k] = k < G ? th_s[k] : INFINITY;
    blist = gated_block_list(a, thk, blk_row, geo.blk_lo, pb0, NS, nb, T, lane, &nbx);
  }
  BlockList bcopy = blist;  // the copies run ahead of the visits on the same list
  uint8_t* const pstage = stage + stream * NST * SB;
  const uint32_t pstage_lds = lds_addr(pstage);

  // This wave's half of block lb into stage st: its K half, its V half, and
  // with one partial instruction (lanes 0..3) the block's K and V norms.
  auto copy_block = [&](int st, int64_t lb) {
    const u32x4 rs = buffer_rsrc(blk_ptr(lb), (uint32_t)L.block_bytes);
    const uint32_t sl = pstage_lds + st * SB;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of this stage are done
#pragma unroll
    for (int r = 0; r < (MODE == kStats ? 1 : 2); r++) {
      const int off = (int)(r == 0 ? L.k_codes : L.v_codes) + half * HB;
#pragma unroll
      for (int k = 0; k < P::kHalfCopies; k++) {
        if (P::kHalfPieces % 64 == 0 || k * 64 + lane < P::kHalfPieces)
          dma16(sl + off + k * 1024, off + k * 1024 + lane * 16, rs);
      }
    }
    if (lane < 4)
      dma16(sl + P::kNormOff + half * 64, (int)(lane < 2 ? L.k_meta : L.v_meta) + (lane & 1) * 16, rs);
  };

  // ---- prologue: LUT, copies, q table ----
  cb_fill_lut<BITS>(lut, tid, kCbWaves * 64);
  if (lane == 0) xflag[wave] = 0;
  constexpr int NQ = (NST + 1) / 2;
  cb_copy_q_row<D>(a, scratch, seq, kvh, wave, lane);
#pragma unroll
  for (int s = 0; s < NQ; s++)
    if (s < nbx) copy_block(s, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : s));
  wait_copies<CP, NQ>(nbx < NQ ? nbx : NQ);  // the q copy preceded every block
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  cb_build_q_table<D>(a, scratch, wave, lane, sbits);
#pragma unroll
  for (int s = NQ; s < NST; s++)
    if (s < nbx) copy_block(s, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : s));
  half8_t bq[NSW];
#pragma unroll
  for (int s = 0; s < NSW; s++)
    bq[s] = *reinterpret_cast<const half8_t*>(scratch + (half * NSW + s) * 1024 + lane * 16);
  __syncthreads();  // the table is consumed: the region becomes the score exchange
  float4_t* const xs = reinterpret_cast<float4_t*>(scratch);  // [wave][parity][lane]

  float4_t o[NTW];
#pragma unroll
  for (int i = 0; i < NTW; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.0f;
  const float lo_sel = hi ? 0.0f : 1.0f;
  // the codebook's value scale 1 / sqrt(D), in the table operands' units
  const float inv_sd = a.c * kCbOperandScale<BITS>;

  // visible slots: linear [vis_lo, vis_hi); ring [0, min(T, W)), unless a
  // trim hides older positions (then each slot's position is computed)
  const int64_t vis_lo = a.window > 0 ? 0 : a.vis_begin;
  const int64_t vis_hi = a.window > 0 ? (T < a.window ? T : a.window) : T;
  const bool ring_trim = a.window > 0 && a.vis_begin > T - a.window;
  // a decode step's new token is the new-token column's (its slot may still
  // hold the position it replaces, or be written meanwhile)
  int64_t ex_slot = -1;
  if (a.new_col && T > 0) ex_slot = a.window > 0 ? (T - 1) % a.window : T - 1;
  // sparse-V: this column's score threshold
  float theta = -INFINITY;
  if constexpr (MODE == kGated) theta = col_valid ? th_s[head] : -INFINITY;

  // this lane's fields: QK slice s, token t = c of the MFMA A rows:
  // 8 indices at bit (t D/2 + 32 s + 8 j) BITS of the K half;
  // PV tile n, dim 16 n + c, tokens 4 j .. 4 j + 3: 4 indices at bit
  // ((16 n + c) 16 + 4 j) BITS of the V half
  const int kbit0 = (c * (D / 2) + 8 * j) * BITS;
  const int vbit0 = (c * 16 + 4 * j) * BITS;

  // slice s moves the K field by 32 BITS bits (a whole number of words),
  // tile n the V field by 256 BITS bits, so a lane's shift stays put
  const uint32_t ksh = kbit0 & 31, vsh = vbit0 & 31;
  auto process = [&](const uint8_t* sp, int64_t b, int it) {
    const uint32_t* kw =
        reinterpret_cast<const uint32_t*>(sp + (int)L.k_codes + half * HB) + (kbit0 >> 5);
    const uint32_t* vw =
        reinterpret_cast<const uint32_t*>(sp + (int)L.v_codes + half * HB) + (vbit0 >> 5);
    // this half's S^T = K . q_rot^T: exact integer centroids (2, 3 bits), or
    // the high and residual centroid parts (4 bits)
    float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NSW; s++) {
      const uint32_t f = lds_field<BITS>(kw, s * BITS, ksh);
      if constexpr (kCbExact<BITS>) {
        const half8_t ak = __builtin_bit_cast(
            half8_t, (u32x4){cb_pair_exact<BITS, 0>(lut_l, f), cb_pair_exact<BITS, 1>(lut_l, f),
                             cb_pair_exact<BITS, 2>(lut_l, f), cb_pair_exact<BITS, 3>(lut_l, f)});
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[s], acc, 0, 0, 0);
      } else {
        uint32_t h4[4], l4[4];
        cb_pair_hl4<0>(lut_l, f, h4[0], l4[0]);
        cb_pair_hl4<1>(lut_l, f, h4[1], l4[1]);
        cb_pair_hl4<2>(lut_l, f, h4[2], l4[2]);
        cb_pair_hl4<3>(lut_l, f, h4[3], l4[3]);
        const half8_t ah = __builtin_bit_cast(half8_t, (u32x4){h4[0], h4[1], h4[2], h4[3]});
        const half8_t al = __builtin_bit_cast(half8_t, (u32x4){l4[0], l4[1], l4[2], l4[3]});
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[s], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[s], acc, 0, 0, 0);
      }
    }
    // the tokens' norms: lane (j, c) holds tokens 4j .. 4j + 3
    const uint2 kn = *reinterpret_cast<const uint2*>(sp + P::kNormOff + half * 64 + 8 * j);
    const uint2 vn = *reinterpret_cast<const uint2*>(sp + P::kNormOff + half * 64 + 32 + 8 * j);

    // exchange the half scores with the partner wave (release orders the
    // data before the flag); both waves add the halves in the same order
    const int par = it & 1;
    xs[(wave * 2 + par) * 64 + lane] = acc;
    __hip_atomic_store(&xflag[wave], it + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(&xflag[wave ^ 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           it + 1)
      __builtin_amdgcn_s_sleep(1);
    const float4_t other = xs[((wave ^ 1) * 2 + par) * 64 + lane];
    const float4_t s0 = half == 0 ? acc : other;
    const float4_t s1 = half == 0 ? other : acc;
    const float kscale[4] = {lo16(kn.x) * inv_sd, hi16(kn.x) * inv_sd, lo16(kn.y) * inv_sd,
                             hi16(kn.y) * inv_sd};
    const float vscale[4] = {lo16(vn.x) * inv_sd, hi16(vn.x) * inv_sd, lo16(vn.y) * inv_sd,
                             hi16(vn.y) * inv_sd};
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float t = s0[i] + s1[i];
      sc[i] = col_valid ? (t + row_ror8(t)) * kscale[i] : -INFINITY;
    }
    // visibility: whole block in the common case, per token at the edges
    const int64_t t0 = b * kBlockTokens;
    const bool full = t0 >= vis_lo && t0 + kBlockTokens <= vis_hi && !ring_trim &&
                      (uint64_t)(ex_slot - t0) >= (uint64_t)kBlockTokens;
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t slot = t0 + 4 * j + i;
        bool vis = slot >= vis_lo && slot < vis_hi && slot != ex_slot;
        if (ring_trim) vis = vis && slot_position(slot, T, a.window) >= a.vis_begin;
        if (!vis) sc[i] = -INFINITY;
      }
    }
    if constexpr (MODE == kGated) {
#pragma unroll
      for (int i = 0; i < 4; i++) sc[i] = sc[i] >= theta ? sc[i] : -INFINITY;
    }
    // online softmax in base 2 (the affine kernel's rule: the reference max
    // moves only on jumps above kRescaleSlack)
    float mb = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    if constexpr (MODE == kStats) {
      // the block's largest score per head, for the gated pass's block skip
      const int64_t rb = b - geo.blk_lo;
      if (half == 0 && j == 0 && hi && rb < a.blk_stride)
        a.blk_max[blk_max_at(a, blk_row, rb, head)] = col_valid ? mb : -INFINITY;
    }
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run + kRescaleSlack)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      if (__any(l_run > 0.0f)) {
#pragma unroll
        for (int i = 0; i < NTW; i++) o[i] *= alpha;
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(sc[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
    if constexpr (MODE == kStats) {
      store_block_scores(a, blk_row, b - geo.blk_lo, head, j, sc, mb, m_run, log2f(a.tau),
                         half == 0 && hi && col_valid);
      return;
    }
    // sparse-V: a block whose weights are all below tau adds nothing to O
    // (the pair's waves hold the same scores: a uniform branch)
    if constexpr (MODE == kGated) {
      if (!__any((p[0] + p[1]) + (p[2] + p[3]) > 0.0f)) return;
    }

    // O^T += V^T . P'^T, P' = p * norm / sqrt D as f16 high (c < 8) and
    // residual (c >= 8) columns
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = p[i] * vscale[i];
    const half2_t h01 = pkrtz(x[0], x[1]);
    const half2_t h23 = pkrtz(x[2], x[3]);
    const half2_t b01 = pkrtz(fmaf(-lo_sel, (float)h01[0], x[0]), fmaf(-lo_sel, (float)h01[1], x[1]));
    const half2_t b23 = pkrtz(fmaf(-lo_sel, (float)h23[0], x[2]), fmaf(-lo_sel, (float)h23[1], x[3]));
    const half4_t bp = cat4(b01, b23);
#pragma unroll
    for (int n = 0; n < NTW; n++) {
      const uint32_t f = lds_field<BITS>(vw, n * 8 * BITS, vsh);
      if constexpr (kCbExact<BITS>) {
        const half4_t av = __builtin_bit_cast(
            half4_t, make_uint2(cb_pair_exact<BITS, 0>(lut_l, f), cb_pair_exact<BITS, 1>(lut_l, f)));
        o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bp, o[n], 0, 0, 0);
      } else {
        uint32_t h2[2], l2[2];
        cb_pair_hl4<0>(lut_l, f, h2[0], l2[0]);
        cb_pair_hl4<1>(lut_l, f, h2[1], l2[1]);
        const half4_t ah = __builtin_bit_cast(half4_t, make_uint2(h2[0], h2[1]));
        const half4_t al = __builtin_bit_cast(half4_t, make_uint2(l2[0], l2[1]));
        o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bp, o[n], 0, 0, 0);
        o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bp, o[n], 0, 0, 0);
      }
    }
  };

  // stage st holds block i; before reading it, wait until only the copies
  // issued after it (the next min(NST - 1, nb - 1 - i) blocks) are pending;
  // once read, the stage is refilled with block i + NST
  int st = 0;
  for (int i = 0; i < nbx; i++) {
    const int rest = nbx - 1 - i;
    wait_copies<CP, NST - 1>(rest < NST - 1 ? rest : NST - 1);
    process(pstage + st * SB, pb0 + (int64_t)NS * (MODE == kGated ? blist.pop() : i), i);
    if (i + NST < nbx)
      copy_block(st, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : i + NST));
    st = st + 1 == NST ? 0 : st + 1;
  }

  // ---- epilogue: merge the four pairs, inverse rotation, store ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
  if constexpr (MODE == kStats) {
    // the split's softmax statistics per head: max and sum over the pairs
    if (hi && col_valid && half == 0 && j == 0) {
      ml_s[stream][head][0] = m_run;
      ml_s[stream][head][1] = l_run;
    }
    __syncthreads();
    if (wave == 0 && lane < G) {
      float M = ml_s[0][lane][0];
#pragma unroll
      for (int q = 1; q < NS; q++) M = fmaxf(M, ml_s[q][lane][0]);
      float Lsum = 0.0f;
#pragma unroll
      for (int q = 0; q < NS; q++)
        Lsum = fmaf(__builtin_amdgcn_exp2f(ml_s[q][lane][0] - M), ml_s[q][lane][1], Lsum);
      const int64_t r = ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G + lane;
      a.part_ml[r * 2 + 0] = M;
      a.part_ml[r * 2 + 1] = Lsum;
      if (split == 0 && a.sv_count) a.sv_count[(int64_t)seq * a.n_q_heads + (int64_t)kvh * G + lane] = 0;
    }
    return;
  }
  // fold the residual columns (c >= 8) into the high-part columns (c < 8)
#pragma unroll
  for (int n = 0; n < NTW; n++)
#pragma unroll
    for (int i = 0; i < 4; i++) o[n][i] = o[n][i] + row_ror8(o[n][i]);
  // the stream's own stages become its merge rows [head][QS] once both of
  // its waves are done with them
  __hip_atomic_store(&xflag[wave], nb + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(&xflag[wave ^ 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
         nb + 1)
    __builtin_amdgcn_s_sleep(1);
  float* const Rp = reinterpret_cast<float*>(pstage);
  if (hi && col_valid) {
#pragma unroll
    for (int n = 0; n < NTW; n++) {
      const int d = half * (D / 2) + n * 16 + 4 * j;
      *reinterpret_cast<float4_t*>(&Rp[head * QS + d]) = o[n];
    }
    if (half == 0 && j == 0) {
      ml_s[stream][head][0] = m_run;
      ml_s[stream][head][1] = l_run;
    }
  }
  __syncthreads();  // every stream's rows are written

  if (wave < G) {  // head w on wave w
    const int hh = wave;
    float M = ml_s[0][hh][0];
#pragma unroll
    for (int q = 1; q < NS; q++) M = fmaxf(M, ml_s[q][hh][0]);
    float wgt[NS], Lsum = 0.0f;
#pragma unroll
    for (int q = 0; q < NS; q++) {
      wgt[q] = __builtin_amdgcn_exp2f(ml_s[q][hh][0] - M);
      Lsum = fmaf(wgt[q], ml_s[q][hh][1], Lsum);
    }
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) {
      float v = 0.0f;
#pragma unroll
      for (int q = 0; q < NS; q++)
        v = fmaf(wgt[q], reinterpret_cast<const float*>(stage + q * NST * SB)[hh * QS + lane * E + i],
                 v);
      x[i] = apply_sign(v, sbits, i);
    }
    wave_fwht_signed<E>(x, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
    const int64_t qh0 = (int64_t)seq * a.n_q_heads + (int64_t)kvh * G;
    if (a.direct) {
      const int64_t o_idx = (qh0 + hh) * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; i++) {
        const float v = Lsum > 0.0f ? (x[i] * cs) / Lsum : 0.0f;
        if (a.out_f32)
          reinterpret_cast<float*>(a.out)[o_idx + i] = v;
        else
          reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
      }
    } else {
      const int64_t pbase = ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G;
      float* dst = a.part_o + (pbase + hh) * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; i++) dst[i] = x[i] * cs;
      if (lane == 0) {
        a.part_ml[(pbase + hh) * 2 + 0] = M;
        a.part_ml[(pbase + hh) * 2 + 1] = Lsum;
      }
    }
  }
}

template <int D, int BITS, int MODE>
hipError_t launch_cb_mode(const AttnArgs& a, dim3 grid, hipStream_t s, hipEvent_t ev0,
                          hipEvent_t ev1) {
  if (ev0 && ev1)
    hipExtLaunchKernelGGL((cb_decode_kernel<D, BITS, MODE>), grid, dim3(kCbWaves * 64), 0, s, ev0,
                          ev1, 0, a);
  else
    hipLaunchKernelGGL((cb_decode_kernel<D, BITS, MODE>), grid, dim3(kCbWaves * 64), 0, s, a);
  return hipGetLastError();
}

template <int D, int BITS>
hipError_t launch_cb_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s, hipEvent_t ev0,
                       hipEvent_t ev1) {
  dim3 grid(n_kv_heads, n_seqs, a.max_splits + a.new_col);
  hipError_t e;
  if (a.tau > 0.0f) {
    // sparse-V as the affine kernel runs it: the stats pass (its statistics
    // in stat_ml; with a decode step's new-token column, which appends the
    // token), the gated pass over every stored token, the combine
    AttnArgs st = a;
    st.part_ml = a.stat_ml;
    if (!st.part_ml) return hipErrorInvalidValue;
    if (a.blk_scores) {
      // the gather in place of the gated pass and the combine (the stats
      // pass stored the candidate blocks' scores and zeroed the counters)
      if ((e = launch_cb_mode<D, BITS, kStats>(st, grid, s, ev0, ev1)) != hipSuccess) return e;
      AttnArgs g = a;
      g.stats_new_col = a.new_col;
      return launch_sparse_gather(g, n_seqs, s);
    }
    if ((e = launch_cb_mode<D, BITS, kStats>(st, grid, s, nullptr, nullptr)) != hipSuccess) return e;
    AttnArgs g = a;
    g.new_col = 0;
    g.stats_new_col = a.new_col;
    if ((e = launch_cb_mode<D, BITS, kGated>(g, dim3(n_kv_heads, n_seqs, a.max_splits), s, ev0,
                                             ev1)) != hipSuccess)
      return e;
    return a.direct ? hipSuccess : launch_combine(g, n_seqs, s);
  }
  e = launch_cb_mode<D, BITS, kDense>(a, grid, s, ev0, ev1);
  if (e != hipSuccess || a.direct) return e;
  return launch_combine(a, n_seqs, s);
}

}  // namespace

hipError_t launch_cb_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                                      hipEvent_t e0, hipEvent_t e1) {
  switch (a.st.layout.head_dim * 16 + a.st.layout.bits) {
    case 128 * 16 + 2: return launch_cb_t<128, 2>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 128 * 16 + 3: return launch_cb_t<128, 3>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 128 * 16 + 4: return launch_cb_t<128, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256 * 16 + 2: return launch_cb_t<256, 2>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256 * 16 + 3: return launch_cb_t<256, 3>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256 * 16 + 4: return launch_cb_t<256, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512 * 16 + 2: return launch_cb_t<512, 2>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512 * 16 + 3: return launch_cb_t<512, 3>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512 * 16 + 4: return launch_cb_t<512, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

// Prefill (chunked) attention over the cache, every mode.
//
// Replaces mlx_rs::fast::scaled_dot_product_attention for L > 1
// (src/model/gemma4_attention.rs:84-104) with the causal mask of
// create_attention_mask and the sliding band of create_sliding_mask
// (src/model/mod.rs:682-753): query position p sees key positions j with
// lo(p) <= j <= p, lo(p) = max(trim, p - W + 1) on sliding layers.
//
// One work-group = 64 query rows (a row is one (position, q head) of the
// KV head's GQA group: 64 / G consecutive positions) of one KV head, four
// wave pairs of 16 rows each. All four pairs read the same staged
// head-block, so one copy HBM -> LDS serves 64 rows. Inside a pair the two
// waves own one half of head_dim each (half the 64-dim groups), exchange
// their partial scores once per block through LDS (flag handshake) and run
// identical softmax bookkeeping, as the decode kernel's pairs do; the
// matrix-core columns are the pair's 16 rows.
//
// Per block (16 keys), affine caches, per 64-dim group g of the wave's half:
//   QK^T  S^T[16 key x 16 row] += K[16 x 32] . Q^T[32 x 16] with K codes as
//         exact f16 integers, q_rot as an f16 high part and an f16 residual
//         (~22 bits), the residual's products first, then the high part's,
//         in one accumulator; then s += scale * acc + bias * sum(q_group). (The decode
//         kernel's 1024 + code operands, one v_perm per two codes, left the
//         residual's contribution on top of a large partial sum here: the
//         worst output error of a 1500-key test rose ~4x; the plain codes
//         cost one packed subtract more per two codes.)
//   PV    O^T[16 dim x 16 row] += V^T[16 dim x 16 key] . P'^T[16 key x 16 row]
//         with P' = p * v_scale as f16 high part + residual (two MFMAs);
//         the bias terms are summed on the side.
// Codebook (TurboQuant) caches, per 32-dim slice / 16-dim tile of the
// wave's half: the indices become f16 centroid operands through the decode
// kernel's LDS lookup table (fmkv_cb_common.h). 2 and 3 bits: the exact
// integer operands 1000 * centroid, S^T = C . q_hi + C . q_lo, scaled per
// key by norm / (1000 sqrt(D)); O^T likewise with P' = p * norm /
// (1000 sqrt(D)) as f16 high part and residual (two MFMAs each). 4 bits: the
// centroids' f16 high part and residual, S^T = C_hi . q_hi + C_lo . q_hi +
// C_hi . q_lo and O^T likewise (three MFMAs each: the fourth product is below
// f32 rounding).
// Plain (bf16) caches read K rows and V columns as bf16 operands
// (v_mfma_f32_16x16x32_bf16 / 16x16x16_bf16) against the raw bf16 q (exact
// products; the softmax scale applies after), P as bf16 high part and
// residual; no rotation.
// Blocks wholly outside a pair's rows' windows are skipped by that pair.
//
// A paged pool runs one sequence per grid z with its own start position and
// block table (linear sequences: the append goes first).
//
// Keys come from two stores: positions below p_split from old_st (the ring
// of a sliding layer, read before the chunk's own append can overwrite
// positions early queries still need), the rest from new_st (a staging
// copy of the chunk, or the cache itself for linear caches). A block that
// straddles p_split is visited once per store with the other part masked.
//
// Copies: each wave issues CP copy instructions per block (the block's
// codes and scale/bias, zero-padded past their end) into one of NST stages;
// a block is used after every wave waited for its own copies and a
// work-group barrier; the next block's copies are then issued into the
// stage the previous block freed.
#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_attn_common.h"
#include "fmkv_cb_common.h"

namespace fmkv {
namespace {

constexpr int kPfWaves = 8;   // four pairs
constexpr int kPfRows = 64;   // query rows per work-group (16 per pair)
constexpr int kPfStages = 3;

template <int D, int BITS, int MODE>
struct PfPlan {
  static constexpr BlockLayout L = make_layout(D, BITS, MODE);
  static constexpr int NG = D / 64;
  static constexpr int GH = NG / 2;  // groups per wave
  static constexpr int NSW = D / 64;  // 32-dim QK slices per wave
  static constexpr int NTW = D / 32;  // 16-dim PV tiles per wave
  // the bytes of a head-block the kernel reads: affine [K codes][V codes]
  // [K meta][V meta]; codebook [K codes][V codes][K norms, padded][V norms];
  // plain [K rows][V columns]
  static constexpr int kBytes = MODE == kAffine     ? (int)(2 * L.code_bytes) + 2 * NG * 64
                                : MODE == kCodebook ? (int)L.v_meta + 2 * kBlockTokens
                                                    : (int)(2 * L.code_bytes);
  static constexpr int kNC = (kBytes + kChunk - 1) / kChunk;
  static constexpr int CP = (kNC + kPfWaves - 1) / kPfWaves;  // copies per wave per block
  static constexpr int kStageBytes = kPfWaves * CP * kChunk;
  static constexpr int kQStride = D + 8;  // 16-bit values per q-table row (padding against bank conflicts)
  // q table: high and residual parts of q_rot (affine: and group sums);
  // plain: the raw bf16 rows
  static constexpr int kQTab = (MODE == kPlain ? 1 : 2) * kPfRows * kQStride * 2 +
                               (MODE == kAffine ? kPfRows * NG * 4 : 0);
  static constexpr int kRStride = D + 4;  // f32 per output row
  static constexpr int kRows = kPfRows * kRStride * 4;
  // codebook: the centroid lookup table follows the stages
  static constexpr int kLutOff = kPfStages * kStageBytes;
  static constexpr int kLutBytes = MODE == kCodebook ? CbLut<BITS == 16 ? 2 : BITS>::kBytes : 0;
  static constexpr int kRegion = cmax(cmax(kLutOff + kLutBytes, kQTab), kRows);
  static_assert(MODE != kAffine || ((int)L.k_meta == (int)(2 * L.code_bytes) &&
                                    (int)L.v_meta == (int)L.k_meta + NG * 64),
                "codes and scale/bias are contiguous in a head-block");
  static_assert(kPfStages * CP <= 63, "vmcnt immediates");
};

// K operand of MFMA s of group g as the plain codes (exact f16 integers).
template <int BITS>
__device__ inline half8_t k_operand_plain(const u32x4 w, int g, int s) {
  if constexpr (BITS == 8) {
    const uint32_t w0 = w[2 * s], w1 = w[2 * s + 1];
    return cat8(u8x2_to_h2(w0, 0x04010400u), u8x2_to_h2(w0, 0x04030402u),
                u8x2_to_h2(w1, 0x04010400u), u8x2_to_h2(w1, 0x04030402u));
  } else {
    return k_operand<BITS>(w, g, s);
  }
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}

template <int D, int BITS, int MODE>
__global__ __launch_bounds__(kPfWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_attn_kernel(PrefillArgs a) {
  using P = PfPlan<D, BITS, MODE>;
  constexpr BlockLayout L = P::L;
  constexpr int NG = P::NG, GH = P::GH, E = D / 64, LPG = 64 / E;
  constexpr int NSW = P::NSW, NTW = P::NTW;
  constexpr int CP = P::CP, NST = kPfStages, SB = P::kStageBytes;
  constexpr int QS = P::kQStride, RS = P::kRStride;
  // codebook index width (the template's BITS; other modes never use it)
  constexpr int CB = MODE == kCodebook ? BITS : 2;

  __shared__ __align__(16) uint8_t region[P::kRegion];
  __shared__ __align__(16) float4_t xs[kPfWaves * 2 * 64];
  __shared__ int xflag[kPfWaves];
  __shared__ float lrow[kPfRows];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pair = wave >> 1, half = wave & 1;
  const int j = lane >> 4, c = lane & 15;
  const int g0 = half * GH;
  const int G = a.group;
  const int QP = kPfRows / G;  // query positions per work-group
  const int kvh = blockIdx.y, seq = blockIdx.z;
  const int qi0 = blockIdx.x * QP;
  // per-sequence start and block table (paged) through scalar loads, which
  // never wait for the copies in flight
  typedef const int32_t __attribute__((address_space(4)))* cint_ptr;
  const int64_t p0 = a.start_pos ? (int64_t)((cint_ptr)(uintptr_t)a.start_pos)[seq] : a.p0;
  const cint_ptr table =
      a.new_st.block_table
          ? (cint_ptr)(uintptr_t)(a.new_st.block_table + (int64_t)seq * a.new_st.table_stride)
          : nullptr;
  const int nq = a.n_q - qi0 < QP ? a.n_q - qi0 : QP;  // valid positions of the tile

  // visible keys of position p: [lo(p), p]
  auto lo_of = [&](int64_t p) -> int64_t {
    int64_t lo = a.vis_begin;
    if (a.window > 0 && p - a.window + 1 > lo) lo = p - a.window + 1;
    return lo < 0 ? 0 : lo;
  };
  // this lane's row = column c of its pair
  const int row = pair * 16 + c;
  const int rq = row / G;
  const bool row_valid = rq < nq;
  const int64_t p_row = p0 + qi0 + rq;
  const int64_t row_lo = lo_of(p_row);
  // the pair's positions [pA, pB] (pair-uniform)
  const int pq0 = (pair * 16) / G;
  int pq1 = (pair * 16 + 15) / G;
  if (pq1 > nq - 1) pq1 = nq - 1;
  const bool pair_any = pq0 <= pq1;
  const int64_t pA = p0 + qi0 + pq0, pB = p0 + qi0 + pq1;
  const int64_t pair_lo_min = lo_of(pA), pair_lo_max = lo_of(pB);
  const bool pair_full_rows = (pair * 16 + 15) / G < nq;  // all 16 rows are real queries

  // ---- virtual blocks of the work-group: [lo(first), last] in 16-key
  // blocks, the part below p_split from old_st, the rest from new_st ----
  const int64_t wg_lo = lo_of(p0 + qi0), wg_hi = p0 + qi0 + nq - 1;
  const int64_t b_lo = wg_lo / kBlockTokens, b_hi = wg_hi / kBlockTokens;
  const int64_t ps = a.p_split;
  int64_t old_last = (ps + kBlockTokens - 1) / kBlockTokens - 1;  // last block with keys < ps
  if (old_last > b_hi) old_last = b_hi;
  const int64_t n_old = old_last >= b_lo ? old_last - b_lo + 1 : 0;
  int64_t new_first = ps / kBlockTokens;
  if (new_first < b_lo) new_first = b_lo;
  const int64_t n_new = b_hi >= new_first ? b_hi - new_first + 1 : 0;
  const int nvb = (int)(n_old + n_new);
  // Per-block tests in 32-bit scalar form (the scalar unit has no 64-bit
  // signed compares, and the vector unit's would cost every block): block
  // rb = b - b_lo. A block that p_split cuts (cut_rb, visited once per
  // store with its own part) takes the 64-bit tests; any other holds keys
  // t0 .. t0 + 15, so the pair sees it when sees_lo <= rb <= sees_hi (a key
  // at or past the pair's smallest lower bound, one at or before its last
  // position) and it is whole for every row of the pair when full_lo <= rb
  // <= full_hi (every key at or past the largest lower bound, at or before
  // the first position). (When the pair has rows, its bounds are at or past
  // b_lo's first key.)
  const int64_t bl16 = b_lo * kBlockTokens;
  auto rel_blk = [&](int64_t x) -> int {  // floor(x / 16) for x >= 0, clamped; -1 below
    if (x < 0) return -1;
    const int64_t q = x / kBlockTokens;
    return (int)(q < INT32_MAX - 1 ? q : INT32_MAX - 1);
  };
  const int sees_lo = pair_any ? rel_blk(pair_lo_min - bl16) : INT32_MAX;
  const int sees_hi = pair_any ? rel_blk(pB - bl16) : -1;
  const int full_lo = pair_any && pair_full_rows ? rel_blk(pair_lo_max - bl16 + kBlockTokens - 1)
                                                  : INT32_MAX;
  const int full_hi = pair_any ? rel_blk(pA - (kBlockTokens - 1) - bl16) : -1;
  const int cut_rb = ps % kBlockTokens != 0 ? rel_blk(ps - bl16) : -1;
  const int new_rb0 = (int)(new_first - b_lo);  // rb of virtual block n_old
  // virtual block i's absolute block and valid key range [vlo, vhi)
  struct VB {
    int64_t b, vlo, vhi;
  };
  auto vb_of = [&](int i) -> VB {
    VB v;
    if (i < n_old) {
      v.b = b_lo + i;
      v.vlo = v.b * kBlockTokens;
      v.vhi = (v.b + 1) * kBlockTokens < ps ? (v.b + 1) * kBlockTokens : ps;
    } else {
      v.b = new_first + (i - n_old);
      v.vlo = v.b * kBlockTokens > ps ? v.b * kBlockTokens : ps;
      v.vhi = (v.b + 1) * kBlockTokens;
    }
    return v;
  };
  // its head-block. A ring's slot block of virtual block i is ring0 + i
  // modulo its nrb blocks (the old keys lie in the last W positions before
  // p_split: n_old <= nrb + 1, so two conditional subtractions reduce it).
  const int nrb = a.ring_slots > 0 ? (int)(a.ring_slots / kBlockTokens) : 0;
  const int ring0 = nrb > 0 ? (int)(b_lo % nrb) : 0;
  const int32_t n_pool = (int32_t)(a.new_st.n_blocks < INT32_MAX ? a.new_st.n_blocks : INT32_MAX);
  auto blk_ptr = [&](int i) -> const uint8_t* {
    if (i < n_old) {
      int64_t phys = b_lo + i;
      if (nrb > 0) {
        int r = ring0 + i;
        r -= r >= nrb ? nrb : 0;
        r -= r >= nrb ? nrb : 0;
        phys = r;
      }
      return a.old_st.base + phys * a.old_st.block_stride + (int64_t)kvh * a.old_st.head_stride;
    }
    const int64_t b = new_first + (i - n_old);
    int64_t phys = b - a.new_blk0;
    if (table) {
      // a table entry outside the pool (or a position past the table's
      // width) reads a valid block rather than faulting
      int32_t e = 0;
      if ((b >> 31) == 0 && (uint32_t)b < (uint32_t)a.new_st.table_stride) e = table[(uint32_t)b];
      phys = e < 0 ? 0 : (e >= n_pool ? n_pool - 1 : e);
    }
    return a.new_st.base + phys * a.new_st.block_stride + (int64_t)kvh * a.new_st.head_stride;
  };

  // ---- q_rot of the 64 rows: rows wave + 8 k, high / residual halves
  // (plain: the raw bf16 rows) ----
  _Float16* const qhi = reinterpret_cast<_Float16*>(region);
  _Float16* const qlo = qhi + kPfRows * QS;
  float* const qsum = reinterpret_cast<float*>(qlo + kPfRows * QS);  // [row][NG] (affine)
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  const float cs_lane = fwht_lane_sign(lane) * a.c;
  if (lane == 0) xflag[wave] = 0;
#pragma unroll 1
  for (int k = 0; k < kPfRows / kPfWaves; k++) {
    const int r = wave + kPfWaves * k;
    const int rq_ = r / G, rh_ = r - (r / G) * G;
    if constexpr (MODE == kPlain) {
      // E consecutive bf16 of the row as stored (zero past the chunk)
      const uint16_t* src =
          a.q + (((int64_t)seq * a.n_q + qi0 + rq_) * a.n_q_heads + (int64_t)kvh * G + rh_) * D +
          lane * E;
      uint16_t* dst = reinterpret_cast<uint16_t*>(qhi + r * QS + lane * E);
#pragma unroll
      for (int i = 0; i < E; i++) dst[i] = rq_ < nq ? src[i] : (uint16_t)0;
      continue;
    }
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = 0.0f;
    if (rq_ < nq) {
      load_row<E>(a.q + (((int64_t)seq * a.n_q + qi0 + rq_) * a.n_q_heads + (int64_t)kvh * G + rh_) * D +
                      lane * E, x);
#pragma unroll
      for (int i = 0; i < E; i++) x[i] = x[i] * a.qscale;
    }
    // the sign-tracking FWHT: a -0 for +0 changes no score or sum
    wave_fwht_signed<E>(x, lane);
    float gs = 0.0f;
    _Float16 hv[E], lv[E];
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float v = apply_sign(x[i] * cs_lane, sbits, i);
      gs += v;
      hv[i] = (_Float16)v;
      lv[i] = (_Float16)(v - (float)hv[i]);
    }
    gs = group_sum<LPG>(gs, lane);
    store_halves<E>(reinterpret_cast<uint8_t*>(qhi + r * QS + lane * E), hv);
    store_halves<E>(reinterpret_cast<uint8_t*>(qlo + r * QS + lane * E), lv);
    if constexpr (MODE == kAffine)
      if ((lane & (LPG - 1)) == 0) qsum[r * NG + ((lane * E) >> 6)] = gs;
  }
  __syncthreads();

  // this wave's B operands: its pair's 16 rows, its groups; the lane (j, c)
  // holds 8 consecutive dims of row `row` at the K-code placement
  // (codebook and plain: slice k = 2 gi + s of the wave's half, dims
  // half * D / 2 + 32 k + 8 j ..; plain B operands are the bf16 bits)
  half8_t bqh[GH][2], bql[GH][2];
  float qs[GH];
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    const int g = g0 + gi;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int d0 = MODE == kAffine ? g * 64 + (BITS == 8 ? j * 16 + s * 8 : s * 32 + j * 8)
                                     : half * (D / 2) + (2 * gi + s) * 32 + j * 8;
      bqh[gi][s] = *reinterpret_cast<const half8_t*>(qhi + row * QS + d0);
      if constexpr (MODE != kPlain) bql[gi][s] = *reinterpret_cast<const half8_t*>(qlo + row * QS + d0);
    }
    qs[gi] = MODE == kAffine ? qsum[row * NG + g] : 0.0f;
  }
  __syncthreads();  // the table is consumed: the region becomes the stages
  // codebook: the centroid lookup table, after the stages (written before
  // the first block's barrier)
  uint8_t* const lut = region + P::kLutOff;
  const uint32_t lut_l = lds_addr(lut) + (lane & (kLutCopies - 1)) * 4;
  if constexpr (MODE == kCodebook) cb_fill_lut<CB>(lut, tid, kPfWaves * 64);

  // ---- copies ----
  const uint32_t stage_lds = lds_addr(region);
  auto copy_vb = [&](int st, int i) {
    const u32x4 rs = buffer_rsrc(blk_ptr(i), (uint32_t)P::kBytes);
    const uint32_t sl = stage_lds + st * SB;
#pragma unroll
    for (int k = 0; k < CP; k++) {
      const int ci = wave + kPfWaves * k;
      dma16(sl + ci * kChunk, ci * kChunk + lane * 16, rs);
    }
  };
#pragma unroll
  for (int s = 0; s < NST - 1; s++)
    if (s < nvb) copy_vb(s, s);

  // ---- main loop ----
  float4_t o[GH * 4];
#pragma unroll
  for (int i = 0; i < GH * 4; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float bacc[GH], psum[GH];
#pragma unroll
  for (int gi = 0; gi < GH; gi++) bacc[gi] = psum[gi] = 0.0f;
  float m_run = -1e30f, l_run = 0.0f;
  float neg_one;
  asm("v_mov_b32 %0, -1.0" : "=v"(neg_one));

  auto codes = [&](const uint8_t* sp, int region_off, int gi) {
    const int g = g0 + gi;
    return lds16(sp + region_off + (BITS == 8 ? g : g / 2) * kChunk + lane * 16);
  };
  auto kmeta = [&](const uint8_t* sp, int gi) {
    return lds16(sp + (int)L.k_meta + (g0 + gi) * 64 + j * 16);
  };
  auto vmeta = [&](const uint8_t* sp, int gi) {
    return lds16(sp + (int)L.v_meta + (g0 + gi) * 64 + j * 16);
  };

  // codebook: this lane's index fields in the wave's half of K (token c,
  // dims 8 j .. of each slice) and V (dim c of each tile, tokens 4 j ..)
  constexpr int HB = D * CB;  // bytes of one half of the K (or V) indices
  const int kbit0 = (c * (D / 2) + 8 * j) * CB, vbit0 = (c * 16 + 4 * j) * CB;
  const uint32_t ksh = kbit0 & 31, vsh = vbit0 & 31;
  // plain: this lane's operand offsets (K row c, dims 8 j .. of each slice;
  // V dim c of each tile, tokens 4 j ..)
  const int pk_off = (int)L.k_codes + (c * D + half * (D / 2) + 8 * j) * 2;
  const int pv_off = (int)L.v_codes + ((half * (D / 2) + c) * kBlockTokens + 4 * j) * 2;

  auto process = [&](const uint8_t* sp, int vi, int it, bool full) {
    float4_t sv = (float4_t){0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == kCodebook) {
      const uint32_t* kw =
          reinterpret_cast<const uint32_t*>(sp + (int)L.k_codes + half * HB) + (kbit0 >> 5);
#pragma unroll
      for (int k = 0; k < NSW; k++) {
        const uint32_t f = lds_field<CB>(kw, k * CB, ksh);
        if constexpr (kCbExact<CB>) {
          const half8_t ak = __builtin_bit_cast(
              half8_t, (u32x4){cb_pair_exact<CB, 0>(lut_l, f), cb_pair_exact<CB, 1>(lut_l, f),
                               cb_pair_exact<CB, 2>(lut_l, f), cb_pair_exact<CB, 3>(lut_l, f)});
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bqh[k >> 1][k & 1], sv, 0, 0, 0);
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bql[k >> 1][k & 1], sv, 0, 0, 0);
        } else {
          uint32_t h4[4], l4[4];
          cb_pair_hl4<0>(lut_l, f, h4[0], l4[0]);
          cb_pair_hl4<1>(lut_l, f, h4[1], l4[1]);
          cb_pair_hl4<2>(lut_l, f, h4[2], l4[2]);
          cb_pair_hl4<3>(lut_l, f, h4[3], l4[3]);
          const half8_t ah = __builtin_bit_cast(half8_t, (u32x4){h4[0], h4[1], h4[2], h4[3]});
          const half8_t al = __builtin_bit_cast(half8_t, (u32x4){l4[0], l4[1], l4[2], l4[3]});
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bqh[k >> 1][k & 1], sv, 0, 0, 0);
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bqh[k >> 1][k & 1], sv, 0, 0, 0);
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bql[k >> 1][k & 1], sv, 0, 0, 0);
        }
      }
    } else if constexpr (MODE == kPlain) {
#pragma unroll
      for (int k = 0; k < NSW; k++)
        sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, lds16(sp + pk_off + k * 64)),
            __builtin_bit_cast(bf16x8_t, bqh[k >> 1][k & 1]), sv, 0, 0, 0);
    } else {
    u32x4 kw = codes(sp, (int)L.k_codes, 0), km = kmeta(sp, 0);
#pragma unroll
    for (int gi = 0; gi < GH; gi++) {
      const u32x4 kw_g = kw, km_g = km;
      if (gi + 1 < GH) {
        if (BITS == 8 || ((g0 + gi + 1) & 1) == 0) kw = codes(sp, (int)L.k_codes, gi + 1);
        km = kmeta(sp, gi + 1);
      }
      const int g = g0 + gi;
      const half8_t k0 = k_operand_plain<BITS>(kw_g, g, 0), k1 = k_operand_plain<BITS>(kw_g, g, 1);
      const float4_t z = (float4_t){0.f, 0.f, 0.f, 0.f};
      // the residual products first, then the high parts, in one accumulator
      float4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, bql[gi][0], z, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, bql[gi][1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, bqh[gi][0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, bqh[gi][1], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++)
        sv[i] = fmaf(lo16(km_g[i]), acc[i], fmaf(hi16(km_g[i]), qs[gi], sv[i]));
      __builtin_amdgcn_sched_barrier(0);
    }
    }

    // exchange the half scores with the partner wave (release / acquire on
    // a per-wave counter); both waves add the halves in the same order
    const int par = it & 1;
    xs[(wave * 2 + par) * 64 + lane] = sv;
    __hip_atomic_store(&xflag[wave], it + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(&xflag[wave ^ 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           it + 1)
      __builtin_amdgcn_s_sleep(1);
    const float4_t so = xs[((wave ^ 1) * 2 + par) * 64 + lane];
    const float4_t s0 = half == 0 ? sv : so;
    const float4_t s1 = half == 0 ? so : sv;
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; i++) s[i] = s0[i] + s1[i];
    // codebook: the keys' norms / sqrt(D) (lane (j, c) holds keys 4 j ..);
    // plain: the softmax scale
    float vscale[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == kCodebook) {
      const uint2 kn = *reinterpret_cast<const uint2*>(sp + (int)L.k_meta + 8 * j);
      const uint2 vn = *reinterpret_cast<const uint2*>(sp + (int)L.v_meta + 8 * j);
      const float ks[4] = {lo16(kn.x), hi16(kn.x), lo16(kn.y), hi16(kn.y)};
      const float vs[4] = {lo16(vn.x), hi16(vn.x), lo16(vn.y), hi16(vn.y)};
      // (1 / sqrt(D) in the table operands' units)
      const float cu = a.c * kCbOperandScale<CB>;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        s[i] = s[i] * (ks[i] * cu);
        vscale[i] = vs[i] * cu;
      }
    } else if constexpr (MODE == kPlain) {
#pragma unroll
      for (int i = 0; i < 4; i++) s[i] = s[i] * a.qscale;
    }

    // masks: the whole block for all rows of the pair in the common case
    if (!full) {
      const VB v = vb_of(vi);
      const int64_t t0 = v.b * kBlockTokens;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t kp = t0 + 4 * j + i;
        const bool vis = row_valid && kp >= v.vlo && kp < v.vhi && kp >= row_lo && kp <= p_row;
        if (!vis) s[i] = -INFINITY;
      }
    }
    float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run + kRescaleSlack)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      if (__any(l_run > 0.0f)) {
#pragma unroll
        for (int i = 0; i < GH * 4; i++) o[i] *= alpha;
#pragma unroll
        for (int gi = 0; gi < GH; gi++) {
          bacc[gi] *= alpha;
          if constexpr (MODE == kAffine && kBiasedCodes<BITS>) psum[gi] *= alpha;
        }
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

    if constexpr (MODE == kCodebook) {
      // O^T += V^T . P'^T, P' = p * norm / sqrt D as f16 high part and
      // residual, the centroids likewise
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; i++) x[i] = p[i] * vscale[i];
      const half2_t h01 = pkrtz(x[0], x[1]);
      const half2_t h23 = pkrtz(x[2], x[3]);
      const half2_t r01 = pkrtz(fmaf(neg_one, (float)h01[0], x[0]), fmaf(neg_one, (float)h01[1], x[1]));
      const half2_t r23 = pkrtz(fmaf(neg_one, (float)h23[0], x[2]), fmaf(neg_one, (float)h23[1], x[3]));
      const half4_t bh = cat4(h01, h23), bl = cat4(r01, r23);
      const uint32_t* vw =
          reinterpret_cast<const uint32_t*>(sp + (int)L.v_codes + half * HB) + (vbit0 >> 5);
#pragma unroll
      for (int n = 0; n < NTW; n++) {
        const uint32_t f = lds_field<CB>(vw, n * 8 * CB, vsh);
        if constexpr (kCbExact<CB>) {
          const half4_t av = __builtin_bit_cast(
              half4_t, make_uint2(cb_pair_exact<CB, 0>(lut_l, f), cb_pair_exact<CB, 1>(lut_l, f)));
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bh, o[n], 0, 0, 0);
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bl, o[n], 0, 0, 0);
        } else {
          uint32_t h2[2], l2[2];
          cb_pair_hl4<0>(lut_l, f, h2[0], l2[0]);
          cb_pair_hl4<1>(lut_l, f, h2[1], l2[1]);
          const half4_t ah = __builtin_bit_cast(half4_t, make_uint2(h2[0], h2[1]));
          const half4_t al = __builtin_bit_cast(half4_t, make_uint2(l2[0], l2[1]));
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, o[n], 0, 0, 0);
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, o[n], 0, 0, 0);
          o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, o[n], 0, 0, 0);
        }
      }
      return;
    } else if constexpr (MODE == kPlain) {
      // O^T += V^T . P^T, P as bf16 high part and residual
      float r[4];
#pragma unroll
      for (int i = 0; i < 4; i++) r[i] = p[i] - bf16_to_f32(f32_to_bf16(p[i]));
      const short4_t bh = __builtin_bit_cast(
          short4_t, make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])));
      const short4_t bl = __builtin_bit_cast(
          short4_t, make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])));
#pragma unroll
      for (int n = 0; n < NTW; n++) {
        const short4_t va =
            __builtin_bit_cast(short4_t, *reinterpret_cast<const uint2*>(sp + pv_off + n * 16 * kBlockTokens * 2));
        o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bh, o[n], 0, 0, 0);
        o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, bl, o[n], 0, 0, 0);
      }
      return;
    } else {
    u32x4 vw = codes(sp, (int)L.v_codes, 0), vm = vmeta(sp, 0);

    // O^T += V^T . P'^T, P' = p * v_scale as f16 high part and residual
    const half2_t one2 = (half2_t){(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int gi = 0; gi < GH; gi++) {
      const u32x4 vw_g = vw, vm_g = vm;
      if (gi + 1 < GH) {
        if (BITS == 8 || ((g0 + gi + 1) & 1) == 0) vw = codes(sp, (int)L.v_codes, gi + 1);
        vm = vmeta(sp, gi + 1);
      }
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] = fmaf(p[i], lo16(vm_g[i]), 0.0f);
        bacc[gi] = fmaf(p[i], hi16(vm_g[i]), bacc[gi]);
      }
      const half2_t h01 = pkrtz(x[0], x[1]);
      const half2_t h23 = pkrtz(x[2], x[3]);
      // residual x - hi (exact) as one mixed-precision fma each (an opaque
      // -1 keeps the f16 operand inside the fma instead of a convert and a
      // subtract)
      const half2_t r01 = pkrtz(fmaf(neg_one, (float)h01[0], x[0]), fmaf(neg_one, (float)h01[1], x[1]));
      const half2_t r23 = pkrtz(fmaf(neg_one, (float)h23[0], x[2]), fmaf(neg_one, (float)h23[1], x[3]));
      const half4_t bh = cat4(h01, h23), bl = cat4(r01, r23);
      if constexpr (kBiasedCodes<BITS>) {
        float t = __builtin_amdgcn_fdot2(h01, one2, psum[gi], false);
        t = __builtin_amdgcn_fdot2(h23, one2, t, false);
        t = __builtin_amdgcn_fdot2(r01, one2, t, false);
        psum[gi] = __builtin_amdgcn_fdot2(r23, one2, t, false);
      }
      const int g = g0 + gi;
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        const half4_t va = v_operand<BITS>(vw_g, g, ct);
        o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bh, o[gi * 4 + ct], 0, 0, 0);
        o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, bl, o[gi * 4 + ct], 0, 0, 0);
      }
    }
    }
  };

  int st = 0, it = 0;
  for (int i = 0; i < nvb; i++) {
    // this wave's copies of block i have landed (only the blocks issued
    // after it may be pending); the barrier makes every wave's copies
    // visible and frees the stage of block i - 1 for block i + NST - 1
    const int rest = nvb - 1 - i;
    wait_copies<CP, NST - 2>(rest < NST - 2 ? rest : NST - 2);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (i + NST - 1 < nvb) copy_vb((i + NST - 1) % NST, i + NST - 1);
    // the pair's rows see this block at all (pair-uniform)
    const int rb = i < n_old ? i : new_rb0 + (i - (int)n_old);
    bool sees = rb >= sees_lo && rb <= sees_hi;
    if (rb == cut_rb) {
      const VB v = vb_of(i);
      sees = pair_any && v.vhi - 1 >= pair_lo_min && v.vlo <= pB;
    }
    if (sees) {
      const bool full = rb >= full_lo && rb <= full_hi && rb != cut_rb;
      process(region + st * SB, i, it, full);
      it++;
    }
    st = st + 1 == NST ? 0 : st + 1;
  }

  // ---- epilogue: normalise, inverse rotation, store ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    bacc[gi] = xor16_sum(bacc[gi]);
    bacc[gi] = xor32_sum(bacc[gi]);
    if constexpr (MODE == kAffine && kBiasedCodes<BITS>) {
      // the V codes entered the MFMAs as 1024 + code
      const float t = xor32_sum(xor16_sum(psum[gi]));
      bacc[gi] = fmaf(-1024.0f, t, bacc[gi]);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the stages are free
  float* const Rr = reinterpret_cast<float*>(region);
  // (tile n of the wave's half: dims half * D / 2 + 16 n + 4 j .., the
  // affine group / column-tile order being the same dims)
#pragma unroll
  for (int gi = 0; gi < GH; gi++)
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      const int d = (g0 + gi) * 64 + ct * 16 + 4 * j;
      *reinterpret_cast<float4_t*>(&Rr[row * RS + d]) =
          MODE == kAffine ? o[gi * 4 + ct] + bacc[gi] : o[gi * 4 + ct];
    }
  if (half == 0 && j == 0) lrow[row] = l_run;
  __syncthreads();
#pragma unroll 1
  for (int k = 0; k < kPfRows / kPfWaves; k++) {
    const int r = wave + kPfWaves * k;
    const int rq_ = r / G, rh_ = r - (r / G) * G;
    if (rq_ >= nq) continue;
    const float l = lrow[r];
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = apply_sign(Rr[r * RS + lane * E + i], sbits, i);
    float cs = cs_lane;
    if constexpr (MODE != kPlain) {
      wave_fwht_signed<E>(x, lane);
    } else {  // no rotation: the row as accumulated
#pragma unroll
      for (int i = 0; i < E; i++) x[i] = Rr[r * RS + lane * E + i];
      cs = 1.0f;
    }
    const int64_t o_idx =
        (((int64_t)seq * a.n_q + qi0 + rq_) * a.n_q_heads + (int64_t)kvh * G + rh_) * D + lane * E;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float v = l > 0.0f ? (x[i] * cs) / l : 0.0f;
      if (a.out_f32)
        reinterpret_cast<float*>(a.out)[o_idx + i] = v;
      else
        reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
    }
  }
}

template <int D, int BITS, int MODE>
hipError_t launch_t(const PrefillArgs& a, hipStream_t s) {
  const int qp = kPfRows / a.group;
  dim3 grid((a.n_q + qp - 1) / qp, a.new_st.n_kv_heads, a.n_seqs);
  hipLaunchKernelGGL((prefill_attn_kernel<D, BITS, MODE>), grid, dim3(kPfWaves * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t s) {
  if (a.n_q <= 0) return hipSuccess;
  const BlockLayout& L = a.new_st.layout;
  if (L.mode == kAffine) {
    switch (L.head_dim * 16 + L.bits) {
      case 128 * 16 + 4: return launch_t<128, 4, kAffine>(a, s);
      case 128 * 16 + 8: return launch_t<128, 8, kAffine>(a, s);
      case 256 * 16 + 4: return launch_t<256, 4, kAffine>(a, s);
      case 256 * 16 + 8: return launch_t<256, 8, kAffine>(a, s);
      case 512 * 16 + 4: return launch_t<512, 4, kAffine>(a, s);
      case 512 * 16 + 8: return launch_t<512, 8, kAffine>(a, s);
    }
  } else if (L.mode == kCodebook) {
    switch (L.head_dim * 16 + L.bits) {
      case 128 * 16 + 2: return launch_t<128, 2, kCodebook>(a, s);
      case 128 * 16 + 3: return launch_t<128, 3, kCodebook>(a, s);
      case 128 * 16 + 4: return launch_t<128, 4, kCodebook>(a, s);
      case 256 * 16 + 2: return launch_t<256, 2, kCodebook>(a, s);
      case 256 * 16 + 3: return launch_t<256, 3, kCodebook>(a, s);
      case 256 * 16 + 4: return launch_t<256, 4, kCodebook>(a, s);
      case 512 * 16 + 2: return launch_t<512, 2, kCodebook>(a, s);
      case 512 * 16 + 3: return launch_t<512, 3, kCodebook>(a, s);
      case 512 * 16 + 4: return launch_t<512, 4, kCodebook>(a, s);
    }
  } else if (L.mode == kPlain) {
    switch (L.head_dim) {
      case 128: return launch_t<128, 16, kPlain>(a, s);
      case 256: return launch_t<256, 16, kPlain>(a, s);
      case 512: return launch_t<512, 16, kPlain>(a, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

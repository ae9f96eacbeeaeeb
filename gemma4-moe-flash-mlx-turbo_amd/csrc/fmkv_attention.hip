// Fused decode attention over the quantized cache (affine mode).
//
// Replaces mlx_rs::fast::scaled_dot_product_attention at decode (L == 1,
// src/model/gemma4_attention.rs:94-103) reading the cache written by
// fmkv_append. One work-group = one (split of consecutive 16-token blocks,
// KV head, sequence) with four wave pairs. Pair p streams whole head-blocks
// b_begin + p, b_begin + p + 4, ...; its two waves each own one half of
// head_dim (half the 64-dim groups), exchange their partial scores once per
// block through LDS (a flag handshake inside the pair, no work-group
// barrier) and then run identical online-softmax bookkeeping. Two waves per
// SIMD hide each other's latencies. The pairs' (m, l, O) meet once, in LDS,
// at the end. Small head-blocks (head_dim 128, head_dim 256 at 4 bits) in
// work-groups of 8 blocks or more use twelve single-wave streams instead
// (b_begin + w, b_begin + w + 12, ...; three waves per SIMD), each wave
// owning every group, with no exchange (AttnPlan).
//
// Memory path: each wave copies its half of its pair's next blocks
// HBM -> LDS with buffer_load_dwordx4 ... lds (16 bytes per lane, no VGPRs
// held while in flight), several stages deep, and waits for a stage with an
// explicit vmcnt. The copies are issued from inline asm, so the compiler
// neither tracks them nor inserts waits of its own on LDS reads; every stage
// read is preceded by the vmcnt wait covering it, computed from the number
// of copies issued after that stage. The compiler issues no vector-memory
// loads of its own in the split columns (the one candidate, the sign-bit
// lookup, is written so that it cannot become one); only the new-token
// column, which tracks no copies, loads through the compiler.
//
// Per block (16 tokens), per 64-dim group g of the wave's half:
//   QK^T  S^T[16 tok x 16 col] += K[16 x 32] . Q^T[32 x 16] on MFMA
//         (v_mfma_f32_16x16x32_f16), K codes entering as the exact f16
//         values 1024 + code (8-bit) or 1 + code / 16 (4-bit), the offset
//         cancelled by the accumulator's start (kCodeOffset); the f16
//         scale/bias apply after the MFMA: s += scale * acc + bias * sum(q_group).
//         Column c = q head (c & 7) of the GQA group, c < 8 carrying the f16
//         high part of q_rot and c >= 8 the residual, so S keeps ~22 bits of
//         q precision; DPP row_ror:8 folds the two halves.
//   PV    O^T[16 dim x 16 col] += V^T[16 dim x 16 tok] . P'^T[16 tok x 16 col]
//         (v_mfma_f32_16x16x16f16) with P' = p * v_scale split hi/lo in the
//         same columns; bias terms are summed on the side.
// The QK output lane layout equals the PV B-operand layout (lane (j, c) holds
// tokens 4j..4j+3 of column c), so no register shuffles are needed.
// (At 4 bits the 1024 + code form would inflate the f32 partial sums ~64x,
// which outlier channels turn into visible error; 1 + code / 16 -- the code
// in the top mantissa bits, one shift and one bit-field insert per two codes
// against four instructions for exact small integers -- inflates them ~3x.)
//
// q_rot = (FWHT(q * scale * log2 e) * c) o s is computed by every work-group
// in its prologue, while its first blocks are in flight: the raw q rows are
// copied to LDS ahead of the blocks and turned into a table of MFMA B
// operands. Epilogue: the pairs' results merge in LDS, the inverse rotation
// o . R^T = c * FWHT(o o s) follows, and the result is the final output (one
// split) or a split partial for combine_kernel.
//
// Decode step (a.new_col): the grid has one more column whose work-groups
// append the step's new token (rotate, quantize, slot write -- the append
// kernel's arithmetic) and contribute its attention as one more partial; the
// split columns leave the new token's slot out. A decode step is then this
// launch and the combine.
#include <hip/hip_ext.h>

#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_prologue.h"
#include "fmkv_quant.h"
#include "fmkv_attn_common.h"

namespace fmkv {
namespace {

// Staging plan of one (head_dim, bits, stream kind). A block stream is a
// wave pair (each wave owns half the 64-dim groups, SW = 0) or a single
// wave owning every group (SW > 0 solo waves per work-group). Pairs finish
// one block soonest; solo streams, with no score exchange, finish more
// blocks per unit of time when a head-block is small (at most 1024 code
// bits per token: head_dim 128, head_dim 256 at 4 bits), so the launch
// picks them for work-groups of many blocks (kSoloMinBlocks). Solo
// work-groups come in two sizes: twelve waves filling a CU's LDS (one
// sequence), or four waves in about 46 KiB, three work-groups sharing a CU
// (a paged batch: one work-group's prologue and epilogue then overlap the
// others' streaming instead of leaving the CU's copies idle).
// A stage holds one head-block as
//   [K codes][V codes][wave 0: K meta, V meta of its groups][wave 1: ...];
// each wave copies its groups' code chunks and, with one partial
// instruction, its groups' scale/bias. Stages per stream: about 136 KiB of
// staging per work-group (144 KiB for twelve single-wave streams, which need
// no score-exchange area; 37 KiB for four), at least two, and the largest
// wait (stages x copies per block) within the 6-bit vmcnt field.
template <int D, int BITS>
constexpr bool kSoloCapable = D * BITS <= 1024;
constexpr int kSoloMinBlocks = 8;  // blocks per work-group from which solo streams pay
#ifndef FMKV_PAGED_SOLO_WAVES
#define FMKV_PAGED_SOLO_WAVES 4
#endif
// solo waves per work-group of a paged batch (4: three work-groups per CU)
constexpr int kPagedSoloWaves = FMKV_PAGED_SOLO_WAVES;

template <int D, int BITS, int SW>
struct AttnPlan {
  static constexpr BlockLayout L = make_layout(D, BITS, kAffine);
  static constexpr int NG = D / 64;
  static constexpr bool kSolo = SW > 0;
  static_assert(!kSolo || kSoloCapable<D, BITS>, "solo streams for small head-blocks only");
  static_assert(SW == 0 || SW == 4 || SW == 12, "pairs, or 4 or 12 solo waves");
  static constexpr int kWPS = kSolo ? 1 : 2;            // waves per stream
  // solo waves run three per SIMD (<= 168 VGPRs each): one work-group of 12
  // or three of 4 per CU
  static constexpr int kWaves = kSolo ? SW : kAttnWaves;
  static constexpr int kWavesPerSimd = kSolo ? 3 : kWaves / 4;
  static constexpr int kStreams = kWaves / kWPS;
  static constexpr int GH = NG / kWPS;  // groups per wave
  static constexpr int kCodeChunks = (int)(L.code_bytes / kChunk);  // per K or V region
  // code chunks a wave copies per region: its groups' chunks (at 4 bits one
  // chunk holds two groups)
  static constexpr int kWaveChunks = BITS == 8 ? GH : (GH >= 2 ? GH / 2 : 1);
  // head_dim 128 at 4 bits: the pair's two groups share the block's one
  // chunk, and each wave keeps its own copy of it in the stage, so that a
  // wave refilling a stage never overwrites a chunk its partner still reads
  static constexpr bool kSharedChunk = !kSolo && BITS == 4 && GH == 1;
  static constexpr int kCodeSlots = kSharedChunk ? 2 : kCodeChunks;  // chunk slots per region
  static constexpr int kMetaHalf = GH * 64;  // one wave's K (or V) scale/bias bytes
  static constexpr int kMetaOff = 2 * kCodeSlots * kChunk;
  static constexpr int kStageBytes = kMetaOff + 2 * kWPS * kMetaHalf;
  static constexpr int kCopies = 2 * kWaveChunks + 1;  // copy instructions per wave per block
  static constexpr int kFit = ((SW == 4 ? 37 : kSolo ? 144 : 136) * 1024) / (kStreams * kStageBytes);
  static constexpr int kStagesA = kFit < 2 ? 2 : (kFit > 8 ? 8 : kFit);
  static constexpr int kStages = kStagesA * kCopies <= 63 ? kStagesA : 63 / kCopies;
  static constexpr int kQS = D + 4;  // padded row stride (LDS banks)
  // a stream's merge rows [8 heads][kQS] floats reuse its own stages
  static constexpr int kStageRegion = kStreams * kStages * kStageBytes;
  static_assert(8 * kQS * 4 <= kStages * kStageBytes, "merge rows fit in a stream's stages");
  // prologue: the raw q rows, then the q table (B operands, group sums of
  // q_rot, group sums of the f16 high and residual parts); loop: the score
  // exchange
  static constexpr int kTabBytes = 2 * NG * kChunk + 8 * NG * 4 + 8 * NG * 8;
  static constexpr int kXBytes = kSolo ? 0 : kWaves * 2 * 64 * 16;
  static constexpr int kScratch = cmax(cmax(kTabBytes, kXBytes), 8 * D * 2);
  static_assert(NG % 2 == 0 && kCodeChunks >= 1, "layout");
  static_assert(kStages * kCopies <= 63, "vmcnt immediates");
  static_assert(8 * GH <= 64, "one partial instruction copies a wave's scale/bias");
};

// Raw bf16 q rows of the GQA heads h = wave, wave + NW, ... of (seq, kvh)
// (D * 2 bytes each) to LDS at dst + h * D * 2, copied by that wave itself
// (lanes < D / 8). NW: waves of the work-group.
template <int D, int NW>
__device__ inline void copy_q_row(const uint16_t* q, int n_q_heads, int group, uint8_t* dst,
                                  int seq, int kvh, int wave, int lane) {
#pragma unroll
  for (int h = wave; h < (NW < 8 ? 8 : NW); h += NW) {
    if (h < group && lane < D / 8) {
      const uint16_t* qh = q + ((int64_t)seq * n_q_heads + (int64_t)kvh * group + h) * D;
      dma16(lds_addr(dst + h * D * 2), lane * 16, buffer_rsrc(qh, (uint32_t)(D * 2)));
    }
  }
}
template <int D, int NW>
__device__ inline void copy_q_row(const AttnArgs& a, uint8_t* dst, int seq, int kvh, int wave,
                                  int lane) {
  copy_q_row<D, NW>(a.q, a.n_q_heads, a.group, dst, seq, kvh, wave, lane);
}

// q_rot = (FWHT(q * qscale) * c) o s of the work-group's GQA heads (q . R,
// R from src/cache.rs:47-62, times the softmax scale in base 2), from the
// raw rows at the start of `tab` (each wave's own row has landed: the
// caller waited for its copy), written over them as the QK B operands:
//   entry e = 2 g + s at e KiB + 16 lane, lane (j, c) = (lane / 16,
//     lane % 16): 8 f16 of head c & 7 -- the f16 high part of q_rot for
//     c < 8, the residual for c >= 8, zero past the group -- times
//     kCodeScale (the codes' operand form);
//   float qsum[8][NG] after the 2 NG entries: per head and group, sum q_rot;
//   float opsum[8][NG][2] after that: per head and group, the sums of the
//     f16 high parts and of the residuals (unscaled: the accumulator start
//     of the offset codes).
// Wave w computes the heads h = w, w + NW, ... (NW waves in the work-group)
// before the first barrier, so the rotation overlaps the other waves' copy
// issue. Every thread of the work-group calls it (it holds two barriers).
// PACK (head_dim 256, at most 2 q heads per KV head): column c of entry
// 2 g + s is (group c >> 2, head (c >> 1) & 1, high part if c is even,
// residual if odd), zero unless c >> 2 == g -- each lane of the packed
// kernel then serves one group of one head.
template <int D, int BITS, int NW, bool PACK = false>
__device__ void build_q_table(const AttnArgs& a, uint8_t* tab, int wave, int lane, uint32_t sbits) {
  constexpr int E = D / 64, NG = D / 64, LPG = 64 / E;
  constexpr int HPW = (8 + NW - 1) / NW;  // table columns (heads) per wave
  const QSlot<E, BITS> qs(lane);
  _Float16 hi[HPW][E], lo[HPW][E];
  float gsum[HPW], hsum[HPW], lsum[HPW];
#pragma unroll
  for (int k = 0; k < HPW; k++) {
    const int h = wave + k * NW;
    const bool hv = h < a.group;
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = 0.0f;
    if (hv) {
      const uint32_t* raw = reinterpret_cast<const uint32_t*>(tab + (h * D + lane * E) * 2);
#pragma unroll
      for (int m = 0; m < E / 2; m++) {
        const uint32_t w = raw[m];
        x[2 * m] = __uint_as_float(w << 16) * a.qscale;
        x[2 * m + 1] = __uint_as_float(w & 0xffff0000u) * a.qscale;
      }
    }
    gsum[k] = 0.0f;
    if (hv) {
      // the sign-tracking FWHT: an exact zero may come out as -0, which no
      // score, sum or code of this kernel can tell from +0
      wave_fwht_signed<E>(x, lane);
      const float cs = fwht_lane_sign(lane) * a.c;
#pragma unroll
      for (int i = 0; i < E; i++) {
        x[i] = apply_sign(x[i] * cs, sbits, i);
        gsum[k] += x[i];
      }
    }
    gsum[k] = group_sum<LPG>(gsum[k], lane);
    hsum[k] = lsum[k] = 0.0f;
#pragma unroll
    for (int i = 0; i < E; i++) {
      hi[k][i] = (_Float16)x[i];
      lo[k][i] = (_Float16)(x[i] - (float)hi[k][i]);
      hsum[k] += (float)hi[k][i];
      lsum[k] += (float)lo[k][i];
      // the stored operands are scaled by kCodeScale (exact); the sums are not
      hi[k][i] = hi[k][i] * (_Float16)kCodeScale<BITS>;
      lo[k][i] = lo[k][i] * (_Float16)kCodeScale<BITS>;
    }
    hsum[k] = group_sum<LPG>(hsum[k], lane);
    lsum[k] = group_sum<LPG>(lsum[k], lane);
  }
  __syncthreads();  // every raw row is read before the table replaces them
  // the 8 columns (zero past the group); heads beyond 8 write nothing
  uint8_t* ent = tab + (2 * qs.g + qs.s) * kChunk + qs.i0 * 2;
#pragma unroll
  for (int k = 0; k < HPW; k++) {
    const int h = wave + k * NW;
    if (PACK ? h < 2 : h < 8) {
      if constexpr (PACK) {
        _Float16 zero[E];
#pragma unroll
        for (int i = 0; i < E; i++) zero[i] = (_Float16)0.0f;
#pragma unroll
        for (int gg = 0; gg < NG; gg++) {
          uint8_t* col = ent + (qs.j * 16 + gg * 4 + h * 2) * 16;
          store_halves<E>(col, gg == qs.g ? hi[k] : zero);
          store_halves<E>(col + 16, gg == qs.g ? lo[k] : zero);
        }
      } else {
        store_halves<E>(ent + (qs.j * 16 + h) * 16, hi[k]);
        store_halves<E>(ent + (qs.j * 16 + h + 8) * 16, lo[k]);
      }
      if ((lane & (LPG - 1)) == 0) {
        reinterpret_cast<float*>(tab + 2 * NG * kChunk)[h * NG + qs.g] = gsum[k];
        float* op = reinterpret_cast<float*>(tab + 2 * NG * kChunk + 8 * NG * 4);
        op[(h * NG + qs.g) * 2 + 0] = hsum[k];
        op[(h * NG + qs.g) * 2 + 1] = lsum[k];
      }
    }
  }
  __syncthreads();
}

// Codes of token t, dims d0 .. d0+E-1, into a head-block's K region. A
// token's K bytes are its own (lane slot (j, t) of each chunk), so whole
// words are written; at 4 bits the 8/E lanes sharing a word OR theirs first.
template <int BITS, int E>
__device__ inline void store_k_codes(uint8_t* kbase, int t, int d0, const uint32_t (&code)[E],
                                     int lane) {
  if constexpr (BITS == 8) {
    int64_t off;
    int sh;
    k_code_pos(8, t, d0, &off, &sh);
    uint8_t* p = kbase + off + sh / 8;  // E consecutive bytes
    uint32_t w[E / 4 > 0 ? E / 4 : 1];
    if constexpr (E >= 4) {
#pragma unroll
      for (int k = 0; k < E / 4; k++)
        w[k] = code[4 * k] | (code[4 * k + 1] << 8) | (code[4 * k + 2] << 16) | (code[4 * k + 3] << 24);
    }
    if constexpr (E == 8)
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    else if constexpr (E == 4)
      *reinterpret_cast<uint32_t*>(p) = w[0];
    else
      *reinterpret_cast<uint16_t*>(p) = (uint16_t)(code[0] | (code[1] << 8));
  } else {
    int64_t off = 0;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < E; i++) {
      int sh;
      k_code_pos(4, t, d0 + i, &off, &sh);  // the same word for the E dims
      w |= code[i] << sh;
    }
    constexpr int N = 8 / E;  // lanes sharing the word
#pragma unroll
    for (int m = 1; m < N; m <<= 1) w |= (uint32_t)__shfl_xor((int)w, m);
    if ((lane & (N - 1)) == 0) *reinterpret_cast<uint32_t*>(kbase + off) = w;
  }
}

// Codes of token t into a head-block's V region, where each 32-bit word
// holds codes of four tokens: byte stores at 8 bits; at 4 bits the token's
// nibble is cleared and set with atomics, leaving the other tokens' nibbles
// untouched at every moment (the split columns may be reading the block).
template <int BITS, int E>
__device__ inline void store_v_codes(uint8_t* vbase, int t, int d0, const uint32_t (&code)[E]) {
#pragma unroll
  for (int i = 0; i < E; i++) {
    int64_t off;
    int sh;
    v_code_pos(BITS, t, d0 + i, &off, &sh);
    if constexpr (BITS == 8) {
      vbase[off + sh / 8] = (uint8_t)code[i];
    } else {
      uint32_t* w = reinterpret_cast<uint32_t*>(vbase + off);
      atomicAnd(w, ~(0xfu << sh));
      atomicOr(w, code[i] << sh);
    }
  }
}

// The new-token column of a decode step, one work-group per (seq, kvh): the
// token at position T - 1 is rotated and quantized exactly as the append
// kernel does it (src/cache.rs:94-129 with the affine codes), written to its
// slot (ring: (T - 1) mod W; paged: through the block table), and -- as the
// reference's current token attends to its own quantized K/V
// (src/cache.rs:295-298) -- contributes partial slot n_splits: m = q_rot .
// k_deq (base 2), l = 1, o = v_deq . R^T, the same row for every head of the
// group. Wave 0 handles K, wave 1 V. With a.k_norm_w the layer's prologue
// runs on the raw projections first, exactly as the append kernel runs it;
// the RoPE (cos, sin) table of position T - 1 is built by every thread of the
// work-group into `rope` (LDS, rope_dims / 2 float2) before the q table's
// barriers. NT: threads of the work-group.
template <int D, int BITS, int NT, bool PACK = false>
__device__ void new_token_column(const AttnArgs& a, uint8_t* tab, float2* rope, int64_t T,
                                 int n_splits, int kvh, int seq, int wave, int lane) {
#pragma clang fp contract(off)
  constexpr BlockLayout L = make_layout(D, BITS, kAffine);
  constexpr int E = D / 64, LPG = 64 / E;
  const int G = a.group;
  const bool pro = a.k_norm_w != nullptr;
  copy_q_row<D, NT / 64>(a, tab, seq, kvh, wave, lane);
  if (pro && T >= 1) {
    for (int j = wave * 64 + lane; j < (a.rope_dims >> 1); j += NT)
      rope[j] = rope_cos_sin(T - 1, rope_inv_freq(j, a.rope_dims, a.rope_theta));
  }
  wait_vmcnt<0>();
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  build_q_table<D, BITS, NT / 64, PACK>(a, tab, wave, lane, sbits);
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
  if (pro) {  // the rope table is complete: build_q_table's barriers passed
    if (!isv) {
      float w[E];
      load_row<E>(a.k_norm_w + d0, w);
      k_norm_row<E>(x, w, a.eps, lane);
      rope_row<E>(x, a.rope_dims, lane, [&](int j) { return rope[j]; });
    } else {
      v_norm_row<E>(x, a.eps, lane);
    }
  }
  wave_fwht_signed<E>(x, lane);
  const float cs = fwht_lane_sign(lane) * a.c;
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = apply_sign(x[i] * cs, sbits, i);
  uint32_t code[E];
  float scale, bias;
  affine_quant<E, BITS>(x, code, scale, bias, lane);
  const uint16_t s16 = f32_to_f16_bits(scale), b16 = f32_to_f16_bits(bias);

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
    if (isv)
      store_v_codes<BITS, E>(blk + L.v_codes, t, d0, code);
    else
      store_k_codes<BITS, E>(blk + L.k_codes, t, d0, code, lane);
    if ((lane & (LPG - 1)) == 0)
      *reinterpret_cast<uint32_t*>(blk + (isv ? L.v_meta : L.k_meta) + scale_pos(lane / LPG, t)) =
          (uint32_t)s16 | ((uint32_t)b16 << 16);
  }

  // the dequantized row in the rotated domain, as the split columns read it
  const float sf = f16_bits_to_f32(s16), bf = f16_bits_to_f32(b16);
  float y[E];
#pragma unroll
  for (int i = 0; i < E; i++) y[i] = (float)code[i] * sf + bf;
  if (!isv) {
    const QSlot<E, BITS> qs(lane);
    const uint8_t* ent = tab + (2 * qs.g + qs.s) * kChunk + qs.i0 * 2;
    for (int h = 0; h < G; h++) {
      // the head's high and residual columns (PACK: those of this lane's group)
      const int ch = PACK ? qs.g * 4 + h * 2 : h, cl = PACK ? ch + 1 : h + 8;
      const _Float16* qh = reinterpret_cast<const _Float16*>(ent + (qs.j * 16 + ch) * 16);
      const _Float16* ql = reinterpret_cast<const _Float16*>(ent + (qs.j * 16 + cl) * 16);
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < E; i++) p += ((float)qh[i] + (float)ql[i]) * y[i];
      // the table holds q_rot * kCodeScale (a power of 2: the quotient is exact)
      p = group_sum<64>(p, lane) * (1.0f / kCodeScale<BITS>);
      if (lane == 0) {
        a.part_ml[(pbase + h) * 2 + 0] = p;
        a.part_ml[(pbase + h) * 2 + 1] = 1.0f;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; i++) y[i] = apply_sign(y[i], sbits, i);
    wave_fwht_signed<E>(y, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int i = 0; i < E; i++) a.part_o[(pbase + h) * D + d0 + i] = y[i] * cs;
  }
}

// Pair work-groups: 8 waves, two per SIMD (register budget <= 256 each);
// solo work-groups: 12 or 4 waves, three waves per SIMD (<= 168).
// Arguments: what a work-group needs before its first copies comes first,
// as 14 dwords of scalars, which the build preloads into SGPRs with the
// dispatch (a scalar load from the argument struct waits 1.5-2 us at a
// work-group's start); the struct follows. geo_len and geo_vis_begin give
// the block range (the visible length, at most the window on a ring; the
// first visible position, 0 on a ring); skew = skew_p | skew_extra << 8;
// flags: bit 2 new-token column, bits 4-7 q heads per KV head, bits 8-31 q
// heads. A linear or ring cache's dense or stats pass needs no struct field
// for its first copies; a paged pool's (PAGED: block table, per-sequence
// lengths) needs the struct from the start. (Measured: 32K global-layer
// step 23.4 -> 23.2 us, 24.0 -> 23.5 us in a HIP graph; the compiler still
// hoists some of the struct's loads above the first copies.)
template <int D, int BITS, int MODE, int SW, bool PAGED, bool PACK>
__global__ __launch_bounds__((AttnPlan<D, BITS, SW>::kWaves * 64))
__attribute__((amdgpu_waves_per_eu(AttnPlan<D, BITS, SW>::kWavesPerSimd,
                                   AttnPlan<D, BITS, SW>::kWavesPerSimd)))
void decode_attn_kernel(const uint8_t* base, const uint16_t* q, int32_t geo_len,
                        int32_t geo_vis_begin, int32_t window, int32_t bps0, int32_t bps,
                        int32_t max_splits, uint32_t skew, int32_t block_stride,
                        int32_t head_stride, uint32_t flags, AttnArgs a) {
  using P = AttnPlan<D, BITS, SW>;
  constexpr BlockLayout L = P::L;
  constexpr int NG = P::NG, GH = P::GH;
  // PACK: dense solo streams of head_dim 256 at 4 bits with at most 2 q heads
  // per KV head -- the 16 matrix-core columns carry (group, head, high /
  // residual) instead of (head, high / residual), so each lane forms the
  // scores and P' of one group only (build_q_table)
  static_assert(!PACK || (MODE == kDense && P::kSolo && D == 256 && BITS == 4),
                "packed columns: dense solo streams, head_dim 256, 4 bits");
  constexpr int E = D / 64;
  constexpr int QS = P::kQS;
  // copy instructions per wave per block (the stats pass copies no V codes)
  constexpr int CP = MODE == kStats ? P::kWaveChunks + 1 : P::kCopies;
  constexpr int NST = P::kStages, SB = P::kStageBytes;
  constexpr int MH = P::kMetaHalf;

  __shared__ __align__(16) uint8_t stage[P::kStageRegion];
  __shared__ __align__(16) uint8_t scratch[P::kScratch];  // q-prep table, then score exchange
  __shared__ float ml_s[P::kStreams][8][2];
  __shared__ int xflag[P::kWaves];
  __shared__ float th_s[8];  // sparse-V gated pass: the group's thresholds
  // paged: the work-group's range of its sequence's block table, for the
  // loop's refills (kTblCap entries; blocks beyond read the table directly)
  constexpr int kTblCap = PAGED ? 1024 : 4;
  __shared__ __align__(16) int32_t tbl_s[kTblCap];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  constexpr int NS = P::kStreams;
  const int stream = P::kSolo ? wave : wave >> 1, half = P::kSolo ? 0 : wave & 1;
  const int j = lane >> 4, c = lane & 15;
  const int head = PACK ? (c >> 1) & 1 : c & 7;
  const bool hi = PACK ? (c & 1) == 0 : c < 8;
  const int grp = c >> 2;  // PACK: this lane's 64-dim group
  const int G = (int)((flags >> 4) & 15u);
  const bool col_valid = head < G;
  const int skew_p = (int)(skew & 255u), skew_extra = (int)(skew >> 8);
  // grid (KV head, sequence, split column): consecutive work-groups, which
  // the dispatcher deals round-robin to the XCDs, are the KV heads of one
  // split and then the sequences, so each XCD gets a like share of the work;
  // the new-token column comes last
  const int kvh = blockIdx.x, seq = blockIdx.y, split = blockIdx.z;
  const int g0 = half * GH;  // this wave's first group

  // the block range from the preloaded arguments (paged: the sequence's
  // length, bounded by the table width)
  int64_t Tg = geo_len;
  if constexpr (PAGED) Tg = a.seq_lens[seq];
  SeqGeom geo = seq_geometry(Tg, window, geo_vis_begin);
  if constexpr (PAGED) {
    if (geo.blk_hi > a.st.table_stride) geo.blk_hi = a.st.table_stride;
    if (geo.blk_hi < geo.blk_lo) geo.blk_hi = geo.blk_lo;
  }
  // one sequence: the host planned max_splits for exactly this block range
  // (no division before the first copies); paged: per sequence
  const int n_splits = PAGED ? n_splits_for(geo, bps0, bps, max_splits, skew_p) : max_splits;
  static_assert(P::kStageRegion >= D / 2 * (int)sizeof(float2), "rope table fits the staging");
  // decode step: the new token's column (dense mode, or the statistics pass
  // of a sparse-V step, whose gated pass then reads the stored token), the
  // grid's last split column
  if constexpr (MODE != kGated) {
    if ((flags & 4u) && split == max_splits) {
      new_token_column<D, BITS, P::kWaves * 64, PACK>(a, scratch, reinterpret_cast<float2*>(stage),
                                                PAGED ? Tg : a.seq_len, n_splits, kvh, seq, wave,
                                                lane);
      return;
    }
  }
  if (split >= n_splits) return;
  int64_t b_begin, b_end;
  split_range(geo, split, bps0, bps, skew_p, skew_extra, &b_begin, &b_end);

  // Table entries are read through the constant address space: a uniform
  // index then becomes a scalar load, which never waits for the copies in
  // flight.
  typedef const int32_t __attribute__((address_space(4)))* table_ptr;
  table_ptr table = nullptr;
  if constexpr (PAGED)
    table = (table_ptr)(uintptr_t)(a.st.block_table + (int64_t)seq * a.st.table_stride);
  const uint8_t* hbase = base + (int64_t)kvh * head_stride;
  auto blk_ptr = [&](int64_t lb) -> const uint8_t* {
    if constexpr (!PAGED) {
      return hbase + lb * block_stride;  // linear or ring: lb is a valid slot block
    } else {
      int64_t phys = (int64_t)table[lb];
      // a bad table entry reads a valid block rather than faulting
      phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
      return hbase + phys * block_stride;
    }
  };
  // The loop's refills take the entry from the work-group's copy of its
  // table range in LDS: a scalar load per refill would hold the stream for a
  // memory round trip at every block (the scalar loads' counter is shared
  // with LDS reads, so no later LDS access could go ahead of it either).
  // (the copy starts at the 16-byte boundary at or below the range's first
  // entry, tsh entries before it, in the same page)
  int64_t n_tbl = 0;
  int tsh = 0;
  if constexpr (PAGED) {
    tsh = (int)(((uintptr_t)(a.st.block_table + (int64_t)seq * a.st.table_stride + b_begin) & 15) >> 2);
    n_tbl = b_end - b_begin;
    n_tbl = n_tbl < 0 ? 0 : (n_tbl > kTblCap - tsh ? kTblCap - tsh : n_tbl);
  }
  auto blk_ptr_loop = [&](int64_t lb) -> const uint8_t* {
    if constexpr (!PAGED) {
      return blk_ptr(lb);
    } else {
      const int64_t r = lb - b_begin;
      int64_t phys = (r >= 0 && r < n_tbl) ? (int64_t)__builtin_amdgcn_readfirstlane(tbl_s[tsh + r])
                                           : (int64_t)table[lb];
      phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
      return hbase + phys * block_stride;
    }
  };

  // this stream's blocks: pb0 + NS i, i < nb
  const int64_t pb0 = b_begin + stream;
  const int nb = pb0 < b_end ? (int)((b_end - pb0 + NS - 1) / NS) : 0;
  // sparse-V: this (sequence, KV head)'s row of block maxima
  int64_t blk_row = 0;
  if constexpr (MODE == kGated) blk_row = ((int64_t)seq * a.st.n_kv_heads + kvh) * a.blk_stride;
  // Sparse-V gated pass: the stream visits only the blocks in which some
  // head's largest score (from the stats pass) reaches its theta, plus the
  // block of the newest token (which the stats pass's split columns leave
  // out when its new-token column attends it); a block whose weights are
  // all below tau adds nothing to O. Lane i tests block i (i < 64; any
  // blocks beyond are always visited); the visits pop the mask's bits in
  // order, as scalars.
  BlockList blist{0ull, 0, nb};
  int nbx = nb;  // blocks visited
  if constexpr (MODE == kGated) {
    gated_thresholds(a, n_splits, seq, kvh, G, split, wave, lane, th_s, P::kWaves);
    float thk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) thk[k] = k < G ? th_s[k] : INFINITY;
    blist = gated_block_list(a, thk, blk_row, geo.blk_lo, pb0, NS, nb, PAGED ? Tg : a.seq_len,
                             lane, &nbx);
  }
  BlockList bcopy = blist;  // the copies run ahead of the visits on the same list
  uint8_t* const pstage = stage + stream * NST * SB;
  const uint32_t pstage_lds = lds_addr(pstage);

  // This wave's part of block lb into stage st: its groups' K and V code
  // chunks, then one partial instruction moving its groups' K and V
  // scale/bias (lanes < 4 GH: K, the next 4 GH: V) to its meta area.
  const int kc0 = BITS == 8 ? g0 : (GH >= 2 ? g0 / 2 : 0);  // first code chunk in HBM
  const int ks0 = P::kSharedChunk ? half : kc0;               // its first chunk slot
  const int mlane = lane < 4 * GH ? lane : lane - 4 * GH;
  const int meta_voff = (lane < 4 * GH ? (int)L.k_meta : (int)L.v_meta) + g0 * 64 + mlane * 16;
  // (a stage's first fill follows no reads of it: no wait, so that the
  // first copies do not wait for the argument struct's scalar loads)
  auto copy_block = [&](int st, int64_t lb, bool refill) {
    const u32x4 rs = buffer_rsrc(refill ? blk_ptr_loop(lb) : blk_ptr(lb), (uint32_t)L.block_bytes);
    const uint32_t sl = pstage_lds + st * SB;
    if (refill) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of this stage are done
#pragma unroll
    for (int k = 0; k < P::kWaveChunks; k++) {
      const int ch = kc0 + k, slot = ks0 + k;
      dma16(sl + slot * kChunk, (int)L.k_codes + ch * kChunk + lane * 16, rs);
      if constexpr (MODE != kStats)
        dma16(sl + (P::kCodeSlots + slot) * kChunk, (int)L.v_codes + ch * kChunk + lane * 16, rs);
    }
    if (lane < 8 * GH) dma16(sl + P::kMetaOff + half * 2 * MH, meta_voff, rs);
  };

  // ---- copies: each wave's raw q row, then the first stages; the q row is
  // waited for alone and rotated while the stages land ----
  constexpr int NE = 2 * NG;  // B-operand entries; the group sums follow
  if (lane == 0) xflag[wave] = 0;
  // The first NQ stages go out before the rotation, the rest after it: the
  // rotation's first barrier then waits for less copy issue, which stalls
  // while the whole chip's first requests queue up.
  constexpr int NQ = (NST + 1) / 2;
  // paged: wave 0 copies the table range first; its q copy and first stages
  // follow, so its wait for the q row covers the table too, and the q
  // table's barrier publishes it to the other waves before any refill
  if constexpr (PAGED) {
    if (wave == 0 && n_tbl > 0) {
      const u32x4 trs = buffer_rsrc(a.st.block_table + (int64_t)seq * a.st.table_stride + b_begin - tsh,
                                    (uint32_t)((n_tbl + tsh) * 4));
      const int nk = (int)((n_tbl + tsh + 255) / 256);
      for (int k = 0; k < nk; k++) dma16(lds_addr(tbl_s) + k * kChunk, k * kChunk + lane * 16, trs);
    }
  }
  copy_q_row<D, P::kWaves>(q, (int)(flags >> 8), G, scratch, seq, kvh, wave, lane);
#pragma unroll
  for (int s = 0; s < NQ; s++)
    if (s < nbx) copy_block(s, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : s), false);
  const int64_t T = PAGED ? Tg : a.seq_len;
  if constexpr (MODE == kStats) blk_row = ((int64_t)seq * a.st.n_kv_heads + kvh) * a.blk_stride;
  wait_copies<CP, NQ>(nbx < NQ ? nbx : NQ);  // the q copy preceded every block
  // this lane's RHT signs, for the q rotation and the inverse rotation
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  build_q_table<D, BITS, P::kWaves, PACK>(a, scratch, wave, lane, sbits);
#pragma unroll
  for (int s = NQ; s < NST; s++)
    if (s < nbx) copy_block(s, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : s), false);

  // B operands of this wave's groups (hi / residual halves of q_rot) and
  // their q sums for the bias term. Pair waves hold the operands in
  // registers; solo waves, which own every group and run at three per SIMD
  // (at most 168 VGPRs), read them from the q table in LDS at each use (no
  // score exchange reuses that region in a solo work-group).
  constexpr int GB = P::kSolo ? 1 : GH;
  half8_t bq[GB][2];
  float qs[GH];
  const float* qsum = reinterpret_cast<const float*>(scratch + NE * kChunk);  // [head][NG]
  auto q_operand = [&](int gi, int s) {
    return *reinterpret_cast<const half8_t*>(scratch + ((g0 + gi) * 2 + s) * kChunk + lane * 16);
  };
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    if constexpr (!P::kSolo) {
#pragma unroll
      for (int s = 0; s < 2; s++) bq[gi][s] = q_operand(gi, s);
    }
    qs[gi] = (hi && col_valid) ? qsum[head * NG + g0 + gi] : 0.0f;
  }
  auto bq_of = [&](int gi, int s) { return P::kSolo ? q_operand(gi, s) : bq[P::kSolo ? 0 : gi][s]; };
  // offset codes: the QK accumulator of group gi starts at -kCodeOffset x
  // this column's q operand summed over the group's 64 dims (the table's
  // high or residual sum of the column's head). Solo waves (three per SIMD,
  // at most 168 VGPRs) keep the offset as one scalar per group and subtract
  // it from the finished accumulator instead of holding four-register
  // accumulator starts.
  constexpr bool kKqInC = !P::kSolo;
  float4_t kq[kKqInC ? GH : 1];
  float kqs[GH];
  const float* opsum = reinterpret_cast<const float*>(scratch + NE * kChunk + 8 * NG * 4);
  const U4Consts u4;
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    const float t = col_valid ? opsum[(head * NG + g0 + gi) * 2 + (hi ? 0 : 1)] : 0.0f;
    kqs[gi] = -kCodeOffset<BITS> * t;
    if constexpr (kKqInC) kq[gi] = (float4_t){kqs[gi], kqs[gi], kqs[gi], kqs[gi]};
  }
  // PACK: this lane's column is one group's: its q sum for the bias term
  // and its offset-code accumulator start
  float qsP = 0.0f, kqP = 0.0f;
  if constexpr (PACK) {
    qsP = (hi && col_valid) ? qsum[head * NG + grp] : 0.0f;
    kqP = col_valid ? -kCodeOffset<BITS> * opsum[(head * NG + grp) * 2 + (hi ? 0 : 1)] : 0.0f;
  }
  __syncthreads();  // pairs: the table is consumed, the region becomes the score exchange
  float4_t* const xs = reinterpret_cast<float4_t*>(scratch);  // [wave][parity][lane]

  // ---- main loop ----
  float4_t o[GH * 4];
#pragma unroll
  for (int i = 0; i < GH * 4; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float bacc[GH];
  float psum[GH];  // offset codes: this lane's running sum of P' per group
#pragma unroll
  for (int gi = 0; gi < GH; gi++) bacc[gi] = psum[gi] = 0.0f;
  // m_run starts finite (-1e30): exp2(-inf - m) is 0 for masked tokens and
  // exp2(m_old - m_new) underflows to 0 at the first visible token, so the
  // softmax needs no special cases.
  float m_run = -1e30f, l_run = 0.0f;
  const float lo_sel = hi ? 0.0f : 1.0f;  // 1 on the residual columns
  const float log2_tau = MODE == kStats ? log2f(a.tau) : 0.0f;

  // visible slots: linear [vis_lo, vis_hi); ring [0, min(T, W)), unless a trim
  // hides older positions (then each slot's position is computed)
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

  // LDS operands, read one group ahead of their use so that the read
  // latency overlaps the previous group's MFMAs
  // region 0: K codes, 1: V codes
  auto codes = [&](const uint8_t* sp, int region, int gi) {
    const int g = g0 + gi;
    const int slot = P::kSharedChunk ? half : (BITS == 8 ? g : g / 2);
    return lds16(sp + (region * P::kCodeSlots + slot) * kChunk + lane * 16);
  };
  auto kmeta = [&](const uint8_t* sp, int gi) {
    return lds16(sp + P::kMetaOff + half * 2 * MH + gi * 64 + j * 16);
  };
  auto vmeta = [&](const uint8_t* sp, int gi) {
    return lds16(sp + P::kMetaOff + half * 2 * MH + MH + gi * 64 + j * 16);
  };

  auto process = [&](const uint8_t* sp, int64_t b, int it) {
    float s[4];
    u32x4 vw, vm;
    if constexpr (PACK) {
      // all groups' QK products into one accumulator (each column sees only
      // its own group's dims: the other groups' q operands are zero there);
      // then the lane's group's scale and bias, and the sum over the four
      // groups and the high / residual columns of the head (commutative at
      // every step: the eight lanes of a head hold the same bits)
      float4_t acc = (float4_t){kqP, kqP, kqP, kqP};
      u32x4 kw = codes(sp, 0, 0);
      const u32x4 km = lds16(sp + P::kMetaOff + grp * 64 + j * 16);
#pragma unroll
      for (int gi = 0; gi < GH; gi++) {
        const u32x4 kw_g = kw;
        if (gi + 1 < GH && (BITS == 8 || ((gi + 1) & 1) == 0)) kw = codes(sp, 0, gi + 1);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand_dec<BITS>(kw_g, gi, 0, u4),
                                                     q_operand(gi, 0), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand_dec<BITS>(kw_g, gi, 1, u4),
                                                     q_operand(gi, 1), acc, 0, 0, 0);
      }
      vw = codes(sp, 1, 0);  // in flight during the softmax
      vm = lds16(sp + P::kMetaOff + MH + grp * 64 + j * 16);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float t0 = fmaf(lo16(km[i]), acc[i], hi16(km[i]) * qsP);
        const float t1 = t0 + row_ror8(t0);
        const float t2 = t1 + row_ror4(t1);
        s[i] = t2 + quad_xor1(t2);
      }
    } else {
    // this half's S^T = K . q_rot^T, * scale + bias * sum(q), per group
    float4_t sv = (float4_t){0.f, 0.f, 0.f, 0.f};
    // (pair waves keep each group's MFMA chain in program order; a solo
    // wave's four independent groups interleave, 2% faster on 4-bit D=256)
    u32x4 kw = codes(sp, 0, 0), km = kmeta(sp, 0);
#pragma unroll
    for (int gi = 0; gi < GH; gi++) {
      const u32x4 kw_g = kw, km_g = km;
      if (gi + 1 < GH) {
        if (BITS == 8 || ((g0 + gi + 1) & 1) == 0) kw = codes(sp, 0, gi + 1);
        km = kmeta(sp, gi + 1);
      }
      const int g = g0 + gi;
      const float4_t acc0 =
          kKqInC ? kq[kKqInC ? gi : 0] : (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
      float4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand_dec<BITS>(kw_g, g, 0, u4),
                                                            bq_of(gi, 0), acc0, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand_dec<BITS>(kw_g, g, 1, u4), bq_of(gi, 1),
                                                   acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ai = kKqInC ? acc[i] : acc[i] + kqs[gi];
        sv[i] = fmaf(lo16(km_g[i]), ai, fmaf(hi16(km_g[i]), qs[gi], sv[i]));
      }
      if constexpr (!P::kSolo) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MODE != kStats) {
      vw = codes(sp, 1, 0);  // in flight during the softmax
      vm = vmeta(sp, 0);
    }

    // pairs: exchange the half scores with the partner wave: publish (the
    // release orders the data before the flag), then wait for the partner's;
    // both waves add the halves in the same order, so they hold identical
    // scores
    if constexpr (P::kSolo) {
#pragma unroll
      for (int i = 0; i < 4; i++) s[i] = sv[i] + row_ror8(sv[i]);
    } else {
      const int par = it & 1;
      xs[(wave * 2 + par) * 64 + lane] = sv;
      __hip_atomic_store(&xflag[wave], it + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      while (__hip_atomic_load(&xflag[wave ^ 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
             it + 1)
        __builtin_amdgcn_s_sleep(1);
      const float4_t sp_other = xs[((wave ^ 1) * 2 + par) * 64 + lane];
      const float4_t s0 = half == 0 ? sv : sp_other;
      const float4_t s1 = half == 0 ? sp_other : sv;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float t = s0[i] + s1[i];
        s[i] = t + row_ror8(t);
      }
    }
    }

    // visibility: whole block in the common case (uniform test), per token
    // only at the edges of the visible range
    const int64_t t0 = b * kBlockTokens;
    const bool full = t0 >= vis_lo && t0 + kBlockTokens <= vis_hi && !ring_trim &&
                      (uint64_t)(ex_slot - t0) >= (uint64_t)kBlockTokens;
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t slot = t0 + 4 * j + i;
        bool vis = slot >= vis_lo && slot < vis_hi && slot != ex_slot;
        if (ring_trim) vis = vis && slot_position(slot, T, a.window) >= a.vis_begin;
        if (!vis) s[i] = -INFINITY;
      }
    }
    if constexpr (MODE == kGated) {
#pragma unroll
      for (int i = 0; i < 4; i++) s[i] = s[i] >= theta ? s[i] : -INFINITY;
    }
    float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    if constexpr (MODE == kStats) {
      // the block's largest score per head, for the gated pass's block skip
      const int64_t rb = b - geo.blk_lo;
      if (half == 0 && j == 0 && hi && rb < a.blk_stride)
        a.blk_max[blk_max_at(a, blk_row, rb, head)] = col_valid ? mb : -INFINITY;
    }
    // The reference max moves only when a score exceeds it by more than
    // kRescaleSlack (base 2): O, l and the bias sums are then rescaled, which
    // costs a multiply per accumulator; below that, p = 2^(s - m_run) stays
    // under 2^kRescaleSlack, exact in f32 and far inside f16 range for
    // p * v_scale. Any reference gives the same softmax.
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run + kRescaleSlack)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      // until something has been accumulated, O and the bias sums are zero
      // and need no rescaling (the common case of the first block)
      if (__any(l_run > 0.0f)) {
#pragma unroll
        for (int i = 0; i < GH * 4; i++) o[i] *= alpha;
#pragma unroll
        for (int gi = 0; gi < GH; gi++) {
          bacc[gi] *= alpha;
          psum[gi] *= alpha;
        }
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
    if constexpr (MODE == kStats) {
      store_block_scores(a, blk_row, b - geo.blk_lo, head, j, s, mb, m_run, log2_tau,
                         half == 0 && hi && col_valid);
      return;
    }
    // sparse-V: a block whose weights are all below tau adds nothing to O
    // (no renormalisation), so its V dequantisation and products are
    // skipped (the pair's waves hold the same scores: a uniform branch)
    if constexpr (MODE == kGated) {
      if (!__any((p[0] + p[1]) + (p[2] + p[3]) > 0.0f)) return;
    }

    // O^T += V^T . P'^T with P' = p * v_scale as f16 hi (c < 8) / residual
    // (c >= 8): x = p * v_scale in f32, hi = f16(x), residual = f16(x - hi),
    // one mixed-precision FMA per element for each
    const half2_t one2 = (half2_t){(_Float16)1.0f, (_Float16)1.0f};
    if constexpr (PACK) {
      // P' of this lane's group (high or residual by column); every group's
      // V tiles against all the columns, of which each lane keeps its own
      // group's at the end
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] = fmaf(p[i], lo16(vm[i]), 0.0f);
        bacc[0] = fmaf(p[i], hi16(vm[i]), bacc[0]);
      }
      const half2_t h01 = pkrtz(x[0], x[1]);
      const half2_t h23 = pkrtz(x[2], x[3]);
      const half2_t b01 = pkrtz(fmaf(-lo_sel, (float)h01[0], x[0]), fmaf(-lo_sel, (float)h01[1], x[1]));
      const half2_t b23 = pkrtz(fmaf(-lo_sel, (float)h23[0], x[2]), fmaf(-lo_sel, (float)h23[1], x[3]));
      const half4_t bp = cat4(b01, b23);
      psum[0] = __builtin_amdgcn_fdot2(b23, one2, __builtin_amdgcn_fdot2(b01, one2, psum[0], false), false);
      u32x4 vwn = vw;
#pragma unroll
      for (int gi = 0; gi < GH; gi++) {
        const u32x4 vw_g = vwn;
        if (gi + 1 < GH && (BITS == 8 || ((gi + 1) & 1) == 0)) vwn = codes(sp, 1, gi + 1);
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
          o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_operand_dec<BITS>(vw_g, gi, ct, u4),
                                                                 bp, o[gi * 4 + ct], 0, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int gi = 0; gi < GH; gi++) {
      const u32x4 vw_g = vw, vm_g = vm;
      if (gi + 1 < GH) {
        if (BITS == 8 || ((g0 + gi + 1) & 1) == 0) vw = codes(sp, 1, gi + 1);
        vm = vmeta(sp, gi + 1);
      }
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] = fmaf(p[i], lo16(vm_g[i]), 0.0f);  // one v_fma_mix; = the rounded product
        bacc[gi] = fmaf(p[i], hi16(vm_g[i]), bacc[gi]);
      }
      const half2_t h01 = pkrtz(x[0], x[1]);
      const half2_t h23 = pkrtz(x[2], x[3]);
      const half2_t b01 = pkrtz(fmaf(-lo_sel, (float)h01[0], x[0]), fmaf(-lo_sel, (float)h01[1], x[1]));
      const half2_t b23 = pkrtz(fmaf(-lo_sel, (float)h23[0], x[2]), fmaf(-lo_sel, (float)h23[1], x[3]));
      const half4_t bp = cat4(b01, b23);
      // the column's sum of P' (exact f16 values) for the code offset
      psum[gi] = __builtin_amdgcn_fdot2(b23, one2, __builtin_amdgcn_fdot2(b01, one2, psum[gi], false), false);
      const int g = g0 + gi;
#pragma unroll
      for (int ct = 0; ct < 4; ct++)
        o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_operand_dec<BITS>(vw_g, g, ct, u4),
                                                               bp, o[gi * 4 + ct], 0, 0, 0);
      if constexpr (!P::kSolo) __builtin_amdgcn_sched_barrier(0);
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
      copy_block(st, pb0 + (int64_t)NS * (MODE == kGated ? bcopy.pop() : i + NST), true);
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
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    bacc[gi] = xor16_sum(bacc[gi]);
    bacc[gi] = xor32_sum(bacc[gi]);
  }
  // fold the residual columns (c >= 8; PACK: odd c) into the high-part
  // columns (c < 8; PACK: even c)
#pragma unroll
  for (int k = 0; k < GH * 4; k++)
#pragma unroll
    for (int i = 0; i < 4; i++) o[k][i] = o[k][i] + (PACK ? quad_xor1(o[k][i]) : row_ror8(o[k][i]));
  if constexpr (PACK) {
    // the lane's group's code-offset term, both columns of its head
    float t = xor32_sum(xor16_sum(psum[0]));
    t = t + quad_xor1(t);
    bacc[0] = fmaf(-kCodeOffset<BITS>, t, bacc[0]);
  } else {
    // the V codes entered the MFMAs as (code + kCodeOffset) / kCodeScale:
    // the merged row is kCodeScale x O less kCodeOffset x the head's P'
    // (both column halves) summed over all tokens, the latter taken
    // together with the bias sum of each group
#pragma unroll
    for (int gi = 0; gi < GH; gi++) {
      float t = xor32_sum(xor16_sum(psum[gi]));
      t = t + row_ror8(t);
      bacc[gi] = fmaf(-kCodeOffset<BITS>, t, bacc[gi]);
    }
  }

  // The stream's own stages become its merge rows [head][QS] as soon as its
  // waves are done with them (all copies were waited for in the last block),
  // without waiting for the other streams.
  if constexpr (!P::kSolo) {
    __hip_atomic_store(&xflag[wave], nb + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(&xflag[wave ^ 1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
           nb + 1)
      __builtin_amdgcn_s_sleep(1);
  }
  float* const Rp = reinterpret_cast<float*>(pstage);
  if constexpr (PACK) {
    if (hi && col_valid) {
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        float4_t oc = o[ct];
#pragma unroll
        for (int gg = 1; gg < GH; gg++) oc = grp == gg ? o[gg * 4 + ct] : oc;
        const int d = grp * 64 + ct * 16 + 4 * j;
        *reinterpret_cast<float4_t*>(&Rp[head * QS + d]) = oc * kCodeScale<BITS> + bacc[0];
      }
      if (j == 0 && grp == 0) {
        ml_s[stream][head][0] = m_run;
        ml_s[stream][head][1] = l_run;
      }
    }
  } else if (hi && col_valid) {
#pragma unroll
    for (int gi = 0; gi < GH; gi++)
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        const int d = (g0 + gi) * 64 + ct * 16 + 4 * j;
        *reinterpret_cast<float4_t*>(&Rp[head * QS + d]) = o[gi * 4 + ct] * kCodeScale<BITS> + bacc[gi];
      }
    if (half == 0 && j == 0) {
      ml_s[stream][head][0] = m_run;
      ml_s[stream][head][1] = l_run;
    }
  }
  __syncthreads();  // every stream's rows are written

  // heads w, w + kWaves, ... on wave w
  for (int hh = wave; hh < G; hh += P::kWaves) {
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
      const int64_t pbase =
          ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G;
      float* dst = a.part_o + (pbase + hh) * D + lane * E;
      if constexpr (E % 4 == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 4)
          *reinterpret_cast<float4_t*>(dst + i) =
              (float4_t){x[i] * cs, x[i + 1] * cs, x[i + 2] * cs, x[i + 3] * cs};
      } else {
#pragma unroll
        for (int i = 0; i < E; i++) dst[i] = x[i] * cs;
      }
      if (lane == 0) {
        a.part_ml[(pbase + hh) * 2 + 0] = M;
        a.part_ml[(pbase + hh) * 2 + 1] = Lsum;
      }
    }
  }
}

// out[seq][h][d] = sum_s 2^(m_s - M) O_s[d] / sum_s 2^(m_s - M) l_s.
// One work-group per (64 dims, q head, sequence); thread (sl, dq) owns dims
// d0 + 4*dq .. +3 and splits sl, sl + 16, ..., merged in one pass with a
// running maximum; the 16 partial merges meet in LDS.
// Arguments: as the split kernel's, what the kernel needs first comes as
// leading scalars (preloaded into SGPRs with the dispatch), the struct last.
// n_cols: split partials per sequence (splits and new-token column), or -1
// for per-sequence counts from the struct (a paged batch); flags: bit 0 f32
// output, bit 1 sparse-V, bits 8-31 q heads.
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(const float* part_o, const float* part_ml,
                                                      void* out, int32_t n_cols,
                                                      int32_t part_stride, uint32_t flags,
                                                      AttnArgs a) {
  __shared__ float4_t red_o[16][16];
  __shared__ float red_m[16][16];
  __shared__ float red_l[16][16];
  const int seq = blockIdx.z, h = blockIdx.y, tid = threadIdx.x;
  const int dq = tid & 15, sl = tid >> 4;
  const int d0 = blockIdx.x * 64 + dq * 4;
  const int nqh = (int)(flags >> 8);
  int n_splits = n_cols;
  if (n_cols < 0) {
    const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
    const SeqGeom geo =
        seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
    n_splits = n_splits_for(geo, a.bps0, a.bps, a.max_splits, a.skew_p) + a.new_col;
  }
  const int64_t stride = (int64_t)nqh;
  const int64_t base = (int64_t)seq * part_stride * stride + h;

  // split maxima are finite (the split kernel starts from -1e30): the first
  // merge scales the empty state by exp2(-inf) = 0
  float M = -INFINITY, den = 0.0f;
  float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = sl; s < n_splits; s += 16) {
    const int64_t r = base + s * stride;
    const float2 ml = *reinterpret_cast<const float2*>(part_ml + r * 2);
    const float4_t ov = *reinterpret_cast<const float4_t*>(part_o + r * D + d0);
    const float mn = fmaxf(M, ml.x);
    const float alpha = exp2f(M - mn);
    const float w = exp2f(ml.x - mn);
    den = fmaf(w, ml.y, den * alpha);
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = fmaf(w, ov[i], acc[i] * alpha);
    M = mn;
  }
  red_o[sl][dq] = acc;
  red_m[sl][dq] = M;
  red_l[sl][dq] = den;
  __syncthreads();
  if (tid < 16) {
    float Mx = red_m[0][tid];
#pragma unroll
    for (int k = 1; k < 16; k++) Mx = fmaxf(Mx, red_m[k][tid]);
    float4_t s = (float4_t){0.f, 0.f, 0.f, 0.f};
    float L = 0.0f;
    if (Mx != -INFINITY) {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const float w = exp2f(red_m[k][tid] - Mx);  // 0 for slots without splits (-inf)
        s += w * red_o[k][tid];
        L = fmaf(w, red_l[k][tid], L);
      }
    }
    const int64_t o_idx = ((int64_t)seq * nqh + h) * D + blockIdx.x * 64 + tid * 4;
    // sparse-V: the kept weights are normalised by the full sum L of the
    // stats pass (no renormalisation, gemma4_attention.rs:226-232), taken at
    // its max M
    const bool sparse = (flags & 2u) != 0;
    float gated = 0.0f;
    if (sparse) {
      const int64_t nh = (int64_t)gridDim.z * nqh, r = (int64_t)seq * nqh + h;
      const float Mf = a.tau_stats[nh + r], Lf = a.tau_stats[2 * nh + r];
      gated = (Lf > 0.0f && Mx != -INFINITY) ? exp2f(Mx - Mf) / Lf : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float v = sparse ? s[i] * gated : (L > 0.0f ? s[i] / L : 0.0f);
      if (flags & 1u)
        reinterpret_cast<float*>(out)[o_idx + i] = v;
      else
        reinterpret_cast<uint16_t*>(out)[o_idx + i] = f32_to_bf16(v);
    }
  }
}

// The split kernel of one mode; with events, they are recorded by the
// dispatch itself (start and end of the kernel's execution, as a kernel
// trace times it), else a plain launch.
template <int D, int BITS, int MODE, int SW, bool PAGED, bool PACK = false>
hipError_t launch_kind(const AttnArgs& a, dim3 grid, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  SplitPre p;
  if (!split_pre(a, &p)) return hipErrorInvalidValue;
  const dim3 block(AttnPlan<D, BITS, SW>::kWaves * 64);
  const auto kern = decode_attn_kernel<D, BITS, MODE, SW, PAGED, PACK>;
  if (ev0 && ev1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, s, ev0, ev1, 0, p.base, p.q, p.geo_len,
                          p.geo_vis_begin, p.window, p.bps0, p.bps, p.max_splits, p.skew,
                          p.block_stride, p.head_stride, p.flags, a);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, s, p.base, p.q, p.geo_len, p.geo_vis_begin, p.window,
                       p.bps0, p.bps, p.max_splits, p.skew, p.block_stride, p.head_stride, p.flags,
                       a);
  return hipGetLastError();
}

template <int D, int BITS, int MODE>
hipError_t launch_split(const AttnArgs& a, dim3 grid, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  // a paged pool has per-sequence lengths; a cache has neither
  if ((a.st.block_table != nullptr) != (a.seq_lens != nullptr)) return hipErrorInvalidValue;
  if constexpr (kSoloCapable<D, BITS>) {
    if (a.bps >= kSoloMinBlocks) {
      // head_dim 256 at 4 bits with at most 2 q heads per KV head (Gemma-4's
      // sliding layers): the packed-column form of the solo streams
      if constexpr (MODE == kDense && D == 256 && BITS == 4) {
        if (a.group <= 2)
          return a.st.block_table
                     ? launch_kind<D, BITS, MODE, kPagedSoloWaves, true, true>(a, grid, s, ev0, ev1)
                     : launch_kind<D, BITS, MODE, 12, false, true>(a, grid, s, ev0, ev1);
      }
      return a.st.block_table ? launch_kind<D, BITS, MODE, kPagedSoloWaves, true>(a, grid, s, ev0, ev1)
                              : launch_kind<D, BITS, MODE, 12, false>(a, grid, s, ev0, ev1);
    }
  }
  return a.st.block_table ? launch_kind<D, BITS, MODE, 0, true>(a, grid, s, ev0, ev1)
                          : launch_kind<D, BITS, MODE, 0, false>(a, grid, s, ev0, ev1);
}

template <int D, int BITS>
hipError_t launch_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                    hipEvent_t ev0, hipEvent_t ev1) {
  dim3 grid(n_kv_heads, n_seqs, a.max_splits + a.new_col);
  hipError_t e;
  if (a.tau > 0.0f) {
    // sparse-V: the stats pass (with a decode step's new-token column, which
    // appends the token), then either the gather (launch_sparse_gather) or
    // the gated pass over every stored token (the new one included; it
    // derives the thresholds from the stats pass's statistics, which sit in
    // a region of their own, stat_ml, so that no gated work-group
    // overwrites what another still reads) and the combine of its splits
    AttnArgs st = a;
    st.part_ml = a.stat_ml;
    if (!st.part_ml) return hipErrorInvalidValue;
    if (a.blk_scores) {
      // the gather in place of the gated pass and the combine (the stats
      // pass stored the candidate blocks' scores and zeroed the counters)
      if ((e = launch_split<D, BITS, kStats>(st, grid, s, ev0, ev1)) != hipSuccess) return e;
      AttnArgs g = a;
      g.stats_new_col = a.new_col;
      return launch_sparse_gather(g, n_seqs, s);
    }
    if ((e = launch_split<D, BITS, kStats>(st, grid, s, nullptr, nullptr)) != hipSuccess) return e;
    AttnArgs g = a;
    g.new_col = 0;
    g.stats_new_col = a.new_col;
    if ((e = launch_split<D, BITS, kGated>(g, dim3(n_kv_heads, n_seqs, a.max_splits), s, ev0, ev1)) !=
        hipSuccess)
      return e;
    return a.direct ? hipSuccess : launch_combine(g, n_seqs, s);
  }
  e = launch_split<D, BITS, kDense>(a, grid, s, ev0, ev1);
  if (e != hipSuccess || a.direct) return e;
  return launch_combine(a, n_seqs, s);
}

}  // namespace

hipError_t launch_combine(const AttnArgs& a, int n_seqs, hipStream_t s) {
  const int D = a.st.layout.head_dim;
  dim3 cgrid(D / 64, a.n_q_heads, n_seqs);
  // one cache: the partial count from the plan, as the split kernel sees it
  int32_t n_cols = -1;
  if (!a.seq_lens && !a.st.block_table && n_seqs == 1) {
    const SeqGeom geo = seq_geometry(a.seq_len, a.window, a.vis_begin);
    n_cols = n_splits_for(geo, a.bps0, a.bps, a.max_splits, a.skew_p) + a.new_col;
  }
  if (a.n_q_heads >= (1 << 24)) return hipErrorInvalidValue;
  const uint32_t flags =
      (a.out_f32 ? 1u : 0u) | (a.tau > 0.0f ? 2u : 0u) | ((uint32_t)a.n_q_heads << 8);
  const float* po = a.part_o;
  const float* pm = a.part_ml;
  if (D == 128)
    hipLaunchKernelGGL((combine_kernel<128>), cgrid, dim3(256), 0, s, po, pm, a.out, n_cols,
                       a.part_stride, flags, a);
  else if (D == 256)
    hipLaunchKernelGGL((combine_kernel<256>), cgrid, dim3(256), 0, s, po, pm, a.out, n_cols,
                       a.part_stride, flags, a);
  else if (D == 512)
    hipLaunchKernelGGL((combine_kernel<512>), cgrid, dim3(256), 0, s, po, pm, a.out, n_cols,
                       a.part_stride, flags, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                                   hipEvent_t e0, hipEvent_t e1) {
  switch (a.st.layout.head_dim * 16 + a.st.layout.bits) {
    case 128 * 16 + 4: return launch_t<128, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 128 * 16 + 8: return launch_t<128, 8>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256 * 16 + 4: return launch_t<256, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256 * 16 + 8: return launch_t<256, 8>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512 * 16 + 4: return launch_t<512, 4>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512 * 16 + 8: return launch_t<512, 8>(a, n_seqs, n_kv_heads, s, e0, e1);
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

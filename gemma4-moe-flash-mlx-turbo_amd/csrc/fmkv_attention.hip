// Fused decode attention over the quantized cache (affine mode).
//
// Replaces mlx_rs::fast::scaled_dot_product_attention at decode (L == 1,
// src/model/gemma4_attention.rs:94-103) reading the cache written by
// fmkv_append. One work-group = one (split of consecutive 16-token blocks,
// KV head, sequence); its NW = D/DW waves each own DW dims of head_dim.
//
// Per block (16 tokens):
//   QK^T  S^T[16 tok x 16 col] += K[16 x 32] . Q^T[32 x 16] on MFMA
//         (v_mfma_f32_16x16x32_f16), K codes converted exactly to f16
//         integers; per 64-dim group the f16 scale/bias are applied after the
//         MFMA: s += scale * acc + bias * sum(q_group). (Codes stay
//         unbiased: an f16 1024 + code operand with the offset cancelled in
//         the accumulator is cheaper but inflates the fp32 partial sums ~64x
//         at 4 bits, which outlier channels turn into visible error.)
//         Column c = q head (c & 7) of the GQA group, c < 8 carrying the f16
//         high part of q_rot and c >= 8 the residual, so S keeps ~22 bits of
//         q precision; DPP row_ror:8 folds the two halves.
//   Waves exchange their partial S through LDS (one barrier per block) and
//   run identical online-softmax bookkeeping (base-2, eager rescale).
//   PV    O^T[16 dim x 16 col] += V^T[16 dim x 16 tok] . P'^T[16 tok x 16 col]
//         (v_mfma_f32_16x16x16f16) with P' = p * v_scale split hi/lo in the
//         same columns; bias terms are summed on the side.
// The QK output lane layout equals the PV B-operand layout (lane (j, c) holds
// tokens 4j..4j+3 of column c), so no register shuffles are needed.
//
// q arrives pre-rotated in the MFMA operand layout (fmkv_qprep.h), so the
// prologue is one load per operand, issued ahead of the first blocks. Each
// wave then keeps DEPTH blocks in flight in as many register sets, refilling
// a set as soon as it has been consumed.
// Epilogue: O is written to LDS, inverse-rotated (o . R^T = c * FWHT(o o s))
// and stored either as the final output (single split) or as a split partial
// (m, l, O) for the combine kernel.
#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_qprep.h"

namespace fmkv {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int BITS, int GW>
struct BlockRegs {
  static constexpr int kCodeLoads = (BITS == 8) ? GW : GW / 2;
  u32x4 k[kCodeLoads];
  u32x4 v[kCodeLoads];
  u32x4 ks[GW];
  u32x4 vs[GW];
};

// One head-block's slice for this wave via buffer loads: the block base is a
// scalar resource (bounded by the block size; out-of-range reads return 0),
// lanes differ only in a 32-bit offset.
// `valid` false gives a zero-size resource: the loads are dropped by the
// hardware (no memory traffic) and return zeros, so callers can issue them
// unconditionally.
template <int D, int BITS, int GW>
__device__ inline void load_block(BlockRegs<BITS, GW>& r, const uint8_t* blk, bool valid, int wave,
                                  int lane) {
  constexpr BlockLayout L = make_layout(D, BITS, kAffine);
  constexpr int kLoads = BlockRegs<BITS, GW>::kCodeLoads;
  // the block base is the same for the whole wave; say so, so that the
  // resource lives in SGPRs
  const uint64_t addr = reinterpret_cast<uint64_t>(blk);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                        valid ? (int)L.block_bytes : 0, 0x00020000);
  const int vo = lane * 16;          // 16 bytes per lane of a 1 KiB chunk
  const int so = (lane >> 4) * 16;   // 4 tokens' {scale, bias} of a group
  const int c0 = wave * kLoads;      // this wave's first code chunk
#pragma unroll
  for (int i = 0; i < kLoads; i++) {
    r.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, (int)L.k_codes + (c0 + i) * 1024, 0);
    r.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, (int)L.v_codes + (c0 + i) * 1024, 0);
  }
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
    const int g = wave * GW + gi;
    r.ks[gi] = __builtin_amdgcn_raw_buffer_load_b128(rs, so, (int)L.k_meta + g * 64, 0);
    r.vs[gi] = __builtin_amdgcn_raw_buffer_load_b128(rs, so, (int)L.v_meta + g * 64, 0);
  }
}

// K codes of group gi (wave-local) for MFMA s in {0, 1}: 8 exact f16 values.
template <int BITS, int GW>
__device__ inline half8_t k_operand(const BlockRegs<BITS, GW>& r, int gi, int s) {
  if constexpr (BITS == 8) {
    const u32x4 u = r.k[gi];
    const uint32_t w0 = u[2 * s], w1 = u[2 * s + 1];
    return cat8(u8x2_to_h2(w0, 0x04010400u), u8x2_to_h2(w0, 0x04030402u),
                u8x2_to_h2(w1, 0x04010400u), u8x2_to_h2(w1, 0x04030402u));
  } else {
    const uint32_t w = r.k[gi >> 1][(gi & 1) * 2 + s];
    return cat8(u4x2_to_h2(w, 0), u4x2_to_h2(w, 1), u4x2_to_h2(w, 2), u4x2_to_h2(w, 3));
  }
}

// V codes of column tile ct (0..3) of group gi: tokens 4j..4j+3 of one dim.
template <int BITS, int GW>
__device__ inline half4_t v_operand(const BlockRegs<BITS, GW>& r, int gi, int ct) {
  if constexpr (BITS == 8) {
    const uint32_t w = r.v[gi][ct];
    return cat4(u8x2_to_h2(w, 0x04010400u), u8x2_to_h2(w, 0x04030402u));
  } else {
    const int ctc = (gi & 1) * 4 + ct;  // column tile inside the 128-dim chunk
    const uint32_t w = r.v[gi >> 1][ctc >> 1];
    const int k0 = (ctc & 1) * 2;
    return cat4(u4x2_to_h2(w, k0), u4x2_to_h2(w, k0 + 1));
  }
}

__device__ inline float lo16(uint32_t w) { return f16_bits_to_f32(w); }
__device__ inline float hi16(uint32_t w) { return f16_bits_to_f32(w >> 16); }

// Waves per SIMD: three with two blocks in flight per wave (register budget
// <= 168), two with three or four (<= 256), one beyond (<= 512 with AGPRs).
template <int D, int BITS, int DW, int DEPTH>
__global__ __launch_bounds__((D / DW) * 64)
__attribute__((amdgpu_waves_per_eu(DEPTH >= 5 ? 1 : (DEPTH >= 3 ? 2 : 3), 8)))
void decode_attn_kernel(AttnArgs a) {
  constexpr int NW = D / DW;
  constexpr int GW = DW / 64;
  static_assert(BITS == 8 || GW % 2 == 0, "4-bit needs 128-dim wave slices");

  constexpr int QS = D + 4;                   // padded row stride (LDS banks)
  __shared__ float qo[8 * QS];                // the split's O, for the epilogue
  __shared__ float4_t sx[2][NW > 1 ? NW : 1][64];  // partial S exchange
  __shared__ float ml_s[8][2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int j = lane >> 4, c = lane & 15;
  const int head = c & 7;
  const bool hi = c < 8;
  const int G = a.group;
  const bool col_valid = head < G;
  const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;

  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps, a.max_splits);
  if (split >= n_splits) return;
  const int64_t b_begin = geo.blk_lo + (int64_t)split * a.bps;
  int64_t b_end = b_begin + a.bps;
  if (b_end > geo.blk_hi) b_end = geo.blk_hi;

  // Table entries are read through the constant address space: a uniform
  // index then becomes a scalar load, counted apart from the vector loads of
  // the block stream, so resolving the next block never waits for the
  // blocks in flight.
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

  // ---- prologue: this wave's q operands first, then the first blocks ----
  constexpr int E = D / 64;
  static_assert(DW == kAttnDW, "q-prep table is laid out for 128-dim wave slices");
  const uint32_t* qp = qprep_entry(a.qprep, seq, (int)gridDim.y, kvh, NW, wave, lane);
  u32x4 qv[kQPrepVecs];
#pragma unroll
  for (int i = 0; i < kQPrepVecs; i++) qv[i] = *reinterpret_cast<const u32x4*>(qp + 4 * i);

  // Loads are issued unconditionally: a block past the split gets a zero-size
  // resource (no traffic), so the loaded registers never merge with stale
  // ones across the loop and no copy forces a wait.
  const int64_t b_last = b_end > b_begin ? b_end - 1 : b_begin;
  auto fetch = [&](BlockRegs<BITS, GW>& r, int64_t lb) {
    const bool valid = lb < b_end;
    load_block<D, BITS, GW>(r, blk_ptr(valid ? lb : b_last), valid, wave, lane);
  };
  BlockRegs<BITS, GW> rs[DEPTH];
#pragma unroll
  for (int s = 0; s < DEPTH; s++) fetch(rs[s], b_begin + s);

  half8_t bq[GW][2];
  float qs[GW];
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
#pragma unroll
    for (int s = 0; s < 2; s++) bq[gi][s] = __builtin_bit_cast(half8_t, qv[gi * 2 + s]);
    qs[gi] = __uint_as_float(qv[2 * GW][gi]);
  }
  const uint32_t sbits = qv[2 * GW][2];

  // ---- main loop ----
  float4_t o[GW * 4];
#pragma unroll
  for (int i = 0; i < GW * 4; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float bacc[GW];
#pragma unroll
  for (int gi = 0; gi < GW; gi++) bacc[gi] = 0.0f;
  // m_run starts finite (-1e30): exp2(-inf - m) is 0 for masked tokens and
  // exp2(m_old - m_new) underflows to 0 at the first visible token, so the
  // softmax needs no special cases.
  float m_run = -1e30f, l_run = 0.0f;
  int par = 0;
  const float lo_sel = hi ? 0.0f : 1.0f;  // 1 on the residual columns

  // visible slots: linear [vis_lo, vis_hi); ring [0, min(T, W)), unless a trim
  // hides older positions (then each slot's position is computed)
  const int64_t vis_lo = a.window > 0 ? 0 : a.vis_begin;
  const int64_t vis_hi = a.window > 0 ? (T < a.window ? T : a.window) : T;
  const bool ring_trim = a.window > 0 && a.vis_begin > T - a.window;

  auto process = [&](const BlockRegs<BITS, GW>& cur, int64_t b) {
    // S^T = K . q_rot^T per 64-dim group, then * scale + bias * sum(q)
    float4_t sv = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
      float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<BITS, GW>(cur, gi, 0), bq[gi][0],
                                                   acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<BITS, GW>(cur, gi, 1), bq[gi][1],
                                                   acc, 0, 0, 0);
      const u32x4 kw = cur.ks[gi];
#pragma unroll
      for (int i = 0; i < 4; i++) sv[i] = fmaf(lo16(kw[i]), acc[i], fmaf(hi16(kw[i]), qs[gi], sv[i]));
    }
    if constexpr (NW > 1) {
      sx[par][wave][lane] = sv;
      __syncthreads();
      sv = sx[par][0][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; w2++) sv += sx[par][w2][lane];
      par ^= 1;
    }
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; i++) s[i] = sv[i] + row_ror8(sv[i]);

    // visibility: whole block in the common case (uniform test), per token
    // only at the edges of the visible range
    const int64_t t0 = b * kBlockTokens;
    const bool full = b < b_end && t0 >= vis_lo && t0 + kBlockTokens <= vis_hi && !ring_trim;
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t slot = t0 + 4 * j + i;
        bool vis = b < b_end && slot >= vis_lo && slot < vis_hi;
        if (ring_trim) vis = vis && slot_position(slot, T, a.window) >= a.vis_begin;
        if (!vis) s[i] = -INFINITY;
      }
    }
    float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int i = 0; i < GW * 4; i++) o[i] *= alpha;
#pragma unroll
      for (int gi = 0; gi < GW; gi++) bacc[gi] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

    // O^T += V^T . P'^T with P' = p * v_scale as f16 hi (c < 8) / residual
    // (c >= 8)
#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
      const u32x4 vw = cur.vs[gi];
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[i] = p[i] * lo16(vw[i]);
        bacc[gi] = fmaf(p[i], hi16(vw[i]), bacc[gi]);
      }
      const half2_t h01 = pkrtz(x[0], x[1]);
      const half2_t h23 = pkrtz(x[2], x[3]);
      const half4_t bp = cat4(
          pkrtz(fmaf(-lo_sel, (float)h01[0], x[0]), fmaf(-lo_sel, (float)h01[1], x[1])),
          pkrtz(fmaf(-lo_sel, (float)h23[0], x[2]), fmaf(-lo_sel, (float)h23[1], x[3])));
#pragma unroll
      for (int ct = 0; ct < 4; ct++)
        o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_operand<BITS, GW>(cur, gi, ct),
                                                               bp, o[gi * 4 + ct], 0, 0, 0);
    }
  };

  // DEPTH register sets in rotation: while one block is processed the others
  // are in flight; a set is reloaded as soon as it has been consumed (no
  // register copies, which would force a wait on every outstanding load).
  // Blocks past the split are skipped (a uniform branch) but still fetched
  // as dropped loads, so every set sees the same load sequence.
  for (int64_t b = b_begin; b < b_end; b += DEPTH) {
#pragma unroll
    for (int s = 0; s < DEPTH; s++) {
      if (b + s < b_end) process(rs[s], b + s);
      fetch(rs[s], b + s + DEPTH);
    }
  }

  // ---- epilogue ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
    bacc[gi] = xor16_sum(bacc[gi]);
    bacc[gi] = xor32_sum(bacc[gi]);
  }
#pragma unroll
  for (int k = 0; k < GW * 4; k++)
#pragma unroll
    for (int i = 0; i < 4; i++) o[k][i] = o[k][i] + row_ror8(o[k][i]);

  __syncthreads();  // all waves are done reading q_rot out of qo
  if (hi && col_valid) {
#pragma unroll
    for (int gi = 0; gi < GW; gi++)
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        const int d = (wave * GW + gi) * 64 + ct * 16 + 4 * j;
        *reinterpret_cast<float4_t*>(&qo[head * QS + d]) = o[gi * 4 + ct] + bacc[gi];
      }
    if (wave == 0 && j == 0) {
      ml_s[head][0] = m_run;
      ml_s[head][1] = l_run;
    }
  }
  __syncthreads();

  // inverse rotation o . R^T = c * FWHT(o o s), one head per wave, then store
  const int64_t qh0 = (int64_t)seq * a.n_q_heads + (int64_t)kvh * G;
  const int64_t pbase = ((int64_t)seq * a.max_splits + split) * a.n_q_heads + (int64_t)kvh * G;
  for (int hh = wave; hh < G; hh += NW) {
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = apply_sign(qo[hh * QS + lane * E + i], sbits, i);
    wave_fwht<E>(x, lane);
    if (a.direct) {
      const float l = ml_s[hh][1];
      const int64_t o_idx = (qh0 + hh) * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; i++) {
        const float v = l > 0.0f ? (x[i] * a.c) / l : 0.0f;
        if (a.out_f32)
          reinterpret_cast<float*>(a.out)[o_idx + i] = v;
        else
          reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
      }
    } else {
      float* dst = a.part_o + (pbase + hh) * D + lane * E;
      if constexpr (E % 4 == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 4)
          *reinterpret_cast<float4_t*>(dst + i) =
              (float4_t){x[i] * a.c, x[i + 1] * a.c, x[i + 2] * a.c, x[i + 3] * a.c};
      } else {
#pragma unroll
        for (int i = 0; i < E; i++) dst[i] = x[i] * a.c;
      }
      if (lane == 0) {
        a.part_ml[(pbase + hh) * 2 + 0] = ml_s[hh][0];
        a.part_ml[(pbase + hh) * 2 + 1] = ml_s[hh][1];
      }
    }
  }
}

// out[seq][h][d] = sum_s 2^(m_s - M) O_s[d] / sum_s 2^(m_s - M) l_s.
// One work-group per (64 dims, q head, sequence); thread (sl, dq) owns dims
// d0 + 4*dq .. +3 and splits sl, sl + 16, ..., merged in one pass with a
// running maximum; the 16 partial merges meet in LDS.
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a) {
  __shared__ float4_t red_o[16][16];
  __shared__ float red_m[16][16];
  __shared__ float red_l[16][16];
  const int seq = blockIdx.z, h = blockIdx.y, tid = threadIdx.x;
  const int dq = tid & 15, sl = tid >> 4;
  const int d0 = blockIdx.x * 64 + dq * 4;
  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps, a.max_splits);
  const int64_t stride = (int64_t)a.n_q_heads;
  const int64_t base = (int64_t)seq * a.max_splits * stride + h;

  // split maxima are finite (the split kernel starts from -1e30): the first
  // merge scales the empty state by exp2(-inf) = 0
  float M = -INFINITY, den = 0.0f;
  float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = sl; s < n_splits; s += 16) {
    const int64_t r = base + s * stride;
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + r * 2);
    const float4_t ov = *reinterpret_cast<const float4_t*>(a.part_o + r * D + d0);
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
    const int64_t o_idx = ((int64_t)seq * a.n_q_heads + h) * D + blockIdx.x * 64 + tid * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float v = L > 0.0f ? s[i] / L : 0.0f;
      if (a.out_f32)
        reinterpret_cast<float*>(a.out)[o_idx + i] = v;
      else
        reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
    }
  }
}

// One work-group per (KV head, sequence).
template <int D, int BITS>
__global__ __launch_bounds__((D / kAttnDW) * 64) void qprep_kernel(QPrepArgs a) {
  qprep_workgroup<D, BITS>(a, (int)gridDim.x, blockIdx.x, blockIdx.y, threadIdx.x);
}

template <int D, int BITS>
hipError_t launch_qprep_t(const QPrepArgs& a, int n_kv_heads, int n_seqs, hipStream_t s) {
  hipLaunchKernelGGL((qprep_kernel<D, BITS>), dim3(n_kv_heads, n_seqs), dim3((D / kAttnDW) * 64),
                     0, s, a);
  return hipGetLastError();
}

template <int D, int BITS>
hipError_t launch_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                    hipEvent_t ev0, hipEvent_t ev1) {
  constexpr int DW = kAttnDW;
  constexpr int NT = (D / DW) * 64;
  dim3 grid(a.max_splits, n_kv_heads, n_seqs);
  if (ev0) (void)hipEventRecord(ev0, s);
  hipLaunchKernelGGL((decode_attn_kernel<D, BITS, DW, kAttnDepth>), grid, dim3(NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (ev1) (void)hipEventRecord(ev1, s);
  if (e != hipSuccess || a.direct) return e;
  dim3 cgrid(D / 64, a.n_q_heads, n_seqs);
  hipLaunchKernelGGL((combine_kernel<D>), cgrid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace

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

hipError_t launch_qprep(const QPrepArgs& a, int head_dim, int bits, int n_kv_heads, int n_seqs,
                        hipStream_t s) {
  if (n_seqs <= 0) return hipSuccess;
  switch (head_dim * 16 + bits) {
    case 128 * 16 + 4: return launch_qprep_t<128, 4>(a, n_kv_heads, n_seqs, s);
    case 128 * 16 + 8: return launch_qprep_t<128, 8>(a, n_kv_heads, n_seqs, s);
    case 256 * 16 + 4: return launch_qprep_t<256, 4>(a, n_kv_heads, n_seqs, s);
    case 256 * 16 + 8: return launch_qprep_t<256, 8>(a, n_kv_heads, n_seqs, s);
    case 512 * 16 + 4: return launch_qprep_t<512, 4>(a, n_kv_heads, n_seqs, s);
    case 512 * 16 + 8: return launch_qprep_t<512, 8>(a, n_kv_heads, n_seqs, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

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
//         MFMA: s += scale * acc + bias * sum(q_group).
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
// Epilogue: O is written to LDS, inverse-rotated (o . R^T = c * FWHT(o o s))
// and stored either as the final output (single split) or as a split partial
// (m, l, O) for fmkv_combine.
#include "fmkv_device.h"
#include "fmkv_internal.h"

namespace fmkv {
namespace {

// Dim of head_dim fed to lane k-group j, element i, of the QK MFMA s (0/1)
// of group g (matches the K-code placement in fmkv_layout.h).
template <int BITS>
__device__ inline int qk_dim(int g, int s, int j, int i) {
  if constexpr (BITS == 8)
    return g * 64 + j * 16 + s * 8 + i;
  else
    return g * 64 + s * 32 + j * 8 + i;
}

template <int BITS, int GW>
struct BlockRegs {
  static constexpr int kCodeLoads = (BITS == 8) ? GW : GW / 2;
  uint4 k[kCodeLoads];
  uint4 v[kCodeLoads];
  uint4 ks[GW];
  uint4 vs[GW];
};

template <int D, int BITS, int GW>
__device__ inline void load_block(BlockRegs<BITS, GW>& r, const uint8_t* blk, int wave, int lane) {
  constexpr BlockLayout L = make_layout(D, BITS, kAffine);
  constexpr int kLoads = BlockRegs<BITS, GW>::kCodeLoads;
  const int j = lane >> 4;
  // chunk index of this wave's first code chunk
  const int c0 = wave * kLoads;
#pragma unroll
  for (int i = 0; i < kLoads; i++) {
    r.k[i] = *reinterpret_cast<const uint4*>(blk + L.k_codes + (c0 + i) * 1024 + lane * 16);
    r.v[i] = *reinterpret_cast<const uint4*>(blk + L.v_codes + (c0 + i) * 1024 + lane * 16);
  }
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
    const int g = wave * GW + gi;
    r.ks[gi] = *reinterpret_cast<const uint4*>(blk + L.k_meta + g * 64 + j * 16);
    r.vs[gi] = *reinterpret_cast<const uint4*>(blk + L.v_meta + g * 64 + j * 16);
  }
}

// K codes of group gi (wave-local) for MFMA s in {0, 1}: 8 exact f16 values.
template <int BITS, int GW>
__device__ inline half8_t k_operand(const BlockRegs<BITS, GW>& r, int gi, int s) {
  if constexpr (BITS == 8) {
    const uint4 u = r.k[gi];
    const uint32_t w0 = s ? u.z : u.x, w1 = s ? u.w : u.y;
    return cat8(u8x2_to_h2(w0, 0x04010400u), u8x2_to_h2(w0, 0x04030402u),
                u8x2_to_h2(w1, 0x04010400u), u8x2_to_h2(w1, 0x04030402u));
  } else {
    const uint4 u = r.k[gi >> 1];
    const int wi = (gi & 1) * 2 + s;
    const uint32_t w = wi == 0 ? u.x : wi == 1 ? u.y : wi == 2 ? u.z : u.w;
    return cat8(u4x2_to_h2(w, 0), u4x2_to_h2(w, 1), u4x2_to_h2(w, 2), u4x2_to_h2(w, 3));
  }
}

// V codes of column tile ct (0..3) of group gi: tokens 4j..4j+3 of one dim.
template <int BITS, int GW>
__device__ inline half4_t v_operand(const BlockRegs<BITS, GW>& r, int gi, int ct) {
  if constexpr (BITS == 8) {
    const uint4 u = r.v[gi];
    const uint32_t w = ct == 0 ? u.x : ct == 1 ? u.y : ct == 2 ? u.z : u.w;
    return cat4(u8x2_to_h2(w, 0x04010400u), u8x2_to_h2(w, 0x04030402u));
  } else {
    const uint4 u = r.v[gi >> 1];
    const int ctc = (gi & 1) * 4 + ct;  // column tile inside the 128-dim chunk
    const int wi = ctc >> 1;
    const uint32_t w = wi == 0 ? u.x : wi == 1 ? u.y : wi == 2 ? u.z : u.w;
    const int k0 = (ctc & 1) * 2;
    return cat4(u4x2_to_h2(w, k0), u4x2_to_h2(w, k0 + 1));
  }
}

__device__ inline float lo16(uint32_t w) { return f16_bits_to_f32(w); }
__device__ inline float hi16(uint32_t w) { return f16_bits_to_f32(w >> 16); }

// Cooperative FWHT over `heads` rows of D floats in LDS (NT threads).
template <int D, int NT>
__device__ inline void lds_fwht(float* buf, int heads) {
  const int n_pairs = heads * D / 2;
  for (int h = 1; h < D; h <<= 1) {
    for (int idx = threadIdx.x; idx < n_pairs; idx += NT) {
      const int i = (idx / h) * 2 * h + (idx % h);
      const float a = buf[i], b = buf[i + h];
      buf[i] = a + b;
      buf[i + h] = a - b;
    }
    __syncthreads();
  }
}

template <int D, int BITS, int DW>
__global__ __launch_bounds__((D / DW) * 64) void decode_attn_kernel(AttnArgs a) {
  constexpr int NW = D / DW;
  constexpr int GW = DW / 64;
  constexpr int NT = NW * 64;
  constexpr int NG = D / 64;
  static_assert(BITS == 8 || GW % 2 == 0, "4-bit needs 128-dim wave slices");

  __shared__ float qo[8 * D];                 // q_rot, then the split's O
  __shared__ float4_t sx[2][NW > 1 ? NW : 1][64];  // partial S exchange
  __shared__ float qsum_s[8][NG];
  __shared__ float ml_s[8][2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  const int32_t* table =
      a.st.block_table ? a.st.block_table + (int64_t)seq * a.st.table_stride : nullptr;
  const uint8_t* hbase = a.st.base + (int64_t)kvh * a.st.head_stride;
  auto blk_ptr = [&](int64_t lb) -> const uint8_t* {
    int64_t phys = table ? (int64_t)table[lb] : lb;
    // a bad table entry reads a valid block rather than faulting
    phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
    return hbase + phys * a.st.block_stride;
  };

  BlockRegs<BITS, GW> nxt;
  if (b_begin < b_end) load_block<D, BITS, GW>(nxt, blk_ptr(b_begin), wave, lane);

  // ---- q prologue: q_rot = (FWHT(q * qscale) * c) o s, per GQA head ----
  const uint16_t* qg = a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G) * D;
  for (int idx = tid; idx < G * D; idx += NT) qo[idx] = bf16_to_f32(qg[idx]) * a.qscale;
  __syncthreads();
  lds_fwht<D, NT>(qo, G);
  for (int idx = tid; idx < G * D; idx += NT) qo[idx] = (qo[idx] * a.c) * a.signs[idx % D];
  __syncthreads();
  for (int idx = tid; idx < G * NG; idx += NT) {
    const int hh = idx / NG, g = idx % NG;
    float s = 0.0f;
    for (int d = 0; d < 64; d++) s += qo[hh * D + g * 64 + d];
    qsum_s[hh][g] = s;
  }
  __syncthreads();

  half8_t bq[GW][2];
  float qs[GW];
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
    const int g = wave * GW + gi;
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float v = col_valid ? qo[head * D + qk_dim<BITS>(g, s, j, i)] : 0.0f;
        const _Float16 vh = (_Float16)v;
        bq[gi][s][i] = hi ? vh : (_Float16)(v - (float)vh);
      }
    }
    qs[gi] = (hi && col_valid) ? qsum_s[head][g] : 0.0f;
  }

  // ---- main loop ----
  float4_t o[GW * 4];
#pragma unroll
  for (int i = 0; i < GW * 4; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float bacc[GW];
#pragma unroll
  for (int gi = 0; gi < GW; gi++) bacc[gi] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  int par = 0;

  for (int64_t b = b_begin; b < b_end; b++) {
    const BlockRegs<BITS, GW> cur = nxt;
    if (b + 1 < b_end) load_block<D, BITS, GW>(nxt, blk_ptr(b + 1), wave, lane);

    float4_t sv = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
      float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<BITS, GW>(cur, gi, 0), bq[gi][0],
                                                   acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<BITS, GW>(cur, gi, 1), bq[gi][1],
                                                   acc, 0, 0, 0);
      const uint4 ks = cur.ks[gi];
      const uint32_t kw[4] = {ks.x, ks.y, ks.z, ks.w};
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

    // visibility of tokens 4j..4j+3 of this block
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int64_t slot = b * kBlockTokens + 4 * j + i;
      const int64_t p = slot_position(slot, T, a.window);
      if (p < 0 || p < a.vis_begin) s[i] = -INFINITY;
    }
    float mb = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    const float m_new = fmaxf(m_run, mb);
    if (__builtin_amdgcn_read_exec() && __any(m_new > m_run)) {
      const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f(m_run - m_new);
#pragma unroll
      for (int i = 0; i < GW * 4; i++) o[i] *= alpha;
#pragma unroll
      for (int gi = 0; gi < GW; gi++) bacc[gi] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = (s[i] == -INFINITY) ? 0.0f : exp2f(s[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

#pragma unroll
    for (int gi = 0; gi < GW; gi++) {
      const uint4 vsr = cur.vs[gi];
      const uint32_t vw[4] = {vsr.x, vsr.y, vsr.z, vsr.w};
      half4_t bp;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float x = p[i] * lo16(vw[i]);
        const _Float16 xh = (_Float16)x;
        bp[i] = hi ? xh : (_Float16)(x - (float)xh);
        bacc[gi] = fmaf(p[i], hi16(vw[i]), bacc[gi]);
      }
#pragma unroll
      for (int ct = 0; ct < 4; ct++)
        o[gi * 4 + ct] = __builtin_amdgcn_mfma_f32_16x16x16f16(v_operand<BITS, GW>(cur, gi, ct),
                                                               bp, o[gi * 4 + ct], 0, 0, 0);
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

  __syncthreads();  // everyone is done reading q_rot out of qo
  if (hi && col_valid) {
#pragma unroll
    for (int gi = 0; gi < GW; gi++)
#pragma unroll
      for (int ct = 0; ct < 4; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int d = (wave * GW + gi) * 64 + ct * 16 + 4 * j + i;
          qo[head * D + d] = (o[gi * 4 + ct][i] + bacc[gi]) * a.signs[d];
        }
    if (wave == 0 && j == 0) {
      ml_s[head][0] = m_run;
      ml_s[head][1] = l_run;
    }
  }
  __syncthreads();
  lds_fwht<D, NT>(qo, G);

  const int64_t qh0 = (int64_t)seq * a.n_q_heads + (int64_t)kvh * G;
  if (a.direct) {
    for (int idx = tid; idx < G * D; idx += NT) {
      const int hh = idx / D;
      const float l = ml_s[hh][1];
      const float v = l > 0.0f ? (qo[idx] * a.c) / l : 0.0f;
      const int64_t o_idx = qh0 * D + idx;
      if (a.out_f32)
        reinterpret_cast<float*>(a.out)[o_idx] = v;
      else
        reinterpret_cast<uint16_t*>(a.out)[o_idx] = f32_to_bf16(v);
    }
  } else {
    const int64_t base = ((int64_t)seq * a.max_splits + split) * a.n_q_heads + (int64_t)kvh * G;
    for (int idx = tid; idx < G * D; idx += NT) a.part_o[base * D + idx] = qo[idx] * a.c;
    if (tid < G) {
      a.part_ml[(base + tid) * 2 + 0] = ml_s[tid][0];
      a.part_ml[(base + tid) * 2 + 1] = ml_s[tid][1];
    }
  }
}

// out[seq][h][d] = sum_s 2^(m_s - M) O_s[d] / sum_s 2^(m_s - M) l_s.
template <int D>
__global__ __launch_bounds__(64) void combine_kernel(AttnArgs a) {
  const int seq = blockIdx.z, h = blockIdx.y;
  const int d = blockIdx.x * 64 + threadIdx.x;
  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps, a.max_splits);
  const int64_t stride = (int64_t)a.n_q_heads;
  const int64_t base = (int64_t)seq * a.max_splits * stride + h;
  float M = -INFINITY;
  for (int s = 0; s < n_splits; s++) M = fmaxf(M, a.part_ml[(base + s * stride) * 2]);
  float num = 0.0f, den = 0.0f;
  if (M != -INFINITY) {
    for (int s = 0; s < n_splits; s++) {
      const int64_t r = base + s * stride;
      const float w = exp2f(a.part_ml[r * 2] - M);
      den = fmaf(w, a.part_ml[r * 2 + 1], den);
      num = fmaf(w, a.part_o[r * D + d], num);
    }
  }
  const float v = den > 0.0f ? num / den : 0.0f;
  const int64_t o_idx = ((int64_t)seq * a.n_q_heads + h) * D + d;
  if (a.out_f32)
    reinterpret_cast<float*>(a.out)[o_idx] = v;
  else
    reinterpret_cast<uint16_t*>(a.out)[o_idx] = f32_to_bf16(v);
}

template <int D, int BITS>
hipError_t launch_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                    hipEvent_t ev0, hipEvent_t ev1) {
  constexpr int DW = 128;
  constexpr int NT = (D / DW) * 64;
  dim3 grid(a.max_splits, n_kv_heads, n_seqs);
  if (ev0) (void)hipEventRecord(ev0, s);
  hipLaunchKernelGGL((decode_attn_kernel<D, BITS, DW>), grid, dim3(NT), 0, s, a);
  hipError_t e = hipGetLastError();
  if (ev1) (void)hipEventRecord(ev1, s);
  if (e != hipSuccess || a.direct) return e;
  dim3 cgrid(D / 64, a.n_q_heads, n_seqs);
  hipLaunchKernelGGL((combine_kernel<D>), cgrid, dim3(64), 0, s, a);
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

}  // namespace fmkv

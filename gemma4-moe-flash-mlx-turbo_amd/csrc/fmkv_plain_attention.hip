// Decode attention over plain (unquantized bf16) caches.
//
// Replaces mlx_rs::fast::scaled_dot_product_attention at decode
// (src/model/gemma4_attention.rs:94-103) over KVCacheInner::Plain
// (src/cache.rs:274-288): K and V are the stored bf16 rows, unrotated.
//
// One work-group of four waves per (KV head, sequence, split of consecutive
// 16-token blocks). Each wave owns a quarter of head_dim and loads its part
// of a head-block straight from HBM into registers, already in matrix-core
// lane order, one block ahead of its use:
//   K  slice k (32 dims), lane (jj, t): dims 32k + 8jj .. + 7 of token t,
//      16 bytes -- an A operand of v_mfma_f32_16x16x32_bf16;
//   V  tile ct (16 dims), lane (q, n): tokens 4q .. 4q + 3 of dim 16ct + n,
//      8 bytes (the dim-major V layout) -- an A operand of
//      v_mfma_f32_16x16x16_bf16.
// q enters the QK product as stored (bf16, exact; B-operand columns c and
// c + 8 both carry head c & 7), so S^T = K . q^T is exact up to the f32
// accumulation and the softmax scale (times log2 e) applies after it. The
// waves' partial scores meet in LDS and are summed in a fixed order; the
// base-2 online softmax is the affine kernel's; P enters the PV product as
// bf16 high (columns < 8) and residual (columns >= 8) parts, which keeps ~16
// bits of each weight. The epilogue writes the output (one split) or a split
// partial for the shared combine kernel.
#include <hip/hip_ext.h>

#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_prologue.h"
#include "fmkv_attn_common.h"

namespace fmkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kPlWaves = 4;
constexpr int kPlThreads = kPlWaves * 64;

template <int D>
struct PlainPlan {
  static constexpr BlockLayout L = make_layout(D, 16, kPlain);
  static constexpr int kSlicesW = D / 32 / kPlWaves;  // QK MFMAs per wave per block
  static constexpr int kTilesW = D / 16 / kPlWaves;   // PV MFMAs per wave per block
  static_assert(kSlicesW >= 1 && kTilesW >= 1, "head_dim split over four waves");
};

// One wave's operands of one head-block.
template <int D>
struct PlainOps {
  u32x4 k[PlainPlan<D>::kSlicesW];
  uint2 v[PlainPlan<D>::kTilesW];
};

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}

__device__ inline float bf16_value(float a) { return __uint_as_float((uint32_t)f32_to_bf16(a) << 16); }

// Decode step's new-token column (the grid's last split column): wave 0
// stores the step's K row, wave 1 its V row, at slot T - 1 (the rows as
// given: a plain cache stores them unchanged), and the token's attention
// goes out as one more partial: m = its base-2 score, l = 1, O = its V row.
// The split columns leave that slot out. With a.k_norm_w the layer's
// prologue runs on the raw projections first, as the append kernel runs it
// (K = RoPE(k_norm(k)), V = v_norm(v) rounded to bf16 for the store); the
// RoPE (cos, sin) table of position T - 1 is built by every thread into
// `rope` (LDS, rope_dims / 2 float2) behind one barrier. Every thread of
// the work-group calls it.
template <int D>
__device__ void plain_new_token_column(const AttnArgs& a, float2* rope, int64_t T, int n_splits,
                                       int kvh, int seq, int wave, int lane) {
#pragma clang fp contract(off)
  constexpr BlockLayout L = make_layout(D, 16, kPlain);
  constexpr int E = D / 64;
  const bool pro = a.k_norm_w != nullptr;
  if (pro) {
    if (T >= 1) {
      for (int j = wave * 64 + lane; j < (a.rope_dims >> 1); j += kPlThreads)
        rope[j] = rope_cos_sin(T - 1, rope_inv_freq(j, a.rope_dims, a.rope_theta));
    }
    __syncthreads();
  }
  if (wave >= 2) return;
  const bool isv = wave == 1;
  const int G = a.group, d0 = lane * E;
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
  const uint16_t* row = (isv ? a.v_new : a.k_new) + ((int64_t)seq * a.st.n_kv_heads + kvh) * D + d0;
  float x[E];
  load_row<E>(row, x);
  if (pro) {
    if (!isv) {
      float w[E];
      load_row<E>(a.k_norm_w + d0, w);
      k_norm_row<E>(x, w, a.eps, lane);
      rope_row<E>(x, a.rope_dims, lane, [&](int j) { return rope[j]; });
    } else {
      v_norm_row<E>(x, a.eps, lane);
    }
  }
  // the stored bf16 values (the rows as given, or the prologue's output
  // rounded to bf16: K is already, V is rounded here)
  uint16_t xb[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    xb[i] = pro ? f32_to_bf16(x[i]) : row[i];
    x[i] = bf16_to_f32(xb[i]);
  }
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
#pragma unroll
    for (int i = 0; i < E; i++)
      *reinterpret_cast<uint16_t*>(blk + (isv ? L.v_codes + plain_v_pos(t, d0 + i)
                                              : L.k_codes + plain_k_pos(D, t, d0 + i))) = xb[i];
  }
  if (!isv) {
    for (int h = 0; h < G; h++) {
      float qx[E];
      load_row<E>(a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G + h) * D + d0, qx);
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < E; i++) dot = fmaf(qx[i], x[i], dot);
      dot = group_sum<64>(dot, lane);
      if (lane == 0) {
        a.part_ml[(pbase + h) * 2 + 0] = dot * a.qscale;
        a.part_ml[(pbase + h) * 2 + 1] = 1.0f;
      }
    }
  } else {
    for (int h = 0; h < G; h++)
#pragma unroll
      for (int i = 0; i < E; i++) a.part_o[(pbase + h) * D + d0 + i] = x[i];
  }
}

// MODE: kDense, or the statistics (kStats: keys only, split (m, l) and block
// maxima) and gated (kGated) passes of sparse-V, as the affine kernel runs
// them.
template <int D, int MODE>
__global__ __launch_bounds__(kPlThreads) void plain_decode_kernel(AttnArgs a) {
  using P = PlainPlan<D>;
  constexpr BlockLayout L = P::L;
  constexpr int SW = P::kSlicesW, TW = P::kTilesW;
  constexpr int E = D / 64;
  __shared__ __align__(16) float4_t xch[2][kPlWaves][64];
  __shared__ __align__(16) float rows[8][D];
  __shared__ float ml_s[8][2];
  __shared__ float th_s[8];  // sparse-V gated pass: the group's thresholds

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane >> 4, c = lane & 15, head = c & 7;
  const bool hi_col = c < 8;
  const int G = a.group;
  const int kvh = blockIdx.x, seq = blockIdx.y, split = blockIdx.z;

  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps0, a.bps, a.max_splits, a.skew_p);
  if constexpr (MODE != kGated) {
    if (a.new_col && split == (int)gridDim.z - 1) {
      static_assert(sizeof(rows) >= D / 2 * sizeof(float2), "rope table fits the row area");
      plain_new_token_column<D>(a, reinterpret_cast<float2*>(rows), T, n_splits, kvh, seq, wave,
                                lane);
      return;
    }
  }
  if (split >= n_splits) return;
  int64_t b_begin, b_end;
  split_range(geo, split, a.bps0, a.bps, a.skew_p, a.skew_extra, &b_begin, &b_end);
  const int nb = (int)(b_end - b_begin);
  // sparse-V: this (sequence, KV head)'s row of block maxima; the gated pass
  // visits only the blocks holding a score at or above a head's threshold
  const int64_t blk_row =
      MODE == kDense ? 0 : ((int64_t)seq * a.st.n_kv_heads + kvh) * a.blk_stride;
  BlockList blist{0ull, 0, nb};
  int nbx = nb;  // blocks visited
  if constexpr (MODE == kGated) {
    gated_thresholds(a, n_splits, seq, kvh, G, split, wave, lane, th_s, kPlWaves);
    float thk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) thk[k] = k < G ? th_s[k] : INFINITY;
    blist = gated_block_list(a, thk, blk_row, geo.blk_lo, b_begin, 1, nb, T, lane, &nbx);
  }
  BlockList bcopy = blist;  // the loads run one block ahead on the same list

  const int32_t* table =
      a.st.block_table ? a.st.block_table + (int64_t)seq * a.st.table_stride : nullptr;
  const uint8_t* hbase = a.st.base + (int64_t)kvh * a.st.head_stride;
  auto blk_ptr = [&](int64_t lb) -> const uint8_t* {
    int64_t phys = table ? (int64_t)table[lb] : lb;
    // a bad table entry reads a valid block rather than faulting
    phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
    return hbase + phys * a.st.block_stride;
  };
  // this lane's operand offsets inside a head-block
  const int k_off = (int)L.k_codes + (c * D + wave * SW * 32 + 8 * j) * 2;         // t = c, jj = j
  const int v_off = (int)L.v_codes + ((wave * TW * 16 + c) * kBlockTokens + 4 * j) * 2;  // n = c, q = j
  auto load_ops = [&](int64_t lb, PlainOps<D>& o) {
    const uint8_t* p = blk_ptr(lb);
#pragma unroll
    for (int s = 0; s < SW; s++) o.k[s] = *reinterpret_cast<const u32x4*>(p + k_off + s * 64);
    if constexpr (MODE != kStats) {
#pragma unroll
      for (int t = 0; t < TW; t++)
        o.v[t] = *reinterpret_cast<const uint2*>(p + v_off + t * 16 * kBlockTokens * 2);
    }
  };
  PlainOps<D> nxt;
  if (nbx > 0) load_ops(b_begin + (MODE == kGated ? bcopy.pop() : 0), nxt);

  // B operands: q of head c & 7 as stored, dims 32k + 8j .. + 7 of this
  // wave's slices (zero past the group)
  u32x4 bq[SW];
  {
    const uint16_t* qh = a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G + head) * D;
#pragma unroll
    for (int s = 0; s < SW; s++)
      bq[s] = head < G ? *reinterpret_cast<const u32x4*>(qh + (wave * SW + s) * 32 + 8 * j)
                       : (u32x4){0u, 0u, 0u, 0u};
  }

  // visible slots: linear [vis_lo, vis_hi); ring [0, min(T, W)), unless a
  // trim hides older positions (then each slot's position is computed)
  const int64_t vis_lo = a.window > 0 ? 0 : a.vis_begin;
  const int64_t vis_hi = a.window > 0 ? (T < a.window ? T : a.window) : T;
  const bool ring_trim = a.window > 0 && a.vis_begin > T - a.window;
  // a decode step's new token is the new-token column's
  int64_t ex_slot = -1;
  if (a.new_col && T > 0) ex_slot = a.window > 0 ? (T - 1) % a.window : T - 1;

  // sparse-V: this column's score threshold
  float theta = -INFINITY;
  if constexpr (MODE == kGated) theta = head < G ? th_s[head] : -INFINITY;

  float4_t o[TW];
#pragma unroll
  for (int t = 0; t < TW; t++) o[t] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.0f;

  for (int i = 0; i < nbx; i++) {
    const int64_t b = b_begin + (MODE == kGated ? blist.pop() : i);
    const PlainOps<D> cur = nxt;
    if (i + 1 < nbx) load_ops(b_begin + (MODE == kGated ? bcopy.pop() : i + 1), nxt);

    // -- this wave's quarter of S^T, summed over the waves in wave order --
    float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SW; s++)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, cur.k[s]),
                                                    __builtin_bit_cast(bf16x8_t, bq[s]), acc, 0, 0, 0);
    const int par = i & 1;
    xch[par][wave][lane] = acc;
    __syncthreads();
    float4_t st = xch[par][0][lane];
#pragma unroll
    for (int w = 1; w < kPlWaves; w++) st += xch[par][w][lane];

    float s4[4];
#pragma unroll
    for (int r = 0; r < 4; r++) s4[r] = head < G ? st[r] * a.qscale : -INFINITY;
    // visibility: whole block in the common case, per token at the edges
    const int64_t t0 = b * kBlockTokens;
    const bool full = t0 >= vis_lo && t0 + kBlockTokens <= vis_hi && !ring_trim &&
                      (uint64_t)(ex_slot - t0) >= (uint64_t)kBlockTokens;
    if (!full) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t slot = t0 + 4 * j + r;
        bool vis = slot >= vis_lo && slot < vis_hi && slot != ex_slot;
        if (ring_trim) vis = vis && slot_position(slot, T, a.window) >= a.vis_begin;
        if (!vis) s4[r] = -INFINITY;
      }
    }
    if constexpr (MODE == kGated) {
#pragma unroll
      for (int r = 0; r < 4; r++) s4[r] = s4[r] >= theta ? s4[r] : -INFINITY;
    }
    // -- online softmax in base 2 (as the affine kernel) --
    float mb = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    if constexpr (MODE == kStats) {
      // the block's largest score per head, for the gated pass's block skip
      // (every wave holds the same scores; wave 0 writes them)
      const int64_t rb = b - geo.blk_lo;
      if (wave == 0 && j == 0 && hi_col && rb < a.blk_stride)
        a.blk_max[blk_max_at(a, blk_row, rb, head)] = head < G ? mb : -INFINITY;
    }
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run + kRescaleSlack)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      if (__any(l_run > 0.0f)) {
#pragma unroll
        for (int t = 0; t < TW; t++) o[t] *= alpha;
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = __builtin_amdgcn_exp2f(s4[r] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
    if constexpr (MODE == kStats) {
      store_block_scores(a, blk_row, b - geo.blk_lo, head, j, s4, mb, m_run, log2f(a.tau),
                         wave == 0 && hi_col && head < G);
      continue;
    }
    // sparse-V: a block whose weights are all below tau adds nothing to O
    // (every wave holds the same scores: a uniform branch)
    if constexpr (MODE == kGated) {
      if (!__any((p[0] + p[1]) + (p[2] + p[3]) > 0.0f)) continue;
    }

    // -- O^T += V^T . P^T, P as bf16 high (c < 8) / residual (c >= 8) --
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; r++) x[r] = hi_col ? p[r] : p[r] - bf16_value(p[r]);
    const short4_t bp = __builtin_bit_cast(
        short4_t, make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])));
#pragma unroll
    for (int t = 0; t < TW; t++)
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, cur.v[t]), bp,
                                                       o[t], 0, 0, 0);
  }

  // ---- epilogue: rows [head][D] in LDS, then store ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
  if constexpr (MODE == kStats) {
    // the split's softmax statistics per head (every wave holds them)
    if (wave == 0 && j == 0 && hi_col && head < G) {
      const int64_t r = ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G + head;
      a.part_ml[r * 2 + 0] = m_run;
      a.part_ml[r * 2 + 1] = l_run;
      if (split == 0 && a.sv_count) a.sv_count[(int64_t)seq * a.n_q_heads + (int64_t)kvh * G + head] = 0;
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < TW; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) o[t][r] = o[t][r] + row_ror8(o[t][r]);
  if (hi_col) {
#pragma unroll
    for (int t = 0; t < TW; t++)
      *reinterpret_cast<float4_t*>(&rows[head][(wave * TW + t) * 16 + 4 * j]) = o[t];
    // every wave holds the same softmax state; wave 0 publishes it per head
    if (wave == 0 && j == 0) {
      ml_s[head][0] = m_run;
      ml_s[head][1] = l_run;
    }
  }
  __syncthreads();
  const int64_t qh0 = (int64_t)seq * a.n_q_heads + (int64_t)kvh * G;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int hh = wave + 4 * r;
    if (hh >= G) continue;
    const float Mh = ml_s[hh][0], Lh = ml_s[hh][1];
    if (a.direct) {
      const int64_t o_idx = (qh0 + hh) * D + lane * E;
#pragma unroll
      for (int e = 0; e < E; e++) {
        const float v = Lh > 0.0f ? rows[hh][lane * E + e] / Lh : 0.0f;
        if (a.out_f32)
          reinterpret_cast<float*>(a.out)[o_idx + e] = v;
        else
          reinterpret_cast<uint16_t*>(a.out)[o_idx + e] = f32_to_bf16(v);
      }
    } else {
      const int64_t pb = ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G + hh;
#pragma unroll
      for (int e = 0; e < E; e++) a.part_o[pb * D + lane * E + e] = rows[hh][lane * E + e];
      if (lane == 0) {
        a.part_ml[pb * 2 + 0] = Mh;
        a.part_ml[pb * 2 + 1] = Lh;
      }
    }
  }
}

template <int D, int MODE>
hipError_t launch_plain_mode(const AttnArgs& a, dim3 grid, hipStream_t s, hipEvent_t ev0,
                             hipEvent_t ev1) {
  if (ev0 && ev1)
    hipExtLaunchKernelGGL((plain_decode_kernel<D, MODE>), grid, dim3(kPlThreads), 0, s, ev0, ev1,
                          0, a);
  else
    hipLaunchKernelGGL((plain_decode_kernel<D, MODE>), grid, dim3(kPlThreads), 0, s, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_plain_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                          hipEvent_t ev0, hipEvent_t ev1) {
  dim3 grid(n_kv_heads, n_seqs, a.max_splits + a.new_col);
  hipError_t e;
  if (a.tau > 0.0f) {
    // sparse-V as the affine kernel runs it: the stats pass (its statistics
    // in stat_ml; with a decode step's new-token column, which stores the
    // token), the gated pass over every stored token, the combine
    AttnArgs st = a;
    st.part_ml = a.stat_ml;
    if (!st.part_ml) return hipErrorInvalidValue;
    if (a.blk_scores) {
      // the gather in place of the gated pass and the combine (the stats
      // pass stored the candidate blocks' scores and zeroed the counters)
      if ((e = launch_plain_mode<D, kStats>(st, grid, s, ev0, ev1)) != hipSuccess) return e;
      AttnArgs g = a;
      g.stats_new_col = a.new_col;
      return launch_sparse_gather(g, n_seqs, s);
    }
    if ((e = launch_plain_mode<D, kStats>(st, grid, s, nullptr, nullptr)) != hipSuccess) return e;
    AttnArgs g = a;
    g.new_col = 0;
    g.stats_new_col = a.new_col;
    if ((e = launch_plain_mode<D, kGated>(g, dim3(n_kv_heads, n_seqs, a.max_splits), s, ev0,
                                          ev1)) != hipSuccess)
      return e;
    return a.direct ? hipSuccess : launch_combine(g, n_seqs, s);
  }
  e = launch_plain_mode<D, kDense>(a, grid, s, ev0, ev1);
  if (e != hipSuccess || a.direct) return e;
  return launch_combine(a, n_seqs, s);
}

}  // namespace

hipError_t launch_plain_decode_attention(const AttnArgs& a, int n_seqs, int n_kv_heads,
                                         hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
  if (a.new_col && (!a.k_new || !a.v_new)) return hipErrorInvalidValue;
  switch (a.st.layout.head_dim) {
    case 128: return launch_plain_t<128>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 256: return launch_plain_t<256>(a, n_seqs, n_kv_heads, s, e0, e1);
    case 512: return launch_plain_t<512>(a, n_seqs, n_kv_heads, s, e0, e1);
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

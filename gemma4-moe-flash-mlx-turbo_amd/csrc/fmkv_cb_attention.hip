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
// One work-group of four waves per (KV head, sequence, split of consecutive
// 16-token blocks). Per block the waves:
//  1. dequantize the block from its LDS copy into f16 matrix-core operand
//     tiles of centroid high and residual parts (a product then keeps ~22
//     bits of the centroid; one f16 alone is off by up to 2^-12 of the
//     value), V laid out for v_mfma_f32_16x16x16f16 with the tokens as the
//     reduction dimension;
//  2. compute S^T = K . q_rot^T on v_mfma_f32_16x16x32_f16, each wave a
//     quarter of head_dim, summed through LDS in a fixed order;
//  3. run the same base-2 online softmax as the affine kernel;
//  4. accumulate O^T += V^T . P'^T with P' = p * norm / sqrt D split into f16
//     high and residual columns, each wave a quarter of head_dim.
// The block's raw bytes for the next block are loaded into registers while
// the current one is processed. The epilogue applies R^T and writes the final
// output (one split) or a split partial for the shared combine kernel.
#include <hip/hip_ext.h>

#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_attn_common.h"

namespace fmkv {
namespace {

// src/cache.rs:67-89 centroids (the same literals as the append's tables).
__constant__ float kCbCent2[4] = {-1.510f, -0.453f, 0.453f, 1.510f};
__constant__ float kCbCent3[8] = {-2.152f, -1.344f, -0.756f, -0.245f, 0.245f, 0.756f, 1.344f, 2.152f};
__constant__ float kCbCent4[16] = {-2.733f, -2.069f, -1.618f, -1.256f, -0.942f, -0.657f,
                                   -0.388f, -0.128f, 0.128f,  0.388f,  0.657f,  0.942f,
                                   1.256f,  1.618f,  2.069f,  2.733f};

constexpr int kCbWaves = 4;
constexpr int kCbThreads = kCbWaves * 64;

template <int D, int BITS>
struct CbPlan {
  static constexpr BlockLayout L = make_layout(D, BITS, kCodebook);
  static constexpr int kRow = D * BITS / 8;               // code bytes of one token row
  static constexpr int kSlices = D / 32;                  // QK MFMAs (32 dims each)
  static constexpr int kTiles = D / 16;                   // PV column tiles (16 dims each)
  static constexpr int kRawChunks = (int)(L.block_bytes / 16);  // the whole head-block
  static constexpr int kLoads = (kRawChunks + kCbThreads - 1) / kCbThreads;  // 16-B loads per thread
  static_assert(kSlices % kCbWaves == 0 && kTiles % kCbWaves == 0, "head_dim split over four waves");
  static constexpr int kSlicesW = kSlices / kCbWaves;
  static constexpr int kTilesW = kTiles / kCbWaves;
  // LDS: q operand table (later the V residual tile), K high / residual
  // tiles, V high tile, raw block, score exchange
  static constexpr int kQTab = kSlices * 1024;
  static constexpr int kKTile = kSlices * 1024;
  static constexpr int kVTile = kTiles * 512;
  static_assert(kVTile <= kQTab, "the V residual tile reuses the q table");
  static constexpr int kXch = kCbWaves * 64 * 16;
};

// Codes of 8 consecutive dims of one row: bits [bit0, bit0 + 8 BITS) of the
// row's little-endian bit stream (index j at bit j * BITS), row 4-byte
// aligned in LDS.
template <int BITS>
__device__ inline uint64_t codes8(const uint8_t* row, int bit0) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + (bit0 >> 5);
  uint64_t v = (uint64_t)w[0];
  if ((bit0 & 31) + 8 * BITS > 32) v |= (uint64_t)w[1] << 32;
  return v >> (bit0 & 31);
}

// The code of one dim (bits [bit, bit + BITS) of a row's bit stream).
template <int BITS>
__device__ inline uint32_t code1(const uint8_t* row, int bit) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + (bit >> 5);
  uint32_t v = w[0] >> (bit & 31);
  if ((bit & 31) + BITS > 32) v |= w[1] << (32 - (bit & 31));
  return v & ((1u << BITS) - 1u);
}

template <int D, int BITS>
__global__ __launch_bounds__(kCbThreads) void cb_decode_kernel(AttnArgs a) {
  using P = CbPlan<D, BITS>;
  constexpr BlockLayout L = P::L;
  constexpr int E = D / 64;  // dims per lane in a row-wise (FWHT) layout
  constexpr int NC = 1 << BITS;
  __shared__ __align__(16) uint8_t qtab[P::kQTab];
  __shared__ __align__(16) uint8_t khi[P::kKTile];
  __shared__ __align__(16) uint8_t klo[P::kKTile];
  __shared__ __align__(16) uint8_t vt[P::kVTile];
  uint8_t* const vlo = qtab;  // once each wave holds its q operands
  __shared__ __align__(16) uint8_t raw[P::kLoads * kCbThreads * 16];
  __shared__ __align__(16) float4_t xch[kCbWaves][64];
  __shared__ uint32_t lut[NC];  // centroid as {f16 high, f16 residual}
  __shared__ float ml_s[8][2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane >> 4, c = lane & 15, head = c & 7;
  const bool hi_col = c < 8;
  const int G = a.group;
  const int kvh = blockIdx.x, seq = blockIdx.y, split = blockIdx.z;

  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps0, a.bps, a.max_splits);
  if (split >= n_splits) return;
  const int64_t b_begin = geo.blk_lo + (split == 0 ? 0 : a.bps0 + (int64_t)(split - 1) * a.bps);
  int64_t b_end = b_begin + (split == 0 ? a.bps0 : a.bps);
  if (b_end > geo.blk_hi) b_end = geo.blk_hi;
  const int nb = (int)(b_end - b_begin);

  const int32_t* table =
      a.st.block_table ? a.st.block_table + (int64_t)seq * a.st.table_stride : nullptr;
  const uint8_t* hbase = a.st.base + (int64_t)kvh * a.st.head_stride;
  auto blk_ptr = [&](int64_t lb) -> const uint8_t* {
    int64_t phys = table ? (int64_t)table[lb] : lb;
    // a bad table entry reads a valid block rather than faulting
    phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
    return hbase + phys * a.st.block_stride;
  };
  // the raw block in 16-byte pieces, kLoads per thread (past the block: zero)
  u32x4 pre[P::kLoads];
  auto load_raw = [&](int64_t lb) {
    const uint8_t* p = blk_ptr(lb);
#pragma unroll
    for (int k = 0; k < P::kLoads; k++) {
      const int ch = k * kCbThreads + tid;
      pre[k] = ch * 16 < (int)L.block_bytes ? *reinterpret_cast<const u32x4*>(p + ch * 16)
                                            : (u32x4){0u, 0u, 0u, 0u};
    }
  };
  auto store_raw = [&]() {
#pragma unroll
    for (int k = 0; k < P::kLoads; k++)
      *reinterpret_cast<u32x4*>(raw + (k * kCbThreads + tid) * 16) = pre[k];
  };
  if (nb > 0) load_raw(b_begin);

  // ---- prologue: centroid table, q_rot as QK B operands ----
  if (tid < NC) {
    const float cv = BITS == 2 ? kCbCent2[tid] : BITS == 3 ? kCbCent3[tid] : kCbCent4[tid];
    const _Float16 h = (_Float16)cv;
    const _Float16 r = (_Float16)(cv - (float)h);
    lut[tid] = (uint32_t)__builtin_bit_cast(uint16_t, h) |
               ((uint32_t)__builtin_bit_cast(uint16_t, r) << 16);
  }
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  // wave w rotates q heads w and w + 4: q_rot = (FWHT(q * qscale) * c) o s;
  // lane l holds dims l E .. l E + E - 1, which in the operand table are
  // slice k = l E / 32, k-group (l E % 32) / 8, element (l E) % 8
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int h = wave + 4 * r;
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = 0.0f;
    if (h < G) {
      const uint16_t* qh = a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G + h) * D + lane * E;
      load_row<E>(qh, x);
#pragma unroll
      for (int i = 0; i < E; i++) x[i] *= a.qscale;
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
    const int d0 = lane * E, k = d0 >> 5, jj = (d0 & 31) >> 3, i0 = d0 & 7;
    uint8_t* ent = qtab + k * 1024 + i0 * 2;
    store_halves<E>(ent + (jj * 16 + h) * 16, hv);
    store_halves<E>(ent + (jj * 16 + h + 8) * 16, lv);
  }

  __syncthreads();
  // this wave's B operands (its quarter of head_dim); the table's memory then
  // holds the V residual tile
  half8_t bq[P::kSlicesW];
#pragma unroll
  for (int s = 0; s < P::kSlicesW; s++)
    bq[s] = *reinterpret_cast<const half8_t*>(qtab + (wave * P::kSlicesW + s) * 1024 + lane * 16);

  // visible slots: linear [vis_lo, vis_hi); ring [0, min(T, W)), unless a
  // trim hides older positions (then each slot's position is computed)
  const int64_t vis_lo = a.window > 0 ? 0 : a.vis_begin;
  const int64_t vis_hi = a.window > 0 ? (T < a.window ? T : a.window) : T;
  const bool ring_trim = a.window > 0 && a.vis_begin > T - a.window;

  float4_t o[P::kTilesW];
#pragma unroll
  for (int i = 0; i < P::kTilesW; i++) o[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f, l_run = 0.0f;
  const float lo_sel = hi_col ? 0.0f : 1.0f;
  const float inv_sd = a.c;  // 1 / sqrt(D): the codebook's value scale

  for (int i = 0; i < nb; i++) {
    const int64_t b = b_begin + i;
    __syncthreads();  // the tiles of the previous block are consumed (and the table written)
    store_raw();
    if (i + 1 < nb) load_raw(b + 1);
    __syncthreads();

    // -- dequantize: K tiles (slice k, lane (jj, t): dims 32k + 8jj .. + 7 of
    // token t) and the V tile (column tile ct, lane (q, n): dim 16ct + n of
    // tokens 4q .. 4q + 3, as 4 halves) --
    const uint8_t* kraw = raw + L.k_codes;
    const uint8_t* vraw = raw + L.v_codes;
#pragma unroll
    for (int it = 0; it < P::kSlices * 64 / kCbThreads; it++) {
      const int item = it * kCbThreads + tid;
      const int k = item >> 6, ln = item & 63, jj = ln >> 4, t = ln & 15;
      const uint64_t cw = codes8<BITS>(kraw + t * P::kRow, (32 * k + 8 * jj) * BITS);
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t a0 = lut[(cw >> (2 * e * BITS)) & (NC - 1)];
        const uint32_t a1 = lut[(cw >> ((2 * e + 1) * BITS)) & (NC - 1)];
        hw[e] = (a0 & 0xffffu) | (a1 << 16);
        lw[e] = (a0 >> 16) | (a1 & 0xffff0000u);
      }
      *reinterpret_cast<u32x4*>(khi + k * 1024 + ln * 16) = (u32x4){hw[0], hw[1], hw[2], hw[3]};
      *reinterpret_cast<u32x4*>(klo + k * 1024 + ln * 16) = (u32x4){lw[0], lw[1], lw[2], lw[3]};
    }
#pragma unroll
    for (int it = 0; it < P::kTiles * 64 / kCbThreads; it++) {
      const int item = it * kCbThreads + tid;
      const int ct = item >> 6, ln = item & 63, q4 = ln >> 4, n = ln & 15;
      const int d = ct * 16 + n;
      uint32_t h4[2], l4[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const uint8_t* r0 = vraw + (4 * q4 + r) * P::kRow;
        const uint32_t a0 = lut[code1<BITS>(r0, d * BITS)];
        const uint32_t a1 = lut[code1<BITS>(r0 + P::kRow, d * BITS)];
        h4[r >> 1] = (a0 & 0xffffu) | (a1 << 16);
        l4[r >> 1] = (a0 >> 16) | (a1 & 0xffff0000u);
      }
      *reinterpret_cast<uint2*>(vt + ct * 512 + ln * 8) = make_uint2(h4[0], h4[1]);
      *reinterpret_cast<uint2*>(vlo + ct * 512 + ln * 8) = make_uint2(l4[0], l4[1]);
    }
    __syncthreads();

    // -- S^T over this wave's quarter of head_dim, summed over the waves --
    float4_t acc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < P::kSlicesW; s++) {
      const int k = wave * P::kSlicesW + s;
      const half8_t ah = *reinterpret_cast<const half8_t*>(khi + k * 1024 + lane * 16);
      const half8_t al = *reinterpret_cast<const half8_t*>(klo + k * 1024 + lane * 16);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[s], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[s], acc, 0, 0, 0);
    }
    xch[wave][lane] = acc;
    __syncthreads();
    float4_t st = xch[0][lane];
#pragma unroll
    for (int w = 1; w < kCbWaves; w++) st += xch[w][lane];
    // per-token value scale norm / sqrt D (f16 norms follow the codes)
    const uint2 kn = *reinterpret_cast<const uint2*>(raw + L.k_meta + 8 * j);
    const uint2 vn = *reinterpret_cast<const uint2*>(raw + L.v_meta + 8 * j);
    const float kscale[4] = {lo16(kn.x) * inv_sd, hi16(kn.x) * inv_sd, lo16(kn.y) * inv_sd,
                             hi16(kn.y) * inv_sd};
    const float vscale[4] = {lo16(vn.x) * inv_sd, hi16(vn.x) * inv_sd, lo16(vn.y) * inv_sd,
                             hi16(vn.y) * inv_sd};
    float s4[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float tv = st[r] + row_ror8(st[r]);  // high + residual columns of q
      s4[r] = (G > head) ? tv * kscale[r] : -INFINITY;
    }
    // visibility: whole block in the common case, per token at the edges
    const int64_t t0 = b * kBlockTokens;
    const bool full = t0 >= vis_lo && t0 + kBlockTokens <= vis_hi && !ring_trim;
    if (!full) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t slot = t0 + 4 * j + r;
        bool vis = slot >= vis_lo && slot < vis_hi;
        if (ring_trim) vis = vis && slot_position(slot, T, a.window) >= a.vis_begin;
        if (!vis) s4[r] = -INFINITY;
      }
    }
    // -- online softmax in base 2 (as the affine kernel) --
    float mb = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3]));
    mb = xor16_max(mb);
    mb = xor32_max(mb);
    const float m_new = fmaxf(m_run, mb);
    if (__any(m_new > m_run + kRescaleSlack)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      if (__any(l_run > 0.0f)) {
#pragma unroll
        for (int tI = 0; tI < P::kTilesW; tI++) o[tI] *= alpha;
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = __builtin_amdgcn_exp2f(s4[r] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
    // -- O^T += V^T . P'^T, P' = p * norm / sqrt D as f16 high / residual columns --
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; r++) x[r] = p[r] * vscale[r];
    const half2_t h01 = pkrtz(x[0], x[1]);
    const half2_t h23 = pkrtz(x[2], x[3]);
    const half2_t b01 = pkrtz(fmaf(-lo_sel, (float)h01[0], x[0]), fmaf(-lo_sel, (float)h01[1], x[1]));
    const half2_t b23 = pkrtz(fmaf(-lo_sel, (float)h23[0], x[2]), fmaf(-lo_sel, (float)h23[1], x[3]));
    const half4_t bp = cat4(b01, b23);
#pragma unroll
    for (int tI = 0; tI < P::kTilesW; tI++) {
      const int ct = wave * P::kTilesW + tI;
      const half4_t av = *reinterpret_cast<const half4_t*>(vt + ct * 512 + lane * 8);
      const half4_t al = *reinterpret_cast<const half4_t*>(vlo + ct * 512 + lane * 8);
      o[tI] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bp, o[tI], 0, 0, 0);
      o[tI] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bp, o[tI], 0, 0, 0);
    }
  }

  // ---- epilogue: rows [head][D] in LDS, inverse rotation, store ----
  l_run = xor16_sum(l_run);
  l_run = xor32_sum(l_run);
  __syncthreads();  // every wave is done with the tiles
  float* rows = reinterpret_cast<float*>(khi);  // [8][D] f32
  static_assert(P::kKTile >= 8 * D * 4, "epilogue rows fit in the K tile");
#pragma unroll
  for (int tI = 0; tI < P::kTilesW; tI++)
#pragma unroll
    for (int r = 0; r < 4; r++) o[tI][r] = o[tI][r] + row_ror8(o[tI][r]);
  if (hi_col) {
#pragma unroll
    for (int tI = 0; tI < P::kTilesW; tI++) {
      const int ct = wave * P::kTilesW + tI;
      *reinterpret_cast<float4_t*>(&rows[head * D + ct * 16 + 4 * j]) = o[tI];
    }
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
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = apply_sign(rows[hh * D + lane * E + i], sbits, i);
    wave_fwht_signed<E>(x, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
    const float Mh = ml_s[hh][0], Lh = ml_s[hh][1];
    if (a.direct) {
      const int64_t o_idx = (qh0 + hh) * D + lane * E;
#pragma unroll
      for (int i = 0; i < E; i++) {
        const float v = Lh > 0.0f ? (x[i] * cs) / Lh : 0.0f;
        if (a.out_f32)
          reinterpret_cast<float*>(a.out)[o_idx + i] = v;
        else
          reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
      }
    } else {
      const int64_t pb = ((int64_t)seq * a.part_stride + split) * a.n_q_heads + (int64_t)kvh * G + hh;
#pragma unroll
      for (int i = 0; i < E; i++) a.part_o[pb * D + lane * E + i] = x[i] * cs;
      if (lane == 0) {
        a.part_ml[pb * 2 + 0] = Mh;
        a.part_ml[pb * 2 + 1] = Lh;
      }
    }
  }
}

template <int D, int BITS>
hipError_t launch_cb_t(const AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s, hipEvent_t ev0,
                       hipEvent_t ev1) {
  dim3 grid(n_kv_heads, n_seqs, a.max_splits);
  if (ev0 && ev1)
    hipExtLaunchKernelGGL((cb_decode_kernel<D, BITS>), grid, dim3(kCbThreads), 0, s, ev0, ev1, 0, a);
  else
    hipLaunchKernelGGL((cb_decode_kernel<D, BITS>), grid, dim3(kCbThreads), 0, s, a);
  hipError_t e = hipGetLastError();
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

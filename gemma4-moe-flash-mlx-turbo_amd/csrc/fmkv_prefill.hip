// Prefill (chunked) attention over the quantized cache (affine mode).
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
// Per block (16 keys), per 64-dim group g of the wave's half:
//   QK^T  S^T[16 key x 16 row] += K[16 x 32] . Q^T[32 x 16] with K codes as
//         exact f16 integers, q_rot as an f16 high part and an f16 residual
//         (~22 bits), each in its own accumulator; then
//         s += scale * (acc_hi + acc_lo) + bias * sum(q_group). (The decode
//         kernel's 1024 + code operands, one v_perm per two codes, left the
//         residual's contribution on top of a large partial sum here: the
//         worst output error of a 1500-key test rose ~4x; the plain codes
//         cost one packed subtract more per two codes.)
//   PV    O^T[16 dim x 16 row] += V^T[16 dim x 16 key] . P'^T[16 key x 16 row]
//         with P' = p * v_scale as f16 high part + residual (two MFMAs);
//         the bias terms are summed on the side.
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

namespace fmkv {
namespace {

constexpr int kPfWaves = 8;   // four pairs
constexpr int kPfRows = 64;   // query rows per work-group (16 per pair)
constexpr int kPfStages = 3;

template <int D, int BITS>
struct PfPlan {
  static constexpr BlockLayout L = make_layout(D, BITS, kAffine);
  static constexpr int NG = D / 64;
  static constexpr int GH = NG / 2;  // groups per wave
  // a head-block's codes and scale/bias: [K codes][V codes][K meta][V meta]
  static constexpr int kBytes = (int)(2 * L.code_bytes) + 2 * NG * 64;
  static constexpr int kNC = (kBytes + kChunk - 1) / kChunk;
  static constexpr int CP = (kNC + kPfWaves - 1) / kPfWaves;  // copies per wave per block
  static constexpr int kStageBytes = kPfWaves * CP * kChunk;
  static constexpr int kQStride = D + 8;  // f16 per q-table row (padding against bank conflicts)
  static constexpr int kQTab = 2 * kPfRows * kQStride * 2 + kPfRows * NG * 4;
  static constexpr int kRStride = D + 4;  // f32 per output row
  static constexpr int kRows = kPfRows * kRStride * 4;
  static constexpr int kRegion = cmax(cmax(kPfStages * kStageBytes, kQTab), kRows);
  static_assert((int)L.k_meta == (int)(2 * L.code_bytes) && (int)L.v_meta == (int)L.k_meta + NG * 64,
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

template <int D, int BITS>
__global__ __launch_bounds__(kPfWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_attn_kernel(PrefillArgs a) {
  using P = PfPlan<D, BITS>;
  constexpr BlockLayout L = P::L;
  constexpr int NG = P::NG, GH = P::GH, E = D / 64, LPG = 64 / E;
  constexpr int CP = P::CP, NST = kPfStages, SB = P::kStageBytes;
  constexpr int QS = P::kQStride, RS = P::kRStride;

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
  // virtual block i: absolute block, valid key range [vlo, vhi), store
  struct VB {
    int64_t b, vlo, vhi;
    const uint8_t* ptr;
  };
  auto vb_of = [&](int i) -> VB {
    VB v;
    if (i < n_old) {
      v.b = b_lo + i;
      v.vlo = v.b * kBlockTokens;
      v.vhi = (v.b + 1) * kBlockTokens < ps ? (v.b + 1) * kBlockTokens : ps;
      int64_t phys = v.b;
      if (a.window > 0) phys = v.b % (a.window / kBlockTokens);
      v.ptr = a.old_st.base + phys * a.old_st.block_stride + (int64_t)kvh * a.old_st.head_stride;
    } else {
      v.b = new_first + (i - n_old);
      v.vlo = v.b * kBlockTokens > ps ? v.b * kBlockTokens : ps;
      v.vhi = (v.b + 1) * kBlockTokens;
      int64_t phys = v.b - a.new_blk0;
      if (table) {
        // a table entry outside the pool (or a position past the table's
        // width) reads a valid block rather than faulting
        phys = v.b < a.new_st.table_stride ? (int64_t)table[v.b] : 0;
        phys = phys < 0 ? 0 : (phys >= a.new_st.n_blocks ? a.new_st.n_blocks - 1 : phys);
      }
      v.ptr = a.new_st.base + phys * a.new_st.block_stride + (int64_t)kvh * a.new_st.head_stride;
    }
    return v;
  };

  // ---- q_rot of the 64 rows: rows wave + 8 k, high / residual halves ----
  _Float16* const qhi = reinterpret_cast<_Float16*>(region);
  _Float16* const qlo = qhi + kPfRows * QS;
  float* const qsum = reinterpret_cast<float*>(qlo + kPfRows * QS);  // [row][NG]
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  const float cs_lane = fwht_lane_sign(lane) * a.c;
  if (lane == 0) xflag[wave] = 0;
#pragma unroll 1
  for (int k = 0; k < kPfRows / kPfWaves; k++) {
    const int r = wave + kPfWaves * k;
    const int rq_ = r / G, rh_ = r - (r / G) * G;
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
    if ((lane & (LPG - 1)) == 0) qsum[r * NG + ((lane * E) >> 6)] = gs;
  }
  __syncthreads();

  // this wave's B operands: its pair's 16 rows, its groups; the lane (j, c)
  // holds 8 consecutive dims of row `row` at the K-code placement
  half8_t bqh[GH][2], bql[GH][2];
  float qs[GH];
#pragma unroll
  for (int gi = 0; gi < GH; gi++) {
    const int g = g0 + gi;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int d0 = g * 64 + (BITS == 8 ? j * 16 + s * 8 : s * 32 + j * 8);
      bqh[gi][s] = *reinterpret_cast<const half8_t*>(qhi + row * QS + d0);
      bql[gi][s] = *reinterpret_cast<const half8_t*>(qlo + row * QS + d0);
    }
    qs[gi] = qsum[row * NG + g];
  }
  __syncthreads();  // the table is consumed: the region becomes the stages

  // ---- copies ----
  const uint32_t stage_lds = lds_addr(region);
  auto copy_vb = [&](int st, int i) {
    const VB v = vb_of(i);
    const u32x4 rs = buffer_rsrc(v.ptr, (uint32_t)P::kBytes);
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

  auto process = [&](const uint8_t* sp, const VB& v, int it) {
    float4_t sv = (float4_t){0.f, 0.f, 0.f, 0.f};
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
      float4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, bqh[gi][0], z, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, bqh[gi][1], acc, 0, 0, 0);
      float4_t acl = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, bql[gi][0], z, 0, 0, 0);
      acl = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, bql[gi][1], acl, 0, 0, 0);
      acc = acc + acl;
#pragma unroll
      for (int i = 0; i < 4; i++)
        sv[i] = fmaf(lo16(km_g[i]), acc[i], fmaf(hi16(km_g[i]), qs[gi], sv[i]));
      __builtin_amdgcn_sched_barrier(0);
    }
    u32x4 vw = codes(sp, (int)L.v_codes, 0), vm = vmeta(sp, 0);

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

    // masks: the whole block for all rows of the pair in the common case
    const int64_t t0 = v.b * kBlockTokens;
    const bool full = pair_full_rows && v.vlo == t0 && v.vhi == t0 + kBlockTokens &&
                      t0 >= pair_lo_max && t0 + kBlockTokens - 1 <= pA;
    if (!full) {
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
          if constexpr (kBiasedCodes<BITS>) psum[gi] *= alpha;
        }
      }
      l_run *= alpha;
      m_run = m_new;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

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
      __builtin_amdgcn_sched_barrier(0);
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
    const VB v = vb_of(i);
    // the pair's rows see this block at all (pair-uniform)
    if (pair_any && v.vhi - 1 >= pair_lo_min && v.vlo <= pB) {
      process(region + st * SB, v, it);
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
    if constexpr (kBiasedCodes<BITS>) {
      // the V codes entered the MFMAs as 1024 + code
      const float t = xor32_sum(xor16_sum(psum[gi]));
      bacc[gi] = fmaf(-1024.0f, t, bacc[gi]);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the stages are free
  float* const Rr = reinterpret_cast<float*>(region);
#pragma unroll
  for (int gi = 0; gi < GH; gi++)
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      const int d = (g0 + gi) * 64 + ct * 16 + 4 * j;
      *reinterpret_cast<float4_t*>(&Rr[row * RS + d]) = o[gi * 4 + ct] + bacc[gi];
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
    wave_fwht_signed<E>(x, lane);
    const int64_t o_idx =
        (((int64_t)seq * a.n_q + qi0 + rq_) * a.n_q_heads + (int64_t)kvh * G + rh_) * D + lane * E;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float v = l > 0.0f ? (x[i] * cs_lane) / l : 0.0f;
      if (a.out_f32)
        reinterpret_cast<float*>(a.out)[o_idx + i] = v;
      else
        reinterpret_cast<uint16_t*>(a.out)[o_idx + i] = f32_to_bf16(v);
    }
  }
}

template <int D, int BITS>
hipError_t launch_t(const PrefillArgs& a, hipStream_t s) {
  const int qp = kPfRows / a.group;
  dim3 grid((a.n_q + qp - 1) / qp, a.new_st.n_kv_heads, a.n_seqs);
  hipLaunchKernelGGL((prefill_attn_kernel<D, BITS>), grid, dim3(kPfWaves * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attention(const PrefillArgs& a, hipStream_t s) {
  if (a.n_q <= 0) return hipSuccess;
  const BlockLayout& L = a.new_st.layout;
  switch (L.head_dim * 16 + L.bits) {
    case 128 * 16 + 4: return launch_t<128, 4>(a, s);
    case 128 * 16 + 8: return launch_t<128, 8>(a, s);
    case 256 * 16 + 4: return launch_t<256, 4>(a, s);
    case 256 * 16 + 8: return launch_t<256, 8>(a, s);
    case 512 * 16 + 4: return launch_t<512, 4>(a, s);
    case 512 * 16 + 8: return launch_t<512, 8>(a, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

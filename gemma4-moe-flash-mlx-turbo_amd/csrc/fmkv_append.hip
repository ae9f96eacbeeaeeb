// Append kernel: rotate -> quantize -> slot write, one work-group per
// (touched head-block, KV head, sequence).
//
// Replaces the store half of KVCache::update_and_fetch (src/cache.rs:266-310)
// and its quantizer turbo_round_trip_kv (src/cache.rs:94-129):
//  - rotation x.R (R from build_rht, src/cache.rs:47-62) as an in-wave fast
//    Walsh-Hadamard transform, stages h = 1, 2, ..., D/2 (registers first,
//    then lane exchanges), then * (1/sqrt D) and the LCG sign;
//  - affine mode: MLX group-64 affine quantization (4/8-bit, f16 scale/bias);
//  - codebook mode: the reference's own TurboQuant Lloyd-Max binning;
//  - slot write: ring slot pos % W for sliding layers, pos for global layers,
//    block table for paged pools;
//  - optionally, the layer's prologue first (src/model/gemma4_attention.rs
//    :52-81): K = RoPE(k_norm(k_proj)) rounded to bf16, V = v_norm(v_proj)
//    in f32 (or v_norm of the raw K for K==V layers).
// Every float op is written out in the oracle's order and the file is built
// with -ffp-contract=off, so codes and scales are bit-identical to it.
#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_quant.h"

namespace fmkv {
namespace {

constexpr int kAppendThreads = 256;

__constant__ float kCbBounds2[3] = {-0.982f, 0.0f, 0.982f};
__constant__ float kCbBounds3[7] = {-1.748f, -1.050f, -0.501f, 0.0f, 0.501f, 1.050f, 1.748f};
__constant__ float kCbBounds4[15] = {-2.401f, -1.844f, -1.437f, -1.099f, -0.800f,
                                     -0.522f, -0.258f, 0.0f,    0.258f,  0.522f,
                                     0.800f,  1.099f,  1.437f,  1.844f,  2.401f};

// Sum of squares in the oracle's order: per-lane left to right, then a
// xor-butterfly over all 64 lanes.
template <int E>
__device__ inline float canonical_sumsq(const float (&x)[E], int lane) {
  float acc = x[0] * x[0];
#pragma unroll
  for (int i = 1; i < E; i++) {
    float sq = x[i] * x[i];
    acc = acc + sq;
  }
  return group_sum<64>(acc, lane);
}

__device__ inline float bf16_round(float v) { return __uint_as_float((uint32_t)f32_to_bf16(v) << 16); }

// Value of lane (lane ^ m) for a runtime m in {1, 2, ..., 32}.
__device__ inline float xor_partner_rt(float v, int m, int lane) {
  switch (m) {
    case 1: return xor_partner<1>(v, lane);
    case 2: return xor_partner<2>(v, lane);
    case 4: return xor_partner<4>(v, lane);
    case 8: return xor_partner<8>(v, lane);
    case 16: return xor_partner<16>(v, lane);
    default: return xor_partner<32>(v, lane);
  }
}

// k_norm then RoPE of one K row (src/model/gemma4_attention.rs:63, :78-81),
// in the oracle's order: fast::rms_norm (x * r) * w with
// r = 1 / sqrt(sum(x^2) / D + eps) (the canonical sum), rounded to bf16;
// then MLX fast::rope (non-traditional): pair (d, d + rope_dims/2) turns by
// a = f32(pos) * f32(theta^(-2i/rope_dims)), cos/sin of the f32 angle taken
// in double; rounded to bf16. The pair partner sits in lane
// lane ^ (rope_dims / 2 / E).
template <int D>
__device__ inline void k_prologue(float (&x)[D / 64], const AppendArgs& a, int64_t pos, int lane) {
  constexpr int E = D / 64;
  const float ms = canonical_sumsq<E>(x, lane) / (float)D;
  const float r = 1.0f / sqrtf(ms + a.eps);
  float w[E];
  load_row<E>(a.k_norm_w + lane * E, w);
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = bf16_round((x[i] * r) * w[i]);
  const int half = a.rope_dims >> 1;
  float p[E];
#pragma unroll
  for (int i = 0; i < E; i++) p[i] = xor_partner_rt(x[i], half / E, lane);
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int d = lane * E + i;
    if (d < a.rope_dims) {
      const bool lower = d < half;
      const int fi = lower ? d : d - half;
      const float f = (float)pow((double)a.rope_theta, -2.0 * (double)fi / (double)a.rope_dims);
      const float ang = (float)pos * f;
      const float c = (float)cos((double)ang), s = (float)sin((double)ang);
      x[i] = lower ? bf16_round((x[i] * c) - (p[i] * s)) : bf16_round((p[i] * s) + (x[i] * c));
    }
  }
}

// v_norm of one V row (src/model/norm.rs:16-29, MLX ops on bf16 in the
// oracle's order): x2 = bf16(x * x); mean = bf16(sum(x2) / D) (canonical
// sum); out = x * (1 / sqrt(mean + eps)) in f32.
template <int D>
__device__ inline void v_prologue(float (&x)[D / 64], float eps, int lane) {
  constexpr int E = D / 64;
  float acc = bf16_round(x[0] * x[0]);
#pragma unroll
  for (int i = 1; i < E; i++) acc = acc + bf16_round(x[i] * x[i]);
  const float mean = bf16_round(group_sum<64>(acc, lane) / (float)D);
  const float rms = 1.0f / sqrtf(mean + eps);
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = x[i] * rms;
}

__device__ inline int cb_index(float z, int bits) {
  int idx = 0;
  if (bits == 2) {
#pragma unroll
    for (int b = 0; b < 3; b++) idx += (z >= kCbBounds2[b]) ? 1 : 0;
  } else if (bits == 3) {
#pragma unroll
    for (int b = 0; b < 7; b++) idx += (z >= kCbBounds3[b]) ? 1 : 0;
  } else {
#pragma unroll
    for (int b = 0; b < 15; b++) idx += (z >= kCbBounds4[b]) ? 1 : 0;
  }
  return idx;
}

// Token owning 32-bit word w of an affine V-code region, for byte/nibble k.
template <int BITS>
__device__ inline uint32_t v_clear_mask(int w, const int* cov) {
  const int q = ((w & 255) >> 2) >> 4;
  uint32_t m = 0;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (cov[4 * q + r] >= 0) m |= 0xffu << (8 * r);
  } else {
#pragma unroll
    for (int p = 0; p < 8; p++)
      if (cov[4 * q + 2 * (p & 1) + (p >> 2)] >= 0) m |= 0xfu << (4 * p);
  }
  return m;
}

template <int D, int BITS, int MODE>
__global__ __launch_bounds__(kAppendThreads) void append_kernel(AppendArgs a) {
  constexpr int E = D / 64;
  constexpr BlockLayout L = make_layout(D, BITS, MODE);
  constexpr int kWords = (int)(L.code_bytes / 4);
  constexpr int kWaves = kAppendThreads / 64;
  constexpr int kRowsPerWave = 2 * kBlockTokens / kWaves;  // K and V rows of 16 slots
  __shared__ uint32_t kst[kWords];
  __shared__ uint32_t vst[kWords];
  __shared__ int cov_row[kBlockTokens];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.y, seq = blockIdx.z, bx = blockIdx.x;
  const int64_t pos0 = a.start_pos ? (int64_t)a.start_pos[seq] : a.start_scalar;
  const int64_t end = pos0 + a.n_new;
  const int64_t W = a.window;
  if (a.n_new <= 0) return;

  int64_t lb, e0 = pos0, s0 = 0;
  if (W > 0) {
    e0 = end - W > pos0 ? end - W : pos0;
    const int64_t n_eff = end - e0;
    s0 = e0 % W;
    const int64_t nb_ring = W / kBlockTokens;
    const int64_t first = s0 / kBlockTokens, last = (s0 + n_eff - 1) / kBlockTokens;
    int64_t count = last - first + 1;
    if (count > nb_ring) count = nb_ring;
    if (bx >= count) return;
    lb = (first + bx) % nb_ring;
  } else {
    const int64_t first = pos0 / kBlockTokens, last = (end - 1) / kBlockTokens;
    if (bx > last - first) return;
    lb = first + bx;
  }

  // input row written to slot t of this block, or -1 (ring: slot - s0 lies
  // in (-W, W), so one conditional add replaces the modulo)
  auto row_of = [&](int t) -> int {
    const int64_t slot = lb * kBlockTokens + t;
    int64_t p = slot;
    if (W > 0) {
      const int64_t d = slot - s0;
      p = e0 + (d < 0 ? d + W : d);
    }
    return (p >= e0 && p < end) ? (int)(p - pos0) : -1;
  };
  int64_t phys = lb;
  if (a.st.block_table) {
    // caller-owned table: positions past its width or entries outside the
    // pool are not written (no out-of-bounds access on bad input)
    if (lb >= a.st.table_stride) return;
    phys = (int64_t)a.st.block_table[(int64_t)seq * a.st.table_stride + lb];
  }
  if (phys < 0 || phys >= a.st.n_blocks) return;
  uint8_t* blk = a.st.base + phys * a.st.block_stride + (int64_t)h * a.st.head_stride;

  // this wave's input rows (r = wave + k * waves: slot r / 2, K or V by
  // r & 1) are loaded first, so that they share one memory round trip with
  // the V-word read below; rows not written here re-read row 0 unused
  const int H = a.st.n_kv_heads;
  float x[kRowsPerWave][E];
  int rows[kRowsPerWave];
#pragma unroll
  for (int k = 0; k < kRowsPerWave; k++) {
    const int r = wv + k * kWaves;
    rows[k] = row_of(r >> 1);
    const int row = rows[k] < 0 ? 0 : rows[k];
    const uint16_t* src = ((r & 1) && !a.v_from_k ? a.v : a.k) +
                          (((int64_t)seq * a.n_new + row) * H + h) * D + lane * E;
    load_row<E>(src, x[k]);
  }
  if (tid < kBlockTokens) cov_row[tid] = row_of(tid);
  __syncthreads();

  bool all_cov = true;
#pragma unroll
  for (int t = 0; t < kBlockTokens; t++) all_cov = all_cov && (cov_row[t] >= 0);

  for (int w = tid; w < kWords; w += kAppendThreads) {
    kst[w] = 0u;
    if constexpr (MODE == kAffine) {
      const uint32_t old =
          all_cov ? 0u : reinterpret_cast<const uint32_t*>(blk + L.v_codes)[w];
      vst[w] = old & ~v_clear_mask<BITS>(w, cov_row);
    } else {
      vst[w] = 0u;
    }
  }
  __syncthreads();

  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
#pragma unroll
  for (int k = 0; k < kRowsPerWave; k++) {
    const int r = wv + k * kWaves;
    const int t = r >> 1, isv = r & 1;
    if (rows[k] < 0) continue;
    uint32_t* stage = isv ? vst : kst;
    if (a.k_norm_w) {
      if (isv)
        v_prologue<D>(x[k], a.eps, lane);
      else
        k_prologue<D>(x[k], a, pos0 + rows[k], lane);
    }
    if constexpr (MODE == kAffine) {
      wave_fwht<E>(x[k], lane);
#pragma unroll
      for (int i = 0; i < E; i++) x[k][i] = apply_sign(x[k][i] * a.c, sbits, i);
      uint32_t code[E];
      float scale, bias;
      affine_quant<E, BITS>(x[k], code, scale, bias, lane);
#pragma unroll
      for (int i = 0; i < E; i++) {
        int64_t off;
        int sh;
        if (isv)
          v_code_pos(BITS, t, lane * E + i, &off, &sh);
        else
          k_code_pos(BITS, t, lane * E + i, &off, &sh);
        atomicOr(&stage[off >> 2], code[i] << sh);
      }
      if ((lane % (64 / E)) == 0) {
        const int g = lane / (64 / E);
        const uint32_t sb = (uint32_t)f32_to_f16_bits(scale) |
                            ((uint32_t)f32_to_f16_bits(bias) << 16);
        *reinterpret_cast<uint32_t*>(blk + (isv ? L.v_meta : L.k_meta) + scale_pos(g, t)) = sb;
      }
    } else {
      constexpr int bits = BITS;
      const float norm = sqrtf(canonical_sumsq<E>(x[k], lane));
      const float den = norm + 1e-8f;
#pragma unroll
      for (int i = 0; i < E; i++) x[k][i] = x[k][i] / den;
      wave_fwht<E>(x[k], lane);
      const int64_t row_bits = (int64_t)D * bits;
#pragma unroll
      for (int i = 0; i < E; i++) {
        const float z = apply_sign(x[k][i] * a.c, sbits, i) * a.sqrt_d;
        const uint32_t idx = (uint32_t)cb_index(z, bits);
        const int64_t bit = t * row_bits + (int64_t)(lane * E + i) * bits;
        const int wi = (int)(bit >> 5), off = (int)(bit & 31);
        atomicOr(&stage[wi], idx << off);
        if (off + bits > 32) atomicOr(&stage[wi + 1], idx >> (32 - off));
      }
      if (lane == 0)
        *reinterpret_cast<uint16_t*>(blk + (isv ? L.v_meta : L.k_meta) + t * 2) =
            f32_to_f16_bits(norm);
    }
  }
  __syncthreads();

  uint32_t* kdst = reinterpret_cast<uint32_t*>(blk + L.k_codes);
  uint32_t* vdst = reinterpret_cast<uint32_t*>(blk + L.v_codes);
  for (int w = tid; w < kWords; w += kAppendThreads) {
    int tk;
    if constexpr (MODE == kAffine) {
      tk = ((w & 255) >> 2) & 15;
      vdst[w] = vst[w];
    } else {
      tk = (int)((int64_t)w * 4 / (L.code_bytes / kBlockTokens));
      if (cov_row[tk] >= 0) vdst[w] = vst[w];
    }
    if (cov_row[tk] >= 0) kdst[w] = kst[w];
  }
}

template <int D, int BITS, int MODE>
hipError_t launch_t(const AppendArgs& a, int n_seqs, int max_tasks, hipStream_t s) {
  dim3 grid(max_tasks, a.st.n_kv_heads, n_seqs);
  hipLaunchKernelGGL((append_kernel<D, BITS, MODE>), grid, dim3(kAppendThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_append(const AppendArgs& a, int n_seqs, int max_tasks, hipStream_t s) {
  const BlockLayout& L = a.st.layout;
  if (n_seqs <= 0) return hipSuccess;
  if (max_tasks <= 0) return hipSuccess;
  if (L.mode == kAffine) {
    switch (L.head_dim * 16 + L.bits) {
      case 128 * 16 + 4: return launch_t<128, 4, kAffine>(a, n_seqs, max_tasks, s);
      case 128 * 16 + 8: return launch_t<128, 8, kAffine>(a, n_seqs, max_tasks, s);
      case 256 * 16 + 4: return launch_t<256, 4, kAffine>(a, n_seqs, max_tasks, s);
      case 256 * 16 + 8: return launch_t<256, 8, kAffine>(a, n_seqs, max_tasks, s);
      case 512 * 16 + 4: return launch_t<512, 4, kAffine>(a, n_seqs, max_tasks, s);
      case 512 * 16 + 8: return launch_t<512, 8, kAffine>(a, n_seqs, max_tasks, s);
    }
  } else {
    switch (L.head_dim * 16 + L.bits) {
      case 128 * 16 + 2: return launch_t<128, 2, kCodebook>(a, n_seqs, max_tasks, s);
      case 128 * 16 + 3: return launch_t<128, 3, kCodebook>(a, n_seqs, max_tasks, s);
      case 128 * 16 + 4: return launch_t<128, 4, kCodebook>(a, n_seqs, max_tasks, s);
      case 256 * 16 + 2: return launch_t<256, 2, kCodebook>(a, n_seqs, max_tasks, s);
      case 256 * 16 + 3: return launch_t<256, 3, kCodebook>(a, n_seqs, max_tasks, s);
      case 256 * 16 + 4: return launch_t<256, 4, kCodebook>(a, n_seqs, max_tasks, s);
      case 512 * 16 + 2: return launch_t<512, 2, kCodebook>(a, n_seqs, max_tasks, s);
      case 512 * 16 + 3: return launch_t<512, 3, kCodebook>(a, n_seqs, max_tasks, s);
      case 512 * 16 + 4: return launch_t<512, 4, kCodebook>(a, n_seqs, max_tasks, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace fmkv

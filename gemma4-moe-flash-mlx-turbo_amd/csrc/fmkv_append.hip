// Append kernel: rotate -> quantize -> slot write, one work-group of 8
// waves per (touched head-block, KV head, sequence).
//
// Replaces the store half of KVCache::update_and_fetch (src/cache.rs:266-310)
// and its quantizer turbo_round_trip_kv (src/cache.rs:94-129):
//  - rotation x.R (R from build_rht, src/cache.rs:47-62) as an in-wave fast
//    Walsh-Hadamard transform, stages h = 1, 2, ..., D/2 (registers first,
//    then lane exchanges), then * (1/sqrt D) and the LCG sign;
//  - affine mode: MLX group-64 affine quantization (4/8-bit, f16 scale/bias);
//  - codebook mode: the reference's own TurboQuant Lloyd-Max binning;
//  - plain mode: the bf16 rows as given (KVCacheInner::Plain,
//    src/cache.rs:274-288), K token-major and V dim-major;
//  - slot write: ring slot pos % W for sliding layers, pos for global layers,
//    block table for paged pools;
//  - optionally, the layer's prologue first (src/model/gemma4_attention.rs
//    :52-81): K = RoPE(k_norm(k_proj)) rounded to bf16, V = v_norm(v_proj)
//    in f32 (or v_norm of the raw K for K==V layers).
// Every float op is written out in the oracle's order and the file is built
// with -ffp-contract=off, so codes and scales are bit-identical to it.
#include "fmkv_device.h"
#include "fmkv_internal.h"
#include "fmkv_prologue.h"
#include "fmkv_quant.h"

namespace fmkv {
namespace {

#ifndef FMKV_APPEND_ROWS
#define FMKV_APPEND_ROWS 2
#endif
// Rows per wave: each half (K, V) of a work-group's 16 tokens takes 16 / R
// waves, so a 2048-token chunk of two KV heads runs 4096 waves at R = 2
// (four per SIMD), whose latencies (lane exchanges, divisions) overlap.
constexpr int kAppendRows = FMKV_APPEND_ROWS;
constexpr int kAppendThreads = 2 * (16 / kAppendRows) * 64;

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

// One work-group per (touched head-block, KV head, sequence), 2 x 16 / R
// waves: wave w handles the K (w < 16 / R) or V rows of the R tokens
// R q .. R q + R - 1, q = w mod 16 / R, all R rows in lockstep (independent
// chains for the scheduler). Codes are combined in registers (the elements
// of one K word; the wave's tokens of a V word) before one LDS atomic per
// word; the block is then copied out with 16-byte stores. PRO: the layer's
// prologue (k_norm + RoPE on K, v_norm on V) runs on the rows first.
template <int D, int BITS, int MODE, bool PRO>
__global__ __launch_bounds__(kAppendThreads) void append_kernel(AppendArgs a) {
  constexpr int E = D / 64;
  constexpr int R = kAppendRows;  // rows per wave
  constexpr int NWH = 16 / R;      // waves per half (K or V)
  constexpr BlockLayout L = make_layout(D, BITS, MODE);
  constexpr int kWords = (int)(L.code_bytes / 4);
  constexpr int kHalfMax = PRO ? D / 2 : 1;
  __shared__ __align__(16) uint32_t kst[kWords];
  __shared__ __align__(16) uint32_t vst[kWords];
  __shared__ int cov_row[kBlockTokens];
  __shared__ float rope_f[kHalfMax];              // f32 theta^(-2i/rope_dims)
  __shared__ float2 rope_cs[NWH][R][kHalfMax];    // per K wave: (cos, sin) per row, angle

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int isv = wv / NWH, quad = wv % NWH;
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

  // the wave's four rows (rows not written here re-read row 0, unused)
  const int H = a.st.n_kv_heads;
  int rows[R];
  bool any = false, allr = true;
  float x[R][E];
#pragma unroll
  for (int r = 0; r < R; r++) {
    rows[r] = row_of(quad * R + r);
    any = any || rows[r] >= 0;
    allr = allr && rows[r] >= 0;
    const int row = rows[r] < 0 ? 0 : rows[r];
    const uint16_t* src = (isv && !a.v_from_k ? a.v : a.k) +
                          (((int64_t)seq * a.n_new + row) * H + h) * D + lane * E;
    load_row<E>(src, x[r]);
  }
  const int half = a.rope_dims >> 1;
  if (tid < kBlockTokens) cov_row[tid] = row_of(tid);
  if constexpr (PRO) {
    for (int i = tid; i < half; i += kAppendThreads)
      rope_f[i] = rope_inv_freq(i, a.rope_dims, a.rope_theta);
  }
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
    } else if constexpr (MODE == kPlain) {
      // a dim's word holds two tokens: start from the stored block, the
      // covered tokens' halves are overwritten below
      vst[w] = all_cov ? 0u : reinterpret_cast<const uint32_t*>(blk + L.v_codes)[w];
    } else {
      // codebook: a word may hold bits of several tokens; the covered tokens'
      // bits are cleared and set below, the others keep the stored ones
      uint32_t keep_k = 0u, keep_v = 0u;
      if (!all_cov) {
        for (int k = 0; k < 32; k++) {
          const int64_t bit = (int64_t)w * 32 + k;
          if (cov_row[cb_k_token_of_bit(D, BITS, bit)] < 0) keep_k |= 1u << k;
          if (cov_row[cb_v_token_of_bit(BITS, bit)] < 0) keep_v |= 1u << k;
        }
      }
      kst[w] = keep_k ? reinterpret_cast<const uint32_t*>(blk + L.k_codes)[w] & keep_k : 0u;
      vst[w] = keep_v ? reinterpret_cast<const uint32_t*>(blk + L.v_codes)[w] & keep_v : 0u;
    }
  }

  if constexpr (PRO) {
    if (!isv) {
      // (cos, sin) of every (row, angle) pair once, spread over the lanes
      for (int j = lane; j < half; j += 64) {
        const float f = rope_f[j];
#pragma unroll
        for (int r = 0; r < R; r++) rope_cs[quad][r][j] = rope_cos_sin(pos0 + (rows[r] < 0 ? 0 : rows[r]), f);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float w[E];
      load_row<E>(a.k_norm_w + lane * E, w);
#pragma unroll
      for (int r = 0; r < R; r++) k_norm_row<E>(x[r], w, a.eps, lane);
#pragma unroll
      for (int r = 0; r < R; r++)
        rope_row<E>(x[r], a.rope_dims, lane, [&](int j) { return rope_cs[quad][r][j]; });
    } else {
#pragma unroll
      for (int r = 0; r < R; r++) v_norm_row<E>(x[r], a.eps, lane);
    }
  }

  // x * (1/sqrt D), the RHT sign and the sign wave_fwht_signed leaves on
  // the lane as one multiplication by +-c (sign flips are exact; a -0 in
  // place of +0 changes no code, scale or bias: min/max, the scale rule,
  // rint and the codebook boundaries treat both zeros alike)
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  const float cl = fwht_lane_sign(lane) * a.c;
  float sc[E];
#pragma unroll
  for (int i = 0; i < E; i++) sc[i] = ((sbits >> i) & 1u) ? -cl : cl;

  uint32_t code[R][E];
  uint32_t meta[R];
  if constexpr (MODE == kPlain) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      meta[r] = 0u;
#pragma unroll
      // exact for rows as given; with the prologue, V (f32 after v_norm) is
      // rounded to the stored bf16 here (RNE)
      for (int i = 0; i < E; i++) code[r][i] = (uint32_t)f32_to_bf16(x[r][i]);
    }
  } else if constexpr (MODE == kAffine) {
#pragma unroll
    for (int r = 0; r < R; r++) wave_fwht_signed<E>(x[r], lane);
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
      for (int i = 0; i < E; i++) x[r][i] = x[r][i] * sc[i];
      float scale, bias;
      affine_quant<E, BITS>(x[r], code[r], scale, bias, lane);
      meta[r] = (uint32_t)f32_to_f16_bits(scale) | ((uint32_t)f32_to_f16_bits(bias) << 16);
    }
  } else {
    float norm[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      norm[r] = sqrtf(canonical_sumsq<E>(x[r], lane));
      const float den = norm[r] + 1e-8f;
#pragma unroll
      for (int i = 0; i < E; i++) x[r][i] = x[r][i] / den;
    }
#pragma unroll
    for (int r = 0; r < R; r++) wave_fwht_signed<E>(x[r], lane);
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
      for (int i = 0; i < E; i++) code[r][i] = (uint32_t)cb_index((x[r][i] * sc[i]) * a.sqrt_d, BITS);
      meta[r] = (uint32_t)f32_to_f16_bits(norm[r]);
    }
  }
  __syncthreads();

  if (any) {
    uint32_t* stage = isv ? vst : kst;
    if constexpr (MODE == kPlain) {
      uint16_t* st16 = reinterpret_cast<uint16_t*>(stage);
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (rows[r] < 0) continue;
        const int t = quad * R + r;
#pragma unroll
        for (int i = 0; i < E; i++) {
          const int d = lane * E + i;
          st16[(isv ? plain_v_pos(t, d) : plain_k_pos(D, t, d)) >> 1] = (uint16_t)code[r][i];
        }
      }
    } else if constexpr (MODE == kAffine) {
      if (!isv) {
        // G consecutive elements of a lane fall into one K word
        constexpr int G = E < 32 / BITS ? E : 32 / BITS;
#pragma unroll
        for (int r = 0; r < R; r++) {
          if (rows[r] < 0) continue;
#pragma unroll
          for (int i0 = 0; i0 < E; i0 += G) {
            int64_t off = 0;
            int sh;
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < G; j++) {
              k_code_pos(BITS, quad * R + r, lane * E + i0 + j, &off, &sh);
              word |= code[r][i0 + j] << sh;
            }
            atomicOr(&stage[off >> 2], word);
          }
        }
      } else {
        // the tokens of a quad 4q .. 4q+3 share each V word; this wave's
        // R of them are or-ed in here
#pragma unroll
        for (int i = 0; i < E; i++) {
          int64_t off = 0;
          int sh;
          uint32_t word = 0;
#pragma unroll
          for (int r = 0; r < R; r++) {
            v_code_pos(BITS, quad * R + r, lane * E + i, &off, &sh);
            if (rows[r] >= 0) word |= code[r][i] << sh;
          }
          atomicOr(&stage[off >> 2], word);
        }
      }
      if ((lane % (64 / E)) == 0) {
        const int g = lane / (64 / E);
        uint32_t* mp = reinterpret_cast<uint32_t*>(blk + (isv ? L.v_meta : L.k_meta) +
                                                   scale_pos(g, quad * R));
        if (allr) {
          if constexpr (R == 4)
            *reinterpret_cast<uint4*>(mp) = make_uint4(meta[0], meta[1], meta[2], meta[3]);
          else if constexpr (R == 2)
            *reinterpret_cast<uint2*>(mp) = make_uint2(meta[0], meta[1]);
          else
            mp[0] = meta[0];
        } else {
#pragma unroll
          for (int r = 0; r < R; r++)
            if (rows[r] >= 0) mp[r] = meta[r];
        }
      }
    } else {
      // K: the lane's E indices are E * bits consecutive bits of the token's
      // half row; V: each index goes to its dim's token run (fmkv_layout.h)
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (rows[r] < 0) continue;
        const int t = quad * R + r;
        if (!isv) {
          uint64_t v = 0;
#pragma unroll
          for (int i = 0; i < E; i++) v |= (uint64_t)code[r][i] << (i * BITS);
          const int64_t bit = cb_k_bit(D, BITS, t, lane * E);
          const int wi = (int)(bit >> 5), off = (int)(bit & 31);
          v <<= off;
          atomicOr(&stage[wi], (uint32_t)v);
          if (off + E * BITS > 32) atomicOr(&stage[wi + 1], (uint32_t)(v >> 32));
        } else {
#pragma unroll
          for (int i = 0; i < E; i++) {
            const int64_t bit = cb_v_bit(BITS, t, lane * E + i);
            const int wi = (int)(bit >> 5), off = (int)(bit & 31);
            const uint64_t v = (uint64_t)code[r][i] << off;
            atomicOr(&stage[wi], (uint32_t)v);
            if (off + BITS > 32) atomicOr(&stage[wi + 1], (uint32_t)(v >> 32));
          }
        }
        if (lane == 0)
          *reinterpret_cast<uint16_t*>(blk + (isv ? L.v_meta : L.k_meta) + (quad * R + r) * 2) =
              (uint16_t)meta[r];
      }
    }
  }
  __syncthreads();

  // 16-byte copy-out; affine K chunks belong to one token each, the other
  // regions are whole (merged with the stored block above)
  uint4* kdst = reinterpret_cast<uint4*>(blk + L.k_codes);
  uint4* vdst = reinterpret_cast<uint4*>(blk + L.v_codes);
  const uint4* ks = reinterpret_cast<const uint4*>(kst);
  const uint4* vs = reinterpret_cast<const uint4*>(vst);
  for (int c = tid; c < kWords / 4; c += kAppendThreads) {
    int tk;
    if constexpr (MODE == kAffine) {
      tk = c & 15;
      vdst[c] = vs[c];
    } else if constexpr (MODE == kPlain) {
      tk = (int)((int64_t)c * 16 / (L.code_bytes / kBlockTokens));
      vdst[c] = vs[c];
    } else {
      kdst[c] = ks[c];
      vdst[c] = vs[c];
      continue;
    }
    if (cov_row[tk] >= 0) kdst[c] = ks[c];
  }
}

template <int D, int BITS, int MODE>
hipError_t launch_t(const AppendArgs& a, int n_seqs, int max_tasks, hipStream_t s) {
  dim3 grid(max_tasks, a.st.n_kv_heads, n_seqs);
  if (a.k_norm_w) {
    hipLaunchKernelGGL((append_kernel<D, BITS, MODE, true>), grid, dim3(kAppendThreads), 0, s, a);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((append_kernel<D, BITS, MODE, false>), grid, dim3(kAppendThreads), 0, s, a);
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
  } else if (L.mode == kPlain) {
    switch (L.head_dim) {
      case 128: return launch_t<128, 16, kPlain>(a, n_seqs, max_tasks, s);
      case 256: return launch_t<256, 16, kPlain>(a, n_seqs, max_tasks, s);
      case 512: return launch_t<512, 16, kPlain>(a, n_seqs, max_tasks, s);
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

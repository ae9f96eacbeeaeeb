// Helpers shared by the decode and prefill attention kernels (gfx950):
// the LDS-DMA copy path (buffer_load_dwordx4 ... lds with explicit vmcnt
// waits), the exact f16 operands built from affine codes for the QK and PV
// matrix-core tiles, and the lane/dim correspondence of those tiles.
#pragma once
#include "fmkv_device.h"
#include "fmkv_internal.h"

namespace fmkv {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 1024;  // bytes per full LDS copy instruction (64 lanes x 16 B)

constexpr int cmax(int a, int b) { return a > b ? a : b; }

// Online softmax: how far (base 2) a score may exceed the running reference
// max before the accumulators are rescaled to a new one.
constexpr float kRescaleSlack = 8.0f;

// Decode kernel modes. Dense: softmax attention. Sparse-V (src/model/
// gemma4_attention.rs:196-234, weights below tau zeroed without
// renormalisation) takes two passes over the cache: kStats streams only the
// keys and writes each split's (m, l) and each block's largest score per
// head; kGated derives every head's threshold theta = M + log2(tau * L)
// from those, visits only the blocks that hold a score at or above it and
// is the dense pass with every score below theta dropped; the combine
// divides by the full L of the stats pass.
constexpr int kDense = 0, kStats = 1, kGated = 2;

// A stream's visiting order in the gated pass: the set bits of `mask` in
// increasing order, then next, next + 1, ... below n (scalar values).
struct BlockList {
  uint64_t mask;
  int next, n;
  __device__ int pop() {
    if (mask) {
      const int i = __builtin_ctzll(mask);
      mask &= mask - 1;
      return i;
    }
    return next < n ? next++ : n;
  }
};

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(p);  // low half of the flat LDS address
}

// Raw buffer resource over [base, base + bytes); reads past the end return 0.
__device__ inline u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;  // stride 0
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}

// One copy instruction: each active lane moves 16 bytes from rsrc + voff to
// LDS at lds + 16 * lane.
__device__ inline void dma16(uint32_t lds, int voff, const u32x4 rs) {
  asm volatile("buffer_load_dwordx4 %1, %2, 0 offen lds" :: "{m0}"(lds), "v"(voff), "s"(rs)
               : "memory");
}

template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Wait until at most `pending` (wave-uniform) blocks' copies, CP
// instructions each, are outstanding; P bounds pending.
template <int CP, int P>
__device__ inline void wait_copies(int pending) {
  if constexpr (P > 0) {
    if (pending >= P) {
      wait_vmcnt<P * CP>();
      return;
    }
    wait_copies<CP, P - 1>(pending);
  } else {
    wait_vmcnt<0>();
  }
}

__device__ inline u32x4 lds16(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// 8-bit codes enter the MFMAs as the exact f16 values 1024 + code (one
// v_perm per two codes): the QK accumulator starts at -1024 * sum(q operand)
// and the PV accumulator loses 1024 * sum(P') at the end, both from the
// exact f16 operand values. At 8 bits the offset costs the f32 partial sums
// at most 3 of their 24 bits; 4-bit codes (range 16) convert exactly
// instead, as the offset would cost them 7.
template <int BITS>
constexpr bool kBiasedCodes = BITS == 8;

// K operand (8 codes as exact f16, + 1024 at 8 bits) of MFMA s of group g;
// `w` is the lane's 16 bytes of the group's chunk (8-bit) or of the two
// groups' chunk (4-bit).
template <int BITS>
__device__ inline half8_t k_operand(const u32x4 w, int g, int s) {
  if constexpr (BITS == 8) {
    const uint32_t w0 = w[2 * s], w1 = w[2 * s + 1];
    return cat8(u8x2_to_h2_biased(w0, 0x04010400u), u8x2_to_h2_biased(w0, 0x04030402u),
                u8x2_to_h2_biased(w1, 0x04010400u), u8x2_to_h2_biased(w1, 0x04030402u));
  } else {
    const uint32_t x = w[(g & 1) * 2 + s];
    return cat8(u4x2_to_h2(x, 0), u4x2_to_h2(x, 1), u4x2_to_h2(x, 2), u4x2_to_h2(x, 3));
  }
}

// V codes of column tile ct (0..3) of group g: tokens 4j..4j+3 of one dim
// (+ 1024 at 8 bits).
template <int BITS>
__device__ inline half4_t v_operand(const u32x4 w, int g, int ct) {
  if constexpr (BITS == 8) {
    const uint32_t x = w[ct];
    return cat4(u8x2_to_h2_biased(x, 0x04010400u), u8x2_to_h2_biased(x, 0x04030402u));
  } else {
    const int ctc = (g & 1) * 4 + ct;  // column tile inside the 128-dim chunk
    const uint32_t x = w[ctc >> 1];
    const int k0 = (ctc & 1) * 2;
    return cat4(u4x2_to_h2(x, k0), u4x2_to_h2(x, k0 + 1));
  }
}

// The decode kernel's operands: a code enters the matrix cores as the exact
// f16 value (code + kCodeOffset) / kCodeScale --
//   8-bit: 1024 + code (k_operand / v_operand: one v_perm per two codes, the
//          code becoming the low mantissa byte of 1024);
//   4-bit: 1 + code / 16 (the code becoming the top four mantissa bits of
//          1.0: one shift and one bit-field insert per two codes, against
//          four instructions for the exact small integer).
// The q operand table is scaled by kCodeScale (exact), the QK accumulator
// starts at -kCodeOffset * (the column's q operand summed over the group), and
// the PV row is kCodeScale * O - kCodeOffset * (the column's P' summed over
// the tokens): exact f16 / f32 scalings, so the products sum to sum(code * q)
// and sum(code * P') up to the f32 rounding of partial sums that the offset
// inflates about 9x at 8 bits and 3x at 4 bits.
template <int BITS>
constexpr float kCodeOffset = BITS == 8 ? 1024.0f : 16.0f;
template <int BITS>
constexpr float kCodeScale = BITS == 8 ? 1.0f : 16.0f;

// The two register constants of the 4-bit operands, made opaque to the
// compiler (which would otherwise rematerialise them at every use): the
// mantissa field mask in an SGPR, 1.0 in both f16 halves in a VGPR.
struct U4Consts {
  uint32_t mask, one;
  __device__ U4Consts() {
    asm volatile("s_mov_b32 %0, 0x3c003c0" : "=s"(mask));
    asm volatile("v_mov_b32 %0, 0x3c003c00" : "=v"(one));
  }
};

// Nibbles k and k + 4 of w (bits 4k and 16 + 4k) as the f16 pair
// {1 + c0 / 16, 1 + c1 / 16}: the codes moved to bits 6..9 of each 16-bit
// half, then merged into 1.0 with one v_and_or_b32 over the register
// constants. (Written in C, not as inline asm: the compiler must see the
// write to insert the wait states an MFMA reading the result right after
// needs.)
__device__ inline half2_t u4x2_to_h2_unit(uint32_t w, int k, const U4Consts& u) {
  const uint32_t x = k == 0 ? w << 6 : k == 1 ? w << 2 : k == 2 ? w >> 2 : w >> 6;
  return __builtin_bit_cast(half2_t, (x & u.mask) | u.one);
}

// K operand of MFMA s of group g in the decode kernel's offset form.
template <int BITS>
__device__ inline half8_t k_operand_dec(const u32x4 w, int g, int s, const U4Consts& u) {
  if constexpr (BITS == 8) {
    return k_operand<8>(w, g, s);
  } else {
    const uint32_t x = w[(g & 1) * 2 + s];
    return cat8(u4x2_to_h2_unit(x, 0, u), u4x2_to_h2_unit(x, 1, u), u4x2_to_h2_unit(x, 2, u),
                u4x2_to_h2_unit(x, 3, u));
  }
}

// V operand of column tile ct of group g in the decode kernel's offset form.
template <int BITS>
__device__ inline half4_t v_operand_dec(const u32x4 w, int g, int ct, const U4Consts& u) {
  if constexpr (BITS == 8) {
    return v_operand<8>(w, g, ct);
  } else {
    const int ctc = (g & 1) * 4 + ct;  // column tile inside the 128-dim chunk
    const uint32_t x = w[ctc >> 1];
    const int k0 = (ctc & 1) * 2;
    return cat4(u4x2_to_h2_unit(x, k0, u), u4x2_to_h2_unit(x, k0 + 1, u));
  }
}

__device__ inline float lo16(uint32_t w) { return f16_bits_to_f32(w); }
__device__ inline float hi16(uint32_t w) { return f16_bits_to_f32(w >> 16); }

// Dim of head_dim fed to lane k-group j, element i, of the QK MFMA s (0/1)
// of group g is g*64 + j*16 + s*8 + i (8-bit) or g*64 + s*32 + j*8 + i
// (4-bit), matching the K-code placement of fmkv_layout.h. For the E = D/64
// consecutive dims of lane l (d0 = l*E) this gives the entry and position
// they occupy: (g, s, j) and the first element i0.
template <int E, int BITS>
struct QSlot {
  int g, s, j, i0;
  __device__ explicit QSlot(int lane) {
    const int d0 = lane * E, o = d0 & 63;
    g = d0 >> 6;
    s = BITS == 8 ? (o >> 3) & 1 : o >> 5;
    j = BITS == 8 ? o >> 4 : (o >> 3) & 3;
    i0 = o & 7;
  }
};

// Sparse-V gated pass (src/model/gemma4_attention.rs:196-234): the score
// thresholds of the work-group's q heads from the statistics pass's split
// (m, l) in a.stat_ml (its split columns and, with stats_new_col, its
// new-token column). Wave w merges q heads kvh * G + h for h = w, w + n_waves,
// ... < G, lane i taking splits i, i + 64, ..., the lanes meeting in a
// butterfly, into the full softmax max M and sum L; theta = M + log2(tau * L),
// so that a weight 2^(s - M) / L >= tau exactly when its base-2 score s >=
// theta (no visible token: +inf). Split column 0 stores theta, M and L in
// tau_stats for the combine. The thresholds land in th_s[0 .. G) (LDS);
// every thread of the work-group calls this (one barrier).
__device__ inline void gated_thresholds(const AttnArgs& a, int n_splits, int seq, int kvh, int G,
                                        int split, int wave, int lane, float* th_s,
                                        int n_waves = 8) {
  for (int h = wave; h < G; h += n_waves) {
    const int n_stat = n_splits + a.stats_new_col;
    const int64_t rbase = (int64_t)seq * a.part_stride * a.n_q_heads + kvh * G + h;
    float M = -INFINITY, Ls = 0.0f;
    for (int sp = lane; sp < n_stat; sp += 64) {
      const float2 ml =
          *reinterpret_cast<const float2*>(a.stat_ml + (rbase + (int64_t)sp * a.n_q_heads) * 2);
      const float mn = fmaxf(M, ml.x);
      Ls = fmaf(ml.y, exp2f(ml.x - mn), Ls * exp2f(M - mn));
      M = mn;
    }
    const float Mw = group_max<64>(M, lane);
    Ls = group_sum<64>(Ls > 0.0f ? Ls * exp2f(M - Mw) : 0.0f, lane);
    const float th = Ls > 0.0f ? Mw + log2f(a.tau * Ls) : INFINITY;
    if (lane == 0) {
      th_s[h] = th;
      if (split == 0) {
        const int64_t nh = (int64_t)gridDim.y * a.n_q_heads;
        const int64_t r = (int64_t)seq * a.n_q_heads + kvh * G + h;
        a.tau_stats[r] = th;
        a.tau_stats[nh + r] = Mw;
        a.tau_stats[2 * nh + r] = Ls;
      }
    }
  }
  __syncthreads();
}

// Sparse-V gated pass: which of a stream's blocks pb0 + ns * i (i < nb) to
// visit -- those in which some head's largest score from the statistics pass
// (blk_max) reaches its threshold thk[head], plus the block holding the
// newest token (whose statistics came from the statistics pass's new-token
// column rather than a block row) and any block beyond the block-maxima
// rows. Lane i tests block i (i < 64); blocks past the 64th are always
// visited. Returns the visiting list; *n_visit is its length.
__device__ inline BlockList gated_block_list(const AttnArgs& a, const float (&thk)[8], int64_t blk_row,
                                             int64_t blk_lo, int64_t pb0, int ns, int nb,
                                             int64_t T, int lane, int* n_visit) {
  const int64_t last_blk =
      T > 0 ? (a.window > 0 ? (T - 1) % a.window : T - 1) / kBlockTokens : -1;
  bool need = false;
  if (lane < nb) {
    const int64_t bl = pb0 + (int64_t)ns * lane, rb = bl - blk_lo;
    need = bl == last_blk || rb >= a.blk_stride;
    if (!need) {
      const float4_t m0 = *reinterpret_cast<const float4_t*>(a.blk_max + (blk_row + rb) * 8);
      const float4_t m1 = *reinterpret_cast<const float4_t*>(a.blk_max + (blk_row + rb) * 8 + 4);
#pragma unroll
      for (int k = 0; k < 4; k++) need = need || m0[k] >= thk[k] || m1[k] >= thk[k + 4];
    }
  }
  const uint64_t mask = __ballot(need);
  *n_visit = __builtin_popcountll(mask) + (nb > 64 ? nb - 64 : 0);
  return BlockList{mask, 64, nb};
}

// Index of the block maximum of (sequence and KV head at blk_row, block rb,
// q head of the group): block-major for the gated pass, head-major for the
// gather.
__device__ inline int64_t blk_max_at(const AttnArgs& a, int64_t blk_row, int64_t rb, int head) {
  return a.blk_scores ? blk_row * 8 + (int64_t)head * a.blk_stride + rb : (blk_row + rb) * 8 + head;
}

// Sparse-V statistics pass, for the gather: the block's scores of the
// lane's head (tokens 4j .. 4j + 3) when the block may hold a kept token. A
// weight 2^(s - M) / L reaches tau only if s >= M + log2(tau) (L >= 1), and a
// split's running reference max m_run (after this block) never exceeds the
// full max M, so a block whose largest score mb for the head is below
// m_run + log2(tau) holds none and is not stored (the test keeps a margin of
// 1/64 against the rounding of either side).
__device__ inline void store_block_scores(const AttnArgs& a, int64_t blk_row, int64_t rb, int head,
                                          int j, const float (&s)[4], float mb, float m_run,
                                          float log2_tau, bool writer) {
  if (a.blk_scores && writer && rb < a.blk_stride && mb + 0.015625f >= m_run + log2_tau)
    *reinterpret_cast<float4_t*>(a.blk_scores + ((blk_row + rb) * 8 + head) * 16 + 4 * j) =
        (float4_t){s[0], s[1], s[2], s[3]};
}

template <int E>
__device__ inline void store_halves(uint8_t* p, const _Float16 (&h)[E]) {
  if constexpr (E == 8)
    *reinterpret_cast<half8_t*>(p) = (half8_t){h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
  else if constexpr (E == 4)
    *reinterpret_cast<half4_t*>(p) = (half4_t){h[0], h[1], h[2], h[3]};
  else
    *reinterpret_cast<half2_t*>(p) = (half2_t){h[0], h[1]};
}

}  // namespace
}  // namespace fmkv

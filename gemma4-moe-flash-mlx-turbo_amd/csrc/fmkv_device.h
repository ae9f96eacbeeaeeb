// Device helpers shared by the fmkv kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmkv_layout.h"

namespace fmkv {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ inline float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet).
__device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

__device__ inline uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ inline float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xffffu));
}

// Lane l receives the value of lane (l & ~15) | ((l + 8) & 15): the other
// half of its 16-lane row (DPP row_ror:8).
__device__ inline float row_ror8(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
}

// Lane l receives the value of lane (l & ~15) | ((l + 4) & 15) (DPP
// row_ror:4).
__device__ inline float row_ror4(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
}

// Lane l receives the value of lane l ^ 1 (DPP quad_perm [1, 0, 3, 2]).
__device__ inline float quad_xor1(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
}

// Sum / max with the lane 16 (resp. 32) apart: permlane swaps return the
// pair {own, partner} in some order, so a commutative op gives both lanes the
// same bits.
__device__ inline float xor16_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor32_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor16_max(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Two 8-bit codes -> two exact f16 values: v_perm builds {c, 0x64} halves,
// i.e. 1024 + c, and the packed subtract removes the 1024 exactly.
// sel 0x04010400 takes bytes (0, 1) of w, 0x04030402 bytes (2, 3).
// The same two codes as the exact f16 values 1024 + c (one v_perm): for
// MFMAs whose accumulator removes the 1024 * sum(other operand) term.
__device__ inline half2_t u8x2_to_h2_biased(uint32_t w, uint32_t sel) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, sel));
}

__device__ inline half2_t u8x2_to_h2(uint32_t w, uint32_t sel) {
  uint32_t x = __builtin_amdgcn_perm(0x64646464u, w, sel);
  return __builtin_bit_cast(half2_t, x) - (half2_t){(_Float16)1024.0f, (_Float16)1024.0f};
}

// Nibbles k and k + 4 of w -> two exact f16 values (same 1024 trick).
__device__ inline half2_t u4x2_to_h2(uint32_t w, int k) {
  uint32_t x = ((w >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
  return __builtin_bit_cast(half2_t, x) - (half2_t){(_Float16)1024.0f, (_Float16)1024.0f};
}

// RHT sign bits of this lane's E = D/64 dims (bit i = dim lane * E + i)
// from the argument words (bit d of the mask = sign of dim d is -1): the
// words are written into lanes 0..D/32-1 of one register and each lane
// fetches its word with a bpermute. (A select chain over the words would be
// turned into a vector load of the argument segment, and kernels that track
// their own vector-memory counts must not get one.)
template <int D>
__device__ inline uint32_t lane_sign_bits(const uint32_t (&bits)[16], int lane) {
  constexpr int E = D / 64;
  int words = 0;
#pragma unroll
  for (int k = 0; k < D / 32; k++)
    asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(words) : "s"(bits[k]), "n"(k));
  const uint32_t word = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane * E) >> 5) * 4, words);
  return (word >> ((lane * E) & 31)) & ((1u << E) - 1u);
}

// x * s with s = -1 where bit i is set, else +1: a sign flip, bit-identical
// to the multiplication.
__device__ inline float apply_sign(float x, uint32_t bits, int i) {
  return __uint_as_float(__float_as_uint(x) ^ (((bits >> i) & 1u) << 31));
}

// Two f32 -> packed f16, round toward zero (v_cvt_pkrtz_f16_f32).
__device__ inline half2_t pkrtz(float a, float b) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

__device__ inline half8_t cat8(half2_t a, half2_t b, half2_t c, half2_t d) {
  return (half8_t){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
__device__ inline half4_t cat4(half2_t a, half2_t b) { return (half4_t){a[0], a[1], b[0], b[1]}; }

// E contiguous bf16 values -> f32 (one 32/64/128-bit load).
template <int E>
__device__ inline void load_row(const uint16_t* src, float (&x)[E]) {
  if constexpr (E == 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(src);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else if constexpr (E == 4) {
    const uint2 u = *reinterpret_cast<const uint2*>(src);
    x[0] = __uint_as_float(u.x << 16);
    x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16);
    x[3] = __uint_as_float(u.y & 0xffff0000u);
  } else {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(src);
    x[0] = __uint_as_float(u << 16);
    x[1] = __uint_as_float(u & 0xffff0000u);
  }
}

// Value of lane (lane ^ M): DPP quad_perm (M = 1, 2) and row_ror:8 (M = 8)
// as plain DPP moves (every lane reads a valid lane, so nothing is
// materialised for masked lanes and the move can fuse into its user), the
// LDS crossbar's swizzle for M = 4 (no VALU), and the permlane swaps for
// M = 16, 32.
template <int M>
__device__ inline float xor_partner(float v, int lane) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (M == 1) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xf, 0xf, true));
  } else if constexpr (M == 2) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xf, 0xf, true));
  } else if constexpr (M == 4) {
    // swizzle bit mode: and 0x1f, or 0, xor 4 within each 32-lane half
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, 0x101F));
  } else if constexpr (M == 8) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x128, 0xf, 0xf, true));
  } else if constexpr (M == 16) {
    auto r = __builtin_amdgcn_permlane16_swap((uint32_t)iv, (uint32_t)iv, false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    auto r = __builtin_amdgcn_permlane32_swap((uint32_t)iv, (uint32_t)iv, false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
  }
}

// Butterfly reductions over aligned groups of LANES lanes (strides 1, 2, ...,
// LANES/2, own value first): every lane of a group ends with the same bits.
template <int LANES>
__device__ inline float group_sum(float v, int lane) {
  if constexpr (LANES > 1) v = v + xor_partner<1>(v, lane);
  if constexpr (LANES > 2) v = v + xor_partner<2>(v, lane);
  if constexpr (LANES > 4) v = v + xor_partner<4>(v, lane);
  if constexpr (LANES > 8) v = v + xor_partner<8>(v, lane);
  if constexpr (LANES > 16) v = v + xor_partner<16>(v, lane);
  if constexpr (LANES > 32) v = v + xor_partner<32>(v, lane);
  return v;
}
template <int LANES>
__device__ inline float group_max(float v, int lane) {
  if constexpr (LANES > 1) v = fmaxf(v, xor_partner<1>(v, lane));
  if constexpr (LANES > 2) v = fmaxf(v, xor_partner<2>(v, lane));
  if constexpr (LANES > 4) v = fmaxf(v, xor_partner<4>(v, lane));
  if constexpr (LANES > 8) v = fmaxf(v, xor_partner<8>(v, lane));
  if constexpr (LANES > 16) v = fmaxf(v, xor_partner<16>(v, lane));
  if constexpr (LANES > 32) v = fmaxf(v, xor_partner<32>(v, lane));
  return v;
}
template <int LANES>
__device__ inline float group_min(float v, int lane) {
  if constexpr (LANES > 1) v = fminf(v, xor_partner<1>(v, lane));
  if constexpr (LANES > 2) v = fminf(v, xor_partner<2>(v, lane));
  if constexpr (LANES > 4) v = fminf(v, xor_partner<4>(v, lane));
  if constexpr (LANES > 8) v = fminf(v, xor_partner<8>(v, lane));
  if constexpr (LANES > 16) v = fminf(v, xor_partner<16>(v, lane));
  if constexpr (LANES > 32) v = fminf(v, xor_partner<32>(v, lane));
  return v;
}

// Partner value for a cross-lane FWHT stage: as xor_partner, with the LDS
// crossbar for M = 16 (swizzle xor 16) and M = 32 (bpermute), so that every
// stage costs one VALU operation besides a fusable DPP move.
template <int M>
__device__ inline float fwht_partner(float v, int lane) {
  if constexpr (M == 16) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  } else if constexpr (M == 32) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __float_as_int(v)));
  } else {
    return xor_partner<M>(v, lane);
  }
}

// Sign carried by a lane's values after wave_fwht_signed: (-1)^popcount(lane).
__device__ inline float fwht_lane_sign(int lane) {
  return (__builtin_popcount(lane & 63) & 1) ? -1.0f : 1.0f;
}

// Canonical unnormalised FWHT of a D = 64*E row held as E contiguous values
// per lane: stages h = 1 .. E/2 in registers, then h = E .. D/2 across lanes
// (lane xor h/E); (a, b) -> (a + b, a - b) exactly as the oracle.
//
// The lane stages carry a per-lane sign instead of selecting add or
// subtract: with z = sigma * y on both lanes of a pair (sigma depends only
// on lane bits other than M), z' = z_own + s * z_partner, s = -1 on the
// upper lane, equals sigma * (a + b) on the lower lane and -sigma * (a - b)
// on the upper one; the product s * z is exact and RN(-x) = -RN(x), so each
// stage is one fma rounding exactly like the add or subtract it stands for.
// On return the true row value is fwht_lane_sign(lane) * x[i], except that
// an exact cancellation can come out as -0 where the oracle has +0.
template <int E>
__device__ inline void wave_fwht_signed(float (&x)[E], int lane) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1)
#pragma unroll
    for (int i = 0; i < E; i += 2 * h)
#pragma unroll
      for (int jj = i; jj < i + h; jj++) {
        const float a = x[jj], b = x[jj + h];
        x[jj] = a + b;
        x[jj + h] = a - b;
      }
#define FMKV_FWHT_STAGE(M)                                                       \
  {                                                                              \
    const float s = (lane & (M)) ? -1.0f : 1.0f;                                 \
    _Pragma("unroll") for (int i = 0; i < E; i++)                                \
        x[i] = __builtin_fmaf(fwht_partner<(M)>(x[i], lane), s, x[i]);           \
  }
  FMKV_FWHT_STAGE(1)
  FMKV_FWHT_STAGE(2)
  FMKV_FWHT_STAGE(4)
  FMKV_FWHT_STAGE(8)
  FMKV_FWHT_STAGE(16)
  FMKV_FWHT_STAGE(32)
#undef FMKV_FWHT_STAGE
}

// The same transform with true values, bit for bit including the sign of
// zero: the sign-tracking stages above turn an exact cancellation's +0 into
// -0 once the lane sign is applied, which only consumers that cannot tell
// the zeros apart (quantizers, sums) may accept. Here the lower lane of a
// pair computes fma(1, own, partner) = own + partner and the upper lane
// fma(-1, own, partner) = partner - own, as the oracle; at M = 16 and 32 the
// permlane swap hands every lane the pair (a, b) (lower lane's value first),
// so fma(+-1, b, a) needs no select.
template <int M, int E>
__device__ inline void fwht_lane_stage(float (&x)[E], int lane) {
  const float sgn = (lane & M) ? -1.0f : 1.0f;
#pragma unroll
  for (int i = 0; i < E; i++) {
    if constexpr (M == 16 || M == 32) {
      const uint32_t u = __float_as_uint(x[i]);
      const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                             : __builtin_amdgcn_permlane32_swap(u, u, false, false);
      x[i] = __builtin_fmaf(sgn, __uint_as_float(r[1]), __uint_as_float(r[0]));
    } else {
      x[i] = __builtin_fmaf(sgn, x[i], xor_partner<M>(x[i], lane));
    }
  }
}

template <int E>
__device__ inline void wave_fwht(float (&x)[E], int lane) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1)
#pragma unroll
    for (int i = 0; i < E; i += 2 * h)
#pragma unroll
      for (int jj = i; jj < i + h; jj++) {
        const float a = x[jj], b = x[jj + h];
        x[jj] = a + b;
        x[jj + h] = a - b;
      }
  fwht_lane_stage<1>(x, lane);
  fwht_lane_stage<2>(x, lane);
  fwht_lane_stage<4>(x, lane);
  fwht_lane_stage<8>(x, lane);
  fwht_lane_stage<16>(x, lane);
  fwht_lane_stage<32>(x, lane);
}

// Visible-position test shared by the attention and combine kernels.
struct SeqGeom {
  int64_t blk_lo, blk_hi;  // logical blocks to scan
};

__host__ __device__ inline SeqGeom seq_geometry(int64_t T, int64_t window, int64_t vis_begin) {
  SeqGeom g;
  if (window > 0) {
    int64_t filled = T < window ? T : window;
    g.blk_lo = 0;
    g.blk_hi = (filled + kBlockTokens - 1) / kBlockTokens;
  } else {
    int64_t vb = vis_begin > 0 ? vis_begin : 0;
    g.blk_lo = vb / kBlockTokens;
    g.blk_hi = (T + kBlockTokens - 1) / kBlockTokens;
    if (g.blk_hi < g.blk_lo) g.blk_hi = g.blk_lo;
  }
  return g;
}

// Blocks to scan for one sequence; paged tables bound it by their width.
__host__ __device__ inline SeqGeom seq_geometry(int64_t T, int64_t window, int64_t vis_begin,
                                                int32_t table_stride, bool paged) {
  SeqGeom g = seq_geometry(T, window, vis_begin);
  if (paged && g.blk_hi > table_stride) g.blk_hi = table_stride;
  if (g.blk_hi < g.blk_lo) g.blk_hi = g.blk_lo;
  return g;
}

// Split count of a sequence (>= 1, so split 0 always writes a result),
// never more than the grid provides.
// Split 0 covers bps0 blocks, every later split bps (bps0 >= bps): a
// sequence's first work-group is its largest, so the dispatcher, which
// takes the grid's split columns in order, starts the big work first and
// fills the tail with small work-groups.
// An XCD-aware plan (skew_p > 0, one sequence) sizes the grid to the
// sequence exactly: every one of its max_splits splits is used.
__host__ __device__ inline int n_splits_for(const SeqGeom& g, int bps0, int bps, int max_splits,
                                            int skew_p = 0) {
  if (skew_p > 0) return max_splits;
  // block counts stay below 2^31 / 16: a 32-bit division suffices
  const uint32_t nb = (uint32_t)(g.blk_hi - g.blk_lo);
  int64_t ns = nb <= (uint32_t)bps0 ? 1 : 1 + (nb - (uint32_t)bps0 + (uint32_t)bps - 1u) / (uint32_t)bps;
  if (ns > max_splits) ns = max_splits;
  return (int)ns;
}

// Blocks [*b_begin, *b_end) of split `split`. Default plan: split 0 has bps0
// blocks, every later one bps. XCD-aware plan (skew_p > 0): every split has
// bps blocks and the first skew_extra splits whose index is a multiple of
// skew_p one more -- the launch puts those on the XCDs that start first.
__device__ inline void split_range(const SeqGeom& g, int split, int bps0, int bps, int skew_p,
                                   int skew_extra, int64_t* b_begin, int64_t* b_end) {
  int64_t first, count;
  if (skew_p > 0) {
    // skew_p is 1, 2 or 4: shifts, not divisions (this runs before a
    // work-group's first copies)
    const int sh = __builtin_ctz((unsigned)skew_p);
    const int before = (split + skew_p - 1) >> sh;  // skewed splits ahead of this one
    first = (int64_t)split * bps + (before < skew_extra ? before : skew_extra);
    count = bps + (((split & (skew_p - 1)) == 0 && (split >> sh) < skew_extra) ? 1 : 0);
  } else {
    first = split == 0 ? 0 : bps0 + (int64_t)(split - 1) * bps;
    count = split == 0 ? bps0 : bps;
  }
  *b_begin = g.blk_lo + first < g.blk_hi ? g.blk_lo + first : g.blk_hi;
  *b_end = *b_begin + count < g.blk_hi ? *b_begin + count : g.blk_hi;
}

}  // namespace fmkv

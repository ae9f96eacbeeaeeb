// Codebook (TurboQuant) operands for the matrix cores, shared by the decode
// and prefill attention kernels: the reference's Lloyd-Max centroids
// (src/cache.rs:67-89) as exact f16 integers (2 and 3 bits) or as f16 high
// part + residual (4 bits), and the lookups that turn a lane's packed
// indices into MFMA operand words through an LDS table replicated
// kLutCopies times (entry e of copy l at (e * kLutCopies + l) * 4, so the
// lanes of a half-wave never hit one bank twice): for 2- and 3-bit indices
// one entry per index pair (two elements); for 4-bit indices one
// {high, residual} entry per index.
#pragma once
#include "fmkv_device.h"
#include "fmkv_attn_common.h"

namespace fmkv {
namespace {

// src/cache.rs:67-89 centroids (the same literals as the append's tables).
__constant__ float kCbCent2[4] = {-1.510f, -0.453f, 0.453f, 1.510f};
__constant__ float kCbCent3[8] = {-2.152f, -1.344f, -0.756f, -0.245f, 0.245f, 0.756f, 1.344f, 2.152f};
__constant__ float kCbCent4[16] = {-2.733f, -2.069f, -1.618f, -1.256f, -0.942f, -0.657f,
                                   -0.388f, -0.128f, 0.128f,  0.388f,  0.657f,  0.942f,
                                   1.256f,  1.618f,  2.069f,  2.733f};

constexpr int kLutCopies = 32;

// The 2- and 3-bit centroids are three-decimal literals whose thousandfold
// values are integers that f16 holds exactly (at most 2152 in magnitude, and
// even where above 2048): as operands n_i = 1000 * centroid_i they need no
// residual part, one matrix-core pass per operand instead of two, and the
// factor 1/1000 joins the value scale norm / sqrt(D) (n_i / 1000 is within
// 2.4e-8 relative of the f32 literal). The 4-bit centroids need 12
// significant bits (2733, 2069) and keep the f16 high part + residual.
template <int BITS>
constexpr bool kCbExact = BITS <= 3;
// what an operand of the table counts in: the value scale's extra factor
template <int BITS>
constexpr float kCbOperandScale = kCbExact<BITS> ? 1e-3f : 1.0f;

// Table size of BITS-bit indices: index pairs (2 and 3 bits; one table of
// the exact integer operands) or single indices (4 bits; one table of
// {high, residual}); 4 bytes per entry and copy.
template <int BITS>
struct CbLut {
  static constexpr bool kPairs = BITS <= 3;
  static constexpr int kEntries = kPairs ? (1 << (2 * BITS)) : 16;
  static constexpr int kHalf = kEntries * kLutCopies * 4;  // one table
  static constexpr int kBytes = kHalf;
};

// Centroid i of an exact table as the f16 integer 1000 * centroid_i.
template <int BITS>
__device__ inline uint16_t cent_int(int i) {
  static_assert(kCbExact<BITS>, "2- and 3-bit tables");
  const float cv = BITS == 2 ? kCbCent2[i] : kCbCent3[i];
  return __builtin_bit_cast(uint16_t, (_Float16)rintf(cv * 1000.0f));
}

// Centroid i as {f16 high part, f16 residual}.
template <int BITS>
__device__ inline uint32_t cent_hl(int i) {
  const float cv = BITS == 2 ? kCbCent2[i] : BITS == 3 ? kCbCent3[i] : kCbCent4[i];
  const _Float16 h = (_Float16)cv;
  const _Float16 r = (_Float16)(cv - (float)h);
  return (uint32_t)__builtin_bit_cast(uint16_t, h) | ((uint32_t)__builtin_bit_cast(uint16_t, r) << 16);
}

// A lane's field: the bits from `sh` on of word `dw` of w (and of the next
// word at 3 bits, where fields straddle words; that word lies inside the LDS
// staging: the K halves are followed by the V halves, the V halves by the
// norms). 2- and 4-bit fields never straddle a word.
template <int BITS>
__device__ inline uint32_t lds_field(const uint32_t* w, int dw, uint32_t sh) {
  if constexpr (BITS == 3)
    return __builtin_amdgcn_alignbit(w[dw + 1], w[dw], sh);
  else
    return w[dw] >> sh;
}

typedef const uint32_t __attribute__((address_space(3)))* lds_u32_ptr;
__device__ inline uint32_t lds_load(uint32_t addr) { return *(lds_u32_ptr)(size_t)addr; }

// Bits [OFF, OFF + W) of x (one v_bfe_u32; written out so that the index
// and the table address stay two instructions).
template <int OFF, int W>
__device__ inline uint32_t bfe(uint32_t x) {
  uint32_t r;
  asm("v_bfe_u32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "n"(OFF), "n"(W));
  return r;
}

// The f16 operand word of two consecutive elements of a field (the field's
// elements 2p and 2p + 1, element e at bits e * BITS) from an exact table
// (2 and 3 bits); base: LDS address of this lane's copy of entry 0.
template <int BITS, int P>
__device__ inline uint32_t cb_pair_exact(uint32_t base, uint32_t field) {
  static_assert(kCbExact<BITS>, "2- and 3-bit tables");
  return lds_load(base + bfe<2 * P * BITS, 2 * BITS>(field) * (kLutCopies * 4));
}

// High and residual f16 operand words of two consecutive elements of a
// 4-bit field (elements 2p and 2p + 1, element e at bits 4e): one
// {high, residual} lookup per element, paired by v_perm; base: LDS address
// of this lane's copy of entry 0.
template <int P>
__device__ inline void cb_pair_hl4(uint32_t base, uint32_t field, uint32_t& hw, uint32_t& lw) {
  const uint32_t e0 = lds_load(base + bfe<8 * P, 4>(field) * (kLutCopies * 4));
  const uint32_t e1 = lds_load(base + bfe<8 * P + 4, 4>(field) * (kLutCopies * 4));
  hw = __builtin_amdgcn_perm(e1, e0, 0x05040100u);  // the high parts
  lw = __builtin_amdgcn_perm(e1, e0, 0x07060302u);  // the residuals
}

// Fills the lookup table at `lut` (CbLut<BITS>::kBytes of LDS); threads
// tid = 0 .. nthreads - 1 of the work-group share the work (no barrier).
template <int BITS>
__device__ inline void cb_fill_lut(uint8_t* lut, int tid, int nthreads) {
  using T = CbLut<BITS>;
  for (int e = tid; e < T::kEntries * kLutCopies; e += nthreads) {
    const int idx = e / kLutCopies;
    if constexpr (kCbExact<BITS>) {
      const uint32_t n0 = cent_int<BITS>(idx & ((1 << BITS) - 1)), n1 = cent_int<BITS>(idx >> BITS);
      *reinterpret_cast<uint32_t*>(lut + e * 4) = n0 | (n1 << 16);
    } else {
      *reinterpret_cast<uint32_t*>(lut + e * 4) = cent_hl<BITS>(idx);
    }
  }
}

}  // namespace
}  // namespace fmkv

// The attention layer's prologue before the cache store
// (src/model/gemma4_attention.rs:52-81), one row at a time in the in-wave
// row layout (lane l holds dims l*E .. l*E+E-1 of a D = 64*E row):
//   K = RoPE(k_norm(k_proj)), each rounded to bf16;
//   V = v_norm(v_proj) in f32 (or v_norm of the raw K on K==V layers).
// Every float op is written out in the oracle's order, with FMA contraction
// off in each helper's body (also in the attention sources, which are built
// with contraction on), so the append kernel and the decode step's new-token
// column, which both use these helpers, store the same codes as the oracle
// does.
#pragma once
#include "fmkv_device.h"

namespace fmkv {
namespace {

// Sum of squares in the oracle's order: per-lane left to right, then a
// xor-butterfly over all 64 lanes.
template <int E>
__device__ inline float canonical_sumsq(const float (&x)[E], int lane) {
#pragma clang fp contract(off)
  float acc = x[0] * x[0];
#pragma unroll
  for (int i = 1; i < E; i++) {
    float sq = x[i] * x[i];
    acc = acc + sq;
  }
  return group_sum<64>(acc, lane);
}

__device__ inline float bf16_round(float v) { return __uint_as_float((uint32_t)f32_to_bf16(v) << 16); }

// Value of v in lane `lane ^ m` via the LDS crossbar (m known only at run
// time). Every lane of the wave must execute it.
__device__ inline float lane_xor_value(float v, int m, int lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, __float_as_int(v)));
}

// RoPE inverse frequency of angle index i: f32(theta^(-2i/dims)), computed
// in double (fast::rope's base ** (-2i/dims) before the f32 multiply).
__device__ inline float rope_inv_freq(int i, int dims, float theta) {
  return (float)pow((double)theta, -2.0 * (double)i / (double)dims);
}

// (cos, sin) of angle f32(pos) * f, evaluated in double, rounded to f32.
__device__ inline float2 rope_cos_sin(int64_t pos, float f) {
  const float ang = (float)pos * f;
  double sn, cs;
  sincos((double)ang, &sn, &cs);
  return make_float2((float)cs, (float)sn);
}

// k_norm (fast::rms_norm with weight w, src/model/norm.rs:5-14):
// x = bf16((x * (1 / sqrt(sum(x^2) / D + eps))) * w), the canonical sum.
template <int E>
__device__ inline void k_norm_row(float (&x)[E], const float (&w)[E], float eps, int lane) {
#pragma clang fp contract(off)
  constexpr int D = 64 * E;
  const float rn = 1.0f / sqrtf(canonical_sumsq<E>(x, lane) / (float)D + eps);
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = bf16_round((x[i] * rn) * w[i]);
}

// RoPE, non-traditional (fast::rope, :78-81): dim d < dims/2 pairs with
// d + dims/2; the partner of lane l's dims sits in lane l ^ (dims / 2 / E).
// cs(j) returns (cos, sin) of angle j < dims/2. Results rounded to bf16; dims
// at or past rope_dims are left as they are. Every lane must call it.
template <int E, typename CS>
__device__ inline void rope_row(float (&x)[E], int rope_dims, int lane, CS cs) {
#pragma clang fp contract(off)
  const int half = rope_dims >> 1;
  const int m = half / E;
  float p[E];
#pragma unroll
  for (int i = 0; i < E; i++) p[i] = lane_xor_value(x[i], m, lane);
  if (lane * E < rope_dims) {
    const bool lower = lane * E < half;
    const int f0 = lower ? lane * E : lane * E - half;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float2 c = cs(f0 + i);
      x[i] = lower ? bf16_round((x[i] * c.x) - (p[i] * c.y)) : bf16_round((p[i] * c.y) + (x[i] * c.x));
    }
  }
}

// v_norm (RMSNormNoScale, src/model/norm.rs:16-29): x2 = bf16(x * x);
// mean = bf16(sum(x2) / D) (canonical sum); x = x * (1 / sqrt(mean + eps)).
template <int E>
__device__ inline void v_norm_row(float (&x)[E], float eps, int lane) {
#pragma clang fp contract(off)
  constexpr int D = 64 * E;
  float acc = bf16_round(x[0] * x[0]);
#pragma unroll
  for (int i = 1; i < E; i++) acc = acc + bf16_round(x[i] * x[i]);
  const float mean = bf16_round(group_sum<64>(acc, lane) / (float)D);
  const float rms = 1.0f / sqrtf(mean + eps);
#pragma unroll
  for (int i = 0; i < E; i++) x[i] = x[i] * rms;
}

}  // namespace
}  // namespace fmkv

// Group-64 affine quantization of one rotated row held by a wave, shared by
// the append kernel and the decode step's new-token column (so both write
// bit-identical codes).
//
// MLX affine_quantize (the quantizer the reference calls at
// src/model/mod.rs:669-675), restated: per group, scale = max((max - min) /
// (2^b - 1), 1e-7), negated unless |min| > |max|; the edge value of larger
// magnitude (max on a tie) is represented exactly: q0 = rint(edge / scale),
// and when q0 != 0 the scale
// becomes edge / q0 and the bias the edge itself, else the bias is 0; codes
// are clip(rint((y - bias) / scale), 0, 2^b - 1) with the f32 scale and
// bias, which are then stored as f16. rint rounds half to even. Every
// operation is written in the oracle's order, with FMA contraction off (the
// pragma in the function body holds in sources built with contraction on).
#pragma once
#include "fmkv_device.h"

namespace fmkv {

// Lane holds E = D/64 consecutive values of the row; the group spans 64/E
// lanes. Returns the codes and the f32 scale and bias of the lane's group.
template <int E, int BITS>
__device__ inline void affine_quant(const float (&y)[E], uint32_t (&code)[E], float& scale_o,
                                    float& bias_o, int lane) {
#pragma clang fp contract(off)
  constexpr int kLanesPerGroup = 64 / E;
  float mx = y[0], mn = y[0];
#pragma unroll
  for (int i = 1; i < E; i++) {
    mx = fmaxf(mx, y[i]);
    mn = fminf(mn, y[i]);
  }
  mx = group_max<kLanesPerGroup>(mx, lane);
  mn = group_min<kLanesPerGroup>(mn, lane);
  const float n_bins = (float)((1 << BITS) - 1);
  float scale = fmaxf((mx - mn) / n_bins, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  // Codes rint((y - bias) / scale) without a division per element: with
  // inv = RN(1 / scale) and t = RN((y - bias) * inv), |t - Q| <= 2^-14 for
  // the exact quotient |Q| < 512 (|Q| <= 2 * (2^b - 1) by the choice of
  // scale), and the correctly rounded quotient lies within 2^-16 of Q. So
  // when t is more than 2^-13 from every half-integer, rint(t) equals rint
  // of the correctly rounded quotient. Lanes with an element closer than
  // that (about 2^-11 of elements), or a non-finite t, divide exactly.
  const float inv = 1.0f / scale;
  float qv[E];
  bool exact = false;
#pragma unroll
  for (int i = 0; i < E; i++) {
    qv[i] = (y[i] - bias) * inv;
    const float fr = qv[i] - floorf(qv[i]);
    exact = exact || !(fabsf(fr - 0.5f) > 0x1p-13f);
  }
  if (exact) {
#pragma unroll
    for (int i = 0; i < E; i++) qv[i] = (y[i] - bias) / scale;
  }
#pragma unroll
  for (int i = 0; i < E; i++) {
    float q = rintf(qv[i]);
    q = fminf(fmaxf(q, 0.0f), n_bins);
    code[i] = (uint32_t)q;
  }
  scale_o = scale;
  bias_o = bias;
}

namespace {

// Lloyd-Max bin of a rotated, normalised value scaled by sqrt(D)
// (src/cache.rs:67-89 boundaries; a value on a boundary goes to the upper
// bin), as the reference's round trip bins it (src/cache.rs:94-129).
__constant__ float kCbBounds2[3] = {-0.982f, 0.0f, 0.982f};
__constant__ float kCbBounds3[7] = {-1.748f, -1.050f, -0.501f, 0.0f, 0.501f, 1.050f, 1.748f};
__constant__ float kCbBounds4[15] = {-2.401f, -1.844f, -1.437f, -1.099f, -0.800f,
                                     -0.522f, -0.258f, 0.0f,    0.258f,  0.522f,
                                     0.800f,  1.099f,  1.437f,  1.844f,  2.401f};

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

}  // namespace

}  // namespace fmkv

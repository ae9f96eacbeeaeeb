// q preparation for the decode kernel, once per (sequence, KV head) and
// step: q_rot = (FWHT(q * qscale) * c) o s (q . R with R from
// src/cache.rs:47-62, times the softmax scale in base 2), stored as the
// decode kernel's MFMA B operands so that every split work-group copies them
// instead of recomputing the rotation.
//
// Table of one (sequence, KV head), (2 NG + 1) KiB with NG = D / 64 groups:
//   entry e = 2 g + s (g < NG, s < 2), at e * 1024 + 16 * lane: the B operand
//     of the QK MFMA s of group g for lane (j, c) = (lane / 16, lane % 16):
//     8 f16 q_rot values of dims qk_dim(g, s, j, i), i < 8, of GQA head c & 7
//     -- the f16 high part for c < 8, the residual for c >= 8; zero for
//     columns beyond the GQA group;
//   at 2 NG * 1024: float qsum[8][NG], per head and group, sum of q_rot.
#pragma once
#include "fmkv_device.h"
#include "fmkv_internal.h"

namespace fmkv {

// Dim of head_dim fed to lane k-group j, element i, of the QK MFMA s (0/1)
// of group g (matches the K-code placement in fmkv_layout.h).
template <int BITS>
__device__ inline int qk_dim(int g, int s, int j, int i) {
  if constexpr (BITS == 8)
    return g * 64 + j * 16 + s * 8 + i;
  else
    return g * 64 + s * 32 + j * 8 + i;
}

// One work-group of kQPrepThreads threads fills the table of (seq, kvh).
// Every thread of the work-group must call it (it holds a barrier).
template <int D, int BITS>
__device__ void qprep_workgroup(const QPrepArgs& a, int n_kv_heads, int kvh, int seq, int tid) {
  constexpr int NG = D / 64;
  constexpr int E = D / 64;
  constexpr int LPG = 64 / E;  // lanes per 64-dim group
  constexpr int QS = D + 4;    // padded row stride (LDS banks)
  constexpr int NWV = kQPrepThreads / 64;
  constexpr int kHPW = (8 + NWV - 1) / NWV;  // GQA heads per wave, at most
  constexpr int NE = 2 * NG;
  __shared__ float qo[8 * QS];
  __shared__ float qsum_s[8][NG];

  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.group;
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  const uint16_t* qg = a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G) * D;
  float qx[kHPW][E];
#pragma unroll
  for (int k = 0; k < kHPW; k++) {
    const int hh = wave + k * NWV;
    load_row<E>(qg + (hh < G ? hh : 0) * D + lane * E, qx[k]);  // rows past G unused
  }
#pragma unroll
  for (int k = 0; k < kHPW; k++) {
    const int hh = wave + k * NWV;
    if (hh >= G) continue;
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = qx[k][i] * a.qscale;
    wave_fwht<E>(x, lane);
    float gsum = 0.0f;
#pragma unroll
    for (int i = 0; i < E; i++) {
      x[i] = apply_sign(x[i] * a.c, sbits, i);
      gsum += x[i];
      qo[hh * QS + lane * E + i] = x[i];
    }
    gsum = group_sum<LPG>(gsum, lane);
    if ((lane & (LPG - 1)) == 0) qsum_s[hh][lane / LPG] = gsum;
  }
  __syncthreads();

  uint8_t* const tab = a.out + ((int64_t)seq * n_kv_heads + kvh) * qprep_bytes(D);
  const int j = lane >> 4, c = lane & 15, head = c & 7;
  const bool hi = c < 8, col_valid = head < G;
  for (int e = wave; e < NE; e += NWV) {
    half8_t b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float v = col_valid ? qo[head * QS + qk_dim<BITS>(e >> 1, e & 1, j, i)] : 0.0f;
      const _Float16 vh = (_Float16)v;
      b[i] = hi ? vh : (_Float16)(v - (float)vh);
    }
    *reinterpret_cast<half8_t*>(tab + e * 1024 + lane * 16) = b;
  }
  for (int t = tid; t < 8 * NG; t += kQPrepThreads)
    reinterpret_cast<float*>(tab + NE * 1024)[t] = (t / NG) < G ? qsum_s[t / NG][t % NG] : 0.0f;
}

}  // namespace fmkv

// q preparation for the decode kernel: q_rot = (FWHT(q * qscale) * c) o s
// (q . R with R from src/cache.rs:47-62, times the softmax scale in base 2),
// laid out as the decode kernel's MFMA B operands, so that its prologue is a
// plain load issued alongside the first cache blocks.
//
// Table layout, per (sequence, KV head, wave w < NW = D/128, lane):
// kQPrepVecs x 16 bytes =
//   [0..3] B operands bq[gi][s] (gi = the wave's two 64-dim groups, s = the
//          two K=32 MFMA halves), 8 f16 each: column c < 8 holds the f16 high
//          part of q_rot of GQA head c, c >= 8 the residual of head c - 8;
//   [4]    {q-group sum of group 0, of group 1 (hi columns; 0 elsewhere),
//          this lane's RHT sign bits (dims lane*E .. lane*E+E-1), 0}.
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

// RHT sign bits of this lane's E dims (bit i = dim lane * E + i), picked from
// the argument words with selects (no dynamic register indexing).
template <int D>
__device__ inline uint32_t lane_sign_bits(const uint32_t (&bits)[16], int lane) {
  constexpr int E = D / 64;
  const int w = (lane * E) >> 5;
  uint32_t word = bits[0];
#pragma unroll
  for (int k = 1; k < D / 32; k++) word = (w == k) ? bits[k] : word;
  return (word >> ((lane * E) & 31)) & ((1u << E) - 1u);
}

// x * s with s = -1 where bit i is set: a sign flip, bit-identical to the
// multiplication.
__device__ inline float apply_sign(float x, uint32_t bits, int i) {
  return __uint_as_float(__float_as_uint(x) ^ (((bits >> i) & 1u) << 31));
}

template <typename W>
__device__ inline W* qprep_entry(W* table, int64_t seq, int n_kv_heads, int kvh, int nw, int wave,
                                 int lane) {
  return table + ((((seq * n_kv_heads + kvh) * nw) + wave) * 64 + lane) * (kQPrepVecs * 4);
}

// One work-group (>= D/128 waves; extra waves idle) prepares the table rows
// of (seq, kvh). Every thread of the work-group must call it (it holds a
// barrier).
template <int D, int BITS>
__device__ void qprep_workgroup(const QPrepArgs& a, int n_kv_heads, int kvh, int seq, int tid) {
  constexpr int NW = D / kAttnDW;
  constexpr int GW = kAttnDW / 64;
  constexpr int E = D / 64;
  constexpr int LPG = 64 / E;              // lanes per 64-dim group
  constexpr int NG = D / 64;
  constexpr int QS = D + 4;                // padded row stride (LDS banks)
  constexpr int kHPW = (8 + NW - 1) / NW;  // GQA heads per wave, at most
  static_assert(GW == 2 && kQPrepVecs == 2 * GW + 1, "table layout assumes two groups per wave");
  __shared__ float qo[8 * QS];
  __shared__ float qsum_s[8][NG];

  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.group;
  const bool active = wave < NW;
  const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
  if (active) {
    const uint16_t* qg = a.q + ((int64_t)seq * a.n_q_heads + (int64_t)kvh * G) * D;
    float qx[kHPW][E];
#pragma unroll
    for (int k = 0; k < kHPW; k++) {
      const int hh = wave + k * NW;
      load_row<E>(qg + (hh < G ? hh : 0) * D + lane * E, qx[k]);
    }
#pragma unroll
    for (int k = 0; k < kHPW; k++) {
      const int hh = wave + k * NW;
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
      }
#pragma unroll
      for (int i = 0; i < E; i++) qo[hh * QS + lane * E + i] = x[i];
      gsum = group_sum<LPG>(gsum, lane);
      if ((lane & (LPG - 1)) == 0) qsum_s[hh][lane / LPG] = gsum;
    }
  }
  __syncthreads();
  if (!active) return;

  const int j = lane >> 4, c = lane & 15, head = c & 7;
  const bool hi = c < 8, col_valid = head < G;
  uint32_t* dst = qprep_entry(a.out, seq, n_kv_heads, kvh, NW, wave, lane);
  float qs[GW];
#pragma unroll
  for (int gi = 0; gi < GW; gi++) {
    const int g = wave * GW + gi;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      half8_t b;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float v = col_valid ? qo[head * QS + qk_dim<BITS>(g, s, j, i)] : 0.0f;
        const _Float16 vh = (_Float16)v;
        b[i] = hi ? vh : (_Float16)(v - (float)vh);
      }
      *reinterpret_cast<uint4*>(dst + (gi * 2 + s) * 4) = __builtin_bit_cast(uint4, b);
    }
    qs[gi] = (hi && col_valid) ? qsum_s[head][g] : 0.0f;
  }
  *reinterpret_cast<uint4*>(dst + 16) =
      make_uint4(__float_as_uint(qs[0]), __float_as_uint(qs[1]), sbits, 0u);
}

}  // namespace fmkv

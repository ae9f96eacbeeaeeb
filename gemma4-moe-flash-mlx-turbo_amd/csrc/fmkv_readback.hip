// Read-side utility kernels:
//  - read_codes: stored codes/scales in a canonical per-slot layout (MLX
//    little-endian packing), for bit-exact comparison with the oracle;
//  - fetch: dequantized, un-rotated K/V of the visible positions in
//    chronological order -- what KVCache::update_and_fetch returns and
//    KVCache::peek_kv reads (src/cache.rs:247-310). In codebook mode this is
//    the reference's round trip output (src/cache.rs:119-125) computed from
//    the stored indices and f16 norm; in plain mode the stored bf16 rows.
#include "fmkv_device.h"
#include "fmkv_internal.h"

namespace fmkv {
namespace {

__constant__ float kCent2[4] = {-1.510f, -0.453f, 0.453f, 1.510f};
__constant__ float kCent3[8] = {-2.152f, -1.344f, -0.756f, -0.245f, 0.245f, 0.756f, 1.344f, 2.152f};
__constant__ float kCent4[16] = {-2.733f, -2.069f, -1.618f, -1.256f, -0.942f, -0.657f,
                                 -0.388f, -0.128f, 0.128f,  0.388f,  0.657f,  0.942f,
                                 1.256f,  1.618f,  2.069f,  2.733f};

__device__ inline float centroid(int bits, uint32_t idx) {
  return bits == 2 ? kCent2[idx] : bits == 3 ? kCent3[idx] : kCent4[idx];
}

__device__ inline uint32_t get_bits(const uint32_t* words, int64_t bit, int bits) {
  const int64_t w = bit >> 5;
  const int off = (int)(bit & 31);
  uint64_t v = words[w] >> off;
  if (off + bits > 32) v |= (uint64_t)words[w + 1] << (32 - off);
  return (uint32_t)(v & ((1u << bits) - 1u));
}

// Code of dim d, token t, of a head-block (plain: the bf16 bits).
__device__ inline uint32_t stored_code(const uint8_t* blk, const BlockLayout& L, int isv, int t,
                                       int d) {
  if (L.mode == kPlain)
    return *reinterpret_cast<const uint16_t*>(
        blk + (isv ? L.v_codes + plain_v_pos(t, d) : L.k_codes + plain_k_pos(L.head_dim, t, d)));
  if (L.mode == kAffine) {
    int64_t off;
    int sh;
    if (isv)
      v_code_pos(L.bits, t, d, &off, &sh);
    else
      k_code_pos(L.bits, t, d, &off, &sh);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(blk + (isv ? L.v_codes : L.k_codes) + off);
    return (w >> sh) & ((1u << L.bits) - 1u);
  }
  const uint32_t* region = reinterpret_cast<const uint32_t*>(blk + (isv ? L.v_codes : L.k_codes));
  return get_bits(region, isv ? cb_v_bit(L.bits, t, d) : cb_k_bit(L.head_dim, L.bits, t, d), L.bits);
}

// One thread per canonical output word; grid.x over slots, grid.y = K/V x heads.
__global__ void read_codes_kernel(ReadArgs a) {
  const BlockLayout L = a.st.layout;
  const int64_t slot = blockIdx.x;
  const int isv = blockIdx.y & 1, h = blockIdx.y >> 1;
  const int H = a.st.n_kv_heads;
  const int D = L.head_dim, bits = L.bits;
  const int words = (D * bits + 31) / 32;
  const int64_t blk_i = slot / kBlockTokens;
  const int t = (int)(slot % kBlockTokens);
  const uint8_t* blk = a.st.base + blk_i * a.st.block_stride + (int64_t)h * a.st.head_stride;
  const int64_t row = (slot * 2 + isv) * H + h;
  for (int wi = threadIdx.x; wi < words; wi += blockDim.x) {
    uint32_t out = 0;
    for (int bit = 0; bit < 32; bit += bits) {
      const int64_t gbit = (int64_t)wi * 32 + bit;
      const int d = (int)(gbit / bits);
      if (d >= D) break;
      if (gbit % bits != 0) continue;
      out |= stored_code(blk, L, isv, t, d) << bit;
    }
    if (bits == 3) {  // codes straddle words: rebuild the exact stream
      out = 0;
      for (int k = 0; k < 32; k++) {
        const int64_t gbit = (int64_t)wi * 32 + k;
        const int d = (int)(gbit / bits);
        if (d >= D) break;
        const uint32_t code = stored_code(blk, L, isv, t, d);
        out |= ((code >> (gbit % bits)) & 1u) << k;
      }
    }
    a.codes[row * words + wi] = out;
  }
  const int n_meta = L.mode == kAffine ? 2 * (D / kGroup) : L.mode == kCodebook ? 1 : 0;
  const uint8_t* meta = blk + (isv ? L.v_meta : L.k_meta);
  for (int mi = threadIdx.x; mi < n_meta; mi += blockDim.x) {
    uint16_t v;
    if (L.mode == kAffine) {
      const uint32_t sb = *reinterpret_cast<const uint32_t*>(meta + scale_pos(mi >> 1, t));
      v = (mi & 1) ? (uint16_t)(sb >> 16) : (uint16_t)(sb & 0xffffu);
    } else {
      v = *reinterpret_cast<const uint16_t*>(meta + t * 2);
    }
    a.meta[row * n_meta + mi] = v;
  }
}

// One wave per (visible position, K/V, head): dequantize in the rotated
// domain, then x = c * FWHT(y o s) (src/cache.rs:122-125 order).
template <int D>
__global__ __launch_bounds__(64) void fetch_kernel(FetchArgs a) {
  constexpr int E = D / 64;
  const BlockLayout L = a.st.layout;
  const int lane = threadIdx.x;
  const int64_t i = blockIdx.x;
  const int isv = blockIdx.y & 1, h = blockIdx.y >> 1;
  const int H = a.st.n_kv_heads;
  const int64_t pos = a.first_pos + i;
  const int64_t slot = a.window > 0 ? pos % a.window : pos;
  const int64_t blk_i = slot / kBlockTokens;
  const int t = (int)(slot % kBlockTokens);
  const uint8_t* blk = a.st.base + blk_i * a.st.block_stride + (int64_t)h * a.st.head_stride;
  float x[E];
  float norm = 1.0f;
  void* dst = isv ? a.v_out : a.k_out;
  const int64_t base = (i * H + h) * D + lane * E;
  if (L.mode == kPlain) {  // the stored rows, no rotation
#pragma unroll
    for (int e = 0; e < E; e++) {
      const uint32_t b = stored_code(blk, L, isv, t, lane * E + e);
      if (a.out_f32)
        reinterpret_cast<float*>(dst)[base + e] = __uint_as_float(b << 16);
      else
        reinterpret_cast<uint16_t*>(dst)[base + e] = (uint16_t)b;
    }
    return;
  }
  if (L.mode == kAffine) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      const int d = lane * E + e;
      const uint32_t sb =
          *reinterpret_cast<const uint32_t*>(blk + (isv ? L.v_meta : L.k_meta) + scale_pos(d / kGroup, t));
      const float y = fmaf((float)stored_code(blk, L, isv, t, d), f16_bits_to_f32(sb),
                           f16_bits_to_f32(sb >> 16));
      x[e] = y * a.signs[d];
    }
  } else {
    norm = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + (isv ? L.v_meta : L.k_meta) + t * 2));
#pragma unroll
    for (int e = 0; e < E; e++) {
      const int d = lane * E + e;
      const float w = centroid(L.bits, stored_code(blk, L, isv, t, d)) * a.c;
      x[e] = w * a.signs[d];
    }
  }
  wave_fwht<E>(x, lane);  // true values: the output is compared bit for bit
#pragma unroll
  for (int e = 0; e < E; e++) {
    const float v = (L.mode == kAffine) ? x[e] * a.c : (x[e] * a.c) * norm;
    if (a.out_f32)
      reinterpret_cast<float*>(dst)[base + e] = v;
    else
      reinterpret_cast<uint16_t*>(dst)[base + e] = f32_to_bf16(v);
  }
}

}  // namespace

hipError_t launch_read_codes(const ReadArgs& a, hipStream_t s) {
  if (a.n_slots <= 0) return hipSuccess;
  dim3 grid((unsigned)a.n_slots, 2 * a.st.n_kv_heads);
  hipLaunchKernelGGL(read_codes_kernel, grid, dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_fetch(const FetchArgs& a, hipStream_t s) {
  if (a.n_pos <= 0) return hipSuccess;
  dim3 grid((unsigned)a.n_pos, 2 * a.st.n_kv_heads);
  switch (a.st.layout.head_dim) {
    case 128: hipLaunchKernelGGL((fetch_kernel<128>), grid, dim3(64), 0, s, a); break;
    case 256: hipLaunchKernelGGL((fetch_kernel<256>), grid, dim3(64), 0, s, a); break;
    case 512: hipLaunchKernelGGL((fetch_kernel<512>), grid, dim3(64), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fmkv

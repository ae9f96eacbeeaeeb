// HBM layout of the quantized KV cache (host and device).
//
// The unit of storage is a "head-block": 16 consecutive token slots of one KV
// head. A head-block holds, back to back:
//
//   [K codes][V codes][K scale/bias][V scale/bias]            (affine mode)
//   [K codes][V codes][K norms][V norms]                      (codebook mode)
//   [K rows][V columns]                                       (plain mode)
//
// Affine mode (4- or 8-bit codes, 64-element groups along head_dim, f16
// scale and bias per group per token) arranges codes for the decode kernel's
// matrix-core tiles, so that one 128-bit load per lane feeds the MFMA operands
// without any shuffle:
//
//  K codes, 8-bit: one 1 KiB chunk per 64-dim group g. Lane L = j*16 + t holds
//    16 bytes: dims g*64 + j*16 + e (e = 0..15) of token t, in dim order.
//  K codes, 4-bit: one 1 KiB chunk per 128-dim pair of groups cg. Lane
//    L = j*16 + t holds 4 words; word w = gl*2 + half carries dims
//    cg*128 + gl*64 + half*32 + j*8 + e (e = 0..7), dim e at nibble
//    (e & 1) * 4 + (e >> 1), so that (word >> 4k) & 0x000F000F yields the
//    pair of dims (2k, 2k+1) as two 16-bit lanes.
//  V codes, 8-bit: one 1 KiB chunk per group g. Lane L = q*16 + n holds 16
//    bytes: byte ct*4 + r is dim g*64 + ct*16 + n of token 4q + r.
//  V codes, 4-bit: one 1 KiB chunk per group pair cg. Lane L = q*16 + n holds
//    4 words; dim cg*128 + ct*16 + n (ct = 0..7) of token 4q + r lives in word
//    ct/2, nibble k + 4*(r & 1) with k = (ct & 1)*2 + (r >> 1).
//  Scale/bias: per group g, 16 tokens x {f16 scale, f16 bias} = 64 bytes;
//    the four tokens 4q..4q+3 of a group are one 16-byte load.
//
// Codebook mode (TurboQuant indices, 2/3/4 bits, index of dim d of token t
// written idx(t, d)) keeps bit streams (little-endian: bit i of the stream is
// bit i & 7 of byte i >> 3) laid out for the decode kernel, whose wave pairs
// each own one half of head_dim:
//  K codes: two halves of D*bits bytes, half h holding dims h*D/2 .. h*D/2 +
//    D/2 - 1; in it token t's D/2 indices follow each other: idx(t, d) at bit
//    (t*D/2 + d - h*D/2) * bits. Eight consecutive dims of a token are
//    8*bits consecutive bits (one matrix-core operand).
//  V codes: dim-major, idx(t, d) at bit (d*16 + t) * bits, so the tokens of
//    one dim are consecutive (four of them are one operand) and each half of
//    head_dim is one contiguous range of D*bits bytes.
//  One f16 L2 norm per token row, for K and for V.
//
// Plain mode (unquantized bf16, bits = 16) keeps K token-major -- row t is
// head_dim bf16 at t * head_dim * 2 -- and V dim-major -- dim d holds the 16
// tokens' bf16 at d * 32 -- so that a lane's 16-byte K load is an operand of
// v_mfma_f32_16x16x32_bf16 (8 consecutive dims of one token) and its 8-byte
// V load one of v_mfma_f32_16x16x16_bf16 (4 consecutive tokens of one dim).
//
// Head-block address: base + phys_block * block_stride + head * head_stride,
// with phys_block = block_table[logical block] for a paged pool and the
// logical block itself otherwise.
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define FMKV_HD __host__ __device__ inline
#else
#define FMKV_HD inline
#endif

namespace fmkv {

constexpr int kBlockTokens = 16;
constexpr int kGroup = 64;

enum Mode : int { kAffine = 0, kCodebook = 1, kPlain = 2 };

struct BlockLayout {
  int head_dim;
  int bits;
  int mode;
  int64_t code_bytes;    // per K or V, whole head-block
  int64_t k_codes;       // offsets inside a head-block
  int64_t v_codes;
  int64_t k_meta;        // affine: scale/bias; codebook: norms
  int64_t v_meta;
  int64_t block_bytes;   // rounded up to 256
};

FMKV_HD constexpr int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

FMKV_HD constexpr BlockLayout make_layout(int head_dim, int bits, int mode) {
  BlockLayout L{};
  L.head_dim = head_dim;
  L.bits = bits;
  L.mode = mode;
  L.code_bytes = (int64_t)kBlockTokens * head_dim * bits / 8;
  L.k_codes = 0;
  L.v_codes = L.code_bytes;
  L.k_meta = 2 * L.code_bytes;
  int64_t meta = (mode == kAffine)     ? (int64_t)(head_dim / kGroup) * kBlockTokens * 4
                 : (mode == kCodebook) ? (int64_t)kBlockTokens * 2
                                       : 0;
  L.v_meta = L.k_meta + round_up(meta, 64);
  L.block_bytes = round_up(L.v_meta + round_up(meta, 64), 256);
  return L;
}

// Byte offset (within the K-code region) of the 32-bit word holding dim d of
// token t, and the bit shift of its code inside that word (affine mode).
FMKV_HD void k_code_pos(int bits, int t, int d, int64_t* word_off, int* shift) {
  if (bits == 8) {
    int g = d >> 6, j = (d & 63) >> 4, e = d & 15;
    int64_t byte = (int64_t)g * 1024 + (j * 16 + t) * 16 + e;
    *word_off = byte & ~(int64_t)3;
    *shift = (int)(byte & 3) * 8;
  } else {
    int cg = d >> 7, o = d & 127;
    int gl = o >> 6, half = (o & 63) >> 5, j = (o & 31) >> 3, e = o & 7;
    int w = gl * 2 + half;
    *word_off = (int64_t)cg * 1024 + (j * 16 + t) * 16 + w * 4;
    *shift = ((e & 1) * 4 + (e >> 1)) * 4;
  }
}

FMKV_HD void v_code_pos(int bits, int t, int d, int64_t* word_off, int* shift) {
  int q = t >> 2, r = t & 3;
  if (bits == 8) {
    int g = d >> 6, ct = (d & 63) >> 4, n = d & 15;
    *word_off = (int64_t)g * 1024 + (q * 16 + n) * 16 + ct * 4;
    *shift = r * 8;
  } else {
    int cg = d >> 7, o = d & 127;
    int ct = o >> 4, n = o & 15;
    int k = (ct & 1) * 2 + (r >> 1);
    *word_off = (int64_t)cg * 1024 + (q * 16 + n) * 16 + (ct >> 1) * 4;
    *shift = (k + 4 * (r & 1)) * 4;
  }
}

// Offset of the {f16 scale, f16 bias} pair of group g, token t (affine).
FMKV_HD int64_t scale_pos(int g, int t) { return (int64_t)(g * kBlockTokens + t) * 4; }

// Plain mode: byte offsets of K dim d of token t and of V dim d of token t.
FMKV_HD int64_t plain_k_pos(int head_dim, int t, int d) { return ((int64_t)t * head_dim + d) * 2; }
FMKV_HD int64_t plain_v_pos(int t, int d) { return ((int64_t)d * kBlockTokens + t) * 2; }

// Codebook mode: bit offsets of idx(t, d) in the K and V code regions.
FMKV_HD int64_t cb_k_bit(int head_dim, int bits, int t, int d) {
  const int hd = head_dim / 2, h = d >= hd ? 1 : 0;
  return ((int64_t)h * kBlockTokens * hd + (int64_t)t * hd + (d - h * hd)) * bits;
}
FMKV_HD int64_t cb_v_bit(int bits, int t, int d) { return ((int64_t)d * kBlockTokens + t) * bits; }
// Codebook mode: the token owning bit `bit` of the K or V code region.
FMKV_HD int cb_k_token_of_bit(int head_dim, int bits, int64_t bit) {
  const int64_t half_bits = (int64_t)kBlockTokens * (head_dim / 2) * bits;
  return (int)((bit % half_bits) / ((int64_t)(head_dim / 2) * bits));
}
FMKV_HD int cb_v_token_of_bit(int bits, int64_t bit) {
  return (int)((bit % ((int64_t)kBlockTokens * bits)) / bits);
}

// Position held by `slot` after `offset` appends (ring of `window` slots, or
// linear when window == 0); -1 when the slot is empty.
FMKV_HD int64_t slot_position(int64_t slot, int64_t offset, int64_t window) {
  if (window <= 0) return slot < offset ? slot : -1;
  if (offset <= 0 || slot >= window) return -1;
  int64_t last = offset - 1;
  int64_t p = last - ((last - slot) % window + window) % window;
  return p >= 0 ? p : -1;
}

}  // namespace fmkv

// Read-side kernels:
//  - read_codes: stored codes/scales in a canonical per-slot layout (MLX
//    little-endian packing), for bit-exact comparison with the oracle;
//  - fetch: dequantized, un-rotated K/V of the visible positions in
//    chronological order -- what KVCache::update_and_fetch returns and
//    KVCache::peek_kv reads (src/cache.rs:247-310). In codebook mode this is
//    the reference's round trip output (src/cache.rs:119-125) computed from
//    the stored indices and f16 norm; in plain mode the stored bf16 rows;
//  - sparse_gather: sparse-V attention's second half, which reads the V
//    rows of the kept tokens only.
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

// acc[e] += w_k V[slot_k][tid + e NT] over the kept list (k = 0 .. n-1, in
// list order), V in the rotated domain the attention kernels read (plain
// caches: the stored row): affine code * scale + bias, codebook
// centroid * c * norm (c = 1/sqrt(D), the centroids in LDS), plain bf16. One
// instance per cache mode and width, so that the words of a batch of tokens
// are all loaded before the first is decoded: a batch of kept rows costs one
// memory round trip (with the mode switched per channel, every load waits
// on its own). Batches of 16 while more than 4 tokens remain, then of 4 (a
// short list pays for no padding). Threads past D load channel D-1 and
// leave acc alone.
template <int MODE, int BITS, int D, int NT, int kUnroll, typename BlockOf>
__device__ inline void accumulate_batch(const int* kept_slot, const float* kept_w, int k0, int n,
                                        const BlockLayout& L, const float* cent, float c,
                                        const BlockOf& block_of, float (&acc)[(D + NT - 1) / NT]) {
  constexpr int ND = (D + NT - 1) / NT;
  constexpr int NW = MODE == kCodebook && BITS == 3 ? 2 : 1;  // 3-bit codes straddle words
  constexpr uint32_t mask = MODE == kPlain ? 0xffffu : (1u << BITS) - 1u;
  const int tid = threadIdx.x;
  {
    uint32_t word[kUnroll][ND][NW];
    uint32_t meta[kUnroll][ND];
    uint32_t nrm[kUnroll];
    int tok[kUnroll];
    float w[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const bool ok = k0 + u < n;
      const int k = ok ? k0 + u : n - 1;
      const int slot = kept_slot[k];
      w[u] = ok ? kept_w[k] : 0.0f;
      const uint8_t* blk = block_of(slot / kBlockTokens);
      const int t = slot % kBlockTokens;
      tok[u] = t;
      nrm[u] = MODE == kCodebook ? *reinterpret_cast<const uint16_t*>(blk + L.v_meta + t * 2) : 0u;
#pragma unroll
      for (int e = 0; e < ND; e++) {
        const int d = tid + e * NT < D ? tid + e * NT : D - 1;
        if (MODE == kAffine) {
          int64_t off;
          int sh;
          v_code_pos(BITS, t, d, &off, &sh);
          word[u][e][0] = *reinterpret_cast<const uint32_t*>(blk + L.v_codes + off);
          meta[u][e] = *reinterpret_cast<const uint32_t*>(blk + L.v_meta + scale_pos(d / kGroup, t));
        } else if (MODE == kCodebook) {
          // the word after a 3-bit code's first is in the block (the V norms
          // follow the V codes)
          const uint32_t* region = reinterpret_cast<const uint32_t*>(blk + L.v_codes);
          const int64_t wi = cb_v_bit(BITS, t, d) >> 5;
#pragma unroll
          for (int i = 0; i < NW; i++) word[u][e][i] = region[wi + i];
        } else {
          word[u][e][0] = *reinterpret_cast<const uint16_t*>(blk + L.v_codes + plain_v_pos(t, d));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int t = tok[u];
#pragma unroll
      for (int e = 0; e < ND; e++) {
        const int d = tid + e * NT < D ? tid + e * NT : D - 1;
        float v;
        if (MODE == kAffine) {
          int64_t off;
          int sh;
          v_code_pos(BITS, t, d, &off, &sh);
          v = fmaf((float)((word[u][e][0] >> sh) & mask), f16_bits_to_f32(meta[u][e]),
                   f16_bits_to_f32(meta[u][e] >> 16));
        } else if (MODE == kCodebook) {
          const int sh = (int)(cb_v_bit(BITS, t, d) & 31);
          uint32_t x = word[u][e][0] >> sh;
          if (NW == 2 && sh + BITS > 32) x |= word[u][e][NW - 1] << (32 - sh);
          v = (cent[x & mask] * c) * f16_bits_to_f32(nrm[u]);
        } else {
          v = __uint_as_float(word[u][e][0] << 16);
        }
        acc[e] = fmaf(w[u], k0 + u < n ? v : 0.0f, acc[e]);
      }
    }
  }
}

template <int MODE, int BITS, int D, int NT, typename BlockOf>
__device__ inline void accumulate_kept(const int* kept_slot, const float* kept_w, int n,
                                       const BlockLayout& L, const float* cent, float c,
                                       const BlockOf& block_of, float (&acc)[(D + NT - 1) / NT]) {
  int k0 = 0;
  for (; n - k0 > 4; k0 += 16)
    accumulate_batch<MODE, BITS, D, NT, 16>(kept_slot, kept_w, k0, n, L, cent, c, block_of, acc);
  for (; k0 < n; k0 += 4)
    accumulate_batch<MODE, BITS, D, NT, 4>(kept_slot, kept_w, k0, n, L, cent, c, block_of, acc);
}

// Exclusive prefix count over the work-group: each thread holds `n` items
// that pass; returns the number of passing items of the threads before it
// and sets *total. Two barriers (the count array is reused by the next call).
template <int NT>
__device__ inline int wg_exclusive_count(int n, int* cnt, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = n;  // inclusive scan inside the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) cnt[wave] = x;
  __syncthreads();
  int before = x - n, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) {
    before += w < wave ? cnt[w] : 0;
    tot += cnt[w];
  }
  __syncthreads();
  *total = tot;
  return before;
}

// Sparse-V attention after the statistics pass (src/model/gemma4_attention.rs
// :196-234: softmax weights below tau zeroed, no renormalisation), without
// a second pass over the cache. Work-group (q head h, sequence, part p of
// n_parts):
//  1. M and L of the head from the statistics pass's split (m, l), the
//     decode step's new-token column included, and theta = M + log2(tau L);
//  2. the candidate blocks: those whose largest score for h reaches theta
//     (every part builds the whole list);
//  3. the kept tokens of the part's share of the candidates, from the
//     scores the statistics pass stored (s >= theta), with weight
//     w = 2^(s - M) / L; part 0 also takes the step's new token when its
//     score (its column's m) reaches theta;
//  4. acc[d] = sum of w * V[token][d] (rotated domain);
//  5. out = acc R^T = c * FWHT(acc o s) (plain caches: out = acc).
// With at most kSoloRows candidates (or one part launched) part 0 takes
// them all and writes out, and the other parts return. Otherwise the
// candidates go to n_act = min(n_parts, ceil(nc / kRowsPerPart)) parts (the
// rest return): part p takes [p nc / n_act, (p + 1) nc / n_act), stores acc
// in its partial row, and the last part to count itself on the (sequence,
// q head)'s counter (zeroed by the statistics pass) sums the rows in part
// order and writes out. Every step's loads are issued together (one memory
// round trip each: block maxima with the statistics, scores, V rows), each
// a coalesced sweep (thread tid takes rows and items k NT + tid); the lists
// are in thread-major order (thread, then k), a fixed order, so the sums
// are deterministic.
// Blocks: at most RPT * 256 visible head-blocks per sequence; the launch
// takes the smallest instance that holds the call's rows, and the one of
// the cache's mode and width (MODE, BITS), so that each kernel holds one
// mode's kept-row loop.
template <int D, int RPT, int MODE, int BITS>
__global__ __launch_bounds__(256) void sparse_gather_kernel(AttnArgs a) {
  constexpr int NT = 256, E = D / 64, ND = (D + NT - 1) / NT;
  static_assert(RPT * NT <= kGatherMaxRows, "block rows per thread");
  constexpr int kRound = 64;                // candidates per score round
  constexpr int IPT = kRound * kBlockTokens / NT;  // score items per thread
  constexpr int SPT = 2;                    // statistics per thread per load round
  constexpr int kSoloRows = 32;
  constexpr int kRowsPerPart = 16;
  __shared__ int cand[RPT * NT];
  __shared__ int kept_slot[kRound * kBlockTokens + 1];
  __shared__ float kept_w[kRound * kBlockTokens + 1];
  __shared__ int cnt[NT / 64];
  __shared__ float red[2][NT / 64];
  __shared__ float xs[D];
  __shared__ float cent[16];
  __shared__ int last_s;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.x, seq = blockIdx.y, part = blockIdx.z;
  const int n_parts = (int)gridDim.z;
  const int G = a.group, kvh = h / G, hl = h - kvh * G;
  const BlockLayout L = a.st.layout;
  const int64_t nqh = a.n_q_heads;
  const int64_t T = a.seq_lens ? (int64_t)a.seq_lens[seq] : a.seq_len;
  const SeqGeom geo =
      seq_geometry(T, a.window, a.vis_begin, a.st.table_stride, a.st.block_table != nullptr);
  const int n_splits = n_splits_for(geo, a.bps0, a.bps, a.max_splits, a.skew_p);
  int64_t nrows = geo.blk_hi - geo.blk_lo;
  if (nrows > a.blk_stride) nrows = a.blk_stride;  // (the host plans rows <= blk_stride)
  if (nrows > RPT * NT) nrows = RPT * NT;          // (and <= gather_rows <= RPT NT)
  const int64_t blk_row = ((int64_t)seq * a.st.n_kv_heads + kvh) * a.blk_stride;

  // 1. the loads of the block maxima (rows k NT + tid), the statistics
  // (partials i NT + tid) and the new token's score, together
  // (the centroid reaches LDS after the loads below have been waited for:
  // written here, its load would be waited for alone, a round trip of its own)
  const float cent_v =
      MODE == kCodebook && tid < (1 << BITS) ? centroid(BITS, tid) : 0.0f;
  const int kmax = (int)((nrows + NT - 1) / NT);  // <= RPT
  float bm[RPT];
#pragma unroll
  for (int k = 0; k < RPT; k++) {
    const int64_t rb = (int64_t)k * NT + tid;
    bm[k] = -INFINITY;
    if (k < kmax && rb < nrows) bm[k] = a.blk_max[blk_row * 8 + (int64_t)hl * a.blk_stride + rb];
  }
  const int n_stat = n_splits + a.stats_new_col;
  const int64_t rbase = (int64_t)seq * a.part_stride * nqh + h;
  float2 ml[SPT];
#pragma unroll
  for (int i = 0; i < SPT; i++) {
    const int sp = i * NT + tid;
    ml[i] = sp < n_stat ? *reinterpret_cast<const float2*>(a.stat_ml + (rbase + (int64_t)sp * nqh) * 2)
                        : make_float2(-INFINITY, 0.0f);
  }
  const float m_nt = a.stats_new_col ? a.stat_ml[(rbase + (int64_t)n_splits * nqh) * 2] : -INFINITY;
  float Mt = fmaxf(ml[0].x, ml[1].x);
  for (int sp = SPT * NT + tid; sp < n_stat; sp += NT)
    Mt = fmaxf(Mt, a.stat_ml[(rbase + (int64_t)sp * nqh) * 2]);
  // the head's M: the work-group maximum
  float v = group_max<64>(Mt, lane);
  if (lane == 0) red[0][wave] = v;
  __syncthreads();
  float M = red[0][0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) M = fmaxf(M, red[0][w]);
  // the head's L at M
  float Lt = 0.0f;
  if (M != -INFINITY) {
#pragma unroll
    for (int i = 0; i < SPT; i++) Lt = fmaf(ml[i].y, exp2f(ml[i].x - M), Lt);
    for (int sp = SPT * NT + tid; sp < n_stat; sp += NT) {
      const float2 m2 = *reinterpret_cast<const float2*>(a.stat_ml + (rbase + (int64_t)sp * nqh) * 2);
      Lt = fmaf(m2.y, exp2f(m2.x - M), Lt);
    }
  }
  v = group_sum<64>(Lt, lane);
  if (lane == 0) red[1][wave] = v;
  __syncthreads();
  float Ls = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) Ls += red[1][w];
  const float theta = Ls > 0.0f ? M + log2f(a.tau * Ls) : INFINITY;
  const float inv_l = Ls > 0.0f ? 1.0f / Ls : 0.0f;

  // 2. candidate rows
  static_assert(RPT <= 64, "one flag word per thread");
  uint64_t flags = 0;
#pragma unroll
  for (int k = 0; k < RPT; k++) flags |= (k < kmax && bm[k] >= theta ? 1ull : 0ull) << k;
  int nc;
  int pos = wg_exclusive_count<NT>(__builtin_popcountll(flags), cnt, &nc);
  while (flags) {
    const int k = __builtin_ctzll(flags);
    flags &= flags - 1;
    cand[pos++] = k * NT + tid;
  }
  if (tid < 16) cent[tid] = cent_v;
  __syncthreads();
  const int n_act = nc <= kSoloRows ? 1 : min(n_parts, (nc + kRowsPerPart - 1) / kRowsPerPart);
  const bool solo = n_act == 1;  // part 0 takes every candidate, no merge
  if (part >= n_act) return;
  const int c0 = solo ? 0 : (int)((int64_t)part * nc / n_act);
  const int c1 = solo ? nc : (int)((int64_t)(part + 1) * nc / n_act);

  // block address of logical slot block lb
  const uint8_t* hbase = a.st.base + (int64_t)kvh * a.st.head_stride;
  auto block_of = [&](int64_t lb) -> const uint8_t* {
    int64_t phys = lb;
    if (a.st.block_table) {
      phys = lb < a.st.table_stride ? (int64_t)a.st.block_table[(int64_t)seq * a.st.table_stride + lb] : 0;
      phys = phys < 0 ? 0 : (phys >= a.st.n_blocks ? a.st.n_blocks - 1 : phys);
    }
    return hbase + phys * a.st.block_stride;
  };

  float acc[ND];
#pragma unroll
  for (int e = 0; e < ND; e++) acc[e] = 0.0f;
  // 3. + 4. the part's candidates, kRound at a time; part 0's first round
  // also takes the decode step's new token (appended to its kept list)
  bool nt_pending = part == 0 && a.stats_new_col && m_nt >= theta;
  for (int r0 = c0; r0 < c1 || nt_pending; r0 += kRound) {
    const int rn = c1 - r0 < kRound ? (c1 > r0 ? c1 - r0 : 0) : kRound;
    float sv[IPT];
    int nk = 0;
#pragma unroll
    for (int k = 0; k < IPT; k++) {
      const int item = k * NT + tid, ci = item / kBlockTokens;
      sv[k] = -INFINITY;
      if (ci < rn) {
        const int64_t rb = cand[r0 + ci];
        sv[k] = a.blk_scores[((blk_row + rb) * 8 + hl) * kBlockTokens + item % kBlockTokens];
      }
      nk += sv[k] >= theta ? 1 : 0;
    }
    int total;
    int at = wg_exclusive_count<NT>(nk, cnt, &total);
#pragma unroll
    for (int k = 0; k < IPT; k++) {
      if (sv[k] >= theta) {
        const int item = k * NT + tid;
        kept_slot[at] =
            (int)((geo.blk_lo + cand[r0 + item / kBlockTokens]) * kBlockTokens + item % kBlockTokens);
        kept_w[at] = exp2f(sv[k] - M) * inv_l;
        at++;
      }
    }
    int n = total;
    if (nt_pending) {
      if (tid == 0) {
        kept_slot[total] = (int)(a.window > 0 ? (T - 1) % a.window : T - 1);
        kept_w[total] = exp2f(m_nt - M) * inv_l;
      }
      n = total + 1;
      nt_pending = false;
    }
    __syncthreads();
    accumulate_kept<MODE, BITS, D, NT>(kept_slot, kept_w, n, L, cent, a.c, block_of, acc);
    __syncthreads();
  }

  // 5. merge (several parts) and the inverse rotation
  float* const orow = a.part_o + (((int64_t)seq * a.part_stride + part) * nqh + h) * D;
  if (!solo) {
    // the row through LDS, so that one wave stores it, releases it (an L2
    // write-back at agent scope, one per work-group rather than per wave)
    // and counts the part
#pragma unroll
    for (int e = 0; e < ND; e++) {
      const int d = tid + e * NT;
      if (d < D) xs[d] = acc[e];
    }
    __syncthreads();
    if (wave == 0) {
      for (int d = lane; d < D; d += 64) orow[d] = xs[d];
      __threadfence();  // release the row (agent scope)
      if (lane == 0) last_s = atomicAdd(&a.sv_count[(int64_t)seq * nqh + h], 1) == n_act - 1;
    }
    __syncthreads();
    if (!last_s) return;
    __threadfence();  // acquire the other parts' rows
    // plain loads after the acquire, 16 parts' rows at a time, all issued
    // before the first is added (atomic loads waited one by one); the sum in
    // part order (rows past n_act read row n_act - 1 and add nothing)
    const float* prow0 = a.part_o + ((int64_t)seq * a.part_stride * nqh + h) * D;
#pragma unroll
    for (int e = 0; e < ND; e++) acc[e] = 0.0f;
    for (int q0 = 0; q0 < n_act; q0 += 16) {
      float v[16][ND];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int64_t q = q0 + i < n_act ? q0 + i : n_act - 1;
#pragma unroll
        for (int e = 0; e < ND; e++) {
          const int d = tid + e * NT < D ? tid + e * NT : D - 1;
          v[i][e] = prow0[q * nqh * D + d];
        }
      }
#pragma unroll
      for (int i = 0; i < 16; i++)
#pragma unroll
        for (int e = 0; e < ND; e++) acc[e] += q0 + i < n_act ? v[i][e] : 0.0f;
    }
  }
  const int64_t o_idx = ((int64_t)seq * nqh + h) * D;
  if constexpr (MODE == kPlain) {
#pragma unroll
    for (int e = 0; e < ND; e++) {
      const int d = tid + e * NT;
      if (d < D) {
        if (a.out_f32)
          reinterpret_cast<float*>(a.out)[o_idx + d] = acc[e];
        else
          reinterpret_cast<uint16_t*>(a.out)[o_idx + d] = f32_to_bf16(acc[e]);
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < ND; e++) {
    const int d = tid + e * NT;
    if (d < D) xs[d] = acc[e];
  }
  __syncthreads();
  if (wave == 0) {
    const uint32_t sbits = lane_sign_bits<D>(a.sign_bits, lane);
    float x[E];
#pragma unroll
    for (int i = 0; i < E; i++) x[i] = apply_sign(xs[lane * E + i], sbits, i);
    wave_fwht_signed<E>(x, lane);
    const float cs = fwht_lane_sign(lane) * a.c;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float y = x[i] * cs;
      if (a.out_f32)
        reinterpret_cast<float*>(a.out)[o_idx + lane * E + i] = y;
      else
        reinterpret_cast<uint16_t*>(a.out)[o_idx + lane * E + i] = f32_to_bf16(y);
    }
  }
}

}  // namespace

// The gather instance for the call's rows: RPT block maxima per thread are
// loaded (unrolled, predicated) and held in registers and RPT * 256 list
// entries in LDS, and each row per thread the instance holds beyond the
// call's costs time. Measured at a 32K step (2049 rows), sparse-V tau 1e-3:
// 64 rows per thread 20.95 us, 32 19.6 us, 16 18.3 us, 9 18.0 us; the
// 1024-slot rings of a 30-layer stack's sliding layers (64 rows) gained
// 0.35 us a layer from 16 to 1.
// Instances: 256 rows (a ring of up to 4096 slots), 2304 (a 36K context),
// 4096, 8192 and 16384.
template <int D, int MODE, int BITS>
hipError_t launch_gather_rows(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if (a.gather_rows <= 1 * 256)
    hipLaunchKernelGGL((sparse_gather_kernel<D, 1, MODE, BITS>), grid, dim3(256), 0, s, a);
  else if (a.gather_rows <= 9 * 256)
    hipLaunchKernelGGL((sparse_gather_kernel<D, 9, MODE, BITS>), grid, dim3(256), 0, s, a);
  else if (a.gather_rows <= 16 * 256)
    hipLaunchKernelGGL((sparse_gather_kernel<D, 16, MODE, BITS>), grid, dim3(256), 0, s, a);
  else if (a.gather_rows <= 32 * 256)
    hipLaunchKernelGGL((sparse_gather_kernel<D, 32, MODE, BITS>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((sparse_gather_kernel<D, 64, MODE, BITS>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_gather_mode(const AttnArgs& a, dim3 grid, hipStream_t s) {
  const BlockLayout& L = a.st.layout;
  if (L.mode == kAffine && L.bits == 8) return launch_gather_rows<D, kAffine, 8>(a, grid, s);
  if (L.mode == kAffine && L.bits == 4) return launch_gather_rows<D, kAffine, 4>(a, grid, s);
  if (L.mode == kCodebook && L.bits == 2) return launch_gather_rows<D, kCodebook, 2>(a, grid, s);
  if (L.mode == kCodebook && L.bits == 3) return launch_gather_rows<D, kCodebook, 3>(a, grid, s);
  if (L.mode == kCodebook && L.bits == 4) return launch_gather_rows<D, kCodebook, 4>(a, grid, s);
  if (L.mode == kPlain) return launch_gather_rows<D, kPlain, 16>(a, grid, s);
  return hipErrorInvalidValue;
}

hipError_t launch_sparse_gather(const AttnArgs& a, int n_seqs, hipStream_t s) {
  if (!a.blk_scores || !a.sv_count || !a.blk_max || !a.stat_ml || !a.part_o || a.group < 1 ||
      a.group > 8 || a.gather_parts < 1 || a.gather_parts > a.part_stride ||
      a.gather_rows < 1 || a.gather_rows > kGatherMaxRows)
    return hipErrorInvalidValue;
  dim3 grid((unsigned)a.n_q_heads, (unsigned)n_seqs, (unsigned)a.gather_parts);
  switch (a.st.layout.head_dim) {
    case 128: return launch_gather_mode<128>(a, grid, s);
    case 256: return launch_gather_mode<256>(a, grid, s);
    case 512: return launch_gather_mode<512>(a, grid, s);
    default: return hipErrorInvalidValue;
  }
}

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

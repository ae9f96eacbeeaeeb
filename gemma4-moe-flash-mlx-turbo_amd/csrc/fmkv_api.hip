// C ABI of the MI355X quantized KV cache (include/fmkv.h).
//
// Host-side state mirrors KVCache (src/cache.rs:166-172): the monotonic
// `offset` (RoPE position), the optional sliding `window`, and the stored
// K/V -- here a preallocated device arena of 16-token head-blocks instead of
// MLX arrays re-concatenated on every append (src/cache.rs:132-148).
// Errors never cross the boundary as exceptions: every entry point returns a
// status and records a message for fmkv_last_error().
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fmkv.h"
#include "fmkv_internal.h"

using fmkv::BlockLayout;

namespace {

thread_local std::string g_err;
int32_t g_bps_override = 0;
// sparse-V after the statistics pass: 1 the gather, 0 the gated pass and the
// combine (fmkv_set_sparse_v_gather)
int32_t g_sparse_gather = 1;

// Kernel-timing records (fmkv_profile_enable / fmkv_profile_collect).
struct Profiler {
  std::vector<hipEvent_t> ev;  // pairs
  int32_t max_records = 0;
  int32_t used = 0;
  void clear_events() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    ev.clear();
    used = 0;
  }
} g_prof;

// Next event pair for a decode launch, or {null, null} when not profiling.
void next_events(hipEvent_t* e0, hipEvent_t* e1) {
  *e0 = *e1 = nullptr;
  if (g_prof.max_records <= 0 || g_prof.used >= g_prof.max_records) return;
  const size_t i = 2 * (size_t)g_prof.used;
  *e0 = g_prof.ev[i];
  *e1 = g_prof.ev[i + 1];
  g_prof.used++;
}

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FMKV_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// src/cache.rs:29-43: MMIX LCG stepped before each draw, +1 iff bit 63 == 0.
std::vector<float> lcg_signs(int n, uint64_t seed) {
  std::vector<float> s(n);
  uint64_t state = seed;
  for (int i = 0; i < n; i++) {
    state = state * 6364136223846793005ull + 1442695040888963407ull;
    s[i] = ((state >> 63) & 1ull) == 0 ? 1.0f : -1.0f;
  }
  return s;
}

int check_desc(const fmkv_cache_desc* d) {
  if (!d) return fail(FMKV_ERR_INVALID_ARG, "descriptor is null");
  if (d->n_kv_heads < 1 || d->n_kv_heads > 256)
    return fail(FMKV_ERR_INVALID_ARG, "n_kv_heads must be in [1, 256]");
  if (d->head_dim != 128 && d->head_dim != 256 && d->head_dim != 512)
    return fail(FMKV_ERR_UNSUPPORTED, "head_dim must be 128, 256 or 512");
  if (d->group_size != 64) return fail(FMKV_ERR_UNSUPPORTED, "group_size must be 64");
  if (d->mode == FMKV_MODE_AFFINE) {
    if (d->bits != 4 && d->bits != 8)
      return fail(FMKV_ERR_UNSUPPORTED, "affine mode supports 4 or 8 bits");
  } else if (d->mode == FMKV_MODE_CODEBOOK) {
    if (d->bits < 2 || d->bits > 4)
      return fail(FMKV_ERR_UNSUPPORTED, "codebook mode supports 2, 3 or 4 bits");
  } else if (d->mode == FMKV_MODE_PLAIN) {
    if (d->bits != 16) return fail(FMKV_ERR_UNSUPPORTED, "plain (bf16) mode has bits = 16");
  } else {
    return fail(FMKV_ERR_UNSUPPORTED, "unknown mode");
  }
  if (d->window < 0) return fail(FMKV_ERR_INVALID_ARG, "window must be >= 0");
  if (d->window > 0) {
    if (d->window > (1 << 30)) return fail(FMKV_ERR_INVALID_ARG, "window must be <= 2^30");
  } else {
    if (d->capacity < 1) return fail(FMKV_ERR_INVALID_ARG, "capacity must be >= 1 for a global cache");
    if (d->capacity > ((int64_t)1 << 31) - 64)
      return fail(FMKV_ERR_INVALID_ARG, "capacity must be < 2^31 - 64");
  }
  return FMKV_OK;
}

// Slots of a ring: the sliding window W rounded up to whole 16-token
// head-blocks. Position p is stored at slot p mod ring_slots, so the ring
// holds the last ring_slots positions; the last W of them are visible
// (visible_begin), the others masked by position.
int64_t ring_slots(const fmkv_cache_desc& d) {
  return d.window > 0 ? fmkv::round_up(d.window, fmkv::kBlockTokens) : 0;
}

int64_t n_slots_of(const fmkv_cache_desc& d) {
  return d.window > 0 ? ring_slots(d) : fmkv::round_up(d.capacity, fmkv::kBlockTokens);
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 256;
  return cus;
}

// Decode work-groups per CU the split plan aims at: the affine and codebook
// kernels' LDS staging fills a CU; the plain kernel's work-groups are about
// half as large (two per CU).
int attn_wg_per_cu(const fmkv_cache_desc& d) {
  return d.mode == FMKV_MODE_PLAIN ? 2 : fmkv::kAttnWgPerCu;
}

// Work-groups per CU of a paged batch's decode kernel when its splits are
// long enough for single-wave streams (at least 8 blocks each): 3 for
// affine head-blocks of at most 1024 code bits per token (four-wave
// work-groups), else 1.
int paged_solo_slots(const fmkv_cache_desc& d) {
  return d.mode == FMKV_MODE_AFFINE && d.head_dim * d.bits <= 1024 ? 3 : 1;
}

// Split-K plan: blocks per split such that the grid has about `wg_per_cu`
// work-groups per CU (each keeps several blocks in flight, so one per CU
// already saturates HBM; more would only add split partials), `reserved` of
// them going to other work of the same launch (the new-token column).
int32_t choose_bps(int64_t total_head_blocks, int cus, int wg_per_cu, int64_t reserved = 0,
                   int64_t min_bps = 1) {
  if (g_bps_override > 0) return g_bps_override;
  int64_t target = (int64_t)wg_per_cu * cus;
  if (target - reserved >= target / 2) target -= reserved;
  int64_t bps = (total_head_blocks + target - 1) / target;
  if (bps < min_bps) bps = min_bps;
  if (bps < 1) bps = 1;
  return (int32_t)bps;
}

// src/cache.rs:29-43 signs as a bit mask (bit d set = -1), the form the
// decode kernel takes them in as a kernel argument.
void sign_bits_of(const fmkv_cache_desc& d, uint32_t out[16]) {
  std::vector<float> s = lcg_signs(d.head_dim, d.sign_seed);
  for (int w = 0; w < 16; w++) out[w] = 0;
  for (int i = 0; i < d.head_dim; i++)
    if (s[i] < 0.0f) out[i >> 5] |= 1u << (i & 31);
}

// Caller-provided device memory standing in for a handle's workspace (the
// no-allocation decode step); ptr null: the handle's own workspace.
struct ExtWorkspace {
  float* ptr = nullptr;
  size_t bytes = 0;
};

struct Workspace {
  float* ptr = nullptr;
  size_t bytes = 0;
  // zero: a new allocation starts zeroed (head-block staging, whose
  // unwritten slots are read, masked, as the cache's own are)
  int ensure(size_t need, bool zero = false) {
    if (need <= bytes) return FMKV_OK;
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
    hipError_t e = hipMalloc(&ptr, need);
    if (e != hipSuccess) return fail(FMKV_ERR_OOM, "workspace allocation failed");
    if (zero) {
      e = hipMemset(ptr, 0, need);
      if (e != hipSuccess) return hip_fail(e, "hipMemset(workspace)");
    }
    bytes = need;
    return FMKV_OK;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
};

}  // namespace

struct fmkv_cache {
  fmkv_cache_desc desc;
  BlockLayout layout;
  uint8_t* arena;
  int64_t n_blocks;
  float* d_signs;
  uint32_t sign_bits[16];
  float c, sqrt_d;
  int64_t offset;
  int64_t vis_begin;
  Workspace ws;
  Workspace stage;  // prefill on a ring: the chunk's quantized rows
  int cus;
};

struct fmkv_pool {
  fmkv_cache_desc desc;
  BlockLayout layout;
  uint8_t* arena;
  int64_t n_blocks;
  float* d_signs;
  uint32_t sign_bits[16];
  float c, sqrt_d;
  Workspace ws;
  int cus;
};

namespace {

fmkv::Store cache_store(const fmkv_cache* c) {
  fmkv::Store s;
  s.base = c->arena;
  s.block_stride = c->layout.block_bytes;
  s.head_stride = c->n_blocks * c->layout.block_bytes;
  s.block_table = nullptr;
  s.table_stride = 0;
  s.n_blocks = c->n_blocks;
  s.n_kv_heads = c->desc.n_kv_heads;
  s.layout = c->layout;
  return s;
}

fmkv::Store pool_store(const fmkv_pool* p, const int32_t* table, int32_t stride) {
  fmkv::Store s;
  s.base = p->arena;
  s.block_stride = p->layout.block_bytes * p->desc.n_kv_heads;
  s.head_stride = p->layout.block_bytes;
  s.block_table = table;
  s.table_stride = stride;
  s.n_blocks = p->n_blocks;
  s.n_kv_heads = p->desc.n_kv_heads;
  s.layout = p->layout;
  return s;
}

int64_t visible_begin(const fmkv_cache* c) {
  int64_t b = c->vis_begin;
  if (c->desc.window > 0 && c->offset - c->desc.window > b) b = c->offset - c->desc.window;
  return b < 0 ? 0 : b;
}

int make_signs(const fmkv_cache_desc& d, float** out) {
  std::vector<float> s = lcg_signs(d.head_dim, d.sign_seed);
  hipError_t e = hipMalloc(out, sizeof(float) * d.head_dim);
  if (e != hipSuccess) return fail(FMKV_ERR_OOM, "sign vector allocation failed");
  e = hipMemcpy(*out, s.data(), sizeof(float) * d.head_dim, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy(signs)");
  return FMKV_OK;
}

int check_attn_args(const fmkv_cache_desc& d, const void* q, int32_t n_q_heads, float tau,
                    const void* out, int32_t out_dtype) {
  if (!q || !out) return fail(FMKV_ERR_INVALID_ARG, "q/out must be device pointers");
  if (n_q_heads < d.n_kv_heads || n_q_heads % d.n_kv_heads != 0)
    return fail(FMKV_ERR_INVALID_ARG, "n_q_heads must be a multiple of n_kv_heads");
  if (n_q_heads / d.n_kv_heads > 8)
    return fail(FMKV_ERR_UNSUPPORTED, "at most 8 query heads per KV head");
  if (!(tau >= 0.0f) || !std::isfinite(tau))
    return fail(FMKV_ERR_INVALID_ARG, "sparse_v_tau must be finite and >= 0");
  if (out_dtype != FMKV_DTYPE_BF16 && out_dtype != FMKV_DTYPE_F32)
    return fail(FMKV_ERR_INVALID_ARG, "out_dtype must be FMKV_DTYPE_BF16 or FMKV_DTYPE_F32");
  return FMKV_OK;
}

// Validation and launch arguments of an append of n tokens at the cache's
// offset (no state change).
// The layer prologue's arguments (no HIP call): a k_norm
// weight, positive finite eps and theta, rope_dims a power of 2 in
// [2 * head_dim / 64, head_dim] (the rotated pairs then sit in different
// lanes of the append kernel's row layout).
int check_prologue(const fmkv_cache_desc& d, const fmkv_kv_prologue* pro) {
  if (!pro) return fail(FMKV_ERR_INVALID_ARG, "prologue is null");
  if (!pro->k_norm_weight) return fail(FMKV_ERR_INVALID_ARG, "k_norm_weight must be a device pointer");
  if (!(pro->eps > 0.0f) || !std::isfinite(pro->eps))
    return fail(FMKV_ERR_INVALID_ARG, "eps must be finite and > 0");
  if (!(pro->rope_theta > 0.0f) || !std::isfinite(pro->rope_theta))
    return fail(FMKV_ERR_INVALID_ARG, "rope_theta must be finite and > 0");
  const int rd = pro->rope_dims;
  if (rd < 2 * (d.head_dim / 64) || rd > d.head_dim || (rd & (rd - 1)) != 0)
    return fail(FMKV_ERR_UNSUPPORTED,
                "rope_dims must be a power of 2 in [2 * head_dim / 64, head_dim]");
  if (pro->v_from_k != 0 && pro->v_from_k != 1)
    return fail(FMKV_ERR_INVALID_ARG, "v_from_k must be 0 or 1");
  return FMKV_OK;
}

void set_prologue(const fmkv_kv_prologue* pro, fmkv::AppendArgs* a) {
  a->k_norm_w = static_cast<const uint16_t*>(pro->k_norm_weight);
  a->eps = pro->eps;
  a->rope_dims = pro->rope_dims;
  a->rope_theta = pro->rope_theta;
  a->v_from_k = pro->v_from_k;
}

int prepare_append(const fmkv_cache* c, const void* k, const void* v, int64_t n,
                   fmkv::AppendArgs* a, int64_t* tasks) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (n < 0) return fail(FMKV_ERR_INVALID_ARG, "n_tokens must be >= 0");
  if (n == 0) return FMKV_OK;
  if (!k || !v) return fail(FMKV_ERR_INVALID_ARG, "k/v must be device pointers");
  if (n > ((int64_t)1 << 30)) return fail(FMKV_ERR_INVALID_ARG, "n_tokens too large");
  const int64_t W = ring_slots(c->desc);  // ring slots (0: linear)
  if (W == 0 && c->offset + n > c->desc.capacity)
    return fail(FMKV_ERR_CAPACITY, "append of " + std::to_string(n) + " tokens at offset " +
                                       std::to_string(c->offset) + " exceeds capacity " +
                                       std::to_string(c->desc.capacity));
  if (c->offset + n > ((int64_t)1 << 31) - 64)
    return fail(FMKV_ERR_CAPACITY, "position counter would exceed 2^31");
  a->st = cache_store(c);
  a->k = static_cast<const uint16_t*>(k);
  a->v = static_cast<const uint16_t*>(v);
  a->start_pos = nullptr;
  a->start_scalar = c->offset;
  a->n_new = (int32_t)n;
  a->window = (int32_t)W;
  std::memcpy(a->sign_bits, c->sign_bits, sizeof(a->sign_bits));
  a->c = c->c;
  a->sqrt_d = c->sqrt_d;
  a->cb_bits = c->desc.bits;
  if (W > 0) {
    const int64_t n_eff = n < W ? n : W;
    *tasks = (n_eff + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens + 1;
    if (*tasks > W / fmkv::kBlockTokens) *tasks = W / fmkv::kBlockTokens;
  } else {
    *tasks = (c->offset + n - 1) / fmkv::kBlockTokens - c->offset / fmkv::kBlockTokens + 1;
  }
  return FMKV_OK;
}

// Split-K plan of one decode attention launch: blocks per split (bps, bps0
// for split 0), split columns per sequence and the XCD-aware skew.
void plan_splits(int cus, int H, int32_t n_seqs, int64_t nblk, int wg_per_cu, int min_bps,
                 int first_mult, int new_col, bool paged, fmkv::AttnArgs* a) {
  if (nblk < 1) nblk = 1;
  // one sequence: the new-token column takes CUs of its own; many sequences:
  // the dispatcher fills CUs as work-groups finish
  const int64_t reserved = n_seqs == 1 ? (int64_t)new_col * H : 0;
  a->bps = choose_bps(nblk * H * n_seqs, cus, wg_per_cu, reserved, min_bps);
  // the split columns are the grid's z dimension (at most 65535)
  if ((nblk + a->bps - 1) / a->bps + new_col > 65535)
    a->bps = (int32_t)((nblk + 65534 - new_col) / (65535 - new_col));
  // split 0 of each sequence takes first_mult x bps blocks
  const int64_t bps0 = (int64_t)a->bps * first_mult;
  a->bps0 = (int32_t)(bps0 < nblk ? bps0 : nblk);
  if (a->bps0 < a->bps) a->bps0 = a->bps;
  a->max_splits = (int32_t)(nblk <= a->bps0 ? 1 : 1 + (nblk - a->bps0 + a->bps - 1) / a->bps);
  a->skew_p = a->skew_extra = 0;
  // XCD-aware plan for one sequence over two KV heads at one work-group per
  // CU: the work-groups (KV head h, split s) go round-robin to the 8 XCDs by
  // linear id h + 2 s, so the splits s = 0 mod 4 land on XCDs 0 and 1, which
  // start first (the others start 1.4 to 4.4 us later). Every CU gets a split
  // of bps blocks and the blocks left over go one each to the splits
  // s = 0 mod p, p = 4 when they fit there (else 2, else 1: the first
  // splits), instead of bps + 1 blocks for every work-group and some CUs
  // left idle.
  if (n_seqs == 1 && H == 2 && wg_per_cu == 1 && !paged &&
      g_bps_override <= 0) {
    const int64_t n_s = (cus - (int64_t)new_col * H) / H;
    const int64_t b = n_s > 0 ? nblk / n_s : 0;
    const int64_t extra = nblk - n_s * b;
    if (n_s >= 8 && b >= fmkv::kAttnPlanMinSkewBlocks) {
      int p = 4;
      while (p > 1 && extra > (n_s + p - 1) / p) p >>= 1;
      a->bps = a->bps0 = (int32_t)b;
      a->max_splits = (int32_t)n_s;
      a->skew_p = p;
      a->skew_extra = (int32_t)extra;
    }
  }
}

// Split-K plan, workspace ([part_o | part_ml]) and launch arguments of
// decode attention; new_col adds the decode step's new-token column.
template <typename Owner>
int prepare_attention_common(Owner* o, const fmkv::Store& st, int32_t n_seqs, int64_t nblk,
                             int64_t blk_cap, const void* q, int32_t n_q_heads, float scale, float tau, void* out,
                             int32_t out_dtype, int wg_per_cu, int min_bps, int first_mult,
                             int new_col, fmkv::AttnArgs* a, ExtWorkspace ext = {}) {
  int rc = check_attn_args(o->desc, q, n_q_heads, tau, out, out_dtype);
  if (rc) return rc;
  const int H = o->desc.n_kv_heads, D = o->desc.head_dim;
  a->st = st;
  a->group = n_q_heads / H;
  a->n_q_heads = n_q_heads;
  a->q = static_cast<const uint16_t*>(q);
  a->qscale = scale * 1.4426950408889634f;
  std::memcpy(a->sign_bits, o->sign_bits, sizeof(a->sign_bits));
  a->c = o->c;
  a->sqrt_d = o->sqrt_d;
  plan_splits(o->cus, H, n_seqs, nblk, wg_per_cu, min_bps, first_mult, new_col,
              st.block_table != nullptr, a);
  a->new_col = new_col;
  a->part_stride = a->max_splits + new_col;
  // sparse-V (tau > 0) always goes through the split partials and the
  // combine, which normalises by the stats pass's full softmax sum
  a->tau = tau;
  a->direct = a->max_splits == 1 && !new_col && tau == 0.0f;
  a->k_new = a->v_new = nullptr;
  a->out = out;
  a->out_f32 = out_dtype == FMKV_DTYPE_F32;
  const size_t n_rows = a->direct ? 0 : (size_t)n_seqs * a->part_stride * n_q_heads;
  // sparse-V: [theta | M | L] per (sequence, q head), then the stats pass's
  // split (m, l) in a region of their own
  const size_t n_stats = tau > 0.0f ? 3 * (size_t)n_seqs * n_q_heads : 0;
  const size_t n_stat_ml = tau > 0.0f ? 2 * n_rows : 0;
  const size_t stat_off = n_rows * (D + 2) + n_stats;
  // sparse-V block maxima, 16-byte aligned (read as float4)
  const size_t blk_off = (stat_off + n_stat_ml + 3) & ~(size_t)3;
  // (rows sized for the most blocks a sequence can hold, so that the
  // library's workspace does not grow as the context does; a caller's
  // scratch holds the call's blocks only)
  a->blk_stride = (int32_t)std::max<int64_t>(std::max<int64_t>(nblk, ext.ptr ? 0 : blk_cap), 1);
  const size_t n_blk = tau > 0.0f ? (size_t)n_seqs * H * a->blk_stride * 8 : 0;
  // sparse-V gather: the candidate blocks' scores (16 per block row and
  // head) after the maxima, then one arrival counter per (sequence, q head);
  // without room for them in a caller's scratch, the gated pass
  bool gather = tau > 0.0f && g_sparse_gather && nblk <= fmkv::kGatherMaxRows;
  const size_t score_off = blk_off + n_blk;  // a multiple of 4 floats
  const size_t cnt_off = score_off + 16 * n_blk;
  const size_t need_gather = (cnt_off + (size_t)n_seqs * n_q_heads) * sizeof(float);
  if (gather && ext.ptr && need_gather > ext.bytes) gather = false;
  const size_t need =
      gather ? need_gather : (n_blk ? blk_off + n_blk : stat_off + n_stat_ml) * sizeof(float);
  float* ws = ext.ptr;
  if (ws) {
    if (need > ext.bytes)
      return fail(FMKV_ERR_CAPACITY, "this call needs " + std::to_string(need) +
                                         " bytes of split partials; the no-allocation scratch "
                                         "holds " + std::to_string(ext.bytes));
  } else {
    // One cache: the workspace is sized once for the largest plan the
    // cache's capacity allows (split count at most the planned work-groups
    // per KV head + 1, a new-token column, sparse-V statistics and block
    // maxima), so that it does not grow as the context does and a decode
    // step captured into a HIP graph stays valid. A paged batch's need
    // depends on each call's batch and grows on demand.
    size_t alloc = need;
    if (n_seqs == 1 && !st.block_table) {
      const int64_t per_head = ((int64_t)wg_per_cu * o->cus + H - 1) / H + 1;
      const int64_t max_splits =
          std::max<int64_t>(g_bps_override > 0 ? blk_cap : std::min<int64_t>(blk_cap, per_head),
                            a->max_splits);
      const size_t rows = (size_t)(max_splits + 1) * n_q_heads;
      const size_t off = (rows * (D + 2) + 3 * (size_t)n_q_heads + 2 * rows + 3) & ~(size_t)3;
      const size_t blks = (size_t)H * std::max<int64_t>(std::max<int64_t>(blk_cap, nblk), 1) * 8;
      alloc = std::max(need, (off + blks * (gather ? 17 : 1) + (gather ? n_q_heads : 0)) * sizeof(float));
    }
    rc = o->ws.ensure(alloc);
    if (rc) return rc;
    ws = o->ws.ptr;
  }
  a->part_o = n_rows ? ws : nullptr;
  a->part_ml = n_rows ? ws + n_rows * D : nullptr;
  a->tau_stats = n_stats ? ws + n_rows * (D + 2) : nullptr;
  a->stat_ml = n_stat_ml ? ws + stat_off : nullptr;
  a->blk_max = n_blk ? ws + blk_off : nullptr;
  a->blk_scores = gather ? ws + score_off : nullptr;
  a->sv_count = gather ? reinterpret_cast<int32_t*>(ws + cnt_off) : nullptr;
  if (gather) {
    // parts per (sequence, q head): the kept tokens, and so the candidate
    // blocks, are at most min(visible tokens, 1 / tau); one part per 128 of
    // them, at most 64 (the gather uses one per 16 candidate blocks)
    const double inv_tau = std::ceil(1.0 / (double)tau);
    const int64_t bound = std::min<int64_t>(nblk * fmkv::kBlockTokens,
                                            inv_tau < 1e15 ? (int64_t)inv_tau : INT64_MAX);
    a->gather_parts = (int32_t)std::clamp<int64_t>((bound + 127) / 128, 1,
                                                   std::min<int64_t>(a->part_stride, 16));
    a->gather_rows = (int32_t)std::max<int64_t>(nblk, 1);
  }
  return FMKV_OK;
}

// Decode attention over the first T positions of a cache.
int prepare_attention(fmkv_cache* c, int64_t T, const void* q, int32_t n_q_heads, float scale,
                      float tau, void* out, int32_t out_dtype, int new_col, fmkv::AttnArgs* a,
                      ExtWorkspace ext = {}) {
  // a ring's slots; its visible positions are the last `window` of the T,
  // which the kernels test per slot whenever that hides stored slots
  const int64_t W = ring_slots(c->desc);
  a->seq_lens = nullptr;
  a->seq_len = T;
  a->window = W;
  a->vis_begin = W > 0 ? std::max<int64_t>(c->vis_begin, T - c->desc.window) : c->vis_begin;
  const int64_t filled = W > 0 ? std::min<int64_t>(T, W) : T;
  const int64_t vb = W > 0 ? 0 : c->vis_begin;
  const int64_t nblk =
      (filled + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens - vb / fmkv::kBlockTokens;
  const int wg_per_cu = attn_wg_per_cu(c->desc);
  const int64_t blk_cap = n_slots_of(c->desc) / fmkv::kBlockTokens;
  return prepare_attention_common(c, cache_store(c), 1, nblk, blk_cap, q, n_q_heads, scale, tau,
                                  out, out_dtype, wg_per_cu, 1, 1, new_col, a, ext);
}

int prepare_paged_append(const fmkv_pool* p, const void* k, const void* v,
                         const int32_t* block_tables, int32_t max_blocks, const int32_t* start_pos,
                         int32_t n_seqs, int32_t n_new, fmkv::AppendArgs* a, int* tasks) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  if (n_seqs < 0 || n_new < 0 || max_blocks < 1)
    return fail(FMKV_ERR_INVALID_ARG, "n_seqs/n_new must be >= 0 and max_blocks >= 1");
  if (n_seqs == 0 || n_new == 0) return FMKV_OK;
  if (!k || !v || !block_tables || !start_pos)
    return fail(FMKV_ERR_INVALID_ARG, "k/v/block_tables/start_pos must be device pointers");
  if (n_seqs > 65535) return fail(FMKV_ERR_INVALID_ARG, "at most 65535 sequences per call");
  a->st = pool_store(p, block_tables, max_blocks);
  a->k = static_cast<const uint16_t*>(k);
  a->v = static_cast<const uint16_t*>(v);
  a->start_pos = start_pos;
  a->start_scalar = 0;
  a->n_new = n_new;
  a->window = 0;
  std::memcpy(a->sign_bits, p->sign_bits, sizeof(a->sign_bits));
  a->c = p->c;
  a->sqrt_d = p->sqrt_d;
  a->cb_bits = p->desc.bits;
  *tasks =(n_new + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens + 1;
  return FMKV_OK;
}

int prepare_paged_attention(fmkv_pool* p, const void* q, const int32_t* block_tables,
                            int32_t max_blocks, const int32_t* seq_lens, int32_t n_seqs,
                            int32_t max_seq_len, int32_t n_q_heads, float scale, float tau,
                            void* out, int32_t out_dtype, int new_col, fmkv::AttnArgs* a) {
  if (n_seqs < 0 || max_seq_len < 0 || max_blocks < 1)
    return fail(FMKV_ERR_INVALID_ARG, "bad n_seqs / max_seq_len / max_blocks");
  if (n_seqs > 0 && (!block_tables || !seq_lens))
    return fail(FMKV_ERR_INVALID_ARG, "block_tables/seq_lens are null");
  if ((int64_t)max_seq_len > (int64_t)max_blocks * fmkv::kBlockTokens)
    return fail(FMKV_ERR_INVALID_ARG, "max_seq_len exceeds max_blocks * 16");
  if (n_seqs > 65535) return fail(FMKV_ERR_INVALID_ARG, "at most 65535 sequences per call");
  a->seq_lens = seq_lens;
  a->seq_len = 0;
  a->window = 0;
  a->vis_begin = 0;
  const int64_t nblk = (max_seq_len + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens;
  // Ragged lengths: the bound counts every sequence at max_seq_len, so the
  // plan aims at several work-groups per CU (the dispatcher balances their
  // uneven sizes), but at least 64 blocks each (a work-group's prologue and
  // epilogue cost about as much as a dozen blocks) -- unless that would
  // leave CUs idle: the floor never exceeds one CU's share of all blocks,
  // so a small batch at long context still spreads over every CU. When the
  // grid holds at least four work-groups per CU, each sequence's first split
  // is four times larger: the big work-groups start first and the small
  // ones fill the tail (32 sequences of 512..16384 tokens: bps 171, 197 us;
  // equal splits at four per CU: 207 us). A grid of fewer work-groups has
  // no tail to fill, and a larger first split would only end last.
  //
  // Affine head-blocks of at most 1024 code bits per token (head_dim 128,
  // head_dim 256 at 4 bits) run as work-groups of four single-wave streams,
  // three to a CU (slots = 3): the plan counts slots instead of CUs, six
  // work-groups per slot, and the floor is at most one slot's share (one
  // sequence of 65536 tokens, Hkv 8, head_dim 256, 4 bits: bps 43, one
  // work-group per slot, 40.7 us; bps 22 or 128: 47.6 / 52.5 us; the 32
  // ragged sequences above at bps 57..96: 173-178 us, against 202 us with
  // twelve-wave work-groups, one per CU).
  const int n_s = n_seqs > 0 ? n_seqs : 1;
  const int64_t total = nblk * p->desc.n_kv_heads * n_s;
  const int slots = paged_solo_slots(p->desc);
  const int64_t n_slots = (int64_t)slots * p->cus;
  const int64_t share = (total + n_slots - 1) / n_slots;
  const int min_bps = (int)std::min<int64_t>(64, std::max<int64_t>(share, 1));
  const int wg_per_cu = 6 * slots * fmkv::kAttnWgPerCu;
  const int64_t bps = choose_bps(total, p->cus, wg_per_cu, 0, min_bps);
  const int first_mult = total >= 4 * n_slots * bps ? 4 : 1;
  return prepare_attention_common(p, pool_store(p, block_tables, max_blocks), n_s, nblk,
                                  max_blocks, q, n_q_heads, scale, tau, out, out_dtype, wg_per_cu,
                                  min_bps, first_mult, new_col, a);
}

int decode_step_impl(fmkv_cache* c, const void* k, const void* v, int64_t n, const void* q,
                     int32_t n_q_heads, float scale, float tau, void* out, int32_t out_dtype,
                     void* stream, ExtWorkspace ext, const fmkv_kv_prologue* pro = nullptr);

// The prologue on the decode step's new-token column (a fused step).
void set_prologue(const fmkv_kv_prologue* pro, fmkv::AttnArgs* a) {
  a->k_norm_w = static_cast<const uint16_t*>(pro->k_norm_weight);
  a->eps = pro->eps;
  a->rope_dims = pro->rope_dims;
  a->rope_theta = pro->rope_theta;
}

// The decode attention kernel of the cache's mode (and the split combine).
hipError_t launch_attention(const fmkv::AttnArgs& a, int n_seqs, int n_kv_heads, hipStream_t s,
                            hipEvent_t e0, hipEvent_t e1) {
  if (a.st.layout.mode == fmkv::kCodebook)
    return fmkv::launch_cb_decode_attention(a, n_seqs, n_kv_heads, s, e0, e1);
  if (a.st.layout.mode == fmkv::kPlain)
    return fmkv::launch_plain_decode_attention(a, n_seqs, n_kv_heads, s, e0, e1);
  return fmkv::launch_decode_attention(a, n_seqs, n_kv_heads, s, e0, e1);
}

}  // namespace

// Device memory of fmkv_decode_step_noalloc: the split partials (and
// sparse-V statistics) of one decode step, as the handle's workspace holds
// them for fmkv_decode_step. Every GPU holds its own copy for the life of the
// process; in host code the name only stands in for it, so the library takes
// each device's address once (noalloc_scratch) and passes that address on.
// The lookup runs at set-up, when a cache handle is created on the device:
// the runtime materialises the symbol's storage on the first lookup (about
// 10 MiB of device memory on one MI355X), which the allocation-free entry
// point must not do. Calls on one GPU share it: every call writes what it
// reads before reading it, and calls that overlap in time on one GPU race.
static __device__ __align__(256) uint8_t scratch[FMKV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device with the
// device current (hipGetSymbolAddress allocates nothing).
int noalloc_scratch(ExtWorkspace* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(FMKV_ERR_UNSUPPORTED, "device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_dev[dev] = p;
  }
  out->ptr = static_cast<float*>(g_scratch_dev[dev]);
  out->bytes = FMKV_NOALLOC_SCRATCH_BYTES;
  return FMKV_OK;
}

}  // namespace

extern "C" {

const char* fmkv_last_error(void) { return g_err.c_str(); }

int fmkv_validate_desc(const fmkv_cache_desc* desc) { return check_desc(desc); }

int fmkv_layout_bytes(const fmkv_cache_desc* desc, int64_t* block_bytes, int64_t* arena_bytes) {
  int rc = check_desc(desc);
  if (rc) return rc;
  const BlockLayout L = fmkv::make_layout(desc->head_dim, desc->bits, desc->mode);
  if (block_bytes) *block_bytes = L.block_bytes;
  if (arena_bytes)
    *arena_bytes = L.block_bytes * desc->n_kv_heads * (n_slots_of(*desc) / fmkv::kBlockTokens);
  return FMKV_OK;
}

int fmkv_cache_create(const fmkv_cache_desc* desc, fmkv_cache** out) {
  int rc = check_desc(desc);
  if (rc) return rc;
  if (!out) return fail(FMKV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  fmkv_cache* c = new fmkv_cache();
  c->desc = *desc;
  c->layout = fmkv::make_layout(desc->head_dim, desc->bits, desc->mode);
  c->n_blocks = n_slots_of(*desc) / fmkv::kBlockTokens;
  c->c = 1.0f / std::sqrt((float)desc->head_dim);
  c->sqrt_d = std::sqrt((float)desc->head_dim);
  c->offset = 0;
  c->vis_begin = 0;
  c->arena = nullptr;
  c->d_signs = nullptr;
  const int64_t bytes = c->layout.block_bytes * c->n_blocks * desc->n_kv_heads;
  hipError_t e = hipMalloc(&c->arena, bytes);
  if (e != hipSuccess) {
    delete c;
    return fail(FMKV_ERR_OOM, "cache arena allocation failed (" + std::to_string(bytes) + " bytes)");
  }
  e = hipMemset(c->arena, 0, bytes);
  if (e != hipSuccess) {
    (void)hipFree(c->arena);
    delete c;
    return hip_fail(e, "hipMemset(arena)");
  }
  rc = make_signs(*desc, &c->d_signs);
  if (rc) {
    (void)hipFree(c->arena);
    delete c;
    return rc;
  }
  sign_bits_of(*desc, c->sign_bits);
  c->cus = device_cus();
  // set-up of the no-allocation decode step's scratch on this device (once
  // per device; later creations find the address recorded)
  ExtWorkspace ext;
  rc = noalloc_scratch(&ext);
  if (rc) {
    (void)fmkv_cache_destroy(c);
    return rc;
  }
  *out = c;
  return FMKV_OK;
}

int fmkv_cache_destroy(fmkv_cache* c) {
  if (!c) return FMKV_OK;
  if (c->arena) (void)hipFree(c->arena);
  if (c->d_signs) (void)hipFree(c->d_signs);
  c->ws.release();
  c->stage.release();
  delete c;
  return FMKV_OK;
}

int fmkv_cache_offset(const fmkv_cache* c, int64_t* out) {
  if (!c || !out) return fail(FMKV_ERR_INVALID_ARG, "null argument");
  *out = c->offset;
  return FMKV_OK;
}

int fmkv_cache_stored_len(const fmkv_cache* c, int64_t* out) {
  if (!c || !out) return fail(FMKV_ERR_INVALID_ARG, "null argument");
  *out = c->offset - visible_begin(c);
  return FMKV_OK;
}

int fmkv_cache_append(fmkv_cache* c, const void* k, const void* v, int64_t n, void* stream) {
  fmkv::AppendArgs a;
  int64_t tasks = 0;
  int rc = prepare_append(c, k, v, n, &a, &tasks);
  if (rc || n == 0) return rc;
  hipError_t e = fmkv::launch_append(a, 1, (int)tasks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "append launch");
  c->offset += n;
  return FMKV_OK;
}

int fmkv_cache_append_projected(fmkv_cache* c, const void* k, const void* v, int64_t n,
                                const fmkv_kv_prologue* pro, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  int rc = check_prologue(c->desc, pro);
  if (rc) return rc;
  fmkv::AppendArgs a;
  int64_t tasks = 0;
  rc = prepare_append(c, k, pro->v_from_k ? k : v, n, &a, &tasks);
  if (rc || n == 0) return rc;
  set_prologue(pro, &a);
  hipError_t e = fmkv::launch_append(a, 1, (int)tasks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "append launch");
  c->offset += n;
  return FMKV_OK;
}

int fmkv_prefill_step(fmkv_cache* c, const void* k, const void* v, int64_t n, const void* q,
                      int32_t n_q_heads, float scale, void* out, int32_t out_dtype, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (n < 1) return fail(FMKV_ERR_INVALID_ARG, "a prefill step appends at least one token");
  int rc = check_attn_args(c->desc, q, n_q_heads, 0.0f, out, out_dtype);
  if (rc) return rc;
  if (!std::isfinite(scale)) return fail(FMKV_ERR_INVALID_ARG, "scale must be finite");
  const int32_t group = n_q_heads / c->desc.n_kv_heads;
  if (n > (int64_t)65535 * (64 / group))
    return fail(FMKV_ERR_INVALID_ARG, "n_tokens too large for one prefill step");
  fmkv::AppendArgs ap;
  int64_t tasks = 0;
  rc = prepare_append(c, k, v, n, &ap, &tasks);
  if (rc) return rc;
  const int64_t p0 = c->offset, W = c->desc.window;  // the sliding window (0: causal only)
  const int H = c->desc.n_kv_heads;
  const int64_t bb = c->layout.block_bytes;
  fmkv::PrefillArgs pa;
  pa.old_st = cache_store(c);
  pa.new_st = pa.old_st;
  pa.p0 = p0;
  pa.start_pos = nullptr;
  pa.n_seqs = 1;
  pa.n_q = (int32_t)n;
  pa.window = W;
  pa.ring_slots = ring_slots(c->desc);
  pa.vis_begin = c->vis_begin;
  pa.p_split = 0;
  pa.new_blk0 = 0;
  pa.group = group;
  pa.n_q_heads = n_q_heads;
  pa.q = static_cast<const uint16_t*>(q);
  pa.qscale = scale * 1.4426950408889634f;
  std::memcpy(pa.sign_bits, c->sign_bits, sizeof(pa.sign_bits));
  pa.c = c->c;
  pa.out = out;
  pa.out_f32 = out_dtype == FMKV_DTYPE_F32 ? 1 : 0;
  fmkv::AppendArgs as = ap;
  int64_t nsb = 0;
  if (W > 0) {
    // the chunk's rows go to a staging store first (block 0 = absolute
    // block p0 / 16), so the ring keeps every position the queries need
    nsb = (p0 % fmkv::kBlockTokens + n + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens;
    rc = c->stage.ensure((size_t)(nsb * H * bb), true);
    if (rc) return rc;
    fmkv::Store st;
    st.base = reinterpret_cast<uint8_t*>(c->stage.ptr);
    st.block_stride = bb;
    st.head_stride = nsb * bb;
    st.block_table = nullptr;
    st.table_stride = 0;
    st.n_blocks = nsb;
    st.n_kv_heads = H;
    st.layout = c->layout;
    as.st = st;
    as.start_scalar = p0 % fmkv::kBlockTokens;
    as.window = 0;
    pa.new_st = st;
    pa.p_split = p0;
    pa.new_blk0 = p0 / fmkv::kBlockTokens;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (W > 0) {
    e = fmkv::launch_append(as, 1, (int)nsb, s);
    if (e != hipSuccess) return hip_fail(e, "staging append launch");
    e = fmkv::launch_prefill_attention(pa, s);
    if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
    e = fmkv::launch_append(ap, 1, (int)tasks, s);
    if (e != hipSuccess) return hip_fail(e, "append launch");
  } else {
    e = fmkv::launch_append(ap, 1, (int)tasks, s);
    if (e != hipSuccess) return hip_fail(e, "append launch");
    e = fmkv::launch_prefill_attention(pa, s);
    if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
  }
  c->offset += n;
  return FMKV_OK;
}

int fmkv_decode_step(fmkv_cache* c, const void* k, const void* v, int64_t n, const void* q,
                     int32_t n_q_heads, float scale, float tau, void* out, int32_t out_dtype,
                     void* stream) {
  return decode_step_impl(c, k, v, n, q, n_q_heads, scale, tau, out, out_dtype, stream, {});
}

int fmkv_decode_step_projected(fmkv_cache* c, const void* k_proj, const void* v_proj, int64_t n,
                               const fmkv_kv_prologue* pro, const void* q, int32_t n_q_heads,
                               float scale, float tau, void* out, int32_t out_dtype, void* stream) {
  if (!pro) return fail(FMKV_ERR_INVALID_ARG, "prologue is null");
  return decode_step_impl(c, k_proj, v_proj, n, q, n_q_heads, scale, tau, out, out_dtype, stream,
                          {}, pro);
}

int fmkv_decode_step_noalloc(fmkv_cache* c, const void* k, const void* v, int64_t n,
                             const void* q, int32_t n_q_heads, float scale, float tau, void* out,
                             int32_t out_dtype, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  ExtWorkspace ext;
  int rc = noalloc_scratch(&ext);
  if (rc) return rc;
  return decode_step_impl(c, k, v, n, q, n_q_heads, scale, tau, out, out_dtype, stream, ext);
}

}  // extern "C"

namespace {

int decode_step_impl(fmkv_cache* c, const void* k, const void* v, int64_t n, const void* q,
                     int32_t n_q_heads, float scale, float tau, void* out, int32_t out_dtype,
                     void* stream, ExtWorkspace ext, const fmkv_kv_prologue* pro) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (n < 1) return fail(FMKV_ERR_INVALID_ARG, "a decode step appends at least one token");
  int rc;
  if (pro && (rc = check_prologue(c->desc, pro))) return rc;
  fmkv::AppendArgs ap;
  int64_t tasks = 0;
  rc = prepare_append(c, k, pro && pro->v_from_k ? k : v, n, &ap, &tasks);
  if (rc) return rc;
  if (pro) set_prologue(pro, &ap);
  // one new token: the attention launch appends it itself (new-token
  // column; with sparse-V the statistics pass does); chunks append first
  const int fused = n == 1 ? 1 : 0;
  fmkv::AttnArgs at;
  rc = prepare_attention(c, c->offset + n, q, n_q_heads, scale, tau, out, out_dtype, fused, &at, ext);
  if (rc) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (fused) {
    at.k_new = ap.k;
    at.v_new = ap.v;
    if (pro) set_prologue(pro, &at);
  } else {
    e = fmkv::launch_append(ap, 1, (int)tasks, s);
    if (e != hipSuccess) return hip_fail(e, "append launch");
    c->offset += n;
  }
  hipEvent_t e0, e1;
  next_events(&e0, &e1);
  e = launch_attention(at, 1, c->desc.n_kv_heads, s, e0, e1);
  if (e != hipSuccess) return hip_fail(e, "decode attention launch");
  if (fused) c->offset += n;
  return FMKV_OK;
}

// Elapsed milliseconds of recorded pair i (waits for it).
int profile_pair_ms(int32_t i, float* ms) {
  hipError_t e = hipEventSynchronize(g_prof.ev[2 * (size_t)i + 1]);
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  *ms = 0.0f;
  e = hipEventElapsedTime(ms, g_prof.ev[2 * (size_t)i], g_prof.ev[2 * (size_t)i + 1]);
  if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  return FMKV_OK;
}

}  // namespace

extern "C" {

int fmkv_cache_trim(fmkv_cache* c, int64_t keep_last) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (keep_last < 0) return fail(FMKV_ERR_INVALID_ARG, "keep_last must be >= 0");
  const int64_t b = c->offset - keep_last;
  if (b > c->vis_begin) c->vis_begin = b;
  return FMKV_OK;
}

int fmkv_decode_attention(fmkv_cache* c, const void* q, int32_t n_q_heads, float scale, float tau,
                          void* out, int32_t out_dtype, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  fmkv::AttnArgs a;
  int rc = prepare_attention(c, c->offset, q, n_q_heads, scale, tau, out, out_dtype, 0, &a);
  if (rc) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t e0, e1;
  next_events(&e0, &e1);
  hipError_t e = launch_attention(a, 1, c->desc.n_kv_heads, s, e0, e1);
  if (e != hipSuccess) return hip_fail(e, "decode attention launch");
  return FMKV_OK;
}

int fmkv_cache_decode_splits(const fmkv_cache* c, int32_t* n_splits) {
  if (!c || !n_splits) return fail(FMKV_ERR_INVALID_ARG, "null argument");
  int64_t filled = c->desc.window > 0 ? std::min<int64_t>(c->offset, ring_slots(c->desc)) : c->offset;
  int64_t vb = c->desc.window > 0 ? 0 : c->vis_begin;
  int64_t nblk = (filled + fmkv::kBlockTokens - 1) / fmkv::kBlockTokens - vb / fmkv::kBlockTokens;
  if (nblk < 1) nblk = 1;
  fmkv::AttnArgs a;
  plan_splits(c->cus, c->desc.n_kv_heads, 1, nblk, attn_wg_per_cu(c->desc), 1, 1, 0, false, &a);
  *n_splits = a.max_splits;
  return FMKV_OK;
}

int fmkv_cache_fetch(const fmkv_cache* c, void* k_out, void* v_out, int32_t out_dtype, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (!k_out || !v_out) return fail(FMKV_ERR_INVALID_ARG, "k_out/v_out must be device pointers");
  if (out_dtype != FMKV_DTYPE_BF16 && out_dtype != FMKV_DTYPE_F32)
    return fail(FMKV_ERR_INVALID_ARG, "bad out_dtype");
  fmkv::FetchArgs a;
  a.st = cache_store(c);
  a.offset = c->offset;
  a.window = ring_slots(c->desc);  // slot of position p: p mod the ring's slots
  a.first_pos = visible_begin(c);
  a.n_pos = c->offset - a.first_pos;
  a.signs = c->d_signs;
  a.c = c->c;
  a.k_out = k_out;
  a.v_out = v_out;
  a.out_f32 = out_dtype == FMKV_DTYPE_F32;
  hipError_t e = fmkv::launch_fetch(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "fetch launch");
  return FMKV_OK;
}

int fmkv_cache_read_codes(const fmkv_cache* c, void* codes, void* meta, void* stream) {
  if (!c) return fail(FMKV_ERR_INVALID_ARG, "cache is null");
  if (!codes || (!meta && c->desc.mode != FMKV_MODE_PLAIN))
    return fail(FMKV_ERR_INVALID_ARG, "codes/meta must be device pointers");
  fmkv::ReadArgs a;
  a.st = cache_store(c);
  a.n_slots = c->desc.window > 0 ? ring_slots(c->desc) : c->desc.capacity;
  a.codes = static_cast<uint32_t*>(codes);
  a.meta = static_cast<uint16_t*>(meta);
  hipError_t e = fmkv::launch_read_codes(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "read_codes launch");
  return FMKV_OK;
}

int fmkv_pool_create(const fmkv_cache_desc* desc, int64_t n_blocks, fmkv_pool** out) {
  if (!desc) return fail(FMKV_ERR_INVALID_ARG, "descriptor is null");
  fmkv_cache_desc d = *desc;
  d.window = 0;
  d.capacity = 1;
  int rc = check_desc(&d);
  if (rc) return rc;
  if (desc->window != 0) return fail(FMKV_ERR_UNSUPPORTED, "paged pools hold global (linear) sequences");
  if (!out) return fail(FMKV_ERR_INVALID_ARG, "out is null");
  if (n_blocks < 1 || n_blocks > ((int64_t)1 << 31) - 1)
    return fail(FMKV_ERR_INVALID_ARG, "n_blocks must be in [1, 2^31)");
  *out = nullptr;
  fmkv_pool* p = new fmkv_pool();
  p->desc = *desc;
  p->layout = fmkv::make_layout(desc->head_dim, desc->bits, desc->mode);
  p->n_blocks = n_blocks;
  p->c = 1.0f / std::sqrt((float)desc->head_dim);
  p->sqrt_d = std::sqrt((float)desc->head_dim);
  p->arena = nullptr;
  p->d_signs = nullptr;
  const int64_t bytes = p->layout.block_bytes * desc->n_kv_heads * n_blocks;
  hipError_t e = hipMalloc(&p->arena, bytes);
  if (e != hipSuccess) {
    delete p;
    return fail(FMKV_ERR_OOM, "pool allocation failed (" + std::to_string(bytes) + " bytes)");
  }
  e = hipMemset(p->arena, 0, bytes);
  if (e != hipSuccess) {
    (void)hipFree(p->arena);
    delete p;
    return hip_fail(e, "hipMemset(pool)");
  }
  rc = make_signs(*desc, &p->d_signs);
  if (rc) {
    (void)hipFree(p->arena);
    delete p;
    return rc;
  }
  sign_bits_of(*desc, p->sign_bits);
  p->cus = device_cus();
  *out = p;
  return FMKV_OK;
}

int fmkv_pool_destroy(fmkv_pool* p) {
  if (!p) return FMKV_OK;
  if (p->arena) (void)hipFree(p->arena);
  if (p->d_signs) (void)hipFree(p->d_signs);
  p->ws.release();
  delete p;
  return FMKV_OK;
}

int fmkv_paged_prefill_step(fmkv_pool* p, const void* k, const void* v,
                            const int32_t* block_tables, int32_t max_blocks,
                            const int32_t* start_pos, int32_t n_seqs, int32_t n_new,
                            const void* q, int32_t n_q_heads, float scale, void* out,
                            int32_t out_dtype, void* stream) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  if (n_seqs < 1 || n_new < 1)
    return fail(FMKV_ERR_INVALID_ARG, "a prefill step needs n_seqs >= 1 and n_new >= 1");
  int rc = check_attn_args(p->desc, q, n_q_heads, 0.0f, out, out_dtype);
  if (rc) return rc;
  if (!std::isfinite(scale)) return fail(FMKV_ERR_INVALID_ARG, "scale must be finite");
  const int32_t group = n_q_heads / p->desc.n_kv_heads;
  if ((int64_t)n_new > (int64_t)65535 * (64 / group))
    return fail(FMKV_ERR_INVALID_ARG, "n_new too large for one prefill step");
  fmkv::AppendArgs ap;
  int tasks = 0;
  rc = prepare_paged_append(p, k, v, block_tables, max_blocks, start_pos, n_seqs, n_new, &ap,
                            &tasks);
  if (rc) return rc;
  fmkv::PrefillArgs pa;
  pa.old_st = ap.st;
  pa.new_st = ap.st;
  pa.p0 = 0;
  pa.start_pos = start_pos;
  pa.n_seqs = n_seqs;
  pa.n_q = n_new;
  pa.window = 0;
  pa.ring_slots = 0;
  pa.vis_begin = 0;
  pa.p_split = 0;
  pa.new_blk0 = 0;
  pa.group = group;
  pa.n_q_heads = n_q_heads;
  pa.q = static_cast<const uint16_t*>(q);
  pa.qscale = scale * 1.4426950408889634f;
  std::memcpy(pa.sign_bits, p->sign_bits, sizeof(pa.sign_bits));
  pa.c = p->c;
  pa.out = out;
  pa.out_f32 = out_dtype == FMKV_DTYPE_F32 ? 1 : 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = fmkv::launch_append(ap, n_seqs, tasks, s);
  if (e != hipSuccess) return hip_fail(e, "paged append launch");
  e = fmkv::launch_prefill_attention(pa, s);
  if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
  return FMKV_OK;
}

int fmkv_paged_append(fmkv_pool* p, const void* k, const void* v, const int32_t* block_tables,
                      int32_t max_blocks, const int32_t* start_pos, int32_t n_seqs, int32_t n_new,
                      void* stream) {
  fmkv::AppendArgs a;
  int tasks = 0;
  int rc = prepare_paged_append(p, k, v, block_tables, max_blocks, start_pos, n_seqs, n_new, &a,
                                &tasks);
  if (rc || n_seqs == 0 || n_new == 0) return rc;
  hipError_t e = fmkv::launch_append(a, n_seqs, tasks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "paged append launch");
  return FMKV_OK;
}

int fmkv_paged_append_projected(fmkv_pool* p, const void* k, const void* v,
                                const int32_t* block_tables, int32_t max_blocks,
                                const int32_t* start_pos, int32_t n_seqs, int32_t n_new,
                                const fmkv_kv_prologue* pro, void* stream) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  int rc = check_prologue(p->desc, pro);
  if (rc) return rc;
  fmkv::AppendArgs a;
  int tasks = 0;
  rc = prepare_paged_append(p, k, pro->v_from_k ? k : v, block_tables, max_blocks, start_pos, n_seqs,
                            n_new, &a, &tasks);
  if (rc || n_seqs == 0 || n_new == 0) return rc;
  set_prologue(pro, &a);
  hipError_t e = fmkv::launch_append(a, n_seqs, tasks, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "paged append launch");
  return FMKV_OK;
}

int fmkv_paged_decode_attention(fmkv_pool* p, const void* q, const int32_t* block_tables,
                                int32_t max_blocks, const int32_t* seq_lens, int32_t n_seqs,
                                int32_t max_seq_len, int32_t n_q_heads, float scale, float tau,
                                void* out, int32_t out_dtype, void* stream) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  fmkv::AttnArgs a;
  int rc = prepare_paged_attention(p, q, block_tables, max_blocks, seq_lens, n_seqs, max_seq_len,
                                   n_q_heads, scale, tau, out, out_dtype, 0, &a);
  if (rc || n_seqs == 0) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t e0, e1;
  next_events(&e0, &e1);
  hipError_t e = launch_attention(a, n_seqs, p->desc.n_kv_heads, s, e0, e1);
  if (e != hipSuccess) return hip_fail(e, "paged decode attention launch");
  return FMKV_OK;
}

}  // extern "C"

namespace {

int paged_decode_step_impl(fmkv_pool* p, const void* k, const void* v,
                           const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* start_pos, const int32_t* seq_lens, int32_t n_seqs,
                           int32_t n_new, int32_t max_seq_len, const void* q, int32_t n_q_heads,
                           float scale, float tau, void* out, int32_t out_dtype, void* stream,
                           const fmkv_kv_prologue* pro) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  if (n_new < 1) return fail(FMKV_ERR_INVALID_ARG, "a decode step appends at least one token");
  int rc;
  if (pro && (rc = check_prologue(p->desc, pro))) return rc;
  fmkv::AppendArgs ap;
  int tasks = 0;
  rc = prepare_paged_append(p, k, pro && pro->v_from_k ? k : v, block_tables, max_blocks,
                            start_pos, n_seqs, n_new, &ap, &tasks);
  if (rc) return rc;
  if (pro) set_prologue(pro, &ap);
  // one new token per sequence: the attention launch appends it itself, at
  // position seq_lens[s] - 1 (= start_pos[s])
  const int fused = n_new == 1 ? 1 : 0;
  fmkv::AttnArgs at;
  rc = prepare_paged_attention(p, q, block_tables, max_blocks, seq_lens, n_seqs, max_seq_len,
                               n_q_heads, scale, tau, out, out_dtype, fused, &at);
  if (rc || n_seqs == 0) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (fused) {
    at.k_new = ap.k;
    at.v_new = ap.v;
    if (pro) set_prologue(pro, &at);
  } else {
    e = fmkv::launch_append(ap, n_seqs, tasks, s);
    if (e != hipSuccess) return hip_fail(e, "paged append launch");
  }
  hipEvent_t e0, e1;
  next_events(&e0, &e1);
  e = launch_attention(at, n_seqs, p->desc.n_kv_heads, s, e0, e1);
  if (e != hipSuccess) return hip_fail(e, "paged decode attention launch");
  return FMKV_OK;
}

}  // namespace

extern "C" {

int fmkv_paged_decode_step(fmkv_pool* p, const void* k, const void* v,
                           const int32_t* block_tables, int32_t max_blocks,
                           const int32_t* start_pos, const int32_t* seq_lens, int32_t n_seqs,
                           int32_t n_new, int32_t max_seq_len, const void* q, int32_t n_q_heads,
                           float scale, float tau, void* out, int32_t out_dtype, void* stream) {
  return paged_decode_step_impl(p, k, v, block_tables, max_blocks, start_pos, seq_lens, n_seqs,
                                n_new, max_seq_len, q, n_q_heads, scale, tau, out, out_dtype,
                                stream, nullptr);
}

int fmkv_paged_decode_step_projected(fmkv_pool* p, const void* k_proj, const void* v_proj,
                                     const int32_t* block_tables, int32_t max_blocks,
                                     const int32_t* start_pos, const int32_t* seq_lens,
                                     int32_t n_seqs, int32_t n_new, int32_t max_seq_len,
                                     const fmkv_kv_prologue* pro, const void* q,
                                     int32_t n_q_heads, float scale, float tau, void* out,
                                     int32_t out_dtype, void* stream) {
  if (!pro) return fail(FMKV_ERR_INVALID_ARG, "prologue is null");
  return paged_decode_step_impl(p, k_proj, v_proj, block_tables, max_blocks, start_pos, seq_lens,
                                n_seqs, n_new, max_seq_len, q, n_q_heads, scale, tau, out,
                                out_dtype, stream, pro);
}

int fmkv_pool_read_codes(const fmkv_pool* p, void* codes, void* meta, void* stream) {
  if (!p) return fail(FMKV_ERR_INVALID_ARG, "pool is null");
  if (!codes || (!meta && p->desc.mode != FMKV_MODE_PLAIN))
    return fail(FMKV_ERR_INVALID_ARG, "codes/meta must be device pointers");
  fmkv::ReadArgs a;
  a.st = pool_store(p, nullptr, 0);
  a.n_slots = p->n_blocks * fmkv::kBlockTokens;
  a.codes = static_cast<uint32_t*>(codes);
  a.meta = static_cast<uint16_t*>(meta);
  hipError_t e = fmkv::launch_read_codes(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "pool read_codes launch");
  return FMKV_OK;
}

int fmkv_set_sparse_v_gather(int32_t on) {
  if (on != 0 && on != 1) return fail(FMKV_ERR_INVALID_ARG, "sparse_v_gather must be 0 or 1");
  g_sparse_gather = on;
  return FMKV_OK;
}

int fmkv_set_blocks_per_split(int32_t bps) {
  if (bps < 0) return fail(FMKV_ERR_INVALID_ARG, "blocks_per_split must be >= 0");
  g_bps_override = bps;
  return FMKV_OK;
}

int fmkv_profile_enable(int32_t max_records) {
  if (max_records < 0 || max_records > (1 << 20))
    return fail(FMKV_ERR_INVALID_ARG, "max_records must be in [0, 2^20]");
  g_prof.clear_events();
  g_prof.max_records = 0;
  if (max_records == 0) return FMKV_OK;
  g_prof.ev.resize(2 * (size_t)max_records, nullptr);
  for (size_t i = 0; i < g_prof.ev.size(); i++) {
    hipError_t e = hipEventCreate(&g_prof.ev[i]);
    if (e != hipSuccess) {
      g_prof.ev.resize(i);
      g_prof.clear_events();
      return hip_fail(e, "hipEventCreate");
    }
  }
  g_prof.max_records = max_records;
  return FMKV_OK;
}

int fmkv_profile_collect(double* total_ms, int32_t* n_records) {
  if (!total_ms || !n_records) return fail(FMKV_ERR_INVALID_ARG, "null argument");
  double sum = 0.0;
  for (int32_t i = 0; i < g_prof.used; i++) {
    float ms;
    int rc = profile_pair_ms(i, &ms);
    if (rc) return rc;
    sum += ms;
  }
  *total_ms = sum;
  *n_records = g_prof.used;
  g_prof.used = 0;
  return FMKV_OK;
}

int fmkv_profile_collect_each(float* ms_out, int32_t capacity, int32_t* n_records) {
  if (!ms_out || !n_records) return fail(FMKV_ERR_INVALID_ARG, "null argument");
  if (capacity < g_prof.used)
    return fail(FMKV_ERR_CAPACITY, std::to_string(g_prof.used) + " records need a buffer of as "
                                   "many floats; capacity is " + std::to_string(capacity));
  for (int32_t i = 0; i < g_prof.used; i++) {
    int rc = profile_pair_ms(i, &ms_out[i]);
    if (rc) return rc;
  }
  *n_records = g_prof.used;
  g_prof.used = 0;
  return FMKV_OK;
}

}  // extern "C"

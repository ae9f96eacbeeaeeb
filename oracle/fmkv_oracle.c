/*
 * CPU oracle for the quantized KV-cache path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker / the timed CPU baseline. The HIP
 * library never links or calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no -ffast-math), so
 * every float operation below rounds exactly once, in the order written.
 *
 * Two kinds of functions live here:
 *  1. Restatements of the reference (Adri96/gemma4-moe-flash-mlx-turbo):
 *     the Sylvester Hadamard, LCG signs, RHT matrices and Lloyd-Max tables
 *     of src/cache.rs, the TurboQuant round trip in the reference's op order
 *     (dense matmuls), the mask semantics of src/model/mod.rs and the SDPA /
 *     sparse-V attention of src/model/gemma4_attention.rs.
 *  2. The canonical arithmetic the kernels reproduce bit for bit: the
 *     fast Walsh-Hadamard transform in a fixed butterfly order (equal to the
 *     reference's x.R up to float reassociation), MLX's affine group
 *     quantizer, the canonical TurboQuant codebook quantizer, and the ring /
 *     paged slot arithmetic.
 */
#include "fmkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
/* Row loops over `rows` run in parallel: every row is computed by one thread in the
 * order written, so the results do not depend on the thread count. */
#define OMP_ROWS _Pragma("omp parallel for schedule(static) if (rows > 64)")
#else
#define OMP_ROWS
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary32 -> binary16, round to nearest even, with subnormals. */
uint16_t ora_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  uint32_t e = ax >> 23;
  if (e < 113) { /* below 2^-14: half subnormal (or zero) */
    if (e < 102) return (uint16_t)sign; /* < 2^-25: rounds to zero */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* value = m * 2^(e-150); unit = 2^-24 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((e - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float ora_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 0x1f) return bits_f32(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    return sign ? -v : v;
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t ora_f32_to_bf16(float f) {
  uint32_t x = f32_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float ora_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

void ora_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = ora_f32_to_f16(x[i]);
}
void ora_f16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = ora_f16_to_f32(x[i]);
}
void ora_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = ora_f32_to_bf16(x[i]);
}
void ora_bf16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = ora_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* reference restatements: src/cache.rs                                      */
/* ------------------------------------------------------------------------ */

/* src/cache.rs:6-26 -- Sylvester construction, then every entry * 1/sqrt(n). */
void ora_generate_hadamard(int n, float* h) {
  memset(h, 0, sizeof(float) * (size_t)n * (size_t)n);
  h[0] = 1.0f;
  for (int size = 1; size < n; size *= 2) {
    for (int i = 0; i < size; i++) {
      for (int j = 0; j < size; j++) {
        float val = h[(size_t)i * n + j];
        h[(size_t)i * n + (j + size)] = val;
        h[(size_t)(i + size) * n + j] = val;
        h[(size_t)(i + size) * n + (j + size)] = -val;
      }
    }
  }
  float scale = 1.0f / sqrtf((float)n);
  for (size_t i = 0; i < (size_t)n * (size_t)n; i++) h[i] *= scale;
}

/* src/cache.rs:29-43 -- MMIX LCG stepped before each draw; +1 iff bit 63 == 0. */
void ora_deterministic_signs(int n, uint64_t seed, float* s) {
  uint64_t state = seed;
  for (int i = 0; i < n; i++) {
    state = state * 6364136223846793005ull + 1442695040888963407ull;
    s[i] = ((state >> 63) & 1ull) == 0 ? 1.0f : -1.0f;
  }
}

/* src/cache.rs:47-62 -- R[i][j] = H[i][j]*s[j], Rt[i][j] = H[i][j]*s[i]. */
void ora_build_rht(int dim, uint64_t seed, float* r, float* rt) {
  float* h = (float*)malloc(sizeof(float) * (size_t)dim * (size_t)dim);
  float* s = (float*)malloc(sizeof(float) * (size_t)dim);
  ora_generate_hadamard(dim, h);
  ora_deterministic_signs(dim, seed, s);
  for (int i = 0; i < dim; i++)
    for (int j = 0; j < dim; j++) {
      r[(size_t)i * dim + j] = h[(size_t)i * dim + j] * s[j];
      rt[(size_t)i * dim + j] = h[(size_t)i * dim + j] * s[i];
    }
  free(h);
  free(s);
}

/* src/cache.rs:67-89 -- literal N(0,1) Lloyd-Max tables. Returns #centroids,
 * or 0 for unsupported bits (the reference panics there). */
int ora_lloyd_max_codebook(int bits, float* centroids, float* bounds) {
  static const float c2[4] = {-1.510f, -0.453f, 0.453f, 1.510f};
  static const float b2[3] = {-0.982f, 0.0f, 0.982f};
  static const float c3[8] = {-2.152f, -1.344f, -0.756f, -0.245f, 0.245f, 0.756f, 1.344f, 2.152f};
  static const float b3[7] = {-1.748f, -1.050f, -0.501f, 0.0f, 0.501f, 1.050f, 1.748f};
  static const float c4[16] = {-2.733f, -2.069f, -1.618f, -1.256f, -0.942f, -0.657f,
                               -0.388f, -0.128f, 0.128f,  0.388f,  0.657f,  0.942f,
                               1.256f,  1.618f,  2.069f,  2.733f};
  static const float b4[15] = {-2.401f, -1.844f, -1.437f, -1.099f, -0.800f,
                               -0.522f, -0.258f, 0.0f,    0.258f,  0.522f,
                               0.800f,  1.099f,  1.437f,  1.844f,  2.401f};
  const float *c, *b;
  int n;
  switch (bits) {
    case 2: c = c2; b = b2; n = 4; break;
    case 3: c = c3; b = b3; n = 8; break;
    case 4: c = c4; b = b4; n = 16; break;
    default: return 0;
  }
  if (centroids) memcpy(centroids, c, sizeof(float) * (size_t)n);
  if (bounds) memcpy(bounds, b, sizeof(float) * (size_t)(n - 1));
  return n;
}

/* src/cache.rs:94-129 in the reference's op order, with the two matmuls
 * written as dense fp32 dot products summed in index order (MLX's BLAS order
 * is unspecified, so this is one admissible order, not MLX's bits):
 *   norm = sqrt(sum x^2); u = x / (norm + 1e-8); z = (u . R) * sqrt(d);
 *   idx = #{b : z >= b}; vals = codebook[idx];
 *   out = bf16(((vals * (1/sqrt d)) . Rt) * norm).                        */
void ora_turbo_round_trip_dense(const uint16_t* x_bf16, int64_t rows, int d, int bits,
                                uint64_t seed, uint16_t* out_bf16) {
  float* r = (float*)malloc(sizeof(float) * (size_t)d * d);
  float* rt = (float*)malloc(sizeof(float) * (size_t)d * d);
  ora_build_rht(d, seed, r, rt);
  ora_turbo_round_trip_rt(x_bf16, rows, d, bits, r, rt, out_bf16);
  free(r);
  free(rt);
}

/* The same with R and Rt built once by the caller (KVCache::
 * new_quantized_with_window keeps them in its TurboQuantConfig,
 * src/cache.rs:206-227). Rows run in parallel. */
void ora_turbo_round_trip_rt(const uint16_t* x_bf16, int64_t rows, int d, int bits, const float* r,
                             const float* rt, uint16_t* out_bf16) {
  float cent[16], bnd[15];
  int nc = ora_lloyd_max_codebook(bits, cent, bnd);
  if (nc == 0) return;
  float sqrt_d = sqrtf((float)d);
  float inv_sqrt_d = 1.0f / sqrtf((float)d);
  const float eps = 1e-8f;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (rows > 1)
#endif
  for (int64_t row = 0; row < rows; row++) {
    float* x = (float*)malloc(sizeof(float) * 3 * (size_t)d);
    float *z = x + d, *w = x + 2 * d;
    const uint16_t* xr = x_bf16 + row * d;
    float ss = 0.0f;
    for (int i = 0; i < d; i++) {
      x[i] = ora_bf16_to_f32(xr[i]);
      ss += x[i] * x[i];
    }
    float norm = sqrtf(ss);
    float den = norm + eps;
    for (int i = 0; i < d; i++) x[i] = x[i] / den;
    /* z_j = sum_i x_i R_ij, summed in i order (the outer loop runs over i
     * so that R is read row by row) */
    for (int j = 0; j < d; j++) z[j] = 0.0f;
    for (int i = 0; i < d; i++)
      for (int j = 0; j < d; j++) z[j] += x[i] * r[(size_t)i * d + j];
    for (int j = 0; j < d; j++) {
      z[j] = z[j] * sqrt_d;
      int idx = 0;
      for (int b = 0; b < nc - 1; b++) idx += (z[j] >= bnd[b]) ? 1 : 0;
      w[j] = cent[idx] * inv_sqrt_d;
    }
    for (int j = 0; j < d; j++) z[j] = 0.0f;
    for (int i = 0; i < d; i++)
      for (int j = 0; j < d; j++) z[j] += w[i] * rt[(size_t)i * d + j];
    for (int j = 0; j < d; j++) out_bf16[row * d + j] = ora_f32_to_bf16(z[j] * norm);
    free(x);
  }
}

/* ------------------------------------------------------------------------ */
/* canonical rotation                                                        */
/* ------------------------------------------------------------------------ */

/* The reference's Hadamard normaliser, src/cache.rs:21: 1.0 / sqrt(n) in f32. */
float ora_inv_sqrt(int n) { return 1.0f / sqrtf((float)n); }

/* Unnormalised FWHT, stages h = 1, 2, 4, ... with (a, b) -> (a + b, a - b).
 * Equals x . H_sylvester(unnormalised); the kernels run the same stages in
 * the same order (low strides in registers, high strides across lanes). */
void ora_fwht(float* x, int n) {
  for (int h = 1; h < n; h <<= 1)
    for (int i = 0; i < n; i += 2 * h)
      for (int j = i; j < i + h; j++) {
        float a = x[j], b = x[j + h];
        x[j] = a + b;
        x[j + h] = a - b;
      }
}

static void fwht_f64(double* x, int n) {
  for (int h = 1; h < n; h <<= 1)
    for (int i = 0; i < n; i += 2 * h)
      for (int j = i; j < i + h; j++) {
        double a = x[j], b = x[j + h];
        x[j] = a + b;
        x[j + h] = a - b;
      }
}

/* y = x . R (src/cache.rs:47-62), canonical order:
 *   y_j = (FWHT(x)_j * c) * s_j,  c = 1/sqrt(d) in f32.                   */
void ora_rotate_rows_f32(const float* x, int64_t rows, int d, const float* signs, float* y) {
  float c = ora_inv_sqrt(d);
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++) {
    float* yr = y + r * d;
    memcpy(yr, x + r * d, sizeof(float) * d);
    ora_fwht(yr, d);
    for (int j = 0; j < d; j++) yr[j] = (yr[j] * c) * signs[j];
  }
}

void ora_rotate_rows(const uint16_t* x_bf16, int64_t rows, int d, const float* signs, float* y) {
  float c = ora_inv_sqrt(d);
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++) {
    float* yr = y + r * d;
    for (int j = 0; j < d; j++) yr[j] = ora_bf16_to_f32(x_bf16[r * d + j]);
    ora_fwht(yr, d);
    for (int j = 0; j < d; j++) yr[j] = (yr[j] * c) * signs[j];
  }
}

/* x = y . Rt in f64 (Rt[i][j] = H[i][j] s[i], H entries +-c with c the f32
 * constant): x_j = c * FWHT(y o s)_j.                                       */
void ora_unrotate_rows_f64(const double* y, int64_t rows, int d, const float* signs, double* x) {
  double c = (double)ora_inv_sqrt(d);
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++) {
    double* xr = x + r * d;
    for (int i = 0; i < d; i++) xr[i] = y[r * d + i] * (double)signs[i];
    fwht_f64(xr, d);
    for (int j = 0; j < d; j++) xr[j] *= c;
  }
}

/* y = x . R with a dense f64 dot product (no rounding to speak of), used to
 * measure how often the canonical f32 FWHT flips a code versus exact math. */
void ora_rotate_rows_dense_f64(const float* x, int64_t rows, int d, const float* r, double* y) {
  for (int64_t row = 0; row < rows; row++)
    for (int j = 0; j < d; j++) {
      double acc = 0.0;
      for (int i = 0; i < d; i++) acc += (double)x[row * d + i] * (double)r[(size_t)i * d + j];
      y[row * d + j] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* MLX affine quantization                                                   */
/* ------------------------------------------------------------------------ */

static void put_bits(uint32_t* words, int64_t bitpos, int bits, uint32_t v) {
  int64_t w = bitpos >> 5;
  int off = (int)(bitpos & 31);
  words[w] |= v << off;
  if (off + bits > 32) words[w + 1] |= v >> (32 - off);
}

static uint32_t get_bits(const uint32_t* words, int64_t bitpos, int bits) {
  int64_t w = bitpos >> 5;
  int off = (int)(bitpos & 31);
  uint64_t v = words[w] >> off;
  if (off + bits > 32) v |= (uint64_t)words[w + 1] << (32 - off);
  return (uint32_t)(v & ((1u << bits) - 1u));
}

/* MLX affine_quantize (mlx/ops.cpp, mlx-sys 0.2.0), restated per group:
 *   scale = max((w_max - w_min) / n_bins, 1e-7)
 *   side  = |w_min| > |w_max|;  scale = side ? scale : -scale
 *   edge  = side ? w_min : w_max;  q0 = rint(edge / scale)
 *   q0 != 0: scale = edge / q0, bias = edge;  else bias = 0
 *   code  = clip(rint((w - bias) / scale), 0, n_bins)
 * All in f32; codes use the f32 scale/bias, which are then stored as f16.
 * Packing: little-endian bit stream in uint32 words (element k of a word at
 * bits [b*k, b*k+b)), as MLX packs 2/4/8-bit codes.                        */
void ora_affine_quantize(const float* y, int64_t rows, int d, int bits, int gs,
                         uint32_t* packed, uint16_t* scales, uint16_t* biases) {
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  int64_t words_per_row = ((int64_t)d * bits + 31) / 32;
  int ng = d / gs;
  memset(packed, 0, sizeof(uint32_t) * (size_t)(words_per_row * rows));
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++) {
    for (int g = 0; g < ng; g++) {
      const float* w = y + r * d + (int64_t)g * gs;
      float w_max = w[0], w_min = w[0];
      for (int i = 1; i < gs; i++) {
        w_max = fmaxf(w_max, w[i]);
        w_min = fminf(w_min, w[i]);
      }
      float scale = fmaxf((w_max - w_min) / n_bins, eps);
      int side = fabsf(w_min) > fabsf(w_max);
      scale = side ? scale : -scale;
      float edge = side ? w_min : w_max;
      float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      for (int i = 0; i < gs; i++) {
        float q = rintf((w[i] - bias) / scale);
        q = fminf(fmaxf(q, 0.0f), n_bins);
        put_bits(packed + r * words_per_row, (int64_t)(g * gs + i) * bits, bits, (uint32_t)q);
      }
      scales[r * ng + g] = ora_f32_to_f16(scale);
      biases[r * ng + g] = ora_f32_to_f16(bias);
    }
  }
}

/* MLX dequantize: w = code * scale + bias, with the stored f16 scale/bias
 * (evaluated in f64, so the only rounding is the f16 storage). */
void ora_affine_dequantize(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                           int64_t rows, int d, int bits, int gs, double* y) {
  int64_t words_per_row = ((int64_t)d * bits + 31) / 32;
  int ng = d / gs;
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++)
    for (int j = 0; j < d; j++) {
      uint32_t c = get_bits(packed + r * words_per_row, (int64_t)j * bits, bits);
      double s = ora_f16_to_f32(scales[r * ng + j / gs]);
      double b = ora_f16_to_f32(biases[r * ng + j / gs]);
      y[r * d + j] = (double)c * s + b;
    }
}

/* ------------------------------------------------------------------------ */
/* TurboQuant codebook mode, canonical order                                 */
/* ------------------------------------------------------------------------ */

/* Sum of squares in the kernels' order: 64 lanes each hold d/64 contiguous
 * elements and sum them left to right (product rounded, then added), then a
 * xor-butterfly over lanes (strides 1, 2, ..., 32).                         */
static float canonical_sumsq(const float* x, int d) {
  float p[64];
  int e = d / 64;
  for (int l = 0; l < 64; l++) {
    float acc = x[l * e] * x[l * e];
    for (int i = 1; i < e; i++) {
      float sq = x[l * e + i] * x[l * e + i];
      acc = acc + sq;
    }
    p[l] = acc;
  }
  for (int m = 1; m < 64; m <<= 1) {
    float q[64];
    for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ m];
    memcpy(p, q, sizeof(p));
  }
  return p[0];
}

/* Canonical form of src/cache.rs:104-118:
 *   norm = sqrt(sumsq) ; u = x / (norm + 1e-8)
 *   z_j = (((FWHT(u)_j * c) * s_j) * sqrt_d)     (= (u . R) * sqrt(d))
 *   idx_j = #{b : z_j >= b}; stored: packed idx (LE bit stream), f16 norm.
 * x_f32 / x_bf16: exactly one of them holds the rows (f32 rows are what the
 * layer prologue leaves for V, bf16 rows what the layer stores). */
static void codebook_quantize_rows(const float* x_f32, const uint16_t* x_bf16, int64_t rows, int d,
                                   int bits, const float* signs, uint32_t* packed,
                                   uint16_t* norms) {
  float bnd[15];
  int nc = ora_lloyd_max_codebook(bits, NULL, bnd);
  if (nc == 0) return;
  float c = ora_inv_sqrt(d);
  float sqrt_d = sqrtf((float)d);
  int64_t words_per_row = ((int64_t)d * bits + 31) / 32;
  memset(packed, 0, sizeof(uint32_t) * (size_t)(words_per_row * rows));
#ifdef _OPENMP
#pragma omp parallel if (rows > 64)
#endif
  {
    float* x = (float*)malloc(sizeof(float) * d);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t r = 0; r < rows; r++) {
      for (int j = 0; j < d; j++)
        x[j] = x_f32 ? x_f32[r * d + j] : ora_bf16_to_f32(x_bf16[r * d + j]);
      float norm = sqrtf(canonical_sumsq(x, d));
      float den = norm + 1e-8f;
      for (int j = 0; j < d; j++) x[j] = x[j] / den;
      ora_fwht(x, d);
      for (int j = 0; j < d; j++) {
        float z = ((x[j] * c) * signs[j]) * sqrt_d;
        int idx = 0;
        for (int b = 0; b < nc - 1; b++) idx += (z >= bnd[b]) ? 1 : 0;
        put_bits(packed + r * words_per_row, (int64_t)j * bits, bits, (uint32_t)idx);
      }
      norms[r] = ora_f32_to_f16(norm);
    }
    free(x);
  }
}

void ora_codebook_quantize(const uint16_t* x_bf16, int64_t rows, int d, int bits,
                           const float* signs, uint32_t* packed, uint16_t* norms) {
  codebook_quantize_rows(NULL, x_bf16, rows, d, bits, signs, packed, norms);
}

void ora_codebook_quantize_f32(const float* x, int64_t rows, int d, int bits, const float* signs,
                               uint32_t* packed, uint16_t* norms) {
  codebook_quantize_rows(x, NULL, rows, d, bits, signs, packed, norms);
}

/* Rotated-domain value of a codebook row: y_j = centroid[idx_j] * norm / sqrt(d). */
void ora_codebook_dequant_rotated(const uint32_t* packed, const uint16_t* norms, int64_t rows,
                                  int d, int bits, double* y) {
  float cent[16];
  ora_lloyd_max_codebook(bits, cent, NULL);
  int64_t words_per_row = ((int64_t)d * bits + 31) / 32;
  double inv = (double)ora_inv_sqrt(d);
  OMP_ROWS
  for (int64_t r = 0; r < rows; r++) {
    double nrm = ora_f16_to_f32(norms[r]);
    for (int j = 0; j < d; j++)
      y[r * d + j] =
          (double)cent[get_bits(packed + r * words_per_row, (int64_t)j * bits, bits)] * inv * nrm;
  }
}

/* Canonical form of src/cache.rs:119-125 from stored codes:
 *   w_i = centroid[idx_i] * (1/sqrt d); t = FWHT(w o s); out_j = bf16((t_j * c) * norm). */
void ora_codebook_round_trip(const uint32_t* packed, const uint16_t* norms, int64_t rows, int d,
                             int bits, const float* signs, uint16_t* out_bf16) {
  float cent[16];
  ora_lloyd_max_codebook(bits, cent, NULL);
  float c = ora_inv_sqrt(d);
  int64_t words_per_row = ((int64_t)d * bits + 31) / 32;
  float* t = (float*)malloc(sizeof(float) * d);
  for (int64_t r = 0; r < rows; r++) {
    float nrm = ora_f16_to_f32(norms[r]);
    for (int i = 0; i < d; i++) {
      float w = cent[get_bits(packed + r * words_per_row, (int64_t)i * bits, bits)] * c;
      t[i] = w * signs[i];
    }
    ora_fwht(t, d);
    for (int j = 0; j < d; j++) out_bf16[r * d + j] = ora_f32_to_bf16((t[j] * c) * nrm);
  }
  free(t);
}

/* ------------------------------------------------------------------------ */
/* pre-append prologue: k_norm, v_norm, RoPE                                 */
/* (src/model/gemma4_attention.rs:52-81, src/model/norm.rs:5-29; MLX         */
/* fast::rms_norm and fast::rope, third-party, restated)                     */
/* ------------------------------------------------------------------------ */

/* Sum in the kernels' order (as canonical_sumsq, of the values themselves). */
static float canonical_sum(const float* x, int d) {
  float p[64];
  int e = d / 64;
  for (int l = 0; l < 64; l++) {
    float acc = x[l * e];
    for (int i = 1; i < e; i++) acc = acc + x[l * e + i];
    p[l] = acc;
  }
  for (int m = 1; m < 64; m <<= 1) {
    float q[64];
    for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ m];
    memcpy(p, q, sizeof(p));
  }
  return p[0];
}

/* MLX fast::rope as gemma4_attention.rs:74-81 calls it (traditional =
 * false, scale 1.0, offset = the cache offset): for i < dims/2 the pair
 * (x_i, x_{i+dims/2}) turns by the angle a = f32(pos) * f_i with
 * f_i = theta^(-2i/dims) rounded to f32; dims >= rope_dims pass through.
 * The angle is formed in f32 as MLX forms it; its cos and sin are taken in
 * double and rounded to f32. */
float ora_rope_inv_freq(int i, int rope_dims, float theta) {
  return (float)pow((double)theta, -2.0 * (double)i / (double)rope_dims);
}

void ora_rope_cos_sin(int64_t pos, int i, int rope_dims, float theta, float* c, float* s) {
  const float a = (float)pos * ora_rope_inv_freq(i, rope_dims, theta);
  *c = (float)cos((double)a);
  *s = (float)sin((double)a);
}

/* One K row (gemma4_attention.rs:63 then :78-81): k_norm = fast::rms_norm
 * (x * r) * w with r = 1 / sqrt(sum(x^2) / d + eps) in f32 (the sum in the
 * kernels' order), rounded to bf16; then RoPE at pos, rounded to bf16. */
void ora_k_prologue(const uint16_t* x_bf16, int d, const uint16_t* w_bf16, float eps, int64_t pos,
                    int rope_dims, float theta, uint16_t* out_bf16) {
  float x[512], y[512];
  for (int j = 0; j < d; j++) x[j] = ora_bf16_to_f32(x_bf16[j]);
  const float ms = canonical_sumsq(x, d) / (float)d;
  const float r = 1.0f / sqrtf(ms + eps);
  for (int j = 0; j < d; j++)
    y[j] = ora_bf16_to_f32(ora_f32_to_bf16((x[j] * r) * ora_bf16_to_f32(w_bf16[j])));
  const int half = rope_dims / 2;
  for (int i = 0; i < half; i++) {
    float c, s;
    ora_rope_cos_sin(pos, i, rope_dims, theta, &c, &s);
    const float x1 = y[i], x2 = y[i + half];
    out_bf16[i] = ora_f32_to_bf16((x1 * c) - (x2 * s));
    out_bf16[i + half] = ora_f32_to_bf16((x1 * s) + (x2 * c));
  }
  for (int j = rope_dims; j < d; j++) out_bf16[j] = ora_f32_to_bf16(y[j]);
}

/* One V row, RMSNormNoScale as norm.rs:16-29 chains MLX ops on a bf16
 * array: x2 = bf16(x * x); mean = bf16(sum(x2) / d) (the sum in the
 * kernels' order); rms = 1 / sqrt(mean + eps) in f32 (the eps Array is f32,
 * so the sum promotes); out = x * rms in f32 (bf16 * f32 promotes). */
void ora_v_prologue(const uint16_t* x_bf16, int d, float eps, float* out) {
  float x2[512];
  for (int j = 0; j < d; j++) {
    const float x = ora_bf16_to_f32(x_bf16[j]);
    x2[j] = ora_bf16_to_f32(ora_f32_to_bf16(x * x));
  }
  const float mean = ora_bf16_to_f32(ora_f32_to_bf16(canonical_sum(x2, d) / (float)d));
  const float rms = 1.0f / sqrtf(mean + eps);
  for (int j = 0; j < d; j++) out[j] = ora_bf16_to_f32(x_bf16[j]) * rms;
}

/* Rows [n][h][d] of one append: token t at position pos0 + t. v_bf16 NULL:
 * a K==V layer, whose V is v_norm of the raw K (gemma4_attention.rs:54-59). */
void ora_kv_prologue(const uint16_t* k_bf16, const uint16_t* v_bf16, int64_t n, int h, int d,
                     int64_t pos0, const uint16_t* w_bf16, float eps, int rope_dims, float theta,
                     uint16_t* k_out_bf16, float* v_out) {
  for (int64_t t = 0; t < n; t++)
    for (int hh = 0; hh < h; hh++) {
      const int64_t r = (t * h + hh) * d;
      ora_k_prologue(k_bf16 + r, d, w_bf16, eps, pos0 + t, rope_dims, theta, k_out_bf16 + r);
      ora_v_prologue((v_bf16 ? v_bf16 : k_bf16) + r, d, eps, v_out + r);
    }
}

/* ------------------------------------------------------------------------ */
/* cache index semantics                                                     */
/* ------------------------------------------------------------------------ */

/* Slot of absolute position `pos` (window 0 = linear growth). A W-slot ring
 * that overwrites slot pos mod W before attending holds exactly the last W
 * positions, which is what tail_along_time (src/cache.rs:140-148) keeps. */
int64_t ora_ring_slot(int64_t pos, int64_t window) { return window > 0 ? pos % window : pos; }

/* Absolute position held by `slot` once `offset` tokens were appended, or -1
 * when the slot is still empty. */
int64_t ora_slot_position(int64_t slot, int64_t offset, int64_t window) {
  if (window <= 0) return slot < offset ? slot : -1;
  if (offset <= 0 || slot >= window) return -1;
  int64_t last = offset - 1;
  int64_t p = last - ((last - slot) % window + window) % window;
  return p >= 0 ? p : -1;
}

/* src/model/mod.rs:682-704 create_attention_mask: rows offset..offset+L-1,
 * col j visible iff j <= row. Additive 0 / -inf, shape [L, offset + L]. */
void ora_causal_mask(int64_t offset, int64_t seq_len, float* mask) {
  int64_t total = offset + seq_len;
  for (int64_t i = 0; i < seq_len; i++)
    for (int64_t j = 0; j < total; j++) mask[i * total + j] = (offset + i >= j) ? 0.0f : -INFINITY;
}

/* src/model/mod.rs:717-753 create_sliding_mask: row i is position stored+i
 * (relative), col j visible iff j <= stored+i and (stored+i) - j < window. */
void ora_sliding_mask(int64_t stored, int64_t seq_len, int64_t window, float* mask) {
  int64_t total = stored + seq_len;
  for (int64_t i = 0; i < seq_len; i++)
    for (int64_t j = 0; j < total; j++) {
      int64_t row = stored + i;
      int vis = (row >= j) && (j > row - window);
      mask[i * total + j] = vis ? 0.0f : -INFINITY;
    }
}

/* Paged address of `pos`: physical block * block_size + offset in block. */
int64_t ora_paged_address(const int32_t* block_table, int64_t pos, int block_size) {
  return (int64_t)block_table[pos / block_size] * block_size + pos % block_size;
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

/* Exact GQA attention for one query position (src/model/gemma4_attention.rs
 * :94-103, and :196-234 when tau > 0). q [hq, d]; k, v [t, hkv, d];
 * q head h reads kv head h / (hq / hkv). softmax(scale * q.k) over valid
 * positions; with tau > 0 weights below tau are zeroed without
 * renormalisation (gemma4_attention.rs:226-229). out [hq, d]. */
void ora_attention_f64(const double* q, const double* k, const double* v, const uint8_t* valid,
                       int64_t t, int hq, int hkv, int d, double scale, double tau, double* out) {
  int rep = hq / hkv;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) if (t * d > 65536)
#endif
  for (int h = 0; h < hq; h++) {
    double* s = (double*)malloc(sizeof(double) * (size_t)(t > 0 ? t : 1));
    int kh = h / rep;
    double m = -INFINITY;
    for (int64_t i = 0; i < t; i++) {
      if (valid && !valid[i]) {
        s[i] = -INFINITY;
        continue;
      }
      double acc = 0.0;
      const double* kr = k + (i * hkv + kh) * d;
      for (int j = 0; j < d; j++) acc += q[h * d + j] * kr[j];
      s[i] = acc * scale;
      if (s[i] > m) m = s[i];
    }
    double l = 0.0;
    for (int64_t i = 0; i < t; i++) {
      s[i] = (s[i] == -INFINITY) ? 0.0 : exp(s[i] - m);
      l += s[i];
    }
    for (int j = 0; j < d; j++) out[h * d + j] = 0.0;
    if (l != 0.0) {
      for (int64_t i = 0; i < t; i++) {
        double w = s[i] / l;
        if (tau > 0.0 && w < tau) continue;
        const double* vr = v + (i * hkv + kh) * d;
        for (int j = 0; j < d; j++) out[h * d + j] += w * vr[j];
      }
    }
    free(s);
  }
}

/* Merge of split partials (m_i, l_i, o_i[d]) where o_i = sum exp(s - m_i) v:
 * out = sum exp(m_i - M) o_i / sum exp(m_i - M) l_i. */
void ora_lse_merge(const double* m, const double* l, const double* o, int n_parts, int d,
                   double* out) {
  double mx = -INFINITY;
  for (int i = 0; i < n_parts; i++)
    if (m[i] > mx) mx = m[i];
  double den = 0.0;
  for (int j = 0; j < d; j++) out[j] = 0.0;
  if (mx == -INFINITY) return;
  for (int i = 0; i < n_parts; i++) {
    double w = exp(m[i] - mx);
    den += w * l[i];
    for (int j = 0; j < d; j++) out[j] += w * o[i * d + j];
  }
  for (int j = 0; j < d; j++) out[j] /= den;
}

/* The reference's decode read on its bf16 cache in the op order of MLX's
 * unfused SDPA: q*scale in bf16, bf16 scores (f32 accumulation), precise
 * softmax in f32 rounded to bf16, bf16 output (f32 accumulation). This is the
 * CPU baseline the benchmark times; it is not a parity target. Every score,
 * the per-head max and sum, and every output element are computed in the
 * same order on any thread count: the scores run in parallel over (head,
 * key), the sums per head, the output over (head, 64-dim slice), each
 * summing its keys in order. */
void ora_sdpa_bf16_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t t,
                          int hq, int hkv, int d, float scale, uint16_t* out, int n_threads) {
  int rep = hq / hkv;
#ifdef _OPENMP
  if (n_threads <= 0) n_threads = omp_get_max_threads();
#endif
  float* qs = (float*)malloc(sizeof(float) * (size_t)hq * d);
  float* s = (float*)malloc(sizeof(float) * (size_t)hq * (size_t)(t > 0 ? t : 1));
  float* lsum = (float*)malloc(sizeof(float) * (size_t)hq);
  for (int h = 0; h < hq; h++)
    for (int j = 0; j < d; j++)
      qs[h * d + j] = ora_bf16_to_f32(ora_f32_to_bf16(ora_bf16_to_f32(q[h * d + j]) * scale));
#ifdef _OPENMP
#pragma omp parallel num_threads(n_threads)
#endif
  {
#ifdef _OPENMP
#pragma omp for collapse(2) schedule(static)
#endif
    for (int h = 0; h < hq; h++)
      for (int64_t i = 0; i < t; i++) {
        const uint16_t* kr = k + (i * hkv + h / rep) * d;
        const float* qh = qs + (size_t)h * d;
        float acc = 0.0f;
        for (int j = 0; j < d; j++) acc += qh[j] * ora_bf16_to_f32(kr[j]);
        s[(size_t)h * t + i] = ora_bf16_to_f32(ora_f32_to_bf16(acc));
      }
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int h = 0; h < hq; h++) {
      float* sh = s + (size_t)h * t;
      float m = -INFINITY;
      for (int64_t i = 0; i < t; i++)
        if (sh[i] > m) m = sh[i];
      float l = 0.0f;
      for (int64_t i = 0; i < t; i++) {
        sh[i] = expf(sh[i] - m);
        l += sh[i];
      }
      lsum[h] = l;
    }
#ifdef _OPENMP
#pragma omp for collapse(2) schedule(static)
#endif
    for (int h = 0; h < hq; h++)
      for (int j0 = 0; j0 < d; j0 += 64) {
        const float* sh = s + (size_t)h * t;
        const float l = lsum[h];
        float o[64];
        const int nj = d - j0 < 64 ? d - j0 : 64;
        for (int j = 0; j < nj; j++) o[j] = 0.0f;
        for (int64_t i = 0; i < t; i++) {
          float w = ora_bf16_to_f32(ora_f32_to_bf16(sh[i] / l));
          const uint16_t* vr = v + (i * hkv + h / rep) * d + j0;
          for (int j = 0; j < nj; j++) o[j] += w * ora_bf16_to_f32(vr[j]);
        }
        for (int j = 0; j < nj; j++) out[h * d + j0 + j] = ora_f32_to_bf16(o[j]);
      }
  }
  free(qs);
  free(s);
  free(lsum);
  (void)n_threads;
}

/* The O(T) store of the reference's update_and_fetch (concat_or_init,
 * src/cache.rs:132-137): a new [t + n, row] array holding the t stored rows
 * followed by the n new ones (MLX's concatenate writes a fresh array). The
 * copy is split over n_threads. */
void ora_concat_rows(const uint16_t* old_rows, int64_t t, const uint16_t* new_rows, int64_t n,
                     int64_t row_elems, uint16_t* out, int n_threads) {
  const int64_t old_elems = t * row_elems, total = (t + n) * row_elems;
  const int64_t chunk = 1 << 18;
#ifdef _OPENMP
  if (n_threads <= 0) n_threads = omp_get_max_threads();
#pragma omp parallel for num_threads(n_threads) schedule(static)
#endif
  for (int64_t c0 = 0; c0 < total; c0 += chunk) {
    int64_t c1 = c0 + chunk < total ? c0 + chunk : total;
    if (c0 < old_elems) {
      int64_t e = c1 < old_elems ? c1 : old_elems;
      memcpy(out + c0, old_rows + c0, sizeof(uint16_t) * (size_t)(e - c0));
    }
    if (c1 > old_elems) {
      int64_t b = c0 > old_elems ? c0 : old_elems;
      memcpy(out + b, new_rows + (b - old_elems), sizeof(uint16_t) * (size_t)(c1 - b));
    }
  }
  (void)n_threads;
}

uint64_t ora_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

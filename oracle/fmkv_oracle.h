/*
 * CPU oracle for the quantized KV-cache path (TEST INFRASTRUCTURE ONLY).
 *
 * This library restates, in plain C, the reference's KV-cache arithmetic and
 * the canonical arithmetic of the MI355X kernels, so that tests and the
 * benchmark's CPU-baseline leg can check the GPU path against it. Nothing in
 * the product (the HIP library, its C ABI, its host mirror) links, loads or
 * calls this code; the product fails loudly when its own HIP library is
 * missing.
 *
 * Reference anchors (files of Adri96/gemma4-moe-flash-mlx-turbo):
 *   src/cache.rs:6-26     generate_hadamard        -> ora_generate_hadamard
 *   src/cache.rs:29-43    deterministic_signs      -> ora_deterministic_signs
 *   src/cache.rs:47-62    build_rht                -> ora_build_rht
 *   src/cache.rs:67-89    lloyd_max_codebook       -> ora_lloyd_max_codebook
 *   src/cache.rs:94-129   turbo_round_trip_kv      -> ora_turbo_round_trip_dense
 *   src/cache.rs:132-137  concat_or_init           -> ora_concat_rows (CPU baseline)
 *   src/cache.rs:140-148  tail_along_time          -> ora_slot_position / ora_ring_slot
 *   src/model/mod.rs:682-753 masks                 -> ora_causal_mask / ora_sliding_mask
 *   src/model/gemma4_attention.rs:94-103 SDPA      -> ora_attention_f64
 *   src/model/gemma4_attention.rs:196-234 sparse-V -> ora_attention_f64 (tau > 0)
 *   MLX affine quantize (mlx-rs 0.25.3 / mlx-sys 0.2.0, called at
 *   src/model/mod.rs:669-675)                      -> ora_affine_quantize
 */
#ifndef FMKV_ORACLE_H
#define FMKV_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar conversions (round-to-nearest-even) */
uint16_t ora_f32_to_f16(float f);
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_bf16(float f);
float ora_bf16_to_f32(uint16_t h);
void ora_f32_to_f16_array(const float* x, uint16_t* y, int64_t n);
void ora_f16_to_f32_array(const uint16_t* x, float* y, int64_t n);
void ora_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n);
void ora_bf16_to_f32_array(const uint16_t* x, float* y, int64_t n);

/* reference restatements (src/cache.rs) */
void ora_generate_hadamard(int n, float* h);
void ora_deterministic_signs(int n, uint64_t seed, float* s);
void ora_build_rht(int dim, uint64_t seed, float* r, float* rt);
int ora_lloyd_max_codebook(int bits, float* centroids, float* bounds);
void ora_turbo_round_trip_dense(const uint16_t* x_bf16, int64_t rows, int d, int bits,
                                uint64_t seed, uint16_t* out_bf16);
void ora_turbo_round_trip_rt(const uint16_t* x_bf16, int64_t rows, int d, int bits, const float* r,
                             const float* rt, uint16_t* out_bf16);

/* canonical rotation arithmetic shared with the kernels */
float ora_inv_sqrt(int n);
void ora_fwht(float* x, int n);
void ora_rotate_rows(const uint16_t* x_bf16, int64_t rows, int d, const float* signs, float* y);
void ora_rotate_rows_f32(const float* x, int64_t rows, int d, const float* signs, float* y);
void ora_unrotate_rows_f64(const double* y, int64_t rows, int d, const float* signs, double* x);
void ora_rotate_rows_dense_f64(const float* x, int64_t rows, int d, const float* r, double* y);

/* MLX affine group quantization (packed uint32, fp16 scale/bias) */
void ora_affine_quantize(const float* y, int64_t rows, int d, int bits, int gs,
                         uint32_t* packed, uint16_t* scales, uint16_t* biases);
void ora_affine_dequantize(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                           int64_t rows, int d, int bits, int gs, double* y);

/* TurboQuant codebook mode in canonical order */
void ora_codebook_quantize(const uint16_t* x_bf16, int64_t rows, int d, int bits,
                           const float* signs, uint32_t* packed, uint16_t* norms);
void ora_codebook_quantize_f32(const float* x, int64_t rows, int d, int bits, const float* signs,
                               uint32_t* packed, uint16_t* norms);
void ora_codebook_dequant_rotated(const uint32_t* packed, const uint16_t* norms, int64_t rows,
                                  int d, int bits, double* y);
void ora_codebook_round_trip(const uint32_t* packed, const uint16_t* norms, int64_t rows, int d,
                             int bits, const float* signs, uint16_t* out_bf16);

/* pre-append prologue: k_norm, v_norm, RoPE */
float ora_rope_inv_freq(int i, int rope_dims, float theta);
void ora_rope_cos_sin(int64_t pos, int i, int rope_dims, float theta, float* c, float* s);
void ora_k_prologue(const uint16_t* x_bf16, int d, const uint16_t* w_bf16, float eps, int64_t pos,
                    int rope_dims, float theta, uint16_t* out_bf16);
void ora_v_prologue(const uint16_t* x_bf16, int d, float eps, float* out);
void ora_kv_prologue(const uint16_t* k_bf16, const uint16_t* v_bf16, int64_t n, int h, int d,
                     int64_t pos0, const uint16_t* w_bf16, float eps, int rope_dims, float theta,
                     uint16_t* k_out_bf16, float* v_out);

/* cache index semantics */
int64_t ora_ring_slot(int64_t pos, int64_t window);
int64_t ora_slot_position(int64_t slot, int64_t offset, int64_t window);
void ora_causal_mask(int64_t offset, int64_t seq_len, float* mask);
void ora_sliding_mask(int64_t stored, int64_t seq_len, int64_t window, float* mask);
int64_t ora_paged_address(const int32_t* block_table, int64_t pos, int block_size);

/* attention */
void ora_attention_f64(const double* q, const double* k, const double* v, const uint8_t* valid,
                       int64_t t, int hq, int hkv, int d, double scale, double tau, double* out);
void ora_lse_merge(const double* m, const double* l, const double* o, int n_parts, int d,
                   double* out);
void ora_sdpa_bf16_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t t,
                          int hq, int hkv, int d, float scale, uint16_t* out, int n_threads);
void ora_concat_rows(const uint16_t* old_rows, int64_t t, const uint16_t* new_rows, int64_t n,
                     int64_t row_elems, uint16_t* out, int n_threads);

/* synthetic inputs: SplitMix64 -> Box-Muller (fp64) */
uint64_t ora_splitmix64(uint64_t* state);

#ifdef __cplusplus
}
#endif
#endif

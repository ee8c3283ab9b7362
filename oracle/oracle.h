/*
 * CPU oracle for the full-attention hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the checker that the HIP path is compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the
 * product library (librdna4attn.so) never links or calls it.
 *
 * Every function restates the reference's arithmetic in plain C (no fast-math,
 * no FP contraction: see oracle/Makefile). Attention accumulates in double, like
 * the reference's scalar oracle tests/check_rope_gpu.hip:103-130.
 *
 * Type codes are the reference's KvType values (include/rdna4/kv.h:89-98):
 *   0 = f32, 1 = f16, 2 = q8_0, 3 = q4_0, 4 = q5_0, 5 = q4_1.
 */
#ifndef RDNA4_ORACLE_H
#define RDNA4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> f32 (reference include/rdna4/fp16.h:16-57). */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* KV tables (reference include/rdna4/kv.h:139-169). -1 / 0 for an unknown type. */
int64_t orc_row_bytes(int type, int head_dim);
double orc_bytes_per_elem(int type);

/* Quantize `width` contiguous f32 values into typed bytes, block-local, exactly
 * like kv_store_row_kernel (kv.h:386-501). width % 32 == 0 for quant types.
 * Returns 0, or -1 on an unknown type / bad width. */
int orc_store_rows(int type, const float *src, void *dst, int64_t width);

/* Dequantize `width` values of typed bytes into f32 (kv.h:174-229). */
int orc_load_rows(int type, const void *src, float *dst, int64_t width);

/* The seeded fill hash (kv.h:508-513) and a fill defined as storing the hash
 * rows: element e of row r is kv_rand(r*head_dim + e, seed). */
float orc_kv_rand(uint32_t idx, uint32_t seed);
int orc_fill(int type, void *dst, int64_t n_rows, int head_dim, uint32_t seed);

/* Single-token GQA decode: q,out [n_head][hd] f32; K/V rows at
 * base + (j*n_head_kv + kvh)*row_bytes; keys 0..t inclusive; t < 0 -> zeros.
 * Double accumulation (check_rope_gpu.hip:103-130). n_threads <= 1: serial. */
int orc_attn_decode(const float *q, const void *k, const void *v, float *out, int t, int n_head,
                    int n_head_kv, int head_dim, float scale, int kt, int vt, int n_threads);

/* Batched: token i has query q[i][n_head][hd] and attends keys 0..pos[i]. */
int orc_attn_batch(const float *q, const void *k, const void *v, float *out, const int *pos,
                   int n_tok, int n_head, int n_head_kv, int head_dim, float scale, int kt, int vt,
                   int n_threads);

/* LSE merge of split partials [n_rows][n_splits][2 + hd] = (m, l, acc[hd])
 * into out [n_rows][hd], double arithmetic (attn.cuh:563-590): all-empty -> 0. */
void orc_merge(const float *partial, float *out, int n_rows, int head_dim, int n_splits);

/* g <- sigmoid(g); y <- y * g, f32 (nn.cuh:110,405-412). */
void orc_sigmoid_gate(float *g, float *y, int64_t n);

/* Split-half RoPE over the first n_rot dims (attn.cuh:30-54): f32 angle, double rotation. */
void orc_rope(float *x, int n_tokens, int n_heads, int head_dim, int n_rot, float freq_base,
              const int *pos);

/* Row RMSNorm in rms_norm_kernel's f32 order (nn.cuh:24-63): 256 chained fmaf
 * partials over elements t, t+256, ..., a halving tree p[t] += p[t+s], then
 * y = (x * scale) * w with scale = 1/sqrt(sum/ncols + eps) correctly rounded
 * (the device rsqrtf is within 1 ulp of it). w may be NULL. */
void orc_rms_norm(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                  float eps);

/* Seeded N(0,1) generator used by every test and bench input (splitmix64 +
 * Box-Muller). Deterministic across platforms. */
void orc_randn(float *dst, int64_t n, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif

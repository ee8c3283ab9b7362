/*
 * rdna4attn -- C ABI of the gfx950 (MI355X) full-attention library.
 *
 * Drop-in boundary for rdna4-infer's attention/KV operator API: every entry
 * point below replaces one `inline` launcher of the reference's headers
 * (cited per function, file:line into Vmarcelo49/rdna4-infer). The C++ header
 * shims in include/rdna4/ keep the reference's `rdna4::` names and signatures
 * and forward here, so graph.cuh / mtp.cuh / main.hip compile unchanged.
 *
 * Conventions (same as the reference):
 *   - all pointers are device pointers unless stated; the caller owns them;
 *   - work is enqueued on `stream` (a hipStream_t, NULL = the null stream) and
 *     never synchronised inside the library;
 *   - KV cache rows are addressed base + (j * n_head_kv + kvh) * row_bytes;
 *   - keys 0..t are attended (inclusive); t < 0 means no keys -> zeros;
 *   - query head h reads kv head h / (n_head / n_head_kv);
 *   - q and out may be the same buffer (in-place).
 * Return value: RD4_OK (0) on success, a negative RD4_E* code otherwise (the
 * reference's `false`). Nothing throws and nothing aborts, except the KV table
 * queries of the C++ shim, which abort on a value outside the enum like the
 * reference's kv_unreachable() (kv.h:58-69).
 */
#ifndef RDNA4ATTN_H
#define RDNA4ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KvType values, never renumbered (kv.h:89-98). */
enum {
  RD4_KV_F32 = 0,
  RD4_KV_F16 = 1,
  RD4_KV_Q8_0 = 2,
  RD4_KV_Q4_0 = 3,
  RD4_KV_Q5_0 = 4,
  RD4_KV_Q4_1 = 5
};

enum {
  RD4_OK = 0,
  RD4_EINVAL = -1,  /* bad shape, head_dim, split count or pointer alignment */
  RD4_ETYPE = -2,   /* KvType outside the enum */
  RD4_ELAUNCH = -3, /* HIP reported an error when the kernel was enqueued */
  RD4_ENOMEM = -4   /* library scratch could not be created */
};

/* ---- library ------------------------------------------------------------ */

/* Version string of this build. */
const char *rd4_version(void);
/* Create the library scratch (split records + merge counters) of the null
 * stream on the current device. Each stream gets its own scratch, so launches
 * on different streams never share records or counters; a stream's scratch is
 * created by its first split launch (hipMalloc plus a stream-ordered fill
 * kernel, no synchronisation) unless rd4_init / rd4_stream_init made it
 * first. Call them at init to keep allocation out of the first step. No
 * counterpart in the reference (its graph owned the partial buffer,
 * graph.cuh:771-778). */
int rd4_init(void);
/* The same for `stream` (a hipStream_t) on the current device. */
int rd4_stream_init(void *stream);
/* Human-readable reason of the last non-OK return on this thread. */
const char *rd4_last_error(void);

/* ---- KV tables (kv.h:100-169) -------------------------------------------- */

/* kv_type_name (kv.h:100): "<unknown-kv-type>" outside the enum. */
const char *rd4_kv_type_name(int type);
/* kv_type_parse (kv.h:129): NULL and *out set on success, else the message. */
const char *rd4_kv_type_parse(const char *name, int *out);
/* kv_bytes_per_elem (kv.h:139): 0.0 outside the enum. */
double rd4_kv_bytes_per_elem(int type);
/* kv_row_bytes (kv.h:155): bytes of one head_dim row; -1 outside the enum. */
int64_t rd4_kv_row_bytes(int type, int head_dim);

/* ---- KV budget (device.h:36-50, 148-190) ----------------------------------- */

/* kv_cache_bytes (device.h:176): bytes of the K and V caches of the reference
 * model shape (16 full-attention layers x 4 kv heads x head_dim 256) at
 * ctx_size tokens, computed exactly as the reference does (a double product,
 * truncated). 0 for a type outside the enum. */
uint64_t rd4_kv_cache_bytes(uint64_t ctx_size, int kt, int vt);
/* The same for any attention shape: n_layers x n_head_kv rows of head_dim
 * elements per token for K and for V. 0 for a bad type or shape. */
uint64_t rd4_kv_cache_bytes_shape(uint64_t ctx_size, int n_layers, int n_head_kv, int head_dim,
                                  int kt, int vt);
/* Largest context whose caches fit in budget_bytes after reserved_bytes (the
 * weights, buffers and the reference's allocator margin), capped at the
 * reference's kMaxCtxSize (2^24, device.h:167). 0 when nothing fits or the
 * arguments are invalid. Sized for a whole GPU: MI355X has 288 GB of HBM. */
uint64_t rd4_kv_max_ctx(uint64_t budget_bytes, uint64_t reserved_bytes, int n_layers, int n_head_kv,
                        int head_dim, int kt, int vt);

/* ---- KV append / fill / dequant (kv.h:386-694) --------------------------- */

/* kv_store_row_launch (kv.h:683): quantize `width` contiguous f32 values into
 * the cache bytes at dst (block-local, so width may span n_tok*n_head_kv*hd).
 * Quantized types need width % 32 == 0; src 4-byte and dst 2-byte aligned. */
int rd4_kv_store_row_launch(int type, const float *src, void *dst, int64_t width, void *stream);
/* kv_fill_launch (kv.h:632): fill n_rows rows with the seeded kv_rand hash
 * (kv.h:508-513), byte-identical to storing those hash values with
 * rd4_kv_store_row_launch. */
int rd4_kv_fill_launch(int type, void *cache, int64_t n_rows, int head_dim, uint32_t seed,
                       void *stream);
/* Dequantize `width` stored values to f32, as kv_load<>/kv_load8<>
 * (kv.h:174-368) return them. Test and inspection hook. */
int rd4_kv_load_rows_launch(int type, const void *src, float *dst, int64_t width, void *stream);

/* ---- decode attention (attn.cuh:200-249, 592-667, 895-956) --------------- */

/* attn_launch (attn.cuh:200): one query token [n_head][head_dim] f32. */
int rd4_attn_launch(const float *q, const void *k, const void *v, float *out, int t, int n_head,
                    int n_head_kv, int head_dim, float scale, int kt, int vt, void *stream);
/* attn_launch_split (attn.cuh:903). n_splits >= 1 is the minimum key split
 * count. `partial` (caller-owned, at least attn_partial_bytes(n_head,
 * head_dim, n_splits) bytes, or NULL) receives the split records when the
 * split count the library runs is at most n_splits, as in attn.cuh:593-608;
 * otherwise the records go to the stream's library scratch. Either way, two
 * streams never share records. A count the scratch cannot hold: RD4_EINVAL. */
int rd4_attn_launch_split(const float *q, const void *k, const void *v, float *out,
                          float *partial, int t, int n_head, int n_head_kv, int head_dim,
                          float scale, int kt, int vt, int n_splits, void *stream);
/* attn_launch_split_wpb (attn.cuh:630): wpb must be 8, 16 or 32 (bench knob of
 * the reference; the gfx950 kernels fix their own CTA shape). */
int rd4_attn_launch_split_wpb(const float *q, const void *k, const void *v, float *out,
                              float *partial, int t, int n_head, int n_head_kv, int head_dim,
                              float scale, int kt, int vt, int n_splits, int wpb, void *stream);
/* attn_partial_bytes (attn.cuh:665). */
size_t rd4_attn_partial_bytes(int n_head, int head_dim, int n_splits);
/* attn_split_wpb (attn.cuh:895): the reference's policy values (16 or 8). */
int rd4_attn_split_wpb(int n_splits);

/* Native decode entry: attention of one token and, when gate != NULL, the
 * sigmoid output gate fused into the epilogue (out *= sigmoid(gate) and gate <-
 * sigmoid(gate), the pair attn_launch_split + sigmoid_gate_launch of
 * graph.cuh:958-981). n_splits = 0 picks the split count for the GPU; n_splits
 * >= 1 forces exactly that many contiguous key splits. */
int rd4_attn_decode(const float *q, const void *k, const void *v, float *out, float *gate, int t,
                    int n_head, int n_head_kv, int head_dim, float scale, int kt, int vt,
                    int n_splits, void *stream);

/* Native decode with the KV append fused in: quantizes k_new / v_new (f32
 * [n_head_kv][head_dim], 16-byte aligned) into cache row t exactly like
 * rd4_kv_store_row_launch, then attends keys 0..t -- the sequence
 * kv_write_batch + attn_launch_split + sigmoid_gate_launch of graph.cuh:954-981
 * in one launch. gate may be NULL. */
int rd4_attn_decode_append(const float *q, const float *k_new, const float *v_new, void *k,
                           void *v, float *out, float *gate, int t, int n_head, int n_head_kv,
                           int head_dim, float scale, int kt, int vt, int n_splits, void *stream);

/* Allocation-free form of rd4_attn_decode_append, same arguments and results
 * within the attention tolerance (bit-identical at the same split count). No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops). It calls no hipMalloc or
 * hipFree: its split records live in a fixed 4 MiB device array of the library
 * (one per GPU, held until the process ends; rd4_init, or the first call on a
 * device, looks up its address). Shapes whose records exceed it (n_head x
 * splits x (head_dim + 2) floats > 1M) are refused with RD4_EINVAL when
 * n_splits is given, and run with fewer splits when it is 0; shapes that take
 * the generic kernel run one split. Calls that overlap on one GPU (two
 * streams, or concurrent graph replays) share the array and race. */
int rd4_attn_decode_append_noalloc(const float *q, const float *k_new, const float *v_new, void *k,
                                   void *v, float *out, float *gate, int t, int n_head,
                                   int n_head_kv, int head_dim, float scale, int kt, int vt,
                                   int n_splits, void *stream);

/* Native multi-token decode (the MTP verify step: N = D+1 drafted tokens,
 * graph.cuh:1494-1527 through attn_split_batch_launch; mtp.cuh:585-596 for the
 * draft token itself): tokens i = 0..n_tok-1 sit at consecutive positions
 * t0 + i and token i attends keys 0..t0+i (the rows were appended before the
 * call). q/out/gate are [n_tok][n_head][head_dim]; gate may be NULL, else
 * fused as in rd4_attn_decode. n_splits = 0 picks the split count for the GPU
 * from the token count; n_splits >= 1 forces it. On the MFMA path (hd 256,
 * GQA group <= 8) one CTA carries two consecutive tokens, so every K/V tile is
 * read and converted once per pair; those queries enter the products as f16
 * (results within the attention tolerance, not bit-identical to per-token
 * decode; rd4_attn_split_batch_launch keeps that identity). */
int rd4_attn_decode_tokens(const float *q, const void *k, const void *v, float *out, float *gate,
                           int t0, int n_tok, int n_head, int n_head_kv, int head_dim, float scale,
                           int kt, int vt, int n_splits, void *stream);

/* ---- batched attention (attn.cuh:373-424, 958-1049) ---------------------- */

/* attn_batch_launch (attn.cuh:373): token i of n_tok attends keys 0..pos[i]
 * (pos is a device int array); q/out [n_tok][n_head][head_dim]. */
int rd4_attn_batch_launch(const float *q, const void *k, const void *v, float *out,
                          const int *pos, int n_tok, int n_head, int n_head_kv, int head_dim,
                          float scale, int kt, int vt, void *stream);
/* attn_split_batch_launch (attn.cuh:958): as above with exactly n_splits key
 * splits per token. `partial` (n_tok * attn_partial_bytes(n_head, head_dim,
 * n_splits) bytes, or NULL) receives the records as in rd4_attn_launch_split. */
int rd4_attn_split_batch_launch(const float *q, const void *k, const void *v, float *out,
                                float *partial, const int *pos, int n_tok, int n_head,
                                int n_head_kv, int head_dim, float scale, int kt, int vt,
                                int n_splits, void *stream);

/* ---- prefill (attn_fa2.cuh:173-207) --------------------------------------- */

/* fa2_prefill_launch (attn_fa2.cuh:173): causal prefill of n_q query tokens at
 * positions pos[i] (device array) over an f16 K/V cache; q/o f32
 * [n_q][n_head][head_dim]; keys 0..min(pos[i], kmax); keys_total rows exist. */
int rd4_fa2_prefill_launch(const float *q, const void *k, const void *v, float *o,
                           const int *pos, int n_q, int kmax, int keys_total, int n_head,
                           int n_head_kv, int head_dim, float scale, void *stream);
/* fa2_prefill_usable (attn_fa2.cuh:192): 1 when rd4_fa2_prefill_launch takes
 * this shape. The gfx950 kernel admits every chunk size and key count for
 * f16/f16 with head_dim 256 (RD_GFX12_FA2_PREFILL=0 still disables it). */
int rd4_fa2_prefill_usable(int kt, int vt, int n_q, int pos0, int n_head, int n_head_kv,
                           int head_dim);

/* Native prefill entry: n_q query tokens at consecutive positions pos0..pos0+n_q-1
 * attend causally to cache rows 0..pos0+i. q_f16 != 0 means q is f16
 * [n_q][n_head][hd], else f32. gate (optional, f32, same shape) is fused:
 * out *= sigmoid(gate), gate <- sigmoid(gate) (graph.cuh:1534-1535). */
int rd4_prefill(const void *q, int q_f16, const void *k, const void *v, float *out, float *gate,
                int pos0, int n_q, int n_head, int n_head_kv, int head_dim, float scale, int kt,
                int vt, void *stream);

/* Prefill with the chunk's K/V append fused into the same launch: the store of
 * graph.cuh:1462 (kv_write_batch -> kv_store_row_launch over the chunk's rows,
 * graph.cuh:1011-1031, kv.h:683) and the prefill + gate of graph.cuh:1479-1535
 * in one pass. k_new / v_new are f32
 * [n_q][n_head_kv][head_dim]; their rows are quantized to dst_type into k_dst /
 * v_dst (rows contiguous, the chunk's first row at the pointer), byte-identical to
 * rd4_kv_store_row_launch. The destination must not overlap the attended rows
 * 0..pos0+n_q-1 of k or v (the launch reads them while it writes): RD4_EINVAL.
 * Shapes the MFMA kernel does not take run the store launches then the prefill. */
int rd4_prefill_append(const void *q, int q_f16, const void *k, const void *v, float *out,
                       float *gate, int pos0, int n_q, int n_head, int n_head_kv, int head_dim,
                       float scale, int kt, int vt, const float *k_new, const float *v_new,
                       void *k_dst, void *v_dst, int dst_type, void *stream);

/* ---- gate / rope ---------------------------------------------------------- */

/* sigmoid_gate_launch (nn.cuh:414): g <- sigmoid(g); y <- y * g. */
int rd4_sigmoid_gate_launch(float *g_io, float *y_io, int64_t n, void *stream);
/* rope_launch (attn.cuh:56): split-half RoPE over the first n_rot dims of each
 * head of x [n_tokens][n_heads][head_dim], positions pos[t] (device). */
int rd4_rope_launch(float *x, int n_tokens, int n_heads, int head_dim, int n_rot,
                    float freq_base, const int *pos, void *stream);

/* ---- pre-attention epilogue (nn.cuh:24-63,239; graph.cuh:914-954) -------- */

/* rms_norm_launch (nn.cuh:239): per row of ncols f32, y = x * scale * w with
 * scale = rsqrtf(sum(x^2) / ncols + eps), the sum in the reference's order (256
 * chained fmaf partials and a halving tree), so y is bit-identical to the
 * reference kernel built for the same GPU. w may be NULL (no weight); y may be x. */
int rd4_rms_norm_launch(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                        float eps, void *stream);

/* Fused pre-attention epilogue: for each of n_tok tokens, the six launches
 * deinterleave_q_gate + rms_norm(q) + rms_norm(k) + rope(q) + rope(k) +
 * kv_write_batch of graph.cuh:914-954 (one token) and graph.cuh:1444-1462 (a
 * chunk) in one launch, with the same bits as that sequence:
 *   qg      [n_tok][n_head][2][head_dim]  projection output, q then gate per head
 *   k_new, v_new [n_tok][n_head_kv][head_dim]
 *   q_norm, k_norm [head_dim] weights (NULL = none); eps as rms_norm
 *   RoPE over the first n_rot dims (even, <= head_dim) at position pos[i]
 *   q_out   [n_tok][n_head][head_dim]  normed, rotated q
 *   gate_out (may be NULL)            the raw gate half, deinterleaved
 *   k_out   (may be NULL, may be k_new) the normed, rotated k
 *   K/V cache rows pos[i] * n_head_kv + h of k / v, quantized as kt / vt.
 * The reference's kv_write_batch stores token i at row pos0 + i; here the row
 * is pos[i], equal for the consecutive positions the graph passes. head_dim is
 * 64, 128, 256 or 512; f32 buffers 16-byte aligned. */
int rd4_qk_norm_rope_append(const float *qg, const float *k_new, const float *v_new,
                            const float *q_norm, const float *k_norm, float eps, int n_rot,
                            float freq_base, const int *pos, int n_tok, int n_head, int n_head_kv,
                            int head_dim, float *q_out, float *gate_out, float *k_out, void *k,
                            void *v, int kt, int vt, void *stream);

/* ---- diagnostics ------------------------------------------------------------ */

/* Streaming read of `bytes` bytes (16-byte aligned, a multiple of 16) by one
 * launch that only loads and discards (sink: a device word written only in an
 * unlikely case). Used by bench.py to measure the practical HBM read rate of a
 * decode-sized launch; no counterpart in the reference. */
int rd4_read_probe(const void *buf, int64_t bytes, void *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif

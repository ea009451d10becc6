/*
 * nnz.h -- C ABI of the MI355X (gfx950) decode hot path.
 *
 * This header is the drop-in boundary that replaces nnmetal's kernel-dispatch
 * API (duanebester/nnzap, nnmetal/src/transformer.zig:384-2387) and the
 * Metal platform calls under it (nnmetal/src/metal.zig).  Every dispatch entry
 * point mirrors one reference `dispatch*` helper: same name (prefixed
 * `nnz_`), same buffer roles, the reference's dims struct passed unchanged.
 * Each declaration cites the reference function it replaces.
 *
 * Differences from the reference, by design:
 *   - Buffers are plain device pointers (hipMalloc'd memory or torch tensors),
 *     not MTLBuffers; quantised weights are described by `nnz_qweight`
 *     (codes / scales / biases pointers) instead of PackedBuffer/Q4Buffer.
 *   - The "encoder" is an `nnz_ctx` that owns a HIP stream; launches are
 *     asynchronous on that stream, in call order (the reference's barriers
 *     become stream order).
 *   - Every function returns an int status (NNZ_OK == 0, negative on error)
 *     instead of asserting; nnz_last_error() returns a message.  Nothing in
 *     this library aborts the process.
 *   - Activation/storage dtypes are parameters where BASELINE configurations
 *     and the reference differ (f32 / f16 / bf16).
 *
 * Threading: one nnz_ctx per host thread.  Nothing here is thread-safe across
 * threads sharing a ctx.
 */
#ifndef NNZ_H
#define NNZ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define NNZ_OK            0
#define NNZ_EINVAL       -1  /* invalid dims / null pointer / bad dtype      */
#define NNZ_EUNSUPPORTED -2  /* legal for the reference, not implemented here */
#define NNZ_EHIP         -3  /* a HIP runtime call failed                     */
#define NNZ_ENOMEM       -4  /* device allocation failed                      */
#define NNZ_ETIMEOUT     -5  /* bounded host wait expired                     */
#define NNZ_ESTATE       -6  /* call not valid in the current state           */

/* ---- element types ------------------------------------------------------ */
#define NNZ_F32  0
#define NNZ_F16  1
#define NNZ_BF16 2

/* ---- dims structs: byte-for-byte the reference's extern structs --------- */

/* transformer.zig:389-393 RMSNormDims */
typedef struct { uint32_t hidden_size, num_tokens; float eps; } nnz_rmsnorm_dims;
/* transformer.zig:396-401 RoPEDims */
typedef struct { uint32_t num_heads, head_dim, position; float rope_theta; } nnz_rope_dims;
/* transformer.zig:404-409 KVUpdateDims */
typedef struct { uint32_t num_kv_heads, head_dim, position, max_context_length; } nnz_kv_update_dims;
/* transformer.zig:412-418 FusedRoPEKVDims */
typedef struct {
    uint32_t num_kv_heads, head_dim, position, max_context_length;
    float rope_theta;
} nnz_fused_rope_kv_dims;
/* transformer.zig:421-427 FusedNormRoPEDims */
typedef struct {
    uint32_t num_heads, head_dim, position;
    float eps, rope_theta;
} nnz_fused_norm_rope_dims;
/* transformer.zig:430-437 FusedKNormRoPEKVDims */
typedef struct {
    uint32_t num_kv_heads, head_dim, position, max_context_length;
    float eps, rope_theta;
} nnz_fused_k_norm_rope_kv_dims;
/* transformer.zig:440-447 GQADims */
typedef struct {
    uint32_t num_query_heads, num_kv_heads, head_dim, seq_len, max_context_length,
             heads_per_kv_group;
} nnz_gqa_dims;
/* transformer.zig:451-461 GQAFusedDims */
typedef struct {
    uint32_t num_query_heads, num_kv_heads, head_dim, seq_len, max_context_length,
             heads_per_kv_group, position;
    float eps, rope_theta;
} nnz_gqa_fused_dims;
/* transformer.zig:464-469 EmbedDims */
typedef struct { uint32_t vocab_size, hidden_size, num_tokens, group_size; } nnz_embed_dims;
/* transformer.zig:475-479 QMVDims (M = output rows, K = input length) */
typedef struct { uint32_t M, K, group_size; } nnz_qmv_dims;

/* Quantised weight matrix [M x K], row-major.  Replaces metal.zig:227-335
 * (PackedBuffer, bits=1: codes + f16 scales, symmetric +-s) and
 * metal.zig:337-469 (Q4Buffer, bits=4: codes + scales + biases, s*n+b).
 * codes: uint32 words, 32 (Q1) or 8 (Q4) columns each, LSB first.
 * scales/biases: one 16-bit value per group of `group_size` columns of a
 * row; `scale_dtype` is NNZ_F16 or NNZ_BF16 (Q1 requires NNZ_F16).
 * All three pointers must be 4-byte aligned device pointers. */
typedef struct {
    const void *codes;
    const void *scales;
    const void *biases;      /* NULL for Q1 */
    uint32_t packed_count;   /* M*K */
    uint32_t group_size;
    uint32_t bits;           /* 1 or 4 */
    uint32_t scale_dtype;    /* NNZ_F16 / NNZ_BF16 */
} nnz_qweight;

typedef struct nnz_ctx nnz_ctx;
typedef struct nnz_graph nnz_graph;

/* ---- context, memory, sync: replaces metal.zig:839-1372 (Device) -------- */

/* Create a context on HIP device `device`.  If `hip_stream` is NULL the
 * context creates its own stream (default priority); otherwise it borrows the
 * caller's stream.  Replaces Device.init (metal.zig:959-1020). */
int nnz_ctx_create(int device, void *hip_stream, nnz_ctx **out);
int nnz_ctx_destroy(nnz_ctx *ctx);
void *nnz_ctx_stream(nnz_ctx *ctx);
const char *nnz_last_error(nnz_ctx *ctx);  /* never NULL */
const char *nnz_version(void);

/* Explicit device memory; replaces shared MTLBuffers (metal.zig:80-469).
 * nnz_alloc zero-fills (metal.zig Rule 21). */
int nnz_alloc(nnz_ctx *ctx, size_t bytes, void **out);
int nnz_free(nnz_ctx *ctx, void *ptr);
int nnz_upload(nnz_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
int nnz_download(nnz_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);
/* Bounded wait for all work on the ctx stream; replaces commitAndWait /
 * commitAndSpinOnFlag (metal.zig:1293-1352), which could spin forever. */
int nnz_stream_sync(nnz_ctx *ctx, uint32_t timeout_ms);

/* Stream capture into a HIP graph (one graph per decode step). */
int nnz_graph_begin(nnz_ctx *ctx);
int nnz_graph_end(nnz_ctx *ctx, nnz_graph **out);
int nnz_graph_replay(nnz_ctx *ctx, nnz_graph *g);
int nnz_graph_destroy(nnz_graph *g);

/* Context options (new; the reference has no counterpart).
 * NNZ_OPT_Q1_MATRIX_CORES selects the kernel of 1-bit QMVs with K = 2048 and
 * group size 128: 0 = the library's choice by shape (default), 1 = the
 * block-scaled MFMA kernel wherever it applies, 2 = never it (the VALU
 * kernels).  Results agree to float32 rounding either way; a captured graph
 * keeps the kernels chosen at capture. */
#define NNZ_OPT_Q1_MATRIX_CORES 1
int nnz_ctx_set_option(nnz_ctx *ctx, int option, int value);

/* Device-side timing on the ctx stream (HIP events). */
int nnz_timer_mark(nnz_ctx *ctx, int slot);           /* slot 0..63 */
int nnz_timer_elapsed_ms(nnz_ctx *ctx, int slot_a, int slot_b, float *ms);

/* ---- QMV family, Q1 (1-bit symmetric) ---------------------------------- */
/* Q1 entry points require bits == 1, K % 32 == 0, group_size % 32 == 0 and
 * K % group_size == 0 (the reference asserts K % 32 and K % gs too). */

/* transformer.zig:1565 dispatchQMV: f32 x[K] -> f32 y[M]. */
int nnz_dispatch_qmv(nnz_ctx *ctx, const nnz_qweight *w, const float *input,
                     float *output, nnz_qmv_dims dims);
/* transformer.zig:1653 dispatchQMVf16in: f16 x -> f32 y (LM head). */
int nnz_dispatch_qmv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                           float *output, nnz_qmv_dims dims);
/* transformer.zig:1728 dispatchQMVf16io: f16 x -> f16 y. */
int nnz_dispatch_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                           void *output, nnz_qmv_dims dims);
/* transformer.zig:1806 dispatchQMVf16ioResadd: residual[r] += (W x)[r]. */
int nnz_dispatch_qmv_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                                  float *residual, nnz_qmv_dims dims);
/* transformer.zig:1120 dispatchQMVFusedPair: two matrices, shared f32 x. */
int nnz_dispatch_qmv_fused_pair(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                const float *input, float *output_a, float *output_b,
                                nnz_qmv_dims dims);
/* transformer.zig:1181 dispatchQMVFusedPairf16in: f16 x, f32 outputs. */
int nnz_dispatch_qmv_fused_pair_f16in(nnz_ctx *ctx, const nnz_qweight *wa,
                                      const nnz_qweight *wb, const void *input,
                                      float *output_a, float *output_b, nnz_qmv_dims dims);
/* transformer.zig:1238 dispatchQMVFusedPairf16io: f16 x, f16 outputs. */
int nnz_dispatch_qmv_fused_pair_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                      const nnz_qweight *wb, const void *input,
                                      void *output_a, void *output_b, nnz_qmv_dims dims);
/* transformer.zig:1309 dispatchQMVFusedPairSiLUf16io: out = f16(silu(Wa x) * (Wb x)). */
int nnz_dispatch_qmv_fused_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                           const nnz_qweight *wb, const void *input,
                                           void *output, nnz_qmv_dims dims);
/* BASELINE config 3 form of the same kernel (no reference counterpart with
 * f32 I/O; same math as transformer.zig:1309): f32 x -> f32 out. */
int nnz_dispatch_qmv_fused_pair_silu(nnz_ctx *ctx, const nnz_qweight *wa,
                                     const nnz_qweight *wb, const float *input,
                                     float *output, nnz_qmv_dims dims);
/* transformer.zig:1373 dispatchFusedNormPairSiLUf16io: x = f16(rmsnorm(res)*w)
 * computed in the kernel from the f32 residual and f32 norm_scale[K]. */
int nnz_dispatch_fused_norm_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                            const nnz_qweight *wb, const float *residual,
                                            void *output, const float *norm_scale,
                                            nnz_qmv_dims dims);
/* transformer.zig:1438 dispatchFusedNormQMVf16io. */
int nnz_dispatch_fused_norm_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                                      void *output, const float *norm_scale, nnz_qmv_dims dims);
/* transformer.zig:1501 dispatchFusedNormPairQMVf16io. */
int nnz_dispatch_fused_norm_pair_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                           const nnz_qweight *wb, const float *residual,
                                           void *output_a, void *output_b,
                                           const float *norm_scale, nnz_qmv_dims dims);

/* One launch for the pair transformer.zig:1438 dispatchFusedNormQMVf16io (Q)
 * + :1501 dispatchFusedNormPairQMVf16io (K, V), which share the normalised
 * input (encodeAttnProjFusedNorm, :3024-3083).  q_dims = {Q rows, K, gs};
 * wk and wv have kv_rows rows each. */
int nnz_dispatch_fused_norm_qkv_f16io(nnz_ctx *ctx, const nnz_qweight *wq, const nnz_qweight *wk,
                                      const nnz_qweight *wv, const float *residual, void *out_q,
                                      void *out_k, void *out_v, const float *norm_scale,
                                      nnz_qmv_dims q_dims, uint32_t kv_rows);
/* One launch for transformer.zig:669 dispatchRMSNorm (rms_norm_f16out) +
 * :1653 dispatchQMVf16in, the final norm + LM head (encodeFinalNormAndLMHead,
 * :2730-2785): the normalised input is rounded to f16 exactly as the
 * reference stores it, logits are f32. */
int nnz_dispatch_fused_norm_qmv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                                      float *output, const float *norm_scale, nnz_qmv_dims dims);

/* ---- QMV family, Q4 (4-bit affine) ------------------------------------- */
/* Q4 entry points require bits == 4, K % 32 == 0, group_size % 32 == 0 and
 * K % group_size == 0.  The `*_f16io*` / `_f16in` forms reproduce the
 * reference's BF16-faithful outputs: results are BF16-truncated before being
 * stored (q4mv_bf16_specialized.metal:52-57) and fused-norm inputs are
 * BF16-truncated before narrowing to f16 (:806). */

/* BASELINE config 1: f32 x -> f32 y, plain fp32 result (no truncation). */
int nnz_dispatch_q4mv(nnz_ctx *ctx, const nnz_qweight *w, const float *input, float *output,
                      nnz_qmv_dims dims);
/* transformer.zig:1903 dispatchQ4MVf16io. */
int nnz_dispatch_q4mv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                            void *output, nnz_qmv_dims dims);
/* transformer.zig:1944 dispatchQ4MVf16in (f32 out, BF16-truncated). */
int nnz_dispatch_q4mv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                            float *output, nnz_qmv_dims dims);
/* transformer.zig:1987 dispatchQ4MVf16ioResadd. */
int nnz_dispatch_q4mv_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                                   float *residual, nnz_qmv_dims dims);
/* transformer.zig:2069 dispatchQ4MVFusedPairf16io. */
int nnz_dispatch_q4mv_fused_pair_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                       const nnz_qweight *wb, const void *input,
                                       void *output_a, void *output_b, nnz_qmv_dims dims);
/* transformer.zig:2118 dispatchQ4MVFusedPairSiLUf16io. */
int nnz_dispatch_q4mv_fused_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                            const nnz_qweight *wb, const void *input,
                                            void *output, nnz_qmv_dims dims);
/* transformer.zig:2166 dispatchQ4FusedNormQMVf16io. */
int nnz_dispatch_q4_fused_norm_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w,
                                         const float *residual, void *output,
                                         const float *norm_scale, nnz_qmv_dims dims);
/* transformer.zig:2237 dispatchQ4FusedNormPairQMVf16io. */
int nnz_dispatch_q4_fused_norm_pair_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                              const nnz_qweight *wb, const float *residual,
                                              void *output_a, void *output_b,
                                              const float *norm_scale, nnz_qmv_dims dims);
/* transformer.zig:2318 dispatchQ4FusedNormPairSiLUf16io. */
int nnz_dispatch_q4_fused_norm_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                               const nnz_qweight *wb, const float *residual,
                                               void *output, const float *norm_scale,
                                               nnz_qmv_dims dims);

/* ---- stacked QMV: many matrices of one shape in one launch ---------------
 * New (the reference has no counterpart; the arithmetic is that of
 * dispatchQMV transformer.zig:1565, dispatchQ4MV :1895 and
 * dispatchQMVFusedPairSiLUf16io :1304 with f32 input and output).  Matrix i
 * (0 <= i < count) has its codes, scales (and biases) at i * codes_stride /
 * i * scales_stride bytes past those of `w` (a pair: `wa` and `wb` advance
 * together), its input at i * input_stride and its output at
 * i * output_stride bytes past `input` / `output`.  One launch streams them
 * all: the stacked-launch form of an HBM-bandwidth measurement and a
 * batched decode of independent matrices.  Strides keep 16-byte alignment
 * (codes, inputs) and 4-byte alignment (scales, outputs).
 * blocks_per_matrix 0 lets the library choose. */
typedef struct {
    uint32_t count;
    uint32_t blocks_per_matrix;
    uint64_t codes_stride, scales_stride, input_stride, output_stride;
} nnz_qmv_stack;
int nnz_dispatch_qmv_stacked(nnz_ctx *ctx, const nnz_qweight *w, const float *input,
                             float *output, nnz_qmv_dims dims, const nnz_qmv_stack *stack);
int nnz_dispatch_q4mv_stacked(nnz_ctx *ctx, const nnz_qweight *w, const float *input,
                              float *output, nnz_qmv_dims dims, const nnz_qmv_stack *stack);
int nnz_dispatch_qmv_fused_pair_silu_stacked(nnz_ctx *ctx, const nnz_qweight *wa,
                                             const nnz_qweight *wb, const float *input,
                                             float *output, nnz_qmv_dims dims,
                                             const nnz_qmv_stack *stack);

/* ---- dequantisation (bit-exact artefact) -------------------------------- */
/* New (no reference kernel; the math of transformer.metal:469-480 / :537-545):
 * out[M*K] = fp32 dequantised weights, Q1 +-s, Q4 fmaf(s, n, b). */
int nnz_dispatch_dequant(nnz_ctx *ctx, const nnz_qweight *w, float *output, nnz_qmv_dims dims);

/* ---- prefill dequant-GEMM (new: reference prefills token by token,
 *      transformer.zig:4032-4068) --------------------------------------------
 * C[P x M] = A[P x K] (f16, row-major) . dequant(W[M x K])^T, fp32 accumulate on
 * MFMA.  Epilogue `mode`: NNZ_GEMM_STORE_F16 (C -> f16 out), NNZ_GEMM_STORE_F32,
 * NNZ_GEMM_RESADD (out_f32[p*M+m] += C), NNZ_GEMM_SILU_PAIR (wb required:
 * out f16 = silu(A.Wa^T) * (A.Wb^T)).  `lda` = K.  Q1 weights: codes 8-byte
 * aligned.  Q4 weights (q4_mlx, bf16 or f16 scales and biases, codes 16-byte
 * aligned): every result is BF16-truncated before its store, += or the
 * SiLU*mul product's store, like the Q4 decode kernels
 * (q4mv_bf16_specialized.metal:52-57).  M, K and the group size multiples of
 * 64, the group size a power of two. */
#define NNZ_GEMM_STORE_F16 0
#define NNZ_GEMM_STORE_F32 1
#define NNZ_GEMM_RESADD    2
#define NNZ_GEMM_SILU_PAIR 3
int nnz_dispatch_dequant_gemm(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                              const void *a_f16, uint32_t num_tokens, void *output,
                              int mode, nnz_qmv_dims dims);

/* ---- transformer kernels (transformer.metal) ----------------------------- */

/* transformer.zig:669 dispatchRMSNorm.  The reference selects a pipeline
 * variant; here `out_dtype` selects it: NNZ_F32 (rms_norm), NNZ_F16
 * (rms_norm_f16out), and `bf16_trunc`=1 with NNZ_F16 gives rms_norm_bf16_f16out.
 * input/scale are f32. */
int nnz_dispatch_rms_norm(nnz_ctx *ctx, const float *input, const float *scale, void *output,
                          int out_dtype, int bf16_trunc, nnz_rmsnorm_dims dims);
/* transformer.zig:700 dispatchSiLU (f32). */
int nnz_dispatch_silu(nnz_ctx *ctx, const float *input, float *output, uint32_t count);
/* transformer.zig:719 dispatchSiLUElementwiseMul; dtype NNZ_F32 or NNZ_F16
 * (silu_elementwise_mul / silu_elementwise_mul_f16). */
int nnz_dispatch_silu_elementwise_mul(nnz_ctx *ctx, const void *gate, const void *up,
                                      void *output, int dtype, uint32_t count);
/* transformer.zig:740 dispatchRoPE: in place, consecutive pairs; dtype
 * NNZ_F32 (rope), NNZ_F16 (rope_f16) or NNZ_BF16. */
int nnz_dispatch_rope(nnz_ctx *ctx, void *data, int dtype, nnz_rope_dims dims);
/* transformer.zig:760 dispatchKVCacheUpdate: K[h][pos][d], V[h][d][pos]
 * (V transposed as in transformer.metal:1092-1112).  proj dtype NNZ_F32 or
 * NNZ_F16; cache dtype NNZ_F16 or NNZ_BF16. */
int nnz_dispatch_kv_cache_update(nnz_ctx *ctx, const void *k_proj, const void *v_proj,
                                 int proj_dtype, void *k_cache, void *v_cache, int cache_dtype,
                                 nnz_kv_update_dims dims);
/* transformer.zig:792 dispatchFusedRoPEKVCache (f16 proj/cache). */
int nnz_dispatch_fused_rope_kv_cache(nnz_ctx *ctx, const void *k_proj, const void *v_proj,
                                     void *k_cache, void *v_cache, nnz_fused_rope_kv_dims dims);
/* transformer.zig:829 dispatchFusedNormRoPE: per-head RMSNorm (f32 scale)
 * + RoPE, f16 in place. */
int nnz_dispatch_fused_norm_rope(nnz_ctx *ctx, void *data, const float *scale,
                                 nnz_fused_norm_rope_dims dims);
/* transformer.zig:866 dispatchFusedKNormRoPEKVCache (f16). */
int nnz_dispatch_fused_k_norm_rope_kv_cache(nnz_ctx *ctx, const void *k_proj,
                                            const void *v_proj, void *k_cache, void *v_cache,
                                            const float *k_scale,
                                            nnz_fused_k_norm_rope_kv_dims dims);

/* Decode attention.  transformer.zig:1030 dispatchGQAAttention / :915
 * dispatchGQAAttentionTG.  One entry point covers both (the reference's
 * seq_len <= 7168 TG variant and the device-scratch variant): the kernel
 * splits the sequence across workgroups (flash-decoding partials + combine),
 * so there is no seq_len limit beyond max_context_length.
 *   q: [Hq x D] in q_dtype (F32/F16/BF16), used as is (already normed/roped)
 *      unless rope_position >= 0, in which case RoPE(rope_position, rope_theta)
 *      is applied to q first;
 *   k_cache: [Hkv][max_ctx][D]; v_cache: [Hkv][D][max_ctx] if v_transposed
 *      (reference layout) else [Hkv][max_ctx][D]; kv_dtype F16 or BF16;
 *   output: [Hq x D] in out_dtype (F32/F16/BF16);
 *   scratch: device workspace of nnz_gqa_scratch_bytes(dims) bytes (replaces
 *      the reference's attn_scratch buffer(4)). */
size_t nnz_gqa_scratch_bytes(nnz_gqa_dims dims);
int nnz_dispatch_gqa_attention(nnz_ctx *ctx, const void *q, int q_dtype, const void *k_cache,
                               const void *v_cache, int kv_dtype, int v_transposed,
                               void *output, int out_dtype, void *scratch, size_t scratch_bytes,
                               int32_t rope_position, float rope_theta, nnz_gqa_dims dims);
/* Allocation-free variant of nnz_dispatch_gqa_attention.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as nnz_dispatch_gqa_attention minus
 * the workspace: the split-sequence partials live in a fixed array of
 * NNZ_GQA_NOALLOC_MAX_BYTES compiled into the library, one per GPU, held until
 * the process ends.  Shapes needing more (nnz_gqa_scratch_bytes(dims) >
 * NNZ_GQA_NOALLOC_MAX_BYTES: 16 query heads x D 128 up to seq_len 64,448)
 * return NNZ_EUNSUPPORTED.  Calls no allocator.  Calls that overlap on one
 * GPU share the array and race: serialise them (one stream per GPU). */
#define NNZ_GQA_NOALLOC_MAX_BYTES ((size_t)8 << 20)
int nnz_dispatch_gqa_attention_noalloc(nnz_ctx *ctx, const void *q, int q_dtype,
                                       const void *k_cache, const void *v_cache, int kv_dtype,
                                       int v_transposed, void *output, int out_dtype,
                                       int32_t rope_position, float rope_theta,
                                       nnz_gqa_dims dims);
/* transformer.zig:962 dispatchGQAAttentionFusedTG: Q/K per-head RMSNorm +
 * RoPE, K/V append at `position`, attention over seq_len = position+1 tokens.
 * f16 q/k_raw/v_raw/output, f16 caches (V transposed), f32 norm scales.
 * No seq_len <= 1024 limit (the reference's fused kernel has one). */
int nnz_dispatch_gqa_attention_fused(nnz_ctx *ctx, const void *q, void *k_cache, void *v_cache,
                                     void *output, const void *k_raw, const void *v_raw,
                                     const float *q_norm_scale, const float *k_norm_scale,
                                     void *scratch, size_t scratch_bytes,
                                     nnz_gqa_fused_dims dims);

/* transformer.zig:962 dispatchGQAAttentionFusedTG again, for graph replay:
 * the same math as nnz_dispatch_gqa_attention_fused with the norm, RoPE,
 * cache append and attention in ONE kernel (plus a merge kernel when the
 * sequence spans several chunks).  Calls sharing one scratch must not
 * overlap.  If `d_seq_len` is non-NULL it points to a device uint32 holding
 * position + 1, read at run time (dims.seq_len is then the largest value it
 * may hold and sizes the launch); otherwise seq_len must be position + 1. */
int nnz_dispatch_gqa_attention_fused_1pass(nnz_ctx *ctx, const void *q, void *k_cache,
                                           void *v_cache, void *output, const void *k_raw,
                                           const void *v_raw, const float *q_norm_scale,
                                           const float *k_norm_scale, void *scratch,
                                           size_t scratch_bytes, const uint32_t *d_seq_len,
                                           nnz_gqa_fused_dims dims);

/* The two halves the decode step uses instead of the call above (no
 * reference counterpart; transformer.zig:3244-3370 encodeAttentionGather
 * followed by :1686 dispatchQMVf16io_resadd on the attention output):
 *   nnz_dispatch_gqa_attention_partials: the same norm/RoPE/append and
 *     attention, leaving per-chunk partials instead of the output --
 *     part_o f32 [nchunks][Hq*D] (unnormalised P.V; within a chunk, column
 *     k = head * D + d sits at ((k >> 2) & 7) * (Hq*D / 8) + (k >> 5) * 4 +
 *     (k & 3), the layout the merge reads with one 16-byte load per lane),
 *     part_ml f32 [nchunks][Hq][2] (max score, exp-sum), nchunks =
 *     nnz_gqa_partial_chunks(dims.seq_len) (64-token chunks);
 *     rope_inv_freq: f32 [D/2] frequencies theta^(-2p/D) or NULL (computed
 *     in the kernel);
 *   nnz_dispatch_qmv_merge_f16io_resadd: residual += W . merge(partials),
 *     the merge rounded to f16 as the attention output would be; W is the
 *     1-bit O projection [M x Hq*D]; at most 16 chunks.
 * d_seq_len as for nnz_dispatch_gqa_attention_fused_1pass. */
uint32_t nnz_gqa_partial_chunks(uint32_t seq_len);
int nnz_dispatch_gqa_attention_partials(nnz_ctx *ctx, const void *q, void *k_cache, void *v_cache,
                                        const void *k_raw, const void *v_raw,
                                        const float *q_norm_scale, const float *k_norm_scale,
                                        const float *rope_inv_freq, float *part_o, float *part_ml,
                                        const uint32_t *d_seq_len, nnz_gqa_fused_dims dims);
int nnz_dispatch_qmv_merge_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const float *part_o,
                                        const float *part_ml, const uint32_t *d_seq_len,
                                        uint32_t seq_len, uint32_t head_dim, float *residual,
                                        nnz_qmv_dims dims);

/* transformer.zig:1072 dispatchEmbeddingLookup (Q1 table, f32 out). */
int nnz_dispatch_embedding_lookup(nnz_ctx *ctx, const uint32_t *token_ids, const void *packed_bits,
                                  const void *scales, float *output, nnz_embed_dims dims);
/* transformer.zig:2625-2691 (Q4 branch): embedding_lookup_q4, BF16 scales. */
int nnz_dispatch_embedding_lookup_q4(nnz_ctx *ctx, const uint32_t *token_ids,
                                     const void *packed_nibs, const void *scales,
                                     const void *biases, float *output, nnz_embed_dims dims);
/* New: gather from a dense bf16 table [vocab x hidden] -> f32 (BASELINE
 * config 5 embeddings). */
int nnz_dispatch_embedding_lookup_bf16(nnz_ctx *ctx, const uint32_t *token_ids,
                                       const void *table, float *output, nnz_embed_dims dims);
/* transformer.zig:1097 dispatchResidualAdd (f32). */
int nnz_dispatch_residual_add(nnz_ctx *ctx, float *residual, const float *addition,
                              uint32_t count);
/* Greedy sampling on device: transformer.zig:3694 argmax (first maximum
 * wins).  out_index is a device uint32; out_value (optional) device f32. */
int nnz_dispatch_argmax(nnz_ctx *ctx, const float *logits, uint32_t count, uint32_t *out_index,
                        float *out_value);

/* ---- sampling (transformer.zig:3692-3908) --------------------------------
 * SamplingParams (transformer.zig:3652-3657): temperature 0 = greedy argmax;
 * top_k 0 = off; top_p >= 1 = off; seed of the random stream. */
typedef struct {
    float temperature;
    uint32_t top_k;
    float top_p;
    uint32_t reserved; /* 0 */
    uint64_t seed;
} nnz_sampling_params;

/* Workspace bytes nnz_dispatch_sample needs for `count` logits. */
size_t nnz_sample_workspace_bytes(uint32_t count);
/* std.Random.DefaultPrng.init(seed) (generate, transformer.zig:3969): write
 * the 4-word xoshiro256++ state expanded by SplitMix64 to device memory
 * d_state[4] (synchronous). */
int nnz_rng_seed(nnz_ctx *ctx, uint64_t seed, uint64_t *d_state);
/* sampleToken (transformer.zig:3860-3894) on device: temperature, top-k,
 * top-p, softmax, inverse-CDF draw with r = the next float of d_rng (the
 * state advances on device).  logits (device f32[count]) are not modified.
 * out_index: device uint32; out_prob (optional): device f32, the chosen
 * token's final probability.  temperature 0 is argmax (no rng, no
 * workspace needed).  count <= 4,194,304. */
int nnz_dispatch_sample(nnz_ctx *ctx, const float *logits, uint32_t count,
                        const nnz_sampling_params *params, uint64_t *d_rng, void *workspace,
                        size_t workspace_bytes, uint32_t *out_index, float *out_prob);

/* Tied bf16 LM head: the LM-head half of encodeFinalNormAndLMHead
 * (transformer.zig:2730-2785) when the head is the bf16 embedding table
 * (tie_word_embeddings, :297; BASELINE config 5 read literally):
 * logits[v] = sum_k table[v][k] * x[k]; table bf16 [vocab][hidden]
 * row-major, x f16 [hidden] (the final norm's output), logits f32 [vocab],
 * f32 accumulation.  table and x 16-byte aligned. */
int nnz_dispatch_lm_head_bf16(nnz_ctx *ctx, const void *table, const void *x, float *logits,
                              uint32_t vocab, uint32_t hidden);

/* ---- decoder model: forwardDecode / generate (transformer.zig:2389-4135) -- */

typedef struct {
    uint32_t vocab_size, hidden_size, intermediate_size, num_layers;
    uint32_t num_query_heads, num_kv_heads, head_dim, max_context_length;
    uint32_t max_prefill_length, group_size;
    float rope_theta, rms_eps;
    uint32_t embed_kind;   /* NNZ_EMBED_Q1, NNZ_EMBED_BF16 or NNZ_EMBED_Q4 */
    uint32_t lm_head_kind; /* NNZ_LMHEAD_Q1 (own 1-bit matrix), NNZ_LMHEAD_TIED_BF16 or NNZ_LMHEAD_Q4 */
    /* transformer.zig:35-55 QuantFormat: NNZ_QUANT_Q1 (q1_0: 1-bit, f16
     * scales) or NNZ_QUANT_Q4 (q4_mlx: 4-bit affine, raw bf16 scales and
     * biases; the reference's BF16-faithful rounding points, transformer.zig
     * :2646, :2743, :2977, :3100).  Q4 models take NNZ_EMBED_Q4 and
     * NNZ_LMHEAD_Q4 (a tied checkpoint uploads its embedding into the head). */
    uint32_t quant_format;
} nnz_model_config;
#define NNZ_EMBED_Q1 0
#define NNZ_EMBED_BF16 1
#define NNZ_EMBED_Q4 2
#define NNZ_LMHEAD_Q1 0
#define NNZ_LMHEAD_TIED_BF16 1
#define NNZ_LMHEAD_Q4 2
#define NNZ_QUANT_Q1 0
#define NNZ_QUANT_Q4 1

/* Tensor ids for nnz_model_tensor (per-layer ids take `layer`). */
#define NNZ_T_EMBED_CODES 0   /* Q1: uint32 codes; BF16: the bf16 table       */
#define NNZ_T_EMBED_SCALES 1  /* Q1 only: f16                                  */
#define NNZ_T_LM_CODES 2
#define NNZ_T_LM_SCALES 3
#define NNZ_T_FINAL_NORM 4    /* f32 [hidden]                                  */
#define NNZ_T_EMBED_BIASES 5  /* Q4 only: bf16 (scales likewise bf16 for Q4)   */
#define NNZ_T_LM_BIASES 6     /* Q4 only                                       */
#define NNZ_T_Q_CODES 10
#define NNZ_T_Q_SCALES 11
#define NNZ_T_K_CODES 12
#define NNZ_T_K_SCALES 13
#define NNZ_T_V_CODES 14
#define NNZ_T_V_SCALES 15
#define NNZ_T_O_CODES 16
#define NNZ_T_O_SCALES 17
#define NNZ_T_GATE_CODES 18
#define NNZ_T_GATE_SCALES 19
#define NNZ_T_UP_CODES 20
#define NNZ_T_UP_SCALES 21
#define NNZ_T_DOWN_CODES 22
#define NNZ_T_DOWN_SCALES 23
#define NNZ_T_ATTN_NORM 24    /* f32 [hidden]   */
#define NNZ_T_FFN_NORM 25     /* f32 [hidden]   */
#define NNZ_T_Q_NORM 26       /* f32 [head_dim] */
#define NNZ_T_K_NORM 27       /* f32 [head_dim] */
#define NNZ_T_K_CACHE 30      /* f16 [Hkv][max_ctx][D]  */
#define NNZ_T_V_CACHE 31      /* f16 [Hkv][D][max_ctx]  */
#define NNZ_T_Q_BIASES 50     /* Q4 only: bf16 biases of each projection      */
#define NNZ_T_K_BIASES 51
#define NNZ_T_V_BIASES 52
#define NNZ_T_O_BIASES 53
#define NNZ_T_GATE_BIASES 54
#define NNZ_T_UP_BIASES 55
#define NNZ_T_DOWN_BIASES 56
#define NNZ_T_LOGITS 40       /* f32 [vocab]            */
#define NNZ_T_RESIDUAL 41     /* f32 [hidden]           */

typedef struct nnz_model nnz_model;

/* Model(Config).init (model.zig:123-166): allocates every weight, KV cache
 * and activation buffer once, in device memory. */
int nnz_model_create(nnz_ctx *ctx, const nnz_model_config *cfg, nnz_model **out);
int nnz_model_destroy(nnz_model *m);
/* Device pointer and byte size of one tensor (upload weights through it). */
int nnz_model_tensor(nnz_model *m, int tensor_id, uint32_t layer, void **ptr, size_t *bytes);
/* forwardDecode (transformer.zig:2566): one token at `position`; logits in
 * NNZ_T_LOGITS.  Enqueued on the ctx stream. */
int nnz_model_forward_decode(nnz_model *m, uint32_t token_id, uint32_t position);
/* Batched prefill (new; the reference prefills token by token through
 * forwardDecode, transformer.zig:4032-4068): tokens[0..n) at positions
 * start..start+n-1 via the dequant-GEMM; leaves the last token's logits in
 * NNZ_T_LOGITS.  `tokens_host` is a host array.  Q4 models use the 4-bit
 * GEMM with the Q4 rounding points. */
int nnz_model_prefill(nnz_model *m, const uint32_t *tokens_host, uint32_t n, uint32_t start);
/* generate (transformer.zig:3942): prefill the prompt, then up to `n_new`
 * decode steps; each step is one replay of a captured hipGraph that picks
 * the next token on the device (argmax, or the sampler set by
 * nnz_model_set_sampling).  Stops early at a stop token (nnz_model_set_eos).
 * Writes the emitted token ids (host), their number to *out_count (optional)
 * and, if non-NULL, per token the top-2 logit margin (greedy) or the
 * sampled token's probability (sampling), and per-step wall ms. */
int nnz_model_generate(nnz_model *m, const uint32_t *prompt_host, uint32_t n_prompt,
                       uint32_t n_new, uint32_t *out_tokens, float *out_margins,
                       float *out_step_ms, int use_graph, uint32_t *out_count);
/* The same loop split for streaming callers and benchmarks (decodeOneToken,
 * transformer.zig:4072, without the per-token host sync):
 *   nnz_model_decode_begin: prefill the prompt, take the greedy first token,
 *     capture the decode-step graphs for up to `max_new` steps (at most 8,
 *     each sized for the sequence lengths of the steps it serves);
 *   nnz_model_decode_steps: enqueue `n` graph replays (asynchronous);
 *   nnz_model_decode_read: copy the first `n` emitted tokens (and margins)
 *     to the host after a bounded sync;
 *   nnz_model_decode_end: release the graphs. */
int nnz_model_decode_begin(nnz_model *m, const uint32_t *prompt_host, uint32_t n_prompt,
                           uint32_t max_new);
int nnz_model_decode_steps(nnz_model *m, uint32_t n);
int nnz_model_decode_read(nnz_model *m, uint32_t n, uint32_t *out_tokens, float *out_margins);
int nnz_model_decode_end(nnz_model *m);
/* Sampling of the decode loop (GenerateOpts.params, transformer.zig:3930):
 * applies from the next generate / decode_begin, which re-seeds the random
 * stream with params->seed.  Default: greedy. */
int nnz_model_set_sampling(nnz_model *m, const nnz_sampling_params *params);
/* Stop tokens (GenerateOpts.eos_ids; isEosToken, transformer.zig:4126): a
 * sampled stop token ends the stream and is not emitted.  n <= 8; n = 0
 * clears them. */
int nnz_model_set_eos(nnz_model *m, const uint32_t *ids, uint32_t n);
/* Tokens emitted so far by the current / last decode stream
 * (GenerateResult.tokens_generated) and whether a stop token ended it;
 * synchronises the stream. */
int nnz_model_decode_status(nnz_model *m, uint32_t *emitted, int *stopped);

/* ---- synthetic data (no reference counterpart) ---------------------------
 * Fill out[0..n) with bf16(scale * N(0,1)) from the counter-based
 * splitmix64 + Box-Muller stream `seed` (bit-identical to the host generator
 * nnzap_amd/synth.py up to last-ulp differences of double log1p/cos, which a
 * bf16 rounding hides).  Used for the benchmark model's embedding table. */
int nnz_synth_normal_bf16(nnz_ctx *ctx, void *out, uint64_t n, uint64_t seed, double scale);

#ifdef __cplusplus
}
#endif
#endif /* NNZ_H */

/*
 * C translation unit over include/nnz.h, linked against libnnzap_amd.so:
 * what a C or Zig caller of the drop-in boundary compiles against.
 *
 *  - compile time: every dims struct has the size and field offsets of the
 *    reference's extern structs (nnmetal/src/transformer.zig:389-479: u32/f32
 *    fields in declaration order, no padding), and nnz_qweight /
 *    nnz_sampling_params / nnz_model_config keep the layout the ctypes table
 *    and include/nnz.zig assume;
 *  - nnz_abi_check_host(): the error paths that need no GPU (null context,
 *    null outputs, host-side size helpers), 0 if all hold, else the number of
 *    the first failed check;
 *  - nnz_abi_qmv_config(): BASELINE config 2 through the C ABI from C --
 *    context, device allocation, upload, nnz_dispatch_qmv, bounded sync,
 *    download, free (needs a GPU; called by a GPU test).
 */
#include <assert.h>
#include <stddef.h>
#include <string.h>

#include "nnz.h"

#define SIZE(T, n) static_assert(sizeof(T) == (n), #T " size")
#define OFF(T, f, n) static_assert(offsetof(T, f) == (n), #T "." #f " offset")

/* transformer.zig:389-393 RMSNormDims */
SIZE(nnz_rmsnorm_dims, 12);
OFF(nnz_rmsnorm_dims, hidden_size, 0); OFF(nnz_rmsnorm_dims, num_tokens, 4);
OFF(nnz_rmsnorm_dims, eps, 8);
/* :396-401 RoPEDims */
SIZE(nnz_rope_dims, 16);
OFF(nnz_rope_dims, num_heads, 0); OFF(nnz_rope_dims, head_dim, 4);
OFF(nnz_rope_dims, position, 8); OFF(nnz_rope_dims, rope_theta, 12);
/* :404-409 KVUpdateDims */
SIZE(nnz_kv_update_dims, 16);
OFF(nnz_kv_update_dims, num_kv_heads, 0); OFF(nnz_kv_update_dims, head_dim, 4);
OFF(nnz_kv_update_dims, position, 8); OFF(nnz_kv_update_dims, max_context_length, 12);
/* :412-418 FusedRoPEKVDims */
SIZE(nnz_fused_rope_kv_dims, 20);
OFF(nnz_fused_rope_kv_dims, num_kv_heads, 0); OFF(nnz_fused_rope_kv_dims, head_dim, 4);
OFF(nnz_fused_rope_kv_dims, position, 8); OFF(nnz_fused_rope_kv_dims, max_context_length, 12);
OFF(nnz_fused_rope_kv_dims, rope_theta, 16);
/* :421-427 FusedNormRoPEDims */
SIZE(nnz_fused_norm_rope_dims, 20);
OFF(nnz_fused_norm_rope_dims, num_heads, 0); OFF(nnz_fused_norm_rope_dims, head_dim, 4);
OFF(nnz_fused_norm_rope_dims, position, 8); OFF(nnz_fused_norm_rope_dims, eps, 12);
OFF(nnz_fused_norm_rope_dims, rope_theta, 16);
/* :430-437 FusedKNormRoPEKVDims */
SIZE(nnz_fused_k_norm_rope_kv_dims, 24);
OFF(nnz_fused_k_norm_rope_kv_dims, num_kv_heads, 0);
OFF(nnz_fused_k_norm_rope_kv_dims, head_dim, 4);
OFF(nnz_fused_k_norm_rope_kv_dims, position, 8);
OFF(nnz_fused_k_norm_rope_kv_dims, max_context_length, 12);
OFF(nnz_fused_k_norm_rope_kv_dims, eps, 16);
OFF(nnz_fused_k_norm_rope_kv_dims, rope_theta, 20);
/* :440-447 GQADims */
SIZE(nnz_gqa_dims, 24);
OFF(nnz_gqa_dims, num_query_heads, 0); OFF(nnz_gqa_dims, num_kv_heads, 4);
OFF(nnz_gqa_dims, head_dim, 8); OFF(nnz_gqa_dims, seq_len, 12);
OFF(nnz_gqa_dims, max_context_length, 16); OFF(nnz_gqa_dims, heads_per_kv_group, 20);
/* :451-461 GQAFusedDims */
SIZE(nnz_gqa_fused_dims, 36);
OFF(nnz_gqa_fused_dims, num_query_heads, 0); OFF(nnz_gqa_fused_dims, num_kv_heads, 4);
OFF(nnz_gqa_fused_dims, head_dim, 8); OFF(nnz_gqa_fused_dims, seq_len, 12);
OFF(nnz_gqa_fused_dims, max_context_length, 16);
OFF(nnz_gqa_fused_dims, heads_per_kv_group, 20); OFF(nnz_gqa_fused_dims, position, 24);
OFF(nnz_gqa_fused_dims, eps, 28); OFF(nnz_gqa_fused_dims, rope_theta, 32);
/* :464-469 EmbedDims */
SIZE(nnz_embed_dims, 16);
OFF(nnz_embed_dims, vocab_size, 0); OFF(nnz_embed_dims, hidden_size, 4);
OFF(nnz_embed_dims, num_tokens, 8); OFF(nnz_embed_dims, group_size, 12);
/* :475-479 QMVDims */
SIZE(nnz_qmv_dims, 12);
OFF(nnz_qmv_dims, M, 0); OFF(nnz_qmv_dims, K, 4); OFF(nnz_qmv_dims, group_size, 8);
/* the stacked-launch descriptor (no reference counterpart): two u32 then four u64 strides */
SIZE(nnz_qmv_stack, 40);
OFF(nnz_qmv_stack, count, 0); OFF(nnz_qmv_stack, blocks_per_matrix, 4);
OFF(nnz_qmv_stack, codes_stride, 8); OFF(nnz_qmv_stack, scales_stride, 16);
OFF(nnz_qmv_stack, input_stride, 24); OFF(nnz_qmv_stack, output_stride, 32);

/* The build's own structs, as the ctypes table and nnz.zig lay them out. */
SIZE(nnz_qweight, 40);
OFF(nnz_qweight, codes, 0); OFF(nnz_qweight, scales, 8); OFF(nnz_qweight, biases, 16);
OFF(nnz_qweight, packed_count, 24); OFF(nnz_qweight, group_size, 28);
OFF(nnz_qweight, bits, 32); OFF(nnz_qweight, scale_dtype, 36);
SIZE(nnz_sampling_params, 24);
OFF(nnz_sampling_params, temperature, 0); OFF(nnz_sampling_params, top_k, 4);
OFF(nnz_sampling_params, top_p, 8); OFF(nnz_sampling_params, seed, 16);
SIZE(nnz_model_config, 60);
OFF(nnz_model_config, rope_theta, 40); OFF(nnz_model_config, rms_eps, 44);
OFF(nnz_model_config, embed_kind, 48); OFF(nnz_model_config, quant_format, 56);

int nnz_abi_check_host(void) {
    int n = 0;
#define CHECK(cond) do { ++n; if (!(cond)) return n; } while (0)
    const nnz_qmv_dims d = {2048, 6144, 128};
    nnz_qweight w;
    memset(&w, 0, sizeof(w));
    float x[1], y[1];
    CHECK(strncmp(nnz_version(), "nnzap_amd", 9) == 0);
    CHECK(strcmp(nnz_last_error(NULL), "null context") == 0);
    /* a null context is refused before anything touches a device */
    CHECK(nnz_dispatch_qmv(NULL, &w, x, y, d) == NNZ_EINVAL);
    CHECK(nnz_dispatch_q4mv(NULL, &w, x, y, d) == NNZ_EINVAL);
    CHECK(nnz_stream_sync(NULL, 10) == NNZ_EINVAL);
    CHECK(nnz_graph_begin(NULL) == NNZ_EINVAL);
    CHECK(nnz_graph_destroy(NULL) == NNZ_EINVAL);
    CHECK(nnz_ctx_destroy(NULL) == NNZ_EINVAL);
    CHECK(nnz_ctx_create(0, NULL, NULL) == NNZ_EINVAL);      /* null out pointer */
    CHECK(nnz_model_forward_decode(NULL, 0, 0) == NNZ_EINVAL);
    CHECK(nnz_model_destroy(NULL) == NNZ_EINVAL);
    const nnz_gqa_dims g = {16, 8, 128, 32768, 32768, 2};
    const nnz_rmsnorm_dims rd = {2048, 1, 1e-6f};
    CHECK(nnz_dispatch_rms_norm(NULL, x, x, y, NNZ_F16, 0, rd) == NNZ_EINVAL);
    CHECK(nnz_dispatch_gqa_attention_noalloc(NULL, x, NNZ_F32, x, x, NNZ_BF16, 0, y, NNZ_F32, -1,
                                             0.f, g) == NNZ_EINVAL);
    /* host-side size helpers */
    const size_t s = nnz_gqa_scratch_bytes(g);
    CHECK(s > (size_t)16 * 512 * 128 * 4 && s <= NNZ_GQA_NOALLOC_MAX_BYTES);
    CHECK(nnz_sample_workspace_bytes(151936) > 151936 * 4);
    CHECK(nnz_gqa_partial_chunks(640) == 10);
#undef CHECK
    return 0;
}

/* y = W x for one 1-bit matrix given as host arrays (codes: M*K/32 words,
 * scales: M*K/gs f16 bit patterns), entirely through the C ABI.  Returns an
 * nnz status; on failure `err` (>= 256 bytes) holds nnz_last_error. */
int nnz_abi_qmv_config(const uint32_t *codes, const uint16_t *scales, const float *x, float *y,
                       uint32_t M, uint32_t K, uint32_t gs, char *err) {
    nnz_ctx *ctx = NULL;
    void *dc = NULL, *ds = NULL, *dx = NULL, *dy = NULL;
    int rc = nnz_ctx_create(0, NULL, &ctx);
    if (rc) return rc;
    const size_t nc = (size_t)M * K / 8, ns = (size_t)M * K / gs * 2;
    if (!rc) rc = nnz_alloc(ctx, nc, &dc);
    if (!rc) rc = nnz_alloc(ctx, ns, &ds);
    if (!rc) rc = nnz_alloc(ctx, (size_t)K * 4, &dx);
    if (!rc) rc = nnz_alloc(ctx, (size_t)M * 4, &dy);
    if (!rc) rc = nnz_upload(ctx, dc, codes, nc);
    if (!rc) rc = nnz_upload(ctx, ds, scales, ns);
    if (!rc) rc = nnz_upload(ctx, dx, x, (size_t)K * 4);
    if (!rc) {
        nnz_qweight w;
        w.codes = dc;
        w.scales = ds;
        w.biases = NULL;
        w.packed_count = M * K;
        w.group_size = gs;
        w.bits = 1;
        w.scale_dtype = NNZ_F16;
        const nnz_qmv_dims d = {M, K, gs};
        rc = nnz_dispatch_qmv(ctx, &w, (const float *)dx, (float *)dy, d);
    }
    if (!rc) rc = nnz_stream_sync(ctx, 10000);
    if (!rc) rc = nnz_download(ctx, y, dy, (size_t)M * 4);
    if (rc && err) {
        strncpy(err, nnz_last_error(ctx), 255);
        err[255] = 0;
    }
    nnz_free(ctx, dc);
    nnz_free(ctx, ds);
    nnz_free(ctx, dx);
    nnz_free(ctx, dy);
    nnz_ctx_destroy(ctx);
    return rc;
}

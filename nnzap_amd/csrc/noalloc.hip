// Allocation-free single-query GQA decode attention.
//
// nnz_dispatch_gqa_attention takes a caller workspace for its split-sequence
// partials.  Callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc) use
// nnz_dispatch_gqa_attention_noalloc instead: the partials live in a
// fixed-size array compiled into the library, one copy per GPU, held until
// the process ends.  The kernels are the same; only the partials' address
// differs.
//
// The array's name is a host-side stand-in in host code.  Its device
// address is looked up once per device with hipGetSymbolAddress when a
// context is created on that device (nnz_ctx_create) and kept per device;
// every host use of the array goes through that address.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one
// GPU (two streams, two threads) race on it.  Nothing in it needs to start
// at zero: each call writes every partial it reads.
#include "internal.h"

#include <mutex>

// 8 MiB: Hq * ceil(seq/64) * (D + 2) * 4 bytes of partials plus Hq * D * 4
// bytes of q must fit (16 query heads x D 128: seq_len <= 64,448).
static __device__ __align__(256) unsigned char scratch[NNZ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES] = {};
}  // namespace

// Called by nnz_ctx_create with `ctx->device` current.
int nnz_noalloc_init(nnz_ctx *ctx) {
    NNZ_REQUIRE(ctx, ctx->device >= 0 && ctx->device < MAX_DEVICES, NNZ_EUNSUPPORTED,
                "noalloc: device index %d >= %d", ctx->device, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[ctx->device]) return NNZ_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return nnz_fail(ctx, NNZ_EHIP, "noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    g_ptr[ctx->device] = p;
    return NNZ_OK;
}

extern "C" int nnz_dispatch_gqa_attention_noalloc(nnz_ctx *ctx, const void *q, int q_dtype,
                                                  const void *k_cache, const void *v_cache,
                                                  int kv_dtype, int v_transposed, void *output,
                                                  int out_dtype, int32_t rope_position,
                                                  float rope_theta, nnz_gqa_dims dims) {
    NNZ_CHECK_CTX(ctx);
    void *ptr = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (ctx->device >= 0 && ctx->device < MAX_DEVICES) ptr = g_ptr[ctx->device];
    }
    NNZ_REQUIRE(ctx, ptr != nullptr, NNZ_ESTATE, "gqa_noalloc: scratch address not set up");
    NNZ_REQUIRE(ctx, dims.num_kv_heads > 0 && dims.seq_len > 0 &&
                         dims.seq_len <= dims.max_context_length,
                NNZ_EINVAL, "gqa_noalloc: bad seq_len/num_kv_heads");
    const size_t need = nnz_gqa_scratch_bytes(dims);
    NNZ_REQUIRE(ctx, need <= NNZ_NOALLOC_SCRATCH_BYTES, NNZ_EUNSUPPORTED,
                "gqa_noalloc: %zu bytes of partials needed, the fixed buffer holds %zu "
                "(use nnz_dispatch_gqa_attention with a workspace)",
                need, (size_t)NNZ_NOALLOC_SCRATCH_BYTES);
    return nnz_attn_launch(ctx, q, q_dtype, k_cache, v_cache, kv_dtype, v_transposed != 0, output,
                           out_dtype, ptr, NNZ_NOALLOC_SCRATCH_BYTES, rope_position, rope_theta,
                           dims);
}

// Context, device memory, bounded synchronisation, graphs and timers.
//
// Replaces the Metal platform layer of nnmetal (nnmetal/src/metal.zig):
// Device.init (:959-1020) -> nnz_ctx_create, shared MTLBuffers (:80-469) ->
// explicit hipMalloc'd buffers uploaded once, commitAndWait / the unbounded
// commitAndSpinOnFlag (:1293-1352) -> nnz_stream_sync with a timeout.
#include "internal.h"

#include <chrono>
#include <thread>

int nnz_fail(nnz_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return code;
}

extern "C" {

const char *nnz_version(void) { return "nnzap_amd 0.1 (gfx950)"; }

int nnz_ctx_create(int device, void *hip_stream, nnz_ctx **out) {
    if (!out) return NNZ_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return NNZ_EHIP;
    if (device < 0 || device >= n) return NNZ_EINVAL;
    if (hipSetDevice(device) != hipSuccess) return NNZ_EHIP;
    nnz_ctx *c = new nnz_ctx();
    c->device = device;
    if (hip_stream) {
        c->stream = (hipStream_t)hip_stream;
    } else {
        if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
            delete c;
            return NNZ_EHIP;
        }
        c->own_stream = true;
    }
    if (int rc = nnz_noalloc_init(c)) {
        if (c->own_stream) hipStreamDestroy(c->stream);
        delete c;
        return rc;
    }
    *out = c;
    return NNZ_OK;
}

int nnz_ctx_destroy(nnz_ctx *ctx) {
    if (!ctx) return NNZ_EINVAL;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (int i = 0; i < 64; ++i)
        if (ctx->ev_ok[i]) hipEventDestroy(ctx->ev[i]);
    if (ctx->own_stream) hipStreamDestroy(ctx->stream);
    delete ctx;
    return NNZ_OK;
}

void *nnz_ctx_stream(nnz_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int nnz_ctx_set_option(nnz_ctx *ctx, int option, int value) {
    NNZ_CHECK_CTX(ctx);
    if (option == NNZ_OPT_Q1_MATRIX_CORES) {
        NNZ_REQUIRE(ctx, value >= 0 && value <= 2, NNZ_EINVAL, "q1 matrix cores: %d (0, 1 or 2)", value);
        ctx->q1_matrix_cores = value;
        return NNZ_OK;
    }
    return nnz_fail(ctx, NNZ_EINVAL, "unknown option %d", option);
}

const char *nnz_last_error(nnz_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int nnz_alloc(nnz_ctx *ctx, size_t bytes, void **out) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, out && bytes > 0, NNZ_EINVAL, "nnz_alloc: bad arguments");
    NNZ_REQUIRE(ctx, !ctx->capturing, NNZ_ESTATE, "nnz_alloc: not allowed during capture");
    *out = nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess)
        return nnz_fail(ctx, NNZ_ENOMEM, "hipMalloc(%zu) failed", bytes);
    hipError_t e = hipMemsetAsync(p, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(p);
        return nnz_fail(ctx, NNZ_EHIP, "zero-fill failed: %s", hipGetErrorString(e));
    }
    *out = p;
    return NNZ_OK;
}

int nnz_free(nnz_ctx *ctx, void *ptr) {
    NNZ_CHECK_CTX(ctx);
    if (!ptr) return NNZ_OK;
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    NNZ_HIP(ctx, hipFree(ptr));
    return NNZ_OK;
}

int nnz_upload(nnz_ctx *ctx, void *dst, const void *src, size_t bytes) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, dst && src, NNZ_EINVAL, "nnz_upload: null pointer");
    if (!bytes) return NNZ_OK;
    NNZ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NNZ_OK;
}

int nnz_download(nnz_ctx *ctx, void *dst, const void *src, size_t bytes) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, dst && src, NNZ_EINVAL, "nnz_download: null pointer");
    if (!bytes) return NNZ_OK;
    NNZ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NNZ_OK;
}

int nnz_stream_sync(nnz_ctx *ctx, uint32_t timeout_ms) {
    NNZ_CHECK_CTX(ctx);
    auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        hipError_t e = hipStreamQuery(ctx->stream);
        if (e == hipSuccess) return NNZ_OK;
        if (e != hipErrorNotReady)
            return nnz_fail(ctx, NNZ_EHIP, "stream error: %s", hipGetErrorString(e));
        auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(
                      std::chrono::steady_clock::now() - t0).count();
        if (ms >= (long long)timeout_ms)
            return nnz_fail(ctx, NNZ_ETIMEOUT, "stream did not drain within %u ms", timeout_ms);
        std::this_thread::sleep_for(std::chrono::microseconds(ms < 2 ? 5 : 200));
    }
}

int nnz_graph_begin(nnz_ctx *ctx) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, !ctx->capturing, NNZ_ESTATE, "capture already active");
    NNZ_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return NNZ_OK;
}

int nnz_graph_end(nnz_ctx *ctx, nnz_graph **out) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, ctx->capturing && out, NNZ_ESTATE, "no capture active");
    ctx->capturing = false;
    nnz_graph *g = new nnz_graph();
    hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g->graph) hipGraphDestroy(g->graph);
        delete g;
        return nnz_fail(ctx, NNZ_EHIP, "graph capture failed: %s", hipGetErrorString(e));
    }
    *out = g;
    return NNZ_OK;
}

int nnz_graph_replay(nnz_ctx *ctx, nnz_graph *g) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, g && g->exec, NNZ_EINVAL, "null graph");
    NNZ_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    return NNZ_OK;
}

int nnz_graph_destroy(nnz_graph *g) {
    if (!g) return NNZ_EINVAL;
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return NNZ_OK;
}

int nnz_timer_mark(nnz_ctx *ctx, int slot) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, slot >= 0 && slot < 64, NNZ_EINVAL, "timer slot out of range");
    if (!ctx->ev_ok[slot]) {
        NNZ_HIP(ctx, hipEventCreate(&ctx->ev[slot]));
        ctx->ev_ok[slot] = true;
    }
    NNZ_HIP(ctx, hipEventRecord(ctx->ev[slot], ctx->stream));
    return NNZ_OK;
}

int nnz_timer_elapsed_ms(nnz_ctx *ctx, int a, int b, float *ms) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, a >= 0 && a < 64 && b >= 0 && b < 64 && ms, NNZ_EINVAL, "bad timer slots");
    NNZ_REQUIRE(ctx, ctx->ev_ok[a] && ctx->ev_ok[b], NNZ_ESTATE, "timer slot never marked");
    NNZ_HIP(ctx, hipEventSynchronize(ctx->ev[b]));
    NNZ_HIP(ctx, hipEventElapsedTime(ms, ctx->ev[a], ctx->ev[b]));
    return NNZ_OK;
}

}  // extern "C"

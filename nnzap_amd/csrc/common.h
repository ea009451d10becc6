// Shared definitions for the gfx950 decode-path library (libnnzap_amd.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string>

#include "../../include/nnz.h"

struct nnz_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    bool capturing = false;
    std::string err;
    hipEvent_t ev[64] = {};
    bool ev_ok[64] = {};
};

struct nnz_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

// Records a formatted error on the context (if any) and returns `code`.
int nnz_fail(nnz_ctx *ctx, int code, const char *fmt, ...);

#define NNZ_CHECK_CTX(ctx) \
    do { if (!(ctx)) return NNZ_EINVAL; } while (0)

#define NNZ_HIP(ctx, call)                                                          \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess)                                                       \
            return nnz_fail((ctx), NNZ_EHIP, "%s failed: %s", #call,                \
                            hipGetErrorString(e_));                                 \
    } while (0)

#define NNZ_LAUNCHED(ctx)                                                           \
    do {                                                                            \
        hipError_t e_ = hipGetLastError();                                          \
        if (e_ != hipSuccess)                                                       \
            return nnz_fail((ctx), NNZ_EHIP, "kernel launch failed: %s (%s:%d)",    \
                            hipGetErrorString(e_), __FILE__, __LINE__);             \
    } while (0)

#define NNZ_REQUIRE(ctx, cond, code, ...)                                           \
    do { if (!(cond)) return nnz_fail((ctx), (code), __VA_ARGS__); } while (0)

// ---------------------------------------------------------------------------
// Element-type helpers (device).  bf16 is carried as raw uint16_t.
// ---------------------------------------------------------------------------

typedef _Float16 f16_t;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

// Round-to-nearest-even float32 -> bfloat16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// The reference's `bf16_round` (q4mv_bf16_specialized.metal:52-57): keep the
// high 16 bits of the float32 (truncation toward zero).
__device__ __forceinline__ float bf16_trunc(float f) {
    return __uint_as_float(__float_as_uint(f) & 0xffff0000u);
}

__device__ __forceinline__ float f16_round(float f) {
    return (float)(f16_t)f;
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void *p, size_t i) {
    if constexpr (DT == NNZ_F32) return ((const float *)p)[i];
    else if constexpr (DT == NNZ_F16) return (float)((const f16_t *)p)[i];
    else return bf16_to_f32(((const uint16_t *)p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void *p, size_t i, float v) {
    if constexpr (DT == NNZ_F32) ((float *)p)[i] = v;
    else if constexpr (DT == NNZ_F16) ((f16_t *)p)[i] = (f16_t)v;
    else ((uint16_t *)p)[i] = f32_to_bf16_rne(v);
}

__device__ __forceinline__ float scale_to_f32(uint16_t raw, int sdt) {
    return sdt == NNZ_BF16 ? bf16_to_f32(raw) : (float)__builtin_bit_cast(f16_t, raw);
}

__host__ __device__ constexpr inline uint32_t ceil_div(uint32_t a, uint32_t b) {
    return (a + b - 1) / b;
}

// Sum across the `width` lanes of an aligned lane group (width a power of 2,
// <= 64).  All lanes of the group receive the result.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Dtype size in bytes for the public element types.
static inline size_t nnz_dtype_size(int dt) {
    return dt == NNZ_F32 ? 4 : 2;
}
static inline bool nnz_dtype_ok(int dt) {
    return dt == NNZ_F32 || dt == NNZ_F16 || dt == NNZ_BF16;
}

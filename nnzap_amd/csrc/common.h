// Shared definitions for the gfx950 decode-path library (libnnzap_amd.so).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
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
    int q1_matrix_cores = 0;   // NNZ_OPT_Q1_MATRIX_CORES
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

// Whole-wave reductions with DPP lane moves (VALU instructions, no LDS
// round trip per step): swap lanes within quads (xor 1, xor 2), mirror
// within 8 and 16 lanes, then broadcast lane 15 of each 16-lane row into
// rows 1 and 3 and lane 31 into rows 2 and 3.  Lanes 48..63 end with the
// total; rows a step leaves unwritten read `neutral`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_move(float v, float neutral) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(neutral), __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xF, false));
}

enum : int {
    DPP_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
    DPP_ROW_MIRROR = 0x140,
    DPP_ROW_HALF_MIRROR = 0x141,
    DPP_ROW_BCAST15 = 0x142,
    DPP_ROW_BCAST31 = 0x143,
};

// Sum over the wave; the total is valid in lane 63.
__device__ __forceinline__ float wave_sum_to_last(float v) {
    v += dpp_move<DPP_XOR1>(v, 0.f);
    v += dpp_move<DPP_XOR2>(v, 0.f);
    v += dpp_move<DPP_ROW_HALF_MIRROR>(v, 0.f);
    v += dpp_move<DPP_ROW_MIRROR>(v, 0.f);
    v += dpp_move<DPP_ROW_BCAST15, 0xA>(v, 0.f);
    v += dpp_move<DPP_ROW_BCAST31, 0xC>(v, 0.f);
    return v;
}

// Totals of V = 1, 2, 4 or 8 per-lane partial sums, each summed over the
// whole wave, by exchange-halving: v_permlane32_swap pairs the values two
// at a time across the wave halves, v_permlane16_swap across 16-lane rows,
// a row mirror across 8-lane halves, then DPP within 8 lanes -- log2(V)
// swaps+adds per level instead of a full 64-lane reduction per value.
// Returns, in every lane, the total of value slot(lane) =
// bit-reverse (log2 V bits) of lane >> (6 - log2 V); lanes 0, 64/V, 2*64/V...
// each hold a different slot.
__device__ __forceinline__ float2 swap32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(a), __float_as_int(b), false, false);
    return make_float2(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float2 swap16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(a), __float_as_int(b), false, false);
    return make_float2(__int_as_float(r[0]), __int_as_float(r[1]));
}

template <int V>
__device__ __forceinline__ float multi_row_sum(const float (&v)[V]) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "1, 2, 4 or 8 values");
    const int lane = threadIdx.x & 63;
    float c[V > 1 ? V / 2 : 1];
    if constexpr (V == 1) {
        const float2 p = swap32(v[0], v[0]);
        c[0] = p.x + p.y;
    } else {
#pragma unroll
        for (int k = 0; k < V / 2; ++k) {      // [slot 2k | slot 2k+1] by wave half
            const float2 p = swap32(v[2 * k], v[2 * k + 1]);
            c[k] = p.x + p.y;
        }
    }
    constexpr int C = V > 1 ? V / 2 : 1;
    float d[C > 1 ? C / 2 : 1];
    if constexpr (C == 1) {
        const float2 p = swap16(c[0], c[0]);
        d[0] = p.x + p.y;
    } else {
#pragma unroll
        for (int k = 0; k < C / 2; ++k) {      // 16-lane rows: slots 4k, 4k+2, 4k+1, 4k+3
            const float2 p = swap16(c[2 * k], c[2 * k + 1]);
            d[k] = p.x + p.y;
        }
    }
    float e;
    if constexpr (V == 8) {                    // 8-lane halves: d[0] low, d[1] high
        const bool hi = lane & 8;
        const float mine = hi ? d[1] : d[0], other = hi ? d[0] : d[1];
        e = mine + dpp_move<DPP_ROW_MIRROR>(other, 0.f);
    } else {
        e = d[0] + dpp_move<DPP_ROW_MIRROR>(d[0], 0.f);
    }
    e += dpp_move<DPP_ROW_HALF_MIRROR>(e, 0.f);
    e += dpp_move<DPP_XOR2>(e, 0.f);
    e += dpp_move<DPP_XOR1>(e, 0.f);
    return e;
}

// Totals over each aligned group of L = 8 or 16 lanes (half or whole DPP
// row) of V per-lane values, by exchange-halving inside the group: at each
// level a lane keeps one half of its values and adds its partner's copy of
// that half (the row mirror pairs the 8-lane halves for L = 16, then the
// half-row mirror, xor 2, xor 1; once one value is left the levels are
// plain pairwise sums).  Afterwards lane l (its index within the group)
// holds in a[0..N) the totals of values prefix * N + j, N = max(V / L, 1),
// prefix = the top log2(V / N) bits of l; with V < L the lanes sharing a
// prefix hold the same totals.
template <int CTRL, int N>
__device__ __forceinline__ void halving_level(float *a, bool upper) {
    if constexpr (N >= 2) {
#pragma unroll
        for (int k = 0; k < N / 2; ++k) {
            const float keep = upper ? a[k + N / 2] : a[k];
            const float send = upper ? a[k] : a[k + N / 2];
            a[k] = keep + dpp_move<CTRL>(send, 0.f);
        }
    } else {
        a[0] += dpp_move<CTRL>(a[0], 0.f);
    }
}

template <int V, int L>
__device__ __forceinline__ void group_multi_sum(float (&a)[V]) {
    static_assert(L == 8 || L == 16, "8 or 16 lanes");
    static_assert(V >= 1 && (V & (V - 1)) == 0, "a power of two of values");
    constexpr int N0 = V, N1 = N0 > 1 ? N0 / 2 : 1, N2 = N1 > 1 ? N1 / 2 : 1, N3 = N2 > 1 ? N2 / 2 : 1;
    const int l = threadIdx.x & (L - 1);
    if constexpr (L == 16) {
        halving_level<DPP_ROW_MIRROR, N0>(a, l & 8);
        halving_level<DPP_ROW_HALF_MIRROR, N1>(a, l & 4);
        halving_level<DPP_XOR2, N2>(a, l & 2);
        halving_level<DPP_XOR1, N3>(a, l & 1);
    } else {
        halving_level<DPP_ROW_HALF_MIRROR, N0>(a, l & 4);
        halving_level<DPP_XOR2, N1>(a, l & 2);
        halving_level<DPP_XOR1, N2>(a, l & 1);
    }
}

// The slot multi_row_sum<V> leaves in this lane.
template <int V>
__device__ __forceinline__ int multi_row_slot() {
    const int lane = threadIdx.x & 63;
    if constexpr (V == 1) return 0;
    else if constexpr (V == 2) return lane >> 5;
    else if constexpr (V == 4) return ((lane >> 4) & 1) * 2 + (lane >> 5);
    else return ((lane >> 3) & 1) * 4 + ((lane >> 4) & 1) * 2 + (lane >> 5);
}

__device__ __forceinline__ float lane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum / max over the wave, returned in every lane.
__device__ __forceinline__ float wave_sum(float v) { return lane63(wave_sum_to_last(v)); }

__device__ __forceinline__ float wave_max(float v) {
    const float n = -INFINITY;
    v = fmaxf(v, dpp_move<DPP_XOR1>(v, n));
    v = fmaxf(v, dpp_move<DPP_XOR2>(v, n));
    v = fmaxf(v, dpp_move<DPP_ROW_HALF_MIRROR>(v, n));
    v = fmaxf(v, dpp_move<DPP_ROW_MIRROR>(v, n));
    v = fmaxf(v, dpp_move<DPP_ROW_BCAST15, 0xA>(v, n));
    v = fmaxf(v, dpp_move<DPP_ROW_BCAST31, 0xC>(v, n));
    return lane63(v);
}

// Dtype size in bytes for the public element types.
static inline size_t nnz_dtype_size(int dt) {
    return dt == NNZ_F32 ? 4 : 2;
}
static inline bool nnz_dtype_ok(int dt) {
    return dt == NNZ_F32 || dt == NNZ_F16 || dt == NNZ_BF16;
}

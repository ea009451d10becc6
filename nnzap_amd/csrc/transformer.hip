// Transformer kernels for the decode path on gfx950: RMSNorm, SiLU, RoPE,
// KV-cache append, GQA decode attention, embedding gathers, residual add,
// on-device argmax and the dequantisation artefact.
//
// Semantics follow nnmetal/src/shaders/transformer.metal; the decomposition
// does not.  In particular decode attention splits the sequence across
// workgroups (flash-decoding partials + a combine kernel) instead of the
// reference's one-threadgroup-per-query-head kernels, so a 32k context keeps
// every CU busy.
#include "internal.h"

#include <math.h>

namespace {

// theta^(-2p/d), evaluated in double and rounded once to float.
__device__ __forceinline__ float rope_inv_freq(int pair, int head_dim, float theta) {
    return (float)exp2(-(2.0 * (double)pair / (double)head_dim) * log2((double)theta));
}

// Rotate element d of a head given its partner (d^1); consecutive-pair RoPE
// (transformer.metal:154-202).
__device__ __forceinline__ float rope_rotate_f(float self, float partner, int d, uint32_t position,
                                               float inv_freq) {
    const float ang = (float)position * inv_freq;
    float s, c;
    sincosf(ang, &s, &c);
    return (d & 1) ? fmaf(partner, s, self * c) : fmaf(self, c, -partner * s);
}

__device__ __forceinline__ float rope_rotate(float self, float partner, int d, uint32_t position,
                                             int head_dim, float theta) {
    return rope_rotate_f(self, partner, d, position, rope_inv_freq(d >> 1, head_dim, theta));
}

// The head_dim/2 frequencies once, for kernels that take them from memory.
__global__ void rope_table_kernel(float *out, uint32_t head_dim, float theta) {
    const uint32_t p = threadIdx.x;
    if (p < head_dim / 2) out[p] = rope_inv_freq((int)p, (int)head_dim, theta);
}

__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float block_max_256(float v, float *red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t = fmaxf(t, red[i]);
    return t;
}

// ---------------------------------------------------------------- RMSNorm --
// transformer.metal:49-104 (rms_norm), :551-608 (rms_norm_f16out),
// :610-677 (rms_norm_bf16_f16out).  One 256-thread block per row.
template <int ODT, bool TRUNC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *in, const float *scale,
                                                       void *out, uint32_t n, float eps) {
    __shared__ float red[4];
    const float *x = in + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) ss += x[i] * x[i];
    ss = block_sum_256(ss, red);
    const float rms = rsqrtf(ss / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        float v = x[i] * rms * scale[i];
        if constexpr (TRUNC) v = bf16_trunc(v);
        store_from_f32<ODT>(out, (size_t)blockIdx.x * n + i, v);
    }
}

// Rows of 256 V floats (hidden 256 .. 4096): one wave per row holding the row
// in registers (V float4 per lane, adjacent lanes on adjacent 16-byte pieces),
// the sum of squares reduced across the wave without LDS or barriers.  Same
// expression as rms_norm_kernel; only the fp32 summation order differs.
template <int ODT, bool TRUNC, int V>
__global__ __launch_bounds__(64) void rms_norm_rows_kernel(const float *in, const float *scale,
                                                            void *out, uint32_t rows, float eps) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    constexpr uint32_t n = 256 * V;
    const uint32_t row = blockIdx.x, lane = threadIdx.x;
    const f4 *x = (const f4 *)(in + (size_t)row * n) + lane;
    const f4 *sc = (const f4 *)scale + lane;
    f4 v[V], w[V];   // the norm weights are loaded with the row, not after the reduction
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = x[64 * i];
#pragma unroll
    for (int i = 0; i < V; ++i) w[i] = sc[64 * i];
#pragma unroll
    for (int i = 0; i < V; ++i) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    const float rms = rsqrtf(wave_sum(ss) / (float)n + eps);
#pragma unroll
    for (int i = 0; i < V; ++i) {
        f4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float t = v[i][e] * rms * w[i][e];
            if constexpr (TRUNC) t = bf16_trunc(t);
            y[e] = t;
        }
        const size_t o = (size_t)row * n / 4 + lane + 64 * i;   // in 4-element units
        if constexpr (ODT == NNZ_F32) ((f4 *)out)[o] = y;
        else ((h4 *)out)[o] = (h4){(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
    }
}

template <int ODT, bool TRUNC>
void launch_rms_norm(nnz_ctx *ctx, const float *in, const float *scale, void *out, uint32_t n,
                     uint32_t rows, float eps) {
    const bool vec = n % 256 == 0 && n <= 4096 && ((uintptr_t)in & 15) == 0 &&
                     ((uintptr_t)scale & 15) == 0 && ((uintptr_t)out & 15) == 0;
    if (!vec) {
        rms_norm_kernel<ODT, TRUNC><<<rows, 256, 0, ctx->stream>>>(in, scale, out, n, eps);
        return;
    }
    const uint32_t g = rows;   // one single-wave workgroup per row, spread over every CU
    switch (n / 256) {
#define NNZ_RMS_CASE(V) \
    case V: rms_norm_rows_kernel<ODT, TRUNC, V><<<g, 64, 0, ctx->stream>>>(in, scale, out, rows, eps); break;
        NNZ_RMS_CASE(1) NNZ_RMS_CASE(2) NNZ_RMS_CASE(3) NNZ_RMS_CASE(4) NNZ_RMS_CASE(5) NNZ_RMS_CASE(6)
        NNZ_RMS_CASE(7) NNZ_RMS_CASE(8) NNZ_RMS_CASE(9) NNZ_RMS_CASE(10) NNZ_RMS_CASE(11) NNZ_RMS_CASE(12)
        NNZ_RMS_CASE(13) NNZ_RMS_CASE(14) NNZ_RMS_CASE(15) NNZ_RMS_CASE(16)
#undef NNZ_RMS_CASE
    }
}

// ------------------------------------------------------------------- SiLU --
__global__ void silu_kernel(const float *in, float *out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float x = in[i]; out[i] = x / (1.f + expf(-x)); }
}

template <int DT>
__global__ void silu_mul_kernel(const void *gate, const void *up, void *out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float g = load_as_f32<DT>(gate, i);
        store_from_f32<DT>(out, i, g / (1.f + expf(-g)) * load_as_f32<DT>(up, i));
    }
}

// ------------------------------------------------------------------- RoPE --
// One thread per (head, pair), in place.
template <int DT>
__global__ void rope_kernel(void *data, uint32_t heads, uint32_t head_dim, uint32_t position,
                            float theta) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t half = head_dim / 2;
    if (gid >= heads * half) return;
    const uint32_t h = gid / half, p = gid % half;
    const size_t base = (size_t)h * head_dim + 2 * p;
    const float a = load_as_f32<DT>(data, base), b = load_as_f32<DT>(data, base + 1);
    const float ang = (float)position * rope_inv_freq((int)p, (int)head_dim, theta);
    float s, c;
    sincosf(ang, &s, &c);
    store_from_f32<DT>(data, base, fmaf(a, c, -b * s));
    store_from_f32<DT>(data, base + 1, fmaf(b, c, a * s));
}

// ------------------------------------------------------------ KV append ----
// transformer.metal:204-257: K[h][pos][d], V[h][d][pos].
template <int PDT, int CDT>
__global__ void kv_update_kernel(const void *kp, const void *vp, void *kc, void *vc,
                                 uint32_t heads, uint32_t head_dim, uint32_t pos, uint32_t max_ctx) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= heads * head_dim) return;
    const uint32_t h = gid / head_dim, d = gid % head_dim;
    const size_t stride = (size_t)max_ctx * head_dim;
    store_from_f32<CDT>(kc, h * stride + (size_t)pos * head_dim + d, load_as_f32<PDT>(kp, gid));
    store_from_f32<CDT>(vc, h * stride + (size_t)d * max_ctx + pos, load_as_f32<PDT>(vp, gid));
}

// Per-head RMSNorm (+ optional scale) and RoPE of one head held by a block of
// head_dim threads (<= 256).  Returns this thread's rotated element.
__device__ __forceinline__ float head_norm_rope(float v, const float *scale, uint32_t head_dim,
                                                uint32_t pos, float eps, float theta,
                                                bool do_norm, float *red) {
    const int d = threadIdx.x;
    if (do_norm) {
        const float ss = block_sum_256(d < (int)head_dim ? v * v : 0.f, red);
        const float rms = rsqrtf(ss / (float)head_dim + eps);
        v = v * rms * (d < (int)head_dim ? scale[d] : 0.f);
    }
    const float partner = __shfl_xor(v, 1, 64);
    return rope_rotate(v, partner, d, pos, (int)head_dim, theta);
}

// transformer.metal:1032-1113 fused_rope_k_kv_cache_update_f16: grid = kv heads.
__global__ __launch_bounds__(256) void fused_rope_kv_kernel(const f16_t *kp, const f16_t *vp,
                                                            f16_t *kc, f16_t *vc, uint32_t head_dim,
                                                            uint32_t pos, uint32_t max_ctx,
                                                            float theta) {
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const float k = d < head_dim ? (float)kp[h * head_dim + d] : 0.f;
    const float kr = head_norm_rope(k, nullptr, head_dim, pos, 0.f, theta, false, red);
    if (d < head_dim) {
        const size_t stride = (size_t)max_ctx * head_dim;
        kc[h * stride + (size_t)pos * head_dim + d] = (f16_t)kr;
        vc[h * stride + (size_t)d * max_ctx + pos] = vp[h * head_dim + d];
    }
}

// transformer.metal:817-912 fused_norm_rope_f16: per-head RMSNorm + RoPE in place.
__global__ __launch_bounds__(256) void fused_norm_rope_kernel(f16_t *data, const float *scale,
                                                              uint32_t head_dim, uint32_t pos,
                                                              float eps, float theta) {
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const float v = d < head_dim ? (float)data[h * head_dim + d] : 0.f;
    const float r = head_norm_rope(v, scale, head_dim, pos, eps, theta, true, red);
    if (d < head_dim) data[h * head_dim + d] = (f16_t)r;
}

// transformer.metal:914-1030 fused_k_norm_rope_kv_cache_f16.
__global__ __launch_bounds__(256) void fused_k_norm_rope_kv_kernel(
    const f16_t *kp, const f16_t *vp, f16_t *kc, f16_t *vc, const float *kscale,
    uint32_t head_dim, uint32_t pos, uint32_t max_ctx, float eps, float theta) {
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const float k = d < head_dim ? (float)kp[h * head_dim + d] : 0.f;
    const float kr = head_norm_rope(k, kscale, head_dim, pos, eps, theta, true, red);
    if (d < head_dim) {
        const size_t stride = (size_t)max_ctx * head_dim;
        kc[h * stride + (size_t)pos * head_dim + d] = (f16_t)kr;
        vc[h * stride + (size_t)d * max_ctx + pos] = vp[h * head_dim + d];
    }
}

// Attention prologue of the fused decode kernel (transformer.metal:1506-1589):
// blocks [0, Hq) normalise+rotate a query head into f32 `qout`; blocks
// [Hq, Hq+Hkv) normalise+rotate a key head into the cache at `pos` and copy V.
// Each KV entry is written by exactly one block.
__global__ __launch_bounds__(256) void attn_prep_kernel(
    const f16_t *q, const f16_t *kr, const f16_t *vr, const float *qn, const float *kn,
    float *qout, f16_t *kc, f16_t *vc, uint32_t hq, uint32_t hkv, uint32_t head_dim, uint32_t pos0,
    const uint32_t *d_pos, uint32_t max_ctx, float eps, float theta) {
    __shared__ float red[4];
    const uint32_t b = blockIdx.x, d = threadIdx.x, z = blockIdx.y;
    const uint32_t pos = (d_pos ? *d_pos : pos0) + z;
    q += (size_t)z * hq * head_dim;
    qout += (size_t)z * hq * head_dim;
    kr += (size_t)z * hkv * head_dim;
    vr += (size_t)z * hkv * head_dim;
    if (b < hq) {
        const float v = d < head_dim ? (float)q[b * head_dim + d] : 0.f;
        const float r = head_norm_rope(v, qn, head_dim, pos, eps, theta, true, red);
        if (d < head_dim) qout[b * head_dim + d] = r;
    } else {
        const uint32_t h = b - hq;
        const float v = d < head_dim ? (float)kr[h * head_dim + d] : 0.f;
        const float r = head_norm_rope(v, kn, head_dim, pos, eps, theta, true, red);
        if (d < head_dim) {
            const size_t stride = (size_t)max_ctx * head_dim;
            kc[h * stride + (size_t)pos * head_dim + d] = (f16_t)r;
            vc[h * stride + (size_t)d * max_ctx + pos] = vr[h * head_dim + d];
        }
    }
}

// The same prologue for a prefill batch: one wave per (head, token), lane p
// holding the rotation pair (2p, 2p+1), so the norm is one wave reduction
// and the rotation needs no shuffle; frequencies from the model's table.
// q goes out as float32 [nq][hq][D], or, with qsplit > 0, as the operands
// of the MFMA prefill attention: x = q * qsplit as f16 hi = f16(x) and
// lo = f16(x - hi), [nq][hq][2][D] (hi row, then lo row).  V rows go to
// the transposed cache from waves of their own, launched first, one per
// (KV head, 64 tokens, 16 dims).  (Written by the k waves, two 2-byte stores
// per lane to 64 different dim rows each, the V copy took 2.6 of the
// kernel's 7.9 us at 512 tokens.)
__global__ __launch_bounds__(256) void attn_prep_waves_kernel(
    const f16_t *q, const f16_t *kr, const f16_t *vr, const float *qn, const float *kn,
    void *qout, f16_t *kc, f16_t *vc, const float *inv_freq, uint32_t hq, uint32_t hkv,
    uint32_t head_dim, uint32_t pos0, uint32_t nq, uint32_t max_ctx, float eps, float qsplit) {
    const uint32_t heads = hq + hkv;
    const uint32_t ng = (nq + 63u) / 64u, ns = (head_dim + 15u) / 16u;
    const uint32_t v_units = hkv * ng * ns;
    const uint32_t uu = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (uu < v_units) {
        // V units first: (KV head, 64-token group, 16-dim slice).  Lane t
        // copies dims 16 s .. 16 s + 15 of token 64 g + t's V row into the
        // transposed cache, one dim row per store instruction, so a store
        // covers 64 consecutive positions (128 bytes) rather than 64 rows.
        const uint32_t sl = uu % ns, g = (uu / ns) % ng, h = uu / (ns * ng);
        const uint32_t z = g * 64u + (threadIdx.x & 63u);
        if (z >= nq) return;
        const uint32_t *row = (const uint32_t *)(vr + ((size_t)z * hkv + h) * head_dim) + 8u * sl;
        const __amdgpu_buffer_rsrc_t dst = __builtin_amdgcn_make_buffer_rsrc(
            vc + (size_t)h * max_ctx * head_dim, (short)0, (int)(max_ctx * head_dim * 2u), 0x00020000);
        const uint32_t voff = (pos0 + z) * 2u, rstride = max_ctx * 2u, nw = head_dim / 2u;
        uint32_t w[8];
#pragma unroll
        for (uint32_t i = 0; i < 8u; ++i)
            if (8u * sl + i < nw) w[i] = row[i];
#pragma unroll
        for (uint32_t i = 0; i < 8u; ++i)
            if (8u * sl + i < nw) {
                const uint32_t d = 2u * (8u * sl + i);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(w[i] & 0xFFFFu), dst, voff, d * rstride, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(w[i] >> 16), dst, voff, (d + 1u) * rstride, 0);
            }
        return;
    }
    const uint32_t u = uu - v_units;
    if (u >= heads * nq) return;   // whole waves only
    const uint32_t z = u / heads, b = u % heads, p = threadIdx.x & 63u;
    const uint32_t pos = pos0 + z;
    const bool on = 2u * p < head_dim;
    const bool isq = b < hq;
    const uint32_t h = isq ? b : b - hq;
    const f16_t *src = isq ? q + ((size_t)z * hq + h) * head_dim : kr + ((size_t)z * hkv + h) * head_dim;
    float x0 = 0.f, x1 = 0.f;
    if (on) {
        const uint32_t w = *(const uint32_t *)(src + 2u * p);
        x0 = (float)__builtin_bit_cast(f16_t, (uint16_t)(w & 0xFFFFu));
        x1 = (float)__builtin_bit_cast(f16_t, (uint16_t)(w >> 16));
    }
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float rms = rsqrtf(ss / (float)head_dim + eps);
    const float *sc = isq ? qn : kn;
    if (!on) return;
    const float v0 = x0 * rms * sc[2u * p], v1 = x1 * rms * sc[2u * p + 1u];
    const float ang = (float)pos * inv_freq[p];
    float sn, cs;
    sincosf(ang, &sn, &cs);
    const float r0 = fmaf(v0, cs, -v1 * sn), r1 = fmaf(v0, sn, v1 * cs);
    if (isq && qsplit > 0.f) {
        const float x0 = r0 * qsplit, x1 = r1 * qsplit;
        const f16_t h0 = (f16_t)x0, h1 = (f16_t)x1;
        const f16_t l0 = (f16_t)(x0 - (float)h0), l1 = (f16_t)(x1 - (float)h1);
        f16_t *row = (f16_t *)qout + ((size_t)z * hq + h) * 2u * head_dim + 2u * p;
        *(uint32_t *)row = (uint32_t)__builtin_bit_cast(uint16_t, h0) |
                           (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
        *(uint32_t *)(row + head_dim) = (uint32_t)__builtin_bit_cast(uint16_t, l0) |
                                        (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
    } else if (isq) {
        *(float2 *)((float *)qout + ((size_t)z * hq + h) * head_dim + 2u * p) = make_float2(r0, r1);
    } else {
        const size_t stride = (size_t)max_ctx * head_dim;
        const uint32_t kw = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)r0) |
                            (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)r1) << 16;
        *(uint32_t *)(kc + h * stride + (size_t)pos * head_dim + 2u * p) = kw;
    }
}

// ------------------------------------------------------ decode attention ---
// Split-sequence GQA decode.  Grid (num_chunks, Hkv); block 256 threads.
// Each block serves the G query heads of one KV head over one chunk of
// `chunk` tokens: scores -> chunk max / exp-sum -> unnormalised P.V partial.
// If the whole sequence is one chunk the block writes the final output.
struct AttnArgs {
    const void *q;        // [Hq][D] in qdt (already normed/roped unless rope_pos >= 0)
    const void *kc;       // [Hkv][max_ctx][D]
    const void *vc;       // [Hkv][D][max_ctx] (VT) or [Hkv][max_ctx][D]
    void *out;            // [Hq][D] in odt (single-chunk case)
    float *part_o;        // [Z][Hq][nchunks][D]
    float *part_ml;       // [Z][Hq][nchunks][2]
    const uint32_t *d_seq;  // if set, seq_len of query 0 is read from device memory
    uint32_t seq_len;     // tokens visible to query 0; query z sees seq_len + z (causal)
    uint32_t max_ctx, chunk, nchunks, hq;
    uint32_t q_stride, o_stride;  // elements between consecutive queries
    int32_t rope_pos;
    int qdt, odt;
    float rope_theta, scale;
};

constexpr int ATT_MAX_CHUNK = 512;
#ifndef NNZ_DEC_TARGET_BLOCKS
#define NNZ_DEC_TARGET_BLOCKS 1024u
#endif

__device__ __forceinline__ float load_dt(const void *p, size_t i, int dt) {
    if (dt == NNZ_F32) return ((const float *)p)[i];
    if (dt == NNZ_F16) return (float)((const f16_t *)p)[i];
    return bf16_to_f32(((const uint16_t *)p)[i]);
}

__device__ __forceinline__ void store_dt(void *p, size_t i, float v, int dt) {
    if (dt == NNZ_F32) ((float *)p)[i] = v;
    else if (dt == NNZ_F16) ((f16_t *)p)[i] = (f16_t)v;
    else ((uint16_t *)p)[i] = f32_to_bf16_rne(v);
}

template <int KVDT>
__device__ __forceinline__ void unpack2(uint32_t w, float &lo, float &hi) {
    if constexpr (KVDT == NNZ_F16) {
        lo = (float)__builtin_bit_cast(f16_t, (uint16_t)(w & 0xFFFFu));
        hi = (float)__builtin_bit_cast(f16_t, (uint16_t)(w >> 16));
    } else {
        lo = bf16_to_f32((uint16_t)(w & 0xFFFFu));
        hi = bf16_to_f32((uint16_t)(w >> 16));
    }
}

template <int D, int G, int KVDT, bool VT>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnArgs a) {
    constexpr int NQ = (G * D + 255) / 256;   // q elements per thread
    __shared__ float qs[G][D];
    __shared__ float ps[G][ATT_MAX_CHUNK];
    __shared__ float red[4];
    __shared__ float ored[4][G][D];

    const int tid = threadIdx.x;
    const uint32_t c = blockIdx.x, h = blockIdx.y, z = blockIdx.z;
    const uint32_t seq = (a.d_seq ? *a.d_seq : a.seq_len) + z;
    const uint32_t t0 = c * a.chunk;
    if (t0 >= seq) return;  // the combine step only reads chunks < ceil(seq/chunk)
    const uint32_t len = min(a.chunk, seq - t0);

    // q of the G heads that share this KV head; optional RoPE (config 4).
    float qv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        qv[k] = (i < G * D) ? load_dt(a.q, (size_t)z * a.q_stride + (size_t)h * G * D + i, a.qdt) : 0.f;
    }
    if (a.rope_pos >= 0) {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int i = tid + 256 * k;
            const float partner = __shfl_xor(qv[k], 1, 64);
            qv[k] = rope_rotate(qv[k], partner, i % D, (uint32_t)a.rope_pos, D, a.rope_theta);
        }
    }
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        if (i < G * D) qs[i / D][i % D] = qv[k];
    }
    __syncthreads();

    // Scores: one thread per token; each streams its K row with 16-byte loads.
    const size_t kv_stride = (size_t)a.max_ctx * D;
    const uint16_t *kb = (const uint16_t *)a.kc + h * kv_stride;
    for (uint32_t t = tid; t < len; t += 256) {
        float dot[G];
#pragma unroll
        for (int g = 0; g < G; ++g) dot[g] = 0.f;
        const uint4 *kr = (const uint4 *)(kb + (size_t)(t0 + t) * D);
#pragma unroll 4
        for (int v = 0; v < D / 8; ++v) {
            const uint4 w = kr[v];
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float k0, k1;
                unpack2<KVDT>(wv[e], k0, k1);
                const int d = v * 8 + 2 * e;
#pragma unroll
                for (int g = 0; g < G; ++g) dot[g] = fmaf(qs[g][d + 1], k1, fmaf(qs[g][d], k0, dot[g]));
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) ps[g][t] = dot[g] * a.scale;
    }
    __syncthreads();

    // Chunk max and exp-sum per head; P overwrites the scores.
    float mval[G], lval[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float m = -INFINITY;
        for (uint32_t t = tid; t < len; t += 256) m = fmaxf(m, ps[g][t]);
        m = block_max_256(m, red);
        float l = 0.f;
        for (uint32_t t = tid; t < len; t += 256) {
            const float e = expf(ps[g][t] - m);
            ps[g][t] = e;
            l += e;
        }
        l = block_sum_256(l, red);
        mval[g] = m;
        lval[g] = l;
    }
    __syncthreads();

    const uint16_t *vb = (const uint16_t *)a.vc + h * kv_stride;
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
    int part;  // which of the 4 partial slots this thread contributes to
    if constexpr (!VT) {
        // V is [t][D]: 16 lanes cover one 256-byte row, 16 token groups.
        constexpr int DP = D / 8, TG = 256 / DP;
        const int dp = tid % DP, tg = tid / DP;
        for (uint32_t t = tg; t < len; t += TG) {
            const uint4 w = *(const uint4 *)(vb + (size_t)(t0 + t) * D + dp * 8);
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v0, v1;
                unpack2<KVDT>(wv[e], v0, v1);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = ps[g][t];
                    o[g][2 * e] = fmaf(p, v0, o[g][2 * e]);
                    o[g][2 * e + 1] = fmaf(p, v1, o[g][2 * e + 1]);
                }
            }
        }
        // Fold the token groups inside the wave (lanes that differ in tg).
#pragma unroll
        for (int off = DP; off < 64; off <<= 1)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] += __shfl_xor(o[g][e], off, 64);
        part = tid >> 6;
        if ((tid & 63) < DP) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) ored[part][g][dp * 8 + e] = o[g][e];
        }
    } else {
        // V is [D][max_ctx]: a thread owns one d and streams 8 tokens per
        // 16-byte load over its share of the chunk.
        constexpr int PARTS = 256 / D;
        const int d = tid % D;
        part = tid / D;
        const uint32_t ngroups = len / 8;
        const uint32_t per = ceil_div(ngroups, PARTS);
        const uint32_t k0 = part * per, k1 = min(ngroups, k0 + per);
        const uint16_t *row = vb + (size_t)d * a.max_ctx + t0;
        for (uint32_t k = k0; k < k1; ++k) {
            const uint4 w = *(const uint4 *)(row + 8 * k);
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v0, v1;
                unpack2<KVDT>(wv[e], v0, v1);
#pragma unroll
                for (int g = 0; g < G; ++g)
                    o[g][0] = fmaf(ps[g][8 * k + 2 * e + 1], v1, fmaf(ps[g][8 * k + 2 * e], v0, o[g][0]));
            }
        }
        if (part == PARTS - 1) {  // ragged tail of the chunk
            for (uint32_t t = ngroups * 8; t < len; ++t) {
                float v;
                if constexpr (KVDT == NNZ_F16) v = (float)__builtin_bit_cast(f16_t, row[t]);
                else v = bf16_to_f32(row[t]);
#pragma unroll
                for (int g = 0; g < G; ++g) o[g][0] = fmaf(ps[g][t], v, o[g][0]);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) ored[part][g][d] = o[g][0];
    }
    __syncthreads();

    constexpr int NPART = VT ? 256 / D : 4;
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float s = 0.f;
#pragma unroll
        for (int p = 0; p < NPART; ++p) s += ored[p][g][d];
        const uint32_t qh = h * G + g;
        if (a.nchunks == 1) {
            store_dt(a.out, (size_t)z * a.o_stride + (size_t)qh * D + d, s / lval[g], a.odt);
        } else {
            const size_t slot = ((size_t)z * a.hq + qh) * a.nchunks + c;
            a.part_o[slot * D + d] = s;
            if (d == 0) {
                a.part_ml[slot * 2 + 0] = mval[g];
                a.part_ml[slot * 2 + 1] = lval[g];
            }
        }
    }
}

// ------------------------------------------------- fused decode attention --
// The attention half of a decode step for one layer:
//   attn_fused_kernel, grid (chunks of FCHUNK tokens, Hkv), 256 threads:
//     * first, every thread issues its K and V loads for the chunk (they do
//       not depend on q), so the q prologue, the scores and P.V wait on one
//       memory round trip instead of three;
//     * per-head RMSNorm + RoPE of the G query heads (kept f32); the block
//       whose chunk holds `pos` also normalises+rotates the new key, rounds
//       it to f16, appends K/V to the caches (transformer.metal:1506-1592)
//       and uses the new row from LDS in place of the prefetched one;
//     * scores with 256/FCHUNK lanes per token, one softmax pass for all G
//       heads, P.V with a thread per (d, token part);
//     * one chunk: f16 output; several: partials (m, l, o) for
//       attn_merge_kernel, which folds them with one round of loads.
// Caches: f16, K [Hkv][max_ctx][D], V [Hkv][D][max_ctx]; seq_len and
// position come from device memory (graph replay) when d_seq is set.
constexpr int FCHUNK = 64;

struct FusedAttnArgs {
    const f16_t *q, *kr, *vr;       // raw projections [Hq*D], [Hkv*D], [Hkv*D]
    const float *qn, *kn;           // per-head norm scales [D]
    f16_t *kc, *vc;                 // caches
    f16_t *out;                     // [Hq*D]
    float *part_o, *part_ml;        // see part_o_at, part_ml_at
    const uint32_t *d_seq;          // device seq_len (= position + 1) or null
    const float *inv_freq;          // [D/2] RoPE frequencies, or null (computed here)
    uint32_t seq_len, max_ctx, nchunks;
    uint32_t unit_major;            // part_o layout: 0 head-major, 1 unit-major
    uint32_t kdim;                  // Hq * D
    uint32_t gfull;                 // query heads per KV head
    uint32_t units;                 // nchunks * Hkv (chunk, KV head) pairs
    uint32_t parts;                 // blocks per unit (query-head groups of G)
    int direct;                     // one chunk and no consumer merge: write out
    float eps, theta, scale;
};

// Offset of partial output (query head qh, chunk c, dim d) in part_o.
// Head-major (attn_merge_kernel): [Hq][nchunks][D].  Unit-major (the O
// projection's merge prologue, qmv.hip): chunk by chunk, column k = qh D + d
// of the K = Hq D columns at ((k >> 2) & 7) K / 8 + (k >> 5) 4 + (k & 3) --
// nibble n of every 32-column unit together, so a lane per unit reads one
// nibble's 4 values with one 16-byte load and a wave's load is contiguous.
// The (max, sum) pair of (qh, c) sits at float2 index part_ml_at: head-major
// [Hq][nchunks], or chunk-major [nchunks][Hq] beside the unit-major part_o
// (a chunk's pairs of all heads are then one contiguous read).
__device__ __forceinline__ size_t part_o_at(const FusedAttnArgs &a, uint32_t qh, uint32_t c, uint32_t d,
                                            uint32_t D) {
    if (!a.unit_major) return ((size_t)qh * a.nchunks + c) * D + d;
    const uint32_t k = qh * D + d;
    return (size_t)c * a.kdim + ((k >> 2) & 7u) * (a.kdim >> 3) + (k >> 5) * 4u + (k & 3u);
}
__device__ __forceinline__ size_t part_ml_at(const FusedAttnArgs &a, uint32_t qh, uint32_t c, uint32_t D) {
    return a.unit_major ? (size_t)c * (a.kdim / D) + qh : (size_t)qh * a.nchunks + c;
}

template <int D, int G>
__global__ __launch_bounds__(256) void attn_fused_kernel(FusedAttnArgs a) {
    static_assert(G * D <= 1024, "group too large");
    constexpr int NQ = (G * D + 255) / 256;
    constexpr int TPT = 256 / FCHUNK;          // lanes per token in the score pass
    constexpr int KV4 = D / 8 / TPT;           // K: 16-byte vectors per lane
    constexpr int PARTS = 256 / D;             // P.V: token parts per d
    constexpr int VT = FCHUNK / PARTS;         // P.V: tokens per thread
    constexpr int VV4 = VT / 8;                // V: 16-byte vectors per thread
    static_assert(KV4 >= 1 && VV4 >= 1, "chunk/head_dim");
    __shared__ float qs[G][D];
    __shared__ float ps[G][FCHUNK];   // scores
    __shared__ float pe[G][FCHUNK];   // exp(score - max)
    __shared__ float knew[D], vnew[D];
    __shared__ float red[4][G];
    __shared__ float ored[PARTS][G][D];
    __shared__ float hsum[G][4];

    const int tid = threadIdx.x;
    // 1-D grid.  Unit u = (chunk c, KV head h); its `parts` blocks serve the
    // query heads [qb, qb + G) of h and sit 8 ids apart, so that workgroups
    // dispatched round-robin over the 8 XCDs put them on one XCD and its L2
    // serves their shared K/V lines once.  The first part appends to the cache.
    const uint32_t bid = blockIdx.x, span = 8 * a.parts;
    const uint32_t j = a.parts == 1 ? 0u : (bid % span) / 8;
    const uint32_t u = a.parts == 1 ? bid : (bid / span) * 8 + bid % 8;
    if (u >= a.units) return;
    const uint32_t c = u % a.nchunks, h = u / a.nchunks, qb = h * a.gfull + j * G;
    const bool writer = j == 0;
    const uint32_t seq = a.d_seq ? *a.d_seq : a.seq_len;
    const uint32_t pos = seq - 1;
    const uint32_t t0 = c * FCHUNK;
    if (t0 >= seq) return;
    const uint32_t len = min((uint32_t)FCHUNK, seq - t0);
    const bool owns_new = pos < t0 + len;   // this chunk holds the new token

    // ---- loads, in the order they are needed: the small q/k/v vectors and
    // norm weights first, then the chunk's K and V (vmcnt counts in order,
    // so the prologue can start while K and V are still in flight)
    float qv[NQ], qnv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        const int ic = i < G * D ? i : 0;
        qv[k] = (float)a.q[(size_t)qb * D + ic];
        qnv[k] = a.qn[ic % D];
    }
    const int kd = tid < D ? tid : 0;
    const float kraw = (float)a.kr[(size_t)h * D + kd];
    const float knw = a.kn[kd];
    const f16_t vraw = a.vr[(size_t)h * D + kd];
    float qfreq[NQ], kfreq;
    if (a.inv_freq) {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int i = tid + 256 * k;
            qfreq[k] = a.inv_freq[((i < G * D ? i : 0) % D) >> 1];
        }
        kfreq = a.inv_freq[kd >> 1];
    } else {
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            const int i = tid + 256 * k;
            qfreq[k] = rope_inv_freq(((i < G * D ? i : 0) % D) >> 1, D, a.theta);
        }
        kfreq = rope_inv_freq(kd >> 1, D, a.theta);
    }

    const size_t kv_stride = (size_t)a.max_ctx * D;
    const int kt = tid / TPT, ksub = tid % TPT;
    const uint32_t ktok = t0 + min((uint32_t)kt, len - 1);
    uint4 kreg[KV4];
    {
        const uint4 *kp = (const uint4 *)(a.kc + h * kv_stride + (size_t)ktok * D) + ksub * KV4;
#pragma unroll
        for (int v = 0; v < KV4; ++v) kreg[v] = kp[v];
    }
    // V: 8-token groups; a group that starts past the chunk's end reads
    // group 0 instead (it stays inside the row) and is masked below.
    const int vd = tid % D, vpart = tid / D;
    uint4 vreg[VV4];
    {
        const f16_t *vrow = a.vc + h * kv_stride + (size_t)vd * a.max_ctx + t0;
#pragma unroll
        for (int v = 0; v < VV4; ++v) {
            const uint32_t g0 = (uint32_t)(vpart * VT + v * 8);
            vreg[v] = *(const uint4 *)(vrow + (g0 < len ? g0 : 0u));
        }
    }

    // ---- q: per-head RMSNorm * q_norm, RoPE; one head = D consecutive slots
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        if (i >= G * D) qv[k] = 0.f;
        // lanes of one wave belong to one head (D >= 64)
        const float s = wave_sum(qv[k] * qv[k]);
        if ((tid & 63) == 0 && i < G * D) hsum[i / D][(i % D) / 64] = s;
    }
    // new key: RMSNorm * k_norm, RoPE, f16; appended to the caches
    if (owns_new) {
        const float kv = tid < D ? kraw : 0.f;
        float ss = wave_sum(kv * kv);
        if (D > 64) {
            if ((tid & 63) == 0) red[tid >> 6][0] = ss;
        }
        __syncthreads();
        if (D > 64) ss = red[0][0] + red[1][0];
        const float kn = kv * rsqrtf(ss / (float)D + a.eps) * knw;
        const float partner = __shfl_xor(kn, 1, 64);
        const float kr = f16_round(rope_rotate_f(kn, partner, tid, pos, kfreq));
        if (tid < D) {
            knew[tid] = kr;
            vnew[tid] = (float)vraw;
            if (writer) {
                a.kc[(size_t)h * kv_stride + (size_t)pos * D + tid] = (f16_t)kr;
                a.vc[(size_t)h * kv_stride + (size_t)tid * a.max_ctx + pos] = vraw;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        const bool ok = i < G * D;
        const int g = ok ? i / D : 0, d = i % D;
        float ss = 0.f;
#pragma unroll
        for (int w = 0; w < D / 64; ++w) ss += hsum[g][w];
        const float v = ok ? qv[k] * rsqrtf(ss / (float)D + a.eps) * qnv[k] : 0.f;
        const float partner = __shfl_xor(v, 1, 64);  // all lanes take part
        if (ok) qs[g][d] = rope_rotate_f(v, partner, d, pos, qfreq[k]);
    }
    __syncthreads();

    // ---- scores: TPT consecutive lanes per token
    {
        float dot[G];
#pragma unroll
        for (int g = 0; g < G; ++g) dot[g] = 0.f;
        const bool is_new = owns_new && t0 + (uint32_t)kt == pos;
#pragma unroll
        for (int v = 0; v < KV4; ++v) {
            const uint32_t wv[4] = {kreg[v].x, kreg[v].y, kreg[v].z, kreg[v].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = (ksub * KV4 + v) * 8 + 2 * e;
                float k0, k1;
                unpack2<NNZ_F16>(wv[e], k0, k1);
                if (is_new) { k0 = knew[d]; k1 = knew[d + 1]; }
#pragma unroll
                for (int g = 0; g < G; ++g) dot[g] = fmaf(qs[g][d + 1], k1, fmaf(qs[g][d], k0, dot[g]));
            }
        }
        // the TPT lanes of a token are consecutive lanes of one quad
        static_assert(TPT <= 4, "lanes per token within a DPP quad");
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if constexpr (TPT >= 2) dot[g] += dpp_move<DPP_XOR1>(dot[g], 0.f);
            if constexpr (TPT >= 4) dot[g] += dpp_move<DPP_XOR2>(dot[g], 0.f);
        }
        if (ksub == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) ps[g][kt] = (uint32_t)kt < len ? dot[g] * a.scale : -INFINITY;
        }
    }
    __syncthreads();

    // ---- softmax over the chunk, all G heads at once: lane l holds tokens
    // l, l + 64, ... so every wave sees the whole chunk and computes the
    // same max and sum (no cross-wave step).
    constexpr int TPL = (FCHUNK + 63) / 64;   // tokens per lane
    float mval[G], lval[G];
    {
        const int lane = tid & 63;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc[TPL];
            float m = -INFINITY;
#pragma unroll
            for (int k = 0; k < TPL; ++k) {
                sc[k] = lane + 64 * k < FCHUNK ? ps[g][lane + 64 * k] : -INFINITY;
                m = fmaxf(m, sc[k]);
            }
            mval[g] = wave_max(m);
            float l = 0.f;
#pragma unroll
            for (int k = 0; k < TPL; ++k) {
                const float e = lane + 64 * k < FCHUNK ? expf(sc[k] - mval[g]) : 0.f;
                l += e;
                if (tid < 64 && lane + 64 * k < FCHUNK) pe[g][lane + 64 * k] = e;
            }
            lval[g] = wave_sum(l);
        }
    }
    __syncthreads();

    // ---- P.V from the prefetched V (new token from LDS)
    {
        float o[G];
#pragma unroll
        for (int g = 0; g < G; ++g) o[g] = 0.f;
        // full chunks without the new token (all but at most two) skip the
        // end and new-token checks (block-uniform branch)
        const bool plain = !owns_new && len == (uint32_t)FCHUNK;
#pragma unroll
        for (int v = 0; v < VV4; ++v) {
            const uint32_t wv[4] = {vreg[v].x, vreg[v].y, vreg[v].z, vreg[v].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = vpart * VT + v * 8 + 2 * e;
                float v0, v1;
                unpack2<NNZ_F16>(wv[e], v0, v1);
                if (!plain) {
                    // past the end: weight 0, value 0 (never NaN * 0)
                    v0 = (uint32_t)t < len ? v0 : 0.f;
                    v1 = (uint32_t)t + 1 < len ? v1 : 0.f;
                    if (owns_new && t0 + t == pos) v0 = vnew[vd];
                    if (owns_new && t0 + t + 1 == pos) v1 = vnew[vd];
                }
#pragma unroll
                for (int g = 0; g < G; ++g) o[g] = fmaf(pe[g][t + 1], v1, fmaf(pe[g][t], v0, o[g]));
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) ored[vpart][g][vd] = o[g];
    }
    __syncthreads();

    // One chunk: final output.  Several: partials for attn_merge_kernel
    // (merging here would need an agent-scope fence between workgroups,
    // which on a multi-XCD part writes back and invalidates the XCD's L2;
    // a kernel boundary is the cheaper synchronisation).
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float s = 0.f;
#pragma unroll
        for (int p = 0; p < PARTS; ++p) s += ored[p][g][d];
        if (a.direct) {
            a.out[(size_t)(qb + g) * D + d] = (f16_t)(s / lval[g]);
        } else {
            const size_t slot = part_ml_at(a, qb + g, c, D);
            a.part_o[part_o_at(a, qb + g, c, d, D)] = s;
            if (d == 0) {
                a.part_ml[slot * 2] = mval[g];
                a.part_ml[slot * 2 + 1] = lval[g];
            }
        }
    }
}

// The decode shape of attn_fused_kernel (head_dim 128, one query head per
// block): same grid, chunking, outputs and cache append, organised by wave
// so that one block barrier remains instead of six.
//   * Every load is issued before the sequence length is read: the chunk's
//     K rows and V groups are clamped to the cache (max_ctx), not to the live
//     length, so they wait on nothing; rows past the length are masked by
//     select (never multiplied), as are the blocks of chunks past it, which
//     exit after issuing their loads.
//   * Wave w owns tokens 16 w .. 16 w + 15 of the chunk.  Each wave normalises
//     and rotates the query itself: lane l holds dims 2l, 2l + 1, a RoPE pair,
//     so the rotation needs no partner exchange.  The scores take 4 lanes per
//     token (32 dims each) and read the query from a wave-private LDS copy.
//   * Softmax per wave (its own maximum and sum); P.V with lane l on dims 2l,
//     2l + 1 over the wave's 16 tokens, the 16 weights read into scalar
//     registers.
//   * The new token (position seq - 1): the wave holding it normalises,
//     rotates and f16-rounds the raw key in the pair layout, scores it with
//     one whole-wave dot product, and takes its value from the raw
//     projection (the writer block appends both to the caches).
//   * The four waves' (m, l, o) meet in LDS after the one barrier; wave 0
//     writes the output (one chunk) or the chunk's partials.
constexpr int WTOK = FCHUNK / 4;   // tokens per wave

__global__ __launch_bounds__(256) void attn_fused_wave_kernel(FusedAttnArgs a) {
    constexpr int D = 128;
    __shared__ __align__(16) float2 qsh[4][64];   // per wave: the rotated query (pair layout)
    __shared__ float2 osh[4][64];                 // per wave: o of dims 2l, 2l + 1
    __shared__ float2 mlsh[4];                    // per wave: (max, sum)

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t bid = blockIdx.x, span = 8 * a.parts;
    const uint32_t j = a.parts == 1 ? 0u : (bid % span) / 8;
    const uint32_t u = a.parts == 1 ? bid : (bid / span) * 8 + bid % 8;
    if (u >= a.units) return;
    const uint32_t c = u % a.nchunks, h = u / a.nchunks, qh = h * a.gfull + j;
    const uint32_t t0 = c * FCHUNK, wt0 = (uint32_t)w * WTOK;

    // ---- loads: q, norm scales, the new K/V projections and the RoPE
    // frequency first (the prologue waits for these only), then K and V
    const uint32_t qpair = ((const uint32_t *)(a.q + (size_t)qh * D))[lane];
    const float2 qn2 = ((const float2 *)a.qn)[lane];
    const uint32_t kpair = ((const uint32_t *)(a.kr + (size_t)h * D))[lane];
    const float2 kn2 = ((const float2 *)a.kn)[lane];
    const uint32_t vpair = ((const uint32_t *)(a.vr + (size_t)h * D))[lane];
    // a null table gets an empty range: the load returns 0 without touching
    // memory (no branch around a load) and the frequency is computed below
    const float freq_t = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.inv_freq), (short)0,
                                          a.inv_freq ? D * 2 : 0, 0x00020000),
        lane * 4, 0, 0));
    const size_t kvh = (size_t)h * a.max_ctx * D;
    const int tk = lane >> 2, sub = lane & 3;
    uint4 kreg[4];
    {
        const uint32_t kt = min(t0 + wt0 + (uint32_t)tk, a.max_ctx - 1);
        const uint4 *kp = (const uint4 *)(a.kc + kvh + (size_t)kt * D + sub * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) kreg[i] = kp[i];
    }
    // V [d][t]: dims 2l, 2l + 1, two 8-token groups each (a group starting
    // at or past max_ctx, which max_ctx % 8 == 0 keeps whole, reads group 0)
    uint4 vreg[2][2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const f16_t *row = a.vc + kvh + (size_t)(2 * lane + e) * a.max_ctx;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t vs = t0 + wt0 + 8u * g;
            vreg[e][g] = *(const uint4 *)(row + (vs < a.max_ctx ? vs : 0u));
        }
    }

    const uint32_t seq = a.d_seq ? *a.d_seq : a.seq_len;
    if (t0 >= seq) return;   // block-uniform: no barrier is pending
    const uint32_t pos = seq - 1;
    const uint32_t len = min((uint32_t)FCHUNK, seq - t0);
    const bool wnew = pos >= t0 + wt0 && pos < t0 + wt0 + WTOK;   // wave-uniform

    // ---- q: RMSNorm * q_norm, RoPE (consecutive pairs), kept f32
    const float freq = a.inv_freq ? freq_t : rope_inv_freq(lane, D, a.theta);
    float sn, cs;
    sincosf((float)pos * freq, &sn, &cs);
    float qe, qo;
    {
        float q0, q1;
        unpack2<NNZ_F16>(qpair, q0, q1);
        const float r = rsqrtf(wave_sum(fmaf(q1, q1, q0 * q0)) / (float)D + a.eps);
        const float x0 = q0 * r * qn2.x, x1 = q1 * r * qn2.y;
        qe = fmaf(x0, cs, -x1 * sn);
        qo = fmaf(x0, sn, x1 * cs);
    }
    qsh[w][lane] = make_float2(qe, qo);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- scores: lanes 4 tk .. 4 tk + 3 share token tk (32 dims each)
    float dot = 0.f;
    {
        const float4 *q4 = (const float4 *)qsh[w] + sub * 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 qa = q4[2 * i], qb = q4[2 * i + 1];
            const float qq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            const uint32_t wv[4] = {kreg[i].x, kreg[i].y, kreg[i].z, kreg[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float k0, k1;
                unpack2<NNZ_F16>(wv[e], k0, k1);
                dot = fmaf(qq[2 * e + 1], k1, fmaf(qq[2 * e], k0, dot));
            }
        }
        dot += dpp_move<DPP_XOR1>(dot, 0.f);
        dot += dpp_move<DPP_XOR2>(dot, 0.f);
    }
    float vn0 = 0.f, vn1 = 0.f;
    if (wnew) {
        // the new key: RMSNorm * k_norm, RoPE, f16; scored here, appended
        // by the writer block
        float k0, k1;
        unpack2<NNZ_F16>(kpair, k0, k1);
        const float r = rsqrtf(wave_sum(fmaf(k1, k1, k0 * k0)) / (float)D + a.eps);
        const float x0 = k0 * r * kn2.x, x1 = k1 * r * kn2.y;
        const float ke = f16_round(fmaf(x0, cs, -x1 * sn));
        const float ko = f16_round(fmaf(x0, sn, x1 * cs));
        const float snew = wave_sum(fmaf(qo, ko, qe * ke));
        if ((uint32_t)tk == pos - t0 - wt0) dot = snew;
        unpack2<NNZ_F16>(vpair, vn0, vn1);
        if (j == 0) {
            const f16_t he = (f16_t)ke, ho = (f16_t)ko;
            ((uint32_t *)(a.kc + kvh + (size_t)pos * D))[lane] =
                (uint32_t)__builtin_bit_cast(uint16_t, he) | ((uint32_t)__builtin_bit_cast(uint16_t, ho) << 16);
            a.vc[kvh + (size_t)(2 * lane) * a.max_ctx + pos] = __builtin_bit_cast(f16_t, (uint16_t)(vpair & 0xFFFFu));
            a.vc[kvh + (size_t)(2 * lane + 1) * a.max_ctx + pos] = __builtin_bit_cast(f16_t, (uint16_t)(vpair >> 16));
        }
    }

    // ---- softmax over the wave's tokens
    const bool tvalid = wt0 + (uint32_t)tk < len;
    const float s = tvalid ? dot * a.scale : -INFINITY;
    const float m = wave_max(s);                  // finite in wave 0 (token 0 is live)
    const float p = tvalid ? expf(s - m) : 0.f;
    const float l = wave_sum(sub == 0 ? p : 0.f);

    // ---- P.V: lane l on dims 2l, 2l + 1
    float pt[WTOK];
#pragma unroll
    for (int t = 0; t < WTOK; ++t) pt[t] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 4 * t));
    const bool plain = wt0 + WTOK <= len && !wnew;   // wave-uniform
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const uint32_t wa[4] = {vreg[0][g].x, vreg[0][g].y, vreg[0][g].z, vreg[0][g].w};
        const uint32_t wb[4] = {vreg[1][g].x, vreg[1][g].y, vreg[1][g].z, vreg[1][g].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 8 * g + 2 * e;
            float a0, a1, b0, b1;
            unpack2<NNZ_F16>(wa[e], a0, a1);
            unpack2<NNZ_F16>(wb[e], b0, b1);
            if (!plain) {
                // past the end: value 0 (the weight is 0 too; never NaN * 0)
                const uint32_t tc = wt0 + (uint32_t)t;
                if (tc >= len) a0 = b0 = 0.f;
                if (tc + 1 >= len) a1 = b1 = 0.f;
                if (t0 + tc == pos) { a0 = vn0; b0 = vn1; }
                if (t0 + tc + 1 == pos) { a1 = vn0; b1 = vn1; }
            }
            o0 = fmaf(pt[t + 1], a1, fmaf(pt[t], a0, o0));
            o1 = fmaf(pt[t + 1], b1, fmaf(pt[t], b0, o1));
        }
    }
    osh[w][lane] = make_float2(o0, o1);
    if (lane == 0) mlsh[w] = make_float2(m, l);
    __syncthreads();

    // ---- the four waves' partials -> the chunk's (m, l, o)
    if (w == 0) {
        float2 ml[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ml[i] = mlsh[i];
        const float M = fmaxf(fmaxf(ml[0].x, ml[1].x), fmaxf(ml[2].x, ml[3].x));
        float lsum = 0.f, r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float wgt = ml[i].x == -INFINITY ? 0.f : expf(ml[i].x - M);
            const float2 o = osh[i][lane];
            lsum = fmaf(wgt, ml[i].y, lsum);
            r0 = fmaf(wgt, o.x, r0);
            r1 = fmaf(wgt, o.y, r1);
        }
        if (a.direct) {
            const f16_t he = (f16_t)(r0 / lsum), ho = (f16_t)(r1 / lsum);
            ((uint32_t *)(a.out + (size_t)qh * D))[lane] =
                (uint32_t)__builtin_bit_cast(uint16_t, he) | ((uint32_t)__builtin_bit_cast(uint16_t, ho) << 16);
        } else {
            // dims 2l, 2l + 1: adjacent in either layout (8-byte aligned)
            const size_t slot = part_ml_at(a, qh, c, D);
            *(float2 *)(a.part_o + part_o_at(a, qh, c, 2u * lane, D)) = make_float2(r0, r1);
            if (lane == 0) ((float2 *)a.part_ml)[slot] = make_float2(M, lsum);
        }
    }
}

// Fold the per-chunk partials of attn_fused_kernel: grid Hq, block 128.
// The first MERGE_PRE chunks' (m, l) pairs and outputs are loaded in one
// round together with seq_len -- (m, l) by one lane per chunk and shared
// through LDS, so the loads stay vector loads; longer sequences loop over
// the rest.
constexpr int MERGE_PRE = 16;

__global__ __launch_bounds__(128) void attn_merge_kernel(const float *part_o, const float *part_ml,
                                                         f16_t *out, const uint32_t *d_seq,
                                                         uint32_t seq_len, uint32_t nchunks,
                                                         uint32_t D) {
    __shared__ float2 ml_s[MERGE_PRE];
    const uint32_t seq = d_seq ? *d_seq : seq_len;
    const uint32_t qh = blockIdx.x, d = threadIdx.x;
    const size_t base = (size_t)qh * nchunks;
    const uint32_t dd = d < D ? d : 0u;
    const float2 mlv = *(const float2 *)(part_ml + (base + min(d % MERGE_PRE, nchunks - 1)) * 2);
    float o[MERGE_PRE];
#pragma unroll
    for (int c = 0; c < MERGE_PRE; ++c) {
        const uint32_t cc = min((uint32_t)c, nchunks - 1);
        o[c] = part_o[(base + cc) * D + dd];
    }
    if (d < MERGE_PRE) ml_s[d] = mlv;
    __syncthreads();
    if (d >= D) return;
    const uint32_t nch = min(nchunks, ceil_div(seq, (uint32_t)FCHUNK));
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < MERGE_PRE; ++c) M = (uint32_t)c < nch ? fmaxf(M, ml_s[c].x) : M;
    for (uint32_t c = MERGE_PRE; c < nch; ++c) M = fmaxf(M, part_ml[(base + c) * 2]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int c = 0; c < MERGE_PRE; ++c) {
        if ((uint32_t)c < nch) {
            const float w = expf(ml_s[c].x - M);
            den = fmaf(w, ml_s[c].y, den);
            num = fmaf(w, o[c], num);
        }
    }
    for (uint32_t c = MERGE_PRE; c < nch; ++c) {
        const float w = expf(part_ml[(base + c) * 2] - M);
        den = fmaf(w, part_ml[(base + c) * 2 + 1], den);
        num = fmaf(w, part_o[(base + c) * D + d], num);
    }
    out[(size_t)qh * D + d] = (f16_t)(num / den);
}

// ------------------------------------------------- single-query attention --
// GQA attention of one query over a cache it does not modify (the public
// gqa entry point): f16 or bf16 caches, V as [Hkv][D][max_ctx] (VT) or
// [Hkv][max_ctx][D], optional RoPE of q, any q/output dtype.
//   * 1-D grid of units (chunk c of `sub` x FCHUNK tokens, KV head h) x
//     parts, placed as in attn_fused_kernel (a unit's parts on one XCD);
//   * a block walks its chunk FCHUNK tokens at a time with an online
//     softmax; the next sub-chunk's K and V are loaded into the other of two
//     register sets while the current one is used, and all loads of a
//     sub-chunk are issued before the first of them is consumed;
//   * scores with 256/FCHUNK lanes per token, P.V from registers;
//   * one chunk: the output; several: partials for the combine (launch_combine).
struct DecAttnArgs {
    const void *q;                  // [Hq][D] in qdt
    const uint16_t *kc, *vc;        // caches (f16 or bf16 bits)
    void *out;                      // [Hq][D] in odt
    float *part_o, *part_ml;        // [Hq][nchunks][D], [Hq][nchunks][2]
    const uint32_t *d_seq;          // device seq_len or null
    uint32_t seq_len, max_ctx, nchunks, sub, gfull, units, parts;
    int32_t rope_pos;
    int qdt, odt;
    float rope_theta, scale;
};

template <int D, int G, int KVDT, bool VT>
__global__ __launch_bounds__(256) void attn_decode_kernel(DecAttnArgs a) {
    constexpr int NQ = (G * D + 255) / 256;
    constexpr int PARTS = 256 / D;               // VT: token parts per d
    constexpr int VTOK = FCHUNK / PARTS;         // VT: tokens per thread
    constexpr int DP = D / 8, TG = 256 / DP;     // lanes per K/V row, token groups
    constexpr int KT = FCHUNK / TG;              // K: tokens (16-byte pieces) per lane
    constexpr int VV4 = VT ? VTOK / 8 : FCHUNK / TG;
    constexpr int NRED = VT ? PARTS : 4;
    constexpr bool QREG = G <= 2;                // this lane's q slice in registers
    static_assert(KT >= 1 && VV4 >= 1 && (DP == 8 || DP == 16) && FCHUNK == 64, "chunk/head_dim");
    __shared__ float qs[G][D];
    __shared__ float ps[G][FCHUNK];
    __shared__ float pe[G][FCHUNK];
    __shared__ float ored[NRED][G][D];

    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t bid = blockIdx.x, span = 8 * a.parts;
    const uint32_t j = a.parts == 1 ? 0u : (bid % span) / 8;
    const uint32_t u = a.parts == 1 ? bid : (bid / span) * 8 + bid % 8;
    if (u >= a.units) return;
    const uint32_t c = u % a.nchunks, h = u / a.nchunks, qb = h * a.gfull + j * G;
    const uint32_t seq = a.d_seq ? *a.d_seq : a.seq_len;
    const uint32_t c0 = c * a.sub * FCHUNK;
    if (c0 >= seq) return;  // the combine step reads chunks < ceil(seq / chunk) only
    const uint32_t ns = min(a.sub, ceil_div(seq - c0, (uint32_t)FCHUNK));

    float qv[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        qv[k] = load_dt(a.q, (size_t)qb * D + (i < G * D ? i : 0), a.qdt);
    }

    const size_t kv_stride = (size_t)a.max_ctx * D;
    const uint16_t *kb = a.kc + h * kv_stride, *vb = a.vc + h * kv_stride;
    const int vd = tid % D, vpart = tid / D;      // VT roles
    const int dp = tid % DP, tg = tid / DP;       // K (and !VT V) roles
    // Loads of sub-chunk s (s < ns): tokens past the end read an in-range
    // token (the last one, or V group 0) and are masked.  K and the
    // row-major V: lane (dp, tg) reads the 16 bytes at dims 8 dp.. of tokens
    // v TG + tg, so one wave instruction reads 64 / DP whole consecutive rows
    // (1 KB at D = 128).
    auto load = [&](uint4 (&kr)[KT], uint4 (&vr)[VV4], uint32_t s) {
        const uint32_t t0 = c0 + s * FCHUNK, len = min((uint32_t)FCHUNK, seq - t0);
#pragma unroll
        for (int v = 0; v < KT; ++v) {
            const uint32_t t = min((uint32_t)(v * TG + tg), len - 1);
            kr[v] = *((const uint4 *)(kb + (size_t)(t0 + t) * D) + dp);
        }
        if constexpr (VT) {
            const uint16_t *row = vb + (size_t)vd * a.max_ctx + t0;
#pragma unroll
            for (int v = 0; v < VV4; ++v) {
                const uint32_t g0 = (uint32_t)(vpart * VTOK + v * 8);
                vr[v] = *(const uint4 *)(row + (g0 < len ? g0 : 0u));
            }
        } else {
#pragma unroll
            for (int v = 0; v < VV4; ++v) {
                const uint32_t t = min((uint32_t)(v * TG + tg), len - 1);
                vr[v] = *((const uint4 *)(vb + (size_t)(t0 + t) * D) + dp);
            }
        }
    };
    uint4 kA[KT], vA[VV4], kB[KT], vB[VV4];
    load(kA, vA, 0);

    // q (optionally RoPE-rotated at rope_pos) -> LDS
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int i = tid + 256 * k;
        float v = i < G * D ? qv[k] : 0.f;
        if (a.rope_pos >= 0) {
            const float partner = __shfl_xor(v, 1, 64);  // all lanes take part
            v = rope_rotate(v, partner, i % D, (uint32_t)a.rope_pos, D, a.rope_theta);
        }
        if (i < G * D) qs[i / D][i % D] = v;
    }
    __syncthreads();

    float qr[QREG ? G : 1][8];   // q at this lane's 8 dims (G <= 2)
    if constexpr (QREG) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) qr[g][i] = qs[g][dp * 8 + i];
    }
    float m_run[G], l_run[G];
    float o[G][VT ? 1 : 8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.f;
#pragma unroll
        for (int e = 0; e < (VT ? 1 : 8); ++e) o[g][e] = 0.f;
    }

    // One sub-chunk from (kr, vr); the caller has already issued the next
    // sub-chunk's loads into the other register set.
    auto compute = [&](const uint4 (&kr)[KT], const uint4 (&vr)[VV4], uint32_t s) {
        const uint32_t t0 = c0 + s * FCHUNK, len = min((uint32_t)FCHUNK, seq - t0);
        {
            // partial q.k over this lane's 8 dims for its KT tokens, value
            // v G + g; then the totals over the DP lanes of each row
            constexpr int NV = KT * G;
            float dot[NV];
#pragma unroll
            for (int i = 0; i < NV; ++i) dot[i] = 0.f;
#pragma unroll
            for (int v = 0; v < KT; ++v) {
                const uint32_t wv[4] = {kr[v].x, kr[v].y, kr[v].z, kr[v].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float k0, k1;
                    unpack2<KVDT>(wv[e], k0, k1);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float q0 = QREG ? qr[QREG ? g : 0][2 * e] : qs[g][dp * 8 + 2 * e];
                        const float q1 = QREG ? qr[QREG ? g : 0][2 * e + 1] : qs[g][dp * 8 + 2 * e + 1];
                        dot[v * G + g] = fmaf(q1, k1, fmaf(q0, k0, dot[v * G + g]));
                    }
                }
            }
            group_multi_sum<NV, DP>(dot);
            constexpr int NF = NV >= DP ? NV / DP : 1;          // totals per lane
            constexpr int LB = DP == 16 ? 4 : 3;
            constexpr int H = NV >= DP ? LB : (NV == 1 ? 0 : (NV == 2 ? 1 : (NV == 4 ? 2 : 3)));
            const int prefix = dp >> (LB - H);
            if ((dp & ((DP >> H) - 1)) == 0) {
#pragma unroll
                for (int jj = 0; jj < NF; ++jj) {
                    const int k = prefix * NF + jj, v = k / G, g = k % G;
                    const uint32_t t = (uint32_t)(v * TG + tg);
                    ps[g][t] = t < len ? dot[jj] * a.scale : -INFINITY;
                }
            }
        }
        __syncthreads();
        // online softmax: every wave sees the whole sub-chunk (one token per
        // lane) and computes the same running max and sum
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float sc = ps[g][lane];
            const float mn = fmaxf(m_run[g], wave_max(sc));
            alpha[g] = expf(m_run[g] - mn);
            const float e = expf(sc - mn);
            if (tid < 64) pe[g][lane] = e;
            l_run[g] = fmaf(l_run[g], alpha[g], wave_sum(e));
            m_run[g] = mn;
        }
        __syncthreads();
        const bool plain = len == (uint32_t)FCHUNK;  // block-uniform
        if constexpr (VT) {
#pragma unroll
            for (int g = 0; g < G; ++g) o[g][0] *= alpha[g];
#pragma unroll
            for (int v = 0; v < VV4; ++v) {
                const uint32_t wv[4] = {vr[v].x, vr[v].y, vr[v].z, vr[v].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = vpart * VTOK + v * 8 + 2 * e;
                    float v0, v1;
                    unpack2<KVDT>(wv[e], v0, v1);
                    if (!plain) {  // past the end: weight 0 and value 0 (never NaN * 0)
                        v0 = (uint32_t)t < len ? v0 : 0.f;
                        v1 = (uint32_t)t + 1 < len ? v1 : 0.f;
                    }
#pragma unroll
                    for (int g = 0; g < G; ++g) o[g][0] = fmaf(pe[g][t + 1], v1, fmaf(pe[g][t], v0, o[g][0]));
                }
            }
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] *= alpha[g];
#pragma unroll
            for (int v = 0; v < VV4; ++v) {
                const int t = v * TG + tg;   // rows past the end are an in-range row, weight 0
                const uint32_t wv[4] = {vr[v].x, vr[v].y, vr[v].z, vr[v].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v0, v1;
                    unpack2<KVDT>(wv[e], v0, v1);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float p = pe[g][t];
                        o[g][2 * e] = fmaf(p, v0, o[g][2 * e]);
                        o[g][2 * e + 1] = fmaf(p, v1, o[g][2 * e + 1]);
                    }
                }
            }
        }
    };

    // Sub-chunks in pairs so the two register sets alternate without moves;
    // loads are never branched around (a clamped index re-reads the last
    // sub-chunk, from L2), only the compute of a missing odd step is skipped.
    for (uint32_t s = 0; s < ns; s += 2) {
        load(kB, vB, min(s + 1, ns - 1));
        compute(kA, vA, s);
        load(kA, vA, min(s + 2, ns - 1));
        if (s + 1 < ns) compute(kB, vB, s + 1);
    }

    // fold the partial P.V sums of the block
    if constexpr (VT) {
#pragma unroll
        for (int g = 0; g < G; ++g) ored[vpart][g][vd] = o[g][0];
    } else {
#pragma unroll
        for (int off = DP; off < 64; off <<= 1)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] += __shfl_xor(o[g][e], off, 64);
        if (lane < DP) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) ored[tid >> 6][g][dp * 8 + e] = o[g][e];
        }
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float s = 0.f;
#pragma unroll
        for (int p = 0; p < NRED; ++p) s += ored[p][g][d];
        if (a.nchunks == 1) {
            store_dt(a.out, (size_t)(qb + g) * D + d, s / l_run[g], a.odt);
        } else {
            const size_t slot = (size_t)(qb + g) * a.nchunks + c;
            a.part_o[slot * D + d] = s;
            if (d == 0) {
                a.part_ml[slot * 2] = m_run[g];
                a.part_ml[slot * 2 + 1] = l_run[g];
            }
        }
    }
}

// ------------------------------------ single-query attention, streaming --
// The single-query attention of attn_decode_kernel for head_dim 128 and 1 or
// 2 query heads per block, with every wave streaming its own tokens:
//   * the block's chunk is cut into 16-token groups; wave w takes groups
//     w, w + 4, ... and keeps its own online softmax (m, l, o), so the loop
//     has no block barrier;
//   * lane (row r = lane / 16, dp = lane % 16) reads the 16 bytes at dims
//     8 dp.. of tokens 4 v + r (v < 4) of a group: each wave instruction
//     reads 4 whole consecutive K (or row-major V) rows, 1 KB;
//   * q.k over the lane's 8 dims, the totals over the 16 lanes of a row by
//     exchange-halving; scores and probabilities go through a per-wave LDS
//     row (one 16-lane row per head for the max and the sum);
//   * P.V from registers (row-major V: the lane's 8 dims over its 4 tokens;
//     V transposed: dims lane and lane + 64 over the group's 16 tokens);
//   * the next group's loads are issued before the current one is used;
//   * the 4 waves' (m, l, o) are merged once at the end: the output (one
//     chunk) or the chunk's partials for the combine (launch_combine).
template <int G, int KVDT, bool VT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))   // <= 128 VGPRs: 4 blocks per CU
void attn_stream_kernel(DecAttnArgs a) {
    constexpr int D = 128, DP = 16, KT = 4, TPI = 16, NR = VT ? 1 : 4;
    static_assert(G == 1 || G == 2, "one or two query heads per block");
    __shared__ float qs[G][D];
    __shared__ float pw[4][G][TPI];
    __shared__ float wml[4][G][2];
    __shared__ float wo[4][NR][G][D];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int row = lane >> 4, dp = lane & 15;
    const uint32_t bid = blockIdx.x, span = 8 * a.parts;
    const uint32_t j = a.parts == 1 ? 0u : (bid % span) / 8;
    const uint32_t u = a.parts == 1 ? bid : (bid / span) * 8 + bid % 8;
    if (u >= a.units) return;
    const uint32_t c = u % a.nchunks, h = u / a.nchunks, qb = h * a.gfull + j * G;
    const uint32_t seq = a.d_seq ? *a.d_seq : a.seq_len;
    const uint32_t c0 = c * a.sub * FCHUNK;
    if (c0 >= seq) return;  // the combine step reads chunks < ceil(seq / chunk) only
    const uint32_t cend = min(c0 + a.sub * FCHUNK, seq);
    const uint32_t ngrp = ceil_div(cend - c0, (uint32_t)TPI);
    const uint32_t nit = ngrp > (uint32_t)w ? ceil_div(ngrp - (uint32_t)w, 4u) : 0u;

    float qv = 0.f;
    if (tid < G * D) qv = load_dt(a.q, (size_t)qb * D + tid, a.qdt);

    const size_t kv_stride = (size_t)a.max_ctx * D;
    const uint16_t *kb = a.kc + h * kv_stride, *vb = a.vc + h * kv_stride;
    // group of this wave's iteration i: past its last group it re-reads the
    // last one (a wave without groups reads group 0), so loads stay in range
    auto grp = [&](uint32_t i) -> uint32_t {
        const uint32_t gi = (uint32_t)w + 4u * i;
        return gi < ngrp ? gi : (nit ? (uint32_t)w + 4u * (nit - 1) : 0u);
    };
    auto load = [&](uint4 (&kr)[KT], uint4 (&vr)[4], uint32_t i) {
        const uint32_t t0 = c0 + grp(i) * TPI, len = min((uint32_t)TPI, cend - t0);
#pragma unroll
        for (int v = 0; v < KT; ++v) {
            const uint32_t t = min((uint32_t)(4 * v + row), len - 1);
            kr[v] = *((const uint4 *)(kb + (size_t)(t0 + t) * D) + dp);
        }
        if constexpr (VT) {
            // dims lane and lane + 64, tokens t0.. in two 8-token halves (a
            // half past the end re-reads the first one; max_ctx % 8 == 0)
            const uint32_t t1 = len > 8 ? t0 + 8 : t0;
            const uint16_t *r0 = vb + (size_t)lane * a.max_ctx, *r1 = vb + (size_t)(lane + 64) * a.max_ctx;
            vr[0] = *(const uint4 *)(r0 + t0);
            vr[1] = *(const uint4 *)(r0 + t1);
            vr[2] = *(const uint4 *)(r1 + t0);
            vr[3] = *(const uint4 *)(r1 + t1);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t t = min((uint32_t)(4 * v + row), len - 1);
                vr[v] = *((const uint4 *)(vb + (size_t)(t0 + t) * D) + dp);
            }
        }
    };
    uint4 kA[KT], vA[4], kB[KT], vB[4];
    load(kA, vA, 0);

    // q (optionally RoPE-rotated at rope_pos) -> LDS -> this lane's 8 dims
    {
        float v = qv;
        if (a.rope_pos >= 0) {
            const float partner = __shfl_xor(v, 1, 64);  // all lanes take part
            v = rope_rotate(v, partner, tid % D, (uint32_t)a.rope_pos, D, a.rope_theta);
        }
        if (tid < G * D) qs[tid / D][tid % D] = v;
    }
    __syncthreads();
    float qr[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) qr[g][i] = qs[g][dp * 8 + i];

    float m_run[G], l_run[G];
    float o[G][VT ? 2 : 8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.f;
#pragma unroll
        for (int e = 0; e < (VT ? 2 : 8); ++e) o[g][e] = 0.f;
    }
    const int sg = (lane >> 4) % G;   // softmax: head of this lane's row

    auto compute = [&](const uint4 (&kr)[KT], const uint4 (&vr)[4], uint32_t i) {
        const uint32_t t0 = c0 + grp(i) * TPI, len = min((uint32_t)TPI, cend - t0);
        // scores: value v G + g = q_g . k of token 4 v + row over 8 dims
        constexpr int NV = KT * G;
        float dot[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) dot[k] = 0.f;
#pragma unroll
        for (int v = 0; v < KT; ++v) {
            const uint32_t wv[4] = {kr[v].x, kr[v].y, kr[v].z, kr[v].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float k0, k1;
                unpack2<KVDT>(wv[e], k0, k1);
#pragma unroll
                for (int g = 0; g < G; ++g)
                    dot[v * G + g] = fmaf(qr[g][2 * e + 1], k1, fmaf(qr[g][2 * e], k0, dot[v * G + g]));
            }
        }
        group_multi_sum<NV, DP>(dot);
        {   // lanes whose low 4 - H bits are 0 hold the total of value dp >> (4 - H)
            constexpr int H = NV == 4 ? 2 : 3;
            if ((dp & ((DP >> H) - 1)) == 0) {
                const int k = dp >> (4 - H), v = k / G, g = k % G;
                const uint32_t tt = (uint32_t)(4 * v + row);
                pw[w][g][tt] = tt < len ? dot[0] * a.scale : -INFINITY;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // online softmax, one 16-lane row per head (rows >= G repeat them)
        float alpha[G];
        {
            const float sc = pw[w][sg][dp];
            float mx = sc;
            mx = fmaxf(mx, dpp_move<DPP_XOR1>(mx, -INFINITY));
            mx = fmaxf(mx, dpp_move<DPP_XOR2>(mx, -INFINITY));
            mx = fmaxf(mx, dpp_move<DPP_ROW_HALF_MIRROR>(mx, -INFINITY));
            mx = fmaxf(mx, dpp_move<DPP_ROW_MIRROR>(mx, -INFINITY));
            const float mo = G == 1 ? m_run[0] : (sg == 0 ? m_run[0] : m_run[G - 1]);
            const float mn = fmaxf(mo, mx);
            const float e = expf(sc - mn);
            float rs = e;
            rs += dpp_move<DPP_XOR1>(rs, 0.f);
            rs += dpp_move<DPP_XOR2>(rs, 0.f);
            rs += dpp_move<DPP_ROW_HALF_MIRROR>(rs, 0.f);
            rs += dpp_move<DPP_ROW_MIRROR>(rs, 0.f);
            if (lane < 16 * G) pw[w][sg][dp] = e;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float mng = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mn), 16 * g));
                const float rsg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rs), 16 * g));
                alpha[g] = expf(m_run[g] - mng);
                l_run[g] = fmaf(l_run[g], alpha[g], rsg);
                m_run[g] = mng;
            }
        }
        __builtin_amdgcn_wave_barrier();
        if constexpr (VT) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                o[g][0] *= alpha[g];
                o[g][1] *= alpha[g];
            }
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const uint32_t w0[4] = {vr[hh].x, vr[hh].y, vr[hh].z, vr[hh].w};
                const uint32_t w1[4] = {vr[2 + hh].x, vr[2 + hh].y, vr[2 + hh].z, vr[2 + hh].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = 8 * hh + 2 * e;
                    float a0, a1, b0, b1;
                    unpack2<KVDT>(w0[e], a0, a1);
                    unpack2<KVDT>(w1[e], b0, b1);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float p0 = pw[w][g][t], p1 = pw[w][g][t + 1];
                        o[g][0] = fmaf(p1, a1, fmaf(p0, a0, o[g][0]));
                        o[g][1] = fmaf(p1, b1, fmaf(p0, b0, o[g][1]));
                    }
                }
            }
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] *= alpha[g];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t wv[4] = {vr[v].x, vr[v].y, vr[v].z, vr[v].w};
                float p[G];
#pragma unroll
                for (int g = 0; g < G; ++g) p[g] = pw[w][g][4 * v + row];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v0, v1;
                    unpack2<KVDT>(wv[e], v0, v1);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        o[g][2 * e] = fmaf(p[g], v0, o[g][2 * e]);
                        o[g][2 * e + 1] = fmaf(p[g], v1, o[g][2 * e + 1]);
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();   // the next group rewrites pw[w]
    };

    // group i + 1 in flight while group i is computed.  The loads in the
    // loop are unconditional (past the wave's last group they re-read it):
    // skipping them by branches leaves the compiler a full wait at every
    // join (L = 32768 27.8 -> 30.0 us); a third register set with two
    // groups in flight measured slower too (29.0 us).  A wave with one
    // group (short chunks) loads it alone.
    if (nit <= 1) {
        if (nit == 1) compute(kA, vA, 0);
    } else {
        for (uint32_t i = 0; i < nit; i += 2) {
            load(kB, vB, i + 1);
            compute(kA, vA, i);
            load(kA, vA, i + 2);
            if (i + 1 < nit) compute(kB, vB, i + 1);
        }
    }

    // the 4 waves' states -> one (m, l, o) per query head
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            wml[w][g][0] = m_run[g];
            wml[w][g][1] = l_run[g];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if constexpr (VT) {
            wo[w][0][g][lane] = o[g][0];
            wo[w][0][g][lane + 64] = o[g][1];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) wo[w][row][g][dp * 8 + e] = o[g][e];
        }
    }
    __syncthreads();
    if (tid < G * D) {
        const int g = tid / D, d = tid % D;
        float M = wml[0][g][0];
#pragma unroll
        for (int k = 1; k < 4; ++k) M = fmaxf(M, wml[k][g][0]);
        float s = 0.f, l = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // a wave without tokens has m = -inf, l = 0, o = 0: weight 0
            const float sc = expf(wml[k][g][0] - M);
            float ok = 0.f;
#pragma unroll
            for (int r = 0; r < NR; ++r) ok += wo[k][r][g][d];
            s = fmaf(sc, ok, s);
            l = fmaf(sc, wml[k][g][1], l);
        }
        if (a.nchunks == 1) {
            store_dt(a.out, (size_t)(qb + g) * D + d, s / l, a.odt);
        } else {
            const size_t slot = (size_t)(qb + g) * a.nchunks + c;
            a.part_o[slot * D + d] = s;
            if (d == 0) {
                a.part_ml[slot * 2] = M;
                a.part_ml[slot * 2 + 1] = l;
            }
        }
    }
}

// -------------------------------------------------------------- embedding --
// transformer.metal:428-481: flat bit index row*hidden + d, group flat/gs.
__global__ void embed_q1_kernel(const uint32_t *ids, const uint8_t *bits, const uint16_t *scales,
                                float *out, uint32_t hidden, uint32_t ntok, uint32_t gs,
                                uint32_t vocab) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= ntok * hidden) return;
    const uint32_t t = gid / hidden, d = gid % hidden;
    uint32_t row = ids[t];
    if (row >= vocab) row = vocab - 1;  // the host validates ids; never read out of bounds
    const uint64_t flat = (uint64_t)row * hidden + d;
    const bool bit = (bits[flat >> 3] >> (flat & 7)) & 1;
    const float s = (float)__builtin_bit_cast(f16_t, scales[flat / gs]);
    out[gid] = bit ? s : -s;
}

// transformer.metal:505-549 embedding_lookup_q4 (BF16 scales/biases, output
// BF16-truncated).
__global__ void embed_q4_kernel(const uint32_t *ids, const uint32_t *words, const uint16_t *scales,
                                const uint16_t *biases, float *out, uint32_t hidden, uint32_t ntok,
                                uint32_t gs, uint32_t vocab) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= ntok * hidden) return;
    const uint32_t t = gid / hidden, d = gid % hidden;
    uint32_t row = ids[t];
    if (row >= vocab) row = vocab - 1;
    const uint64_t flat = (uint64_t)row * hidden + d;
    const uint32_t n = (words[flat >> 3] >> ((flat & 7) * 4)) & 0xFu;
    const uint64_t g = flat / gs;
    out[gid] = bf16_trunc(bf16_to_f32(scales[g]) * (float)n + bf16_to_f32(biases[g]));
}

__global__ void embed_bf16_kernel(const uint32_t *ids, const uint16_t *table, float *out,
                                  uint32_t hidden, uint32_t ntok, uint32_t vocab) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= ntok * hidden) return;
    const uint32_t t = gid / hidden, d = gid % hidden;
    uint32_t row = ids[t];
    if (row >= vocab) row = vocab - 1;
    out[gid] = bf16_to_f32(table[(size_t)row * hidden + d]);
}

__global__ void residual_add_kernel(float *r, const float *a, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) r[i] += a[i];
}

// ----------------------------------------------------------------- argmax --
// First maximum wins (transformer.zig:3694-3707); NaN never wins.  One block
// of 1024 threads; also reports the runner-up value for margin logging.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *x, uint32_t n, uint32_t *oi,
                                                      float *ov) {
    __shared__ float sv[1024], sv2[1024];
    __shared__ uint32_t si[1024];
    float best = -INFINITY, second = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        if (v > best) { second = best; best = v; bi = i; }
        else if (v > second) second = v;
    }
    sv[threadIdx.x] = best; sv2[threadIdx.x] = second; si[threadIdx.x] = bi;
    __syncthreads();
    for (uint32_t s = 512; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const float a = sv[threadIdx.x], b = sv[threadIdx.x + s];
            const uint32_t ia = si[threadIdx.x], ib = si[threadIdx.x + s];
            const bool take_b = (b > a) || (b == a && ib < ia);
            const float lo = take_b ? a : b;
            const float s2 = fmaxf(fmaxf(sv2[threadIdx.x], sv2[threadIdx.x + s]), lo);
            sv[threadIdx.x] = take_b ? b : a;
            si[threadIdx.x] = take_b ? ib : ia;
            sv2[threadIdx.x] = s2;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        oi[0] = si[0] == 0xFFFFFFFFu ? 0u : si[0];
        if (ov) { ov[0] = sv[0]; ov[1] = sv2[0]; }
    }
}

// ---------------------------------------------------------------- dequant --
__global__ void dequant_kernel(const uint32_t *codes, const uint16_t *scales, const uint16_t *biases,
                               float *out, uint32_t M, uint32_t K, uint32_t gs, int bits, int sdt) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)M * K) return;
    const uint64_t r = gid / K, c = gid % K;
    const uint64_t g = r * (K / gs) + c / gs;
    if (bits == 1) {
        const uint32_t w = codes[r * (K / 32) + c / 32];
        const float s = (float)__builtin_bit_cast(f16_t, scales[g]);
        out[gid] = ((w >> (c & 31)) & 1) ? s : -s;
    } else {
        const uint32_t w = codes[r * (K / 8) + c / 8];
        const float n = (float)((w >> ((c & 7) * 4)) & 0xFu);
        out[gid] = fmaf(scale_to_f32(scales[g], sdt), n, scale_to_f32(biases[g], sdt));
    }
}

inline uint32_t grid1d(uint64_t n, uint32_t block) { return (uint32_t)((n + block - 1) / block); }

}  // namespace

// ---------------------------------------------------------------------------
// Attention host helpers shared with the model code.
// ---------------------------------------------------------------------------

// Choose the chunk length: small enough to give >= ~2 blocks per CU at long
// context, >= 64 tokens, a multiple of 8, and <= ATT_MAX_CHUNK.
uint32_t nnz_attn_chunk(uint32_t seq_len, uint32_t hkv) {
    const uint32_t want_blocks = 512;
    const uint32_t per = ceil_div(seq_len * hkv, want_blocks);
    uint32_t chunk = 64;
    while (chunk < per && chunk < (uint32_t)ATT_MAX_CHUNK) chunk <<= 1;
    return chunk;
}

size_t nnz_attn_scratch_bytes_impl(uint32_t hq, uint32_t head_dim, uint32_t seq_len,
                                   uint32_t hkv) {
    // the fused decode path splits into FCHUNK-token chunks, the split
    // kernel into nnz_attn_chunk ones (never shorter): size for the former
    const uint32_t nch = ceil_div(seq_len, (uint32_t)FCHUNK);
    (void)hkv;
    // partial outputs + (m, l) pairs + one f32 q buffer for the fused path
    return ((size_t)hq * nch * head_dim + (size_t)hq * nch * 2 + (size_t)hq * head_dim) * 4 + 256;
}

// Few chunks: one wave per (query head, query, 64 dims), lane = dim,
// no barrier: every lane reads the chunks' (m, l) pairs (wave-uniform
// addresses) and its dim of each partial, all issued before the first is
// used, and folds them itself -- one memory round trip.
template <int D>
__global__ __launch_bounds__(64) void attn_combine_wave_kernel(AttnArgs a) {
    constexpr int U = 16;   // chunks per batch of loads (one batch up to 16 chunks)
    const uint32_t qh = blockIdx.x, z = blockIdx.y / (D / 64), d = (blockIdx.y % (D / 64)) * 64 + threadIdx.x;
    const size_t base = ((size_t)z * a.hq + qh) * a.nchunks;
    const float2 *ml = (const float2 *)(a.part_ml + base * 2);
    const float *po = a.part_o + base * D + d;
    const uint32_t seq = (a.d_seq ? *a.d_seq : a.seq_len) + z;
    const uint32_t nch = min(a.nchunks, ceil_div(seq, a.chunk));
    // online fold: running maximum, rescaled sums
    float m = -INFINITY, num = 0.f, den = 0.f;
    for (uint32_t c0 = 0; c0 < nch; c0 += U) {
        float2 mlc[U];
        float oc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t c = c0 + (uint32_t)u < nch ? c0 + (uint32_t)u : 0u;
            mlc[u] = ml[c];
            oc[u] = po[(size_t)c * D];
        }
        float mb = m;
#pragma unroll
        for (int u = 0; u < U; ++u) mb = c0 + (uint32_t)u < nch ? fmaxf(mb, mlc[u].x) : mb;
        const float sc = m == -INFINITY ? 0.f : expf(m - mb);
        num *= sc;
        den *= sc;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // past the live count: weight 0 by selection (never NaN * 0)
            const bool live = c0 + (uint32_t)u < nch;
            const float w = expf(mlc[u].x - mb);
            den = live ? fmaf(w, mlc[u].y, den) : den;
            num = live ? fmaf(w, oc[u], num) : num;
        }
        m = mb;
    }
    store_dt(a.out, (size_t)z * a.o_stride + (size_t)qh * D + d, num / den, a.odt);
}

// More chunks: one wave per (query head, query, 8 dims), lane = chunk (64
// per pass), no barrier: a lane loads its chunk's (m, l) pair and the
// slice's 8 partial values (two 16-byte loads), all issued before any is
// used; the maximum is a wave reduction, and the exp-sum and the 8 weighted
// sums are one exchange-halving reduction, whose 8 slots land in lanes 8 k
// (slot multi_row_slot<8>) and are stored from there.  Over 64 chunks each
// lane folds its chunks c, c + 64, ... after a first pass for the maximum.
// Hq * D / 8 waves: 256 for 16 heads of 128.
template <int D>
__global__ __launch_bounds__(64) void attn_combine_slice_kernel(AttnArgs a) {
    constexpr int SL = D / 8;   // slices per head
    const uint32_t lane = threadIdx.x;
    const uint32_t qh = blockIdx.x, z = blockIdx.y / SL, d0 = (blockIdx.y % SL) * 8;
    const size_t base = ((size_t)z * a.hq + qh) * a.nchunks;
    const float2 *ml = (const float2 *)(a.part_ml + base * 2);
    const float4 *po = (const float4 *)(a.part_o + base * D + d0);
    const uint32_t last = a.nchunks - 1;
    const uint32_t c0 = min(lane, last);
    const float2 m0 = ml[c0];
    const float4 oa = po[(size_t)c0 * (D / 4)], ob = po[(size_t)c0 * (D / 4) + 1];
    const uint32_t seq = (a.d_seq ? *a.d_seq : a.seq_len) + z;
    const uint32_t nch = min(a.nchunks, ceil_div(seq, a.chunk));

    float m = lane < nch ? m0.x : -INFINITY;
    for (uint32_t c = lane + 64; c < nch; c += 64) m = fmaxf(m, ml[c].x);
    const float M = wave_max(m);
    // past the live count: weight 0 by selection (never NaN * 0)
    const bool live = lane < nch;
    const float w0 = expf(m0.x - M);
    float v[9] = {live ? w0 * m0.y : 0.f,
                  live ? w0 * oa.x : 0.f, live ? w0 * oa.y : 0.f,
                  live ? w0 * oa.z : 0.f, live ? w0 * oa.w : 0.f,
                  live ? w0 * ob.x : 0.f, live ? w0 * ob.y : 0.f,
                  live ? w0 * ob.z : 0.f, live ? w0 * ob.w : 0.f};
    for (uint32_t c = lane + 64; c < nch; c += 64) {
        const float2 mc = ml[c];
        const float4 xa = po[(size_t)c * (D / 4)], xb = po[(size_t)c * (D / 4) + 1];
        const float w = expf(mc.x - M);
        v[0] = fmaf(w, mc.y, v[0]);
        v[1] = fmaf(w, xa.x, v[1]); v[2] = fmaf(w, xa.y, v[2]);
        v[3] = fmaf(w, xa.z, v[3]); v[4] = fmaf(w, xa.w, v[4]);
        v[5] = fmaf(w, xb.x, v[5]); v[6] = fmaf(w, xb.y, v[6]);
        v[7] = fmaf(w, xb.z, v[7]); v[8] = fmaf(w, xb.w, v[8]);
    }
    const float den = wave_sum(v[0]);
    const float num[8] = {v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8]};
    const float t = multi_row_sum<8>(num);
    if ((lane & 7) == 0)
        store_dt(a.out, (size_t)z * a.o_stride + (size_t)qh * D + d0 + multi_row_slot<8>(), t / den, a.odt);
}

template <int D>
static void launch_combine(nnz_ctx *ctx, const AttnArgs &a, uint32_t nq) {
    // measured at config 4: L = 512 (8 chunks) 7.49 -> 7.18 us with the
    // one-wave form; more chunks take a wave per 8-dim slice
    if (a.nchunks <= 8)
        attn_combine_wave_kernel<D><<<dim3(a.hq, nq * (D / 64)), 64, 0, ctx->stream>>>(a);
    else
        attn_combine_slice_kernel<D><<<dim3(a.hq, nq * (D / 8)), 64, 0, ctx->stream>>>(a);
}

template <int D, int G, int KVDT, bool VT>
static int launch_attn_t(nnz_ctx *ctx, const AttnArgs &a, uint32_t hkv, uint32_t nq) {
    dim3 grid(a.nchunks, hkv, nq);
    attn_split_kernel<D, G, KVDT, VT><<<grid, 256, 0, ctx->stream>>>(a);
    NNZ_LAUNCHED(ctx);
    if (a.nchunks > 1) {
        launch_combine<D>(ctx, a, nq);
        NNZ_LAUNCHED(ctx);
    }
    return NNZ_OK;
}

template <int D, int G>
static int launch_attn_g(nnz_ctx *ctx, const AttnArgs &a, uint32_t hkv, uint32_t nq, int kvdt, bool vt) {
    if (kvdt == NNZ_F16)
        return vt ? launch_attn_t<D, G, NNZ_F16, true>(ctx, a, hkv, nq)
                  : launch_attn_t<D, G, NNZ_F16, false>(ctx, a, hkv, nq);
    return vt ? launch_attn_t<D, G, NNZ_BF16, true>(ctx, a, hkv, nq)
              : launch_attn_t<D, G, NNZ_BF16, false>(ctx, a, hkv, nq);
}

template <int D>
static int launch_attn_d(nnz_ctx *ctx, const AttnArgs &a, uint32_t hkv, uint32_t nq, uint32_t g, int kvdt,
                         bool vt) {
    switch (g) {
    case 1: return launch_attn_g<D, 1>(ctx, a, hkv, nq, kvdt, vt);
    case 2: return launch_attn_g<D, 2>(ctx, a, hkv, nq, kvdt, vt);
    case 4: return launch_attn_g<D, 4>(ctx, a, hkv, nq, kvdt, vt);
    default: return launch_attn_g<D, 8>(ctx, a, hkv, nq, kvdt, vt);
    }
}

// Full-control attention launch used by the public entry points and by the
// decoder (prefill: nq causal queries; decode graph: seq_len read from d_seq).
static int attn_validate(nnz_ctx *ctx, const NnzAttnCall &c) {
    const nnz_gqa_dims &d = c.dims;
    NNZ_REQUIRE(ctx, c.q && c.kc && c.vc && c.out && c.part_o && c.part_ml, NNZ_EINVAL,
                "gqa: null buffer");
    NNZ_REQUIRE(ctx, d.num_query_heads > 0 && d.num_kv_heads > 0 && (d.seq_len > 0 || c.d_seq),
                NNZ_EINVAL, "gqa: zero dims");
    NNZ_REQUIRE(ctx, d.num_query_heads % d.num_kv_heads == 0 &&
                         d.heads_per_kv_group == d.num_query_heads / d.num_kv_heads,
                NNZ_EINVAL, "gqa: heads_per_kv_group mismatch");
    NNZ_REQUIRE(ctx, d.heads_per_kv_group == 1 || d.heads_per_kv_group == 2 ||
                         d.heads_per_kv_group == 4 || d.heads_per_kv_group == 8,
                NNZ_EUNSUPPORTED, "gqa: heads_per_kv_group %u (supported: 1, 2, 4, 8)",
                d.heads_per_kv_group);
    NNZ_REQUIRE(ctx, d.head_dim == 64 || d.head_dim == 128, NNZ_EUNSUPPORTED,
                "gqa: head_dim %u (supported: 64, 128)", d.head_dim);
    NNZ_REQUIRE(ctx, d.max_context_length % 8 == 0, NNZ_EUNSUPPORTED,
                "gqa: max_context_length must be a multiple of 8");
    NNZ_REQUIRE(ctx, nnz_dtype_ok(c.qdt) && nnz_dtype_ok(c.odt) &&
                         (c.kvdt == NNZ_F16 || c.kvdt == NNZ_BF16),
                NNZ_EINVAL, "gqa: bad dtype");
    NNZ_REQUIRE(ctx, ((uintptr_t)c.kc & 15) == 0 && ((uintptr_t)c.vc & 15) == 0, NNZ_EINVAL,
                "gqa: caches must be 16-byte aligned");
    NNZ_REQUIRE(ctx, ((uintptr_t)c.part_o & 15) == 0 && ((uintptr_t)c.part_ml & 7) == 0, NNZ_EINVAL,
                "gqa: partial buffers must be 16-byte (o) and 8-byte (m, l) aligned");
    return NNZ_OK;
}

int nnz_attn_launch_ex(nnz_ctx *ctx, const NnzAttnCall &c) {
    const nnz_gqa_dims &d = c.dims;
    if (int rc = attn_validate(ctx, c)) return rc;
    NNZ_REQUIRE(ctx, c.chunk >= 8 && c.chunk % 8 == 0 && c.chunk <= (uint32_t)ATT_MAX_CHUNK &&
                         c.nchunks >= 1 && c.nq >= 1,
                NNZ_EINVAL, "gqa: bad chunking");
    NNZ_REQUIRE(ctx, c.d_seq || ((uint64_t)d.seq_len + c.nq - 1 <= d.max_context_length &&
                                 (uint64_t)d.seq_len + c.nq - 1 <= (uint64_t)c.chunk * c.nchunks),
                NNZ_EINVAL, "gqa: sequence exceeds max_context_length or the chunk plan");
    AttnArgs a{};
    a.q = c.q;
    a.kc = c.kc;
    a.vc = c.vc;
    a.out = c.out;
    a.part_o = c.part_o;
    a.part_ml = c.part_ml;
    a.d_seq = c.d_seq;
    a.seq_len = d.seq_len;
    a.max_ctx = d.max_context_length;
    a.chunk = c.chunk;
    a.nchunks = c.nchunks;
    a.hq = d.num_query_heads;
    a.q_stride = c.q_stride ? c.q_stride : d.num_query_heads * d.head_dim;
    a.o_stride = c.o_stride ? c.o_stride : d.num_query_heads * d.head_dim;
    a.qdt = c.qdt;
    a.odt = c.odt;
    a.rope_pos = c.rope_pos;
    a.rope_theta = c.rope_theta;
    a.scale = 1.0f / sqrtf((float)d.head_dim);
    if (d.head_dim == 128)
        return launch_attn_d<128>(ctx, a, d.num_kv_heads, c.nq, d.heads_per_kv_group, c.kvdt, c.vt);
    return launch_attn_d<64>(ctx, a, d.num_kv_heads, c.nq, d.heads_per_kv_group, c.kvdt, c.vt);
}

// Single-query launch with the partials carved out of a caller scratch buffer.
int nnz_attn_launch(nnz_ctx *ctx, const void *q, int qdt, const void *kc, const void *vc, int kvdt,
                    bool vt, void *out, int odt, void *scratch, size_t scratch_bytes,
                    int32_t rope_pos, float theta, const nnz_gqa_dims &d) {
    NNZ_REQUIRE(ctx, d.num_kv_heads > 0 && d.seq_len > 0 && d.seq_len <= d.max_context_length,
                NNZ_EINVAL, "gqa: bad seq_len/num_kv_heads");
    const size_t need = nnz_attn_scratch_bytes_impl(d.num_query_heads, d.head_dim, d.seq_len,
                                                    d.num_kv_heads);
    NNZ_REQUIRE(ctx, scratch && scratch_bytes >= need, NNZ_EINVAL,
                "gqa: scratch of %zu bytes needed, %zu given", need, scratch_bytes);
    // chunks of `sub` x FCHUNK tokens: sub doubles (up to 8) while at least
    // NNZ_DEC_TARGET_BLOCKS (chunk, KV head) units remain, so long contexts
    // keep every CU busy with few partials to combine.  The streaming kernel
    // (head_dim 128, <= 2 query heads per KV head) does best with about one
    // unit per CU and long chunks (sub up to 32; measured at L = 4096: 11.1
    // -> 9.2 us, at L = 32768: 29.7 -> 29.0 us).
    const bool stream_shape = d.head_dim == 128 && d.heads_per_kv_group <= 2;
    const uint32_t target = stream_shape ? 256u : NNZ_DEC_TARGET_BLOCKS, max_sub = stream_shape ? 32u : 8u;
    const uint32_t nch64 = ceil_div(d.seq_len, (uint32_t)FCHUNK);
    uint32_t sub = 1;
    while (sub < max_sub && (uint64_t)ceil_div(nch64, 2 * sub) * d.num_kv_heads >= target) sub *= 2;
    NnzAttnCall c{};
    c.q = q;
    c.qdt = qdt;
    c.kc = kc;
    c.vc = vc;
    c.kvdt = kvdt;
    c.vt = vt;
    c.out = out;
    c.odt = odt;
    c.chunk = sub * FCHUNK;
    c.nchunks = ceil_div(nch64, sub);  // <= the ceil(seq / FCHUNK) the scratch is sized for
    float *base = (float *)(((uintptr_t)scratch + 255) & ~(uintptr_t)255);
    c.part_o = base;
    c.part_ml = base + (size_t)d.num_query_heads * c.nchunks * d.head_dim;
    c.nq = 1;
    c.rope_pos = rope_pos;
    c.rope_theta = theta;
    c.dims = d;
    if (int rc = attn_validate(ctx, c)) return rc;

    const uint32_t G = d.heads_per_kv_group;
    DecAttnArgs a{};
    a.q = q;
    a.kc = (const uint16_t *)kc;
    a.vc = (const uint16_t *)vc;
    a.out = out;
    a.part_o = c.part_o;
    a.part_ml = c.part_ml;
    a.d_seq = nullptr;
    a.seq_len = d.seq_len;
    a.max_ctx = d.max_context_length;
    a.nchunks = c.nchunks;
    a.sub = sub;
    a.gfull = G;
    a.units = c.nchunks * d.num_kv_heads;
    // few units leave CUs idle: split each KV group over blocks of one query head
    const uint32_t gb = a.units < 128 ? 1u : G;
    a.parts = G / gb;
    a.rope_pos = rope_pos;
    a.qdt = qdt;
    a.odt = odt;
    a.rope_theta = theta;
    a.scale = 1.0f / sqrtf((float)d.head_dim);
    const uint32_t blocks = a.parts == 1 ? a.units : ceil_div(a.units, 8u) * 8u * a.parts;
#define DEC(DD, GG, KK, VV) attn_decode_kernel<DD, GG, KK, VV><<<blocks, 256, 0, ctx->stream>>>(a)
#define DEC_KV(DD, GG)                                                       \
    do {                                                                     \
        if (kvdt == NNZ_F16) { if (vt) DEC(DD, GG, NNZ_F16, true); else DEC(DD, GG, NNZ_F16, false); } \
        else { if (vt) DEC(DD, GG, NNZ_BF16, true); else DEC(DD, GG, NNZ_BF16, false); }             \
    } while (0)
#define DEC_G(DD)                                                            \
    do {                                                                     \
        switch (gb) {                                                        \
        case 1: DEC_KV(DD, 1); break;                                        \
        case 2: DEC_KV(DD, 2); break;                                        \
        case 4: DEC_KV(DD, 4); break;                                        \
        default: DEC_KV(DD, 8); break;                                       \
        }                                                                    \
    } while (0)
    if (d.head_dim == 128 && gb <= 2) {
#define STR(GG)                                                                                         \
    do {                                                                                                \
        if (kvdt == NNZ_F16) {                                                                          \
            if (vt) attn_stream_kernel<GG, NNZ_F16, true><<<blocks, 256, 0, ctx->stream>>>(a);          \
            else attn_stream_kernel<GG, NNZ_F16, false><<<blocks, 256, 0, ctx->stream>>>(a); \
        } else {                                                                                        \
            if (vt) attn_stream_kernel<GG, NNZ_BF16, true><<<blocks, 256, 0, ctx->stream>>>(a);         \
            else attn_stream_kernel<GG, NNZ_BF16, false><<<blocks, 256, 0, ctx->stream>>>(a); \
        }                                                                                               \
    } while (0)
        if (gb == 1) STR(1);
        else STR(2);
#undef STR
    } else if (d.head_dim == 128) {
        DEC_G(128);
    } else {
        DEC_G(64);
    }
#undef DEC_G
#undef DEC_KV
#undef DEC
    NNZ_LAUNCHED(ctx);
    if (a.nchunks > 1) {
        AttnArgs m{};
        m.out = out;
        m.part_o = c.part_o;
        m.part_ml = c.part_ml;
        m.seq_len = d.seq_len;
        m.chunk = c.chunk;
        m.nchunks = c.nchunks;
        m.hq = d.num_query_heads;
        m.o_stride = d.num_query_heads * d.head_dim;
        m.odt = odt;
        if (d.head_dim == 128) launch_combine<128>(ctx, m, 1);
        else launch_combine<64>(ctx, m, 1);
        NNZ_LAUNCHED(ctx);
    }
    return NNZ_OK;
}

// Chunk length of the fused decode attention (fixed: the kernel prefetches
// a whole chunk into registers).
uint32_t nnz_attn_fused_chunk(uint32_t, uint32_t) { return (uint32_t)FCHUNK; }

// Fused decode attention (see attn_fused_kernel).  `max_seq` sizes the grid;
// the live seq_len is d_seq ? *d_seq : max_seq.  part_o / part_ml hold
// Hq * nchunks partials for the chunk from nnz_attn_fused_chunk.
int nnz_attn_fused1_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                           const float *qn, const float *kn, void *kc, void *vc, void *out,
                           float *part_o, float *part_ml, const uint32_t *d_seq, uint32_t max_seq,
                           uint32_t hq, uint32_t hkv, uint32_t head_dim, uint32_t max_ctx, float eps,
                           float theta, const float *inv_freq, bool partials_only) {
    NNZ_REQUIRE(ctx, q && kr && vr && qn && kn && kc && vc && (out || partials_only) && part_o && part_ml,
                NNZ_EINVAL, "gqa_fused_1pass: null buffer");
    NNZ_REQUIRE(ctx, hkv > 0 && hq % hkv == 0 && max_seq > 0 && max_seq <= max_ctx, NNZ_EINVAL,
                "gqa_fused_1pass: bad dims");
    NNZ_REQUIRE(ctx, head_dim == 64 || head_dim == 128, NNZ_EUNSUPPORTED,
                "gqa_fused_1pass: head_dim %u (supported: 64, 128)", head_dim);
    NNZ_REQUIRE(ctx, max_ctx % 8 == 0 && ((uintptr_t)kc & 15) == 0 && ((uintptr_t)vc & 15) == 0,
                NNZ_EUNSUPPORTED, "gqa_fused_1pass: caches must be 16-byte aligned, max_ctx %% 8 == 0");
    const uint32_t G = hq / hkv;
    FusedAttnArgs a{};
    a.q = (const f16_t *)q;
    a.kr = (const f16_t *)kr;
    a.vr = (const f16_t *)vr;
    a.qn = qn;
    a.kn = kn;
    a.kc = (f16_t *)kc;
    a.vc = (f16_t *)vc;
    a.out = (f16_t *)out;
    a.part_o = part_o;
    a.part_ml = part_ml;
    a.d_seq = d_seq;
    a.inv_freq = inv_freq;
    a.seq_len = max_seq;
    a.max_ctx = max_ctx;
    a.nchunks = ceil_div(max_seq, (uint32_t)FCHUNK);
    a.direct = a.nchunks == 1 && !partials_only;
    // partials for the O projection's merge: its unit-major layout
    a.unit_major = partials_only ? 1u : 0u;
    a.kdim = hq * head_dim;
    a.eps = eps;
    a.theta = theta;
    a.scale = 1.0f / sqrtf((float)head_dim);
    // Few chunks x KV heads leave CUs idle: split each KV group over blocks
    // of one query head, placed on one XCD so the K/V repeats hit its L2.
    a.gfull = G;
    const uint32_t gb = (a.nchunks * hkv < 128) ? 1u : G;
    a.units = a.nchunks * hkv;
    a.parts = G / gb;
    const dim3 grid(a.parts == 1 ? a.units : ceil_div(a.units, 8u) * 8u * a.parts);
#define FUSED(DD, GG) attn_fused_kernel<DD, GG><<<grid, 256, 0, ctx->stream>>>(a)
    if (gb == 1) {
        if (head_dim == 128) attn_fused_wave_kernel<<<grid, 256, 0, ctx->stream>>>(a);
        else FUSED(64, 1);
    } else if (head_dim == 128) {
        if (G == 2) FUSED(128, 2);
        else if (G == 4) FUSED(128, 4);
        else if (G == 8) FUSED(128, 8);
        else return nnz_fail(ctx, NNZ_EUNSUPPORTED, "gqa_fused_1pass: group %u", G);
    } else {
        if (G == 2) FUSED(64, 2);
        else if (G == 4) FUSED(64, 4);
        else if (G == 8) FUSED(64, 8);
        else return nnz_fail(ctx, NNZ_EUNSUPPORTED, "gqa_fused_1pass: group %u", G);
    }
#undef FUSED
    NNZ_LAUNCHED(ctx);
    if (a.nchunks > 1 && !partials_only) {
        attn_merge_kernel<<<hq, 128, 0, ctx->stream>>>(part_o, part_ml, (f16_t *)out, d_seq, max_seq,
                                                       a.nchunks, head_dim);
        NNZ_LAUNCHED(ctx);
    }
    return NNZ_OK;
}

// RoPE frequency table [head_dim / 2] (same values the kernels compute).
int nnz_rope_table_launch(nnz_ctx *ctx, float *out, uint32_t head_dim, float theta) {
    NNZ_REQUIRE(ctx, out && head_dim >= 2 && head_dim <= 256 && head_dim % 2 == 0, NNZ_EINVAL,
                "rope table: bad head_dim %u", head_dim);
    rope_table_kernel<<<1, 128, 0, ctx->stream>>>(out, head_dim, theta);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

// q buffer (f32) inside the attention scratch, used by the fused path.
float *nnz_attn_scratch_q(void *scratch, const nnz_gqa_dims &d) {
    // after the partials of the finest chunking any launcher uses (FCHUNK
    // tokens), as nnz_attn_scratch_bytes_impl sizes them
    const uint32_t nch = ceil_div(d.seq_len, (uint32_t)FCHUNK);
    float *base = (float *)(((uintptr_t)scratch + 255) & ~(uintptr_t)255);
    return base + (size_t)d.num_query_heads * nch * d.head_dim + (size_t)d.num_query_heads * nch * 2;
}

// Batched attention prologue: nq tokens at positions (d_pos ? *d_pos : pos) + z.
int nnz_attn_prep_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                         const float *qn, const float *kn, float *qout, void *kc, void *vc,
                         uint32_t hq, uint32_t hkv, uint32_t head_dim, uint32_t pos,
                         const uint32_t *d_pos, uint32_t nq, uint32_t max_ctx, float eps,
                         float theta) {
    attn_prep_kernel<<<dim3(hq + hkv, nq), 256, 0, ctx->stream>>>(
        (const f16_t *)q, (const f16_t *)kr, (const f16_t *)vr, qn, kn, qout, (f16_t *)kc,
        (f16_t *)vc, hq, hkv, head_dim, pos, d_pos, max_ctx, eps, theta);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_attn_prep_waves_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                               const float *qn, const float *kn, void *qout, void *kc, void *vc,
                               const float *inv_freq, uint32_t hq, uint32_t hkv, uint32_t head_dim,
                               uint32_t pos0, uint32_t nq, uint32_t max_ctx, float eps, float qsplit) {
    NNZ_REQUIRE(ctx, head_dim % 2 == 0 && head_dim <= 128, NNZ_EUNSUPPORTED,
                "attn_prep: head_dim %u (even, <= 128)", head_dim);
    // (KV head, 64-token group, 16-dim slice) units for V, then (token, head) units for q and k
    const uint32_t units = hkv * ceil_div(nq, 64u) * ceil_div(head_dim, 16u) + (hq + hkv) * nq;
    attn_prep_waves_kernel<<<ceil_div(units, 4u), 256, 0, ctx->stream>>>(
        (const f16_t *)q, (const f16_t *)kr, (const f16_t *)vr, qn, kn, qout, (f16_t *)kc,
        (f16_t *)vc, inv_freq, hq, hkv, head_dim, pos0, nq, max_ctx, eps, qsplit);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_argmax_launch(nnz_ctx *ctx, const float *x, uint32_t n, uint32_t *oi, float *ov) {
    argmax_kernel<<<1, 1024, 0, ctx->stream>>>(x, n, oi, ov);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

extern "C" {

int nnz_dispatch_rms_norm(nnz_ctx *ctx, const float *input, const float *scale, void *output,
                          int out_dtype, int trunc, nnz_rmsnorm_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, input && scale && output, NNZ_EINVAL, "rms_norm: null buffer");
    NNZ_REQUIRE(ctx, d.hidden_size > 0 && d.num_tokens > 0, NNZ_EINVAL, "rms_norm: zero dims");
    if (out_dtype == NNZ_F32 && !trunc)
        launch_rms_norm<NNZ_F32, false>(ctx, input, scale, output, d.hidden_size, d.num_tokens, d.eps);
    else if (out_dtype == NNZ_F16 && !trunc)
        launch_rms_norm<NNZ_F16, false>(ctx, input, scale, output, d.hidden_size, d.num_tokens, d.eps);
    else if (out_dtype == NNZ_F16 && trunc)
        launch_rms_norm<NNZ_F16, true>(ctx, input, scale, output, d.hidden_size, d.num_tokens, d.eps);
    else
        return nnz_fail(ctx, NNZ_EINVAL, "rms_norm: unsupported output variant");
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_silu(nnz_ctx *ctx, const float *input, float *output, uint32_t count) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, input && output && count > 0, NNZ_EINVAL, "silu: bad arguments");
    silu_kernel<<<grid1d(count, 256), 256, 0, ctx->stream>>>(input, output, count);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_silu_elementwise_mul(nnz_ctx *ctx, const void *gate, const void *up, void *output,
                                      int dtype, uint32_t count) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, gate && up && output && count > 0, NNZ_EINVAL, "silu_mul: bad arguments");
    if (dtype == NNZ_F32)
        silu_mul_kernel<NNZ_F32><<<grid1d(count, 256), 256, 0, ctx->stream>>>(gate, up, output, count);
    else if (dtype == NNZ_F16)
        silu_mul_kernel<NNZ_F16><<<grid1d(count, 256), 256, 0, ctx->stream>>>(gate, up, output, count);
    else
        return nnz_fail(ctx, NNZ_EINVAL, "silu_mul: dtype must be f32 or f16");
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_rope(nnz_ctx *ctx, void *data, int dtype, nnz_rope_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, data && d.num_heads > 0 && d.head_dim >= 2 && d.head_dim % 2 == 0, NNZ_EINVAL,
                "rope: bad arguments");
    const uint32_t n = d.num_heads * d.head_dim / 2;
    if (dtype == NNZ_F32)
        rope_kernel<NNZ_F32><<<grid1d(n, 256), 256, 0, ctx->stream>>>(data, d.num_heads, d.head_dim, d.position, d.rope_theta);
    else if (dtype == NNZ_F16)
        rope_kernel<NNZ_F16><<<grid1d(n, 256), 256, 0, ctx->stream>>>(data, d.num_heads, d.head_dim, d.position, d.rope_theta);
    else if (dtype == NNZ_BF16)
        rope_kernel<NNZ_BF16><<<grid1d(n, 256), 256, 0, ctx->stream>>>(data, d.num_heads, d.head_dim, d.position, d.rope_theta);
    else
        return nnz_fail(ctx, NNZ_EINVAL, "rope: bad dtype");
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_kv_cache_update(nnz_ctx *ctx, const void *k_proj, const void *v_proj, int pdt,
                                 void *k_cache, void *v_cache, int cdt, nnz_kv_update_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, k_proj && v_proj && k_cache && v_cache, NNZ_EINVAL, "kv_update: null buffer");
    NNZ_REQUIRE(ctx, d.num_kv_heads > 0 && d.head_dim > 0 && d.position < d.max_context_length,
                NNZ_EINVAL, "kv_update: bad dims");
    const uint32_t n = d.num_kv_heads * d.head_dim;
    const uint32_t g = grid1d(n, 256);
#define KVU(P, C) kv_update_kernel<P, C><<<g, 256, 0, ctx->stream>>>(k_proj, v_proj, k_cache, v_cache, d.num_kv_heads, d.head_dim, d.position, d.max_context_length)
    if (pdt == NNZ_F32 && cdt == NNZ_F16) KVU(NNZ_F32, NNZ_F16);
    else if (pdt == NNZ_F16 && cdt == NNZ_F16) KVU(NNZ_F16, NNZ_F16);
    else if (pdt == NNZ_F32 && cdt == NNZ_BF16) KVU(NNZ_F32, NNZ_BF16);
    else if (pdt == NNZ_BF16 && cdt == NNZ_BF16) KVU(NNZ_BF16, NNZ_BF16);
    else return nnz_fail(ctx, NNZ_EINVAL, "kv_update: unsupported dtype pair");
#undef KVU
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_fused_rope_kv_cache(nnz_ctx *ctx, const void *k_proj, const void *v_proj,
                                     void *k_cache, void *v_cache, nnz_fused_rope_kv_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, k_proj && v_proj && k_cache && v_cache, NNZ_EINVAL, "fused_rope_kv: null buffer");
    NNZ_REQUIRE(ctx, d.num_kv_heads > 0 && d.head_dim >= 2 && d.head_dim <= 256 && d.head_dim % 2 == 0 &&
                         d.position < d.max_context_length,
                NNZ_EINVAL, "fused_rope_kv: bad dims");
    fused_rope_kv_kernel<<<d.num_kv_heads, 256, 0, ctx->stream>>>(
        (const f16_t *)k_proj, (const f16_t *)v_proj, (f16_t *)k_cache, (f16_t *)v_cache, d.head_dim,
        d.position, d.max_context_length, d.rope_theta);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_fused_norm_rope(nnz_ctx *ctx, void *data, const float *scale,
                                 nnz_fused_norm_rope_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, data && scale, NNZ_EINVAL, "fused_norm_rope: null buffer");
    NNZ_REQUIRE(ctx, d.num_heads > 0 && d.head_dim >= 2 && d.head_dim <= 256 && d.head_dim % 2 == 0,
                NNZ_EINVAL, "fused_norm_rope: bad dims");
    fused_norm_rope_kernel<<<d.num_heads, 256, 0, ctx->stream>>>((f16_t *)data, scale, d.head_dim,
                                                                 d.position, d.eps, d.rope_theta);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_fused_k_norm_rope_kv_cache(nnz_ctx *ctx, const void *k_proj, const void *v_proj,
                                            void *k_cache, void *v_cache, const float *k_scale,
                                            nnz_fused_k_norm_rope_kv_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, k_proj && v_proj && k_cache && v_cache && k_scale, NNZ_EINVAL,
                "fused_k_norm_rope_kv: null buffer");
    NNZ_REQUIRE(ctx, d.num_kv_heads > 0 && d.head_dim >= 2 && d.head_dim <= 256 && d.head_dim % 2 == 0 &&
                         d.position < d.max_context_length,
                NNZ_EINVAL, "fused_k_norm_rope_kv: bad dims");
    fused_k_norm_rope_kv_kernel<<<d.num_kv_heads, 256, 0, ctx->stream>>>(
        (const f16_t *)k_proj, (const f16_t *)v_proj, (f16_t *)k_cache, (f16_t *)v_cache, k_scale,
        d.head_dim, d.position, d.max_context_length, d.eps, d.rope_theta);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

size_t nnz_gqa_scratch_bytes(nnz_gqa_dims d) {
    if (!d.num_kv_heads || !d.seq_len) return 0;
    return nnz_attn_scratch_bytes_impl(d.num_query_heads, d.head_dim, d.seq_len, d.num_kv_heads);
}

int nnz_dispatch_gqa_attention(nnz_ctx *ctx, const void *q, int q_dtype, const void *k_cache,
                               const void *v_cache, int kv_dtype, int v_transposed, void *output,
                               int out_dtype, void *scratch, size_t scratch_bytes,
                               int32_t rope_position, float rope_theta, nnz_gqa_dims dims) {
    NNZ_CHECK_CTX(ctx);
    return nnz_attn_launch(ctx, q, q_dtype, k_cache, v_cache, kv_dtype, v_transposed != 0, output,
                           out_dtype, scratch, scratch_bytes, rope_position, rope_theta, dims);
}

int nnz_dispatch_gqa_attention_fused(nnz_ctx *ctx, const void *q, void *k_cache, void *v_cache,
                                     void *output, const void *k_raw, const void *v_raw,
                                     const float *q_norm_scale, const float *k_norm_scale,
                                     void *scratch, size_t scratch_bytes, nnz_gqa_fused_dims fd) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, q && k_cache && v_cache && output && k_raw && v_raw && q_norm_scale && k_norm_scale,
                NNZ_EINVAL, "gqa_fused: null buffer");
    NNZ_REQUIRE(ctx, fd.position < fd.max_context_length && fd.seq_len == fd.position + 1, NNZ_EINVAL,
                "gqa_fused: seq_len must be position + 1 (< max_context_length)");
    nnz_gqa_dims d{fd.num_query_heads, fd.num_kv_heads, fd.head_dim, fd.seq_len,
                   fd.max_context_length, fd.heads_per_kv_group};
    const size_t need = nnz_gqa_scratch_bytes(d);
    NNZ_REQUIRE(ctx, scratch && scratch_bytes >= need, NNZ_EINVAL,
                "gqa_fused: scratch of %zu bytes needed", need);
    NNZ_REQUIRE(ctx, fd.head_dim == 64 || fd.head_dim == 128, NNZ_EUNSUPPORTED,
                "gqa_fused: head_dim %u (supported: 64, 128)", fd.head_dim);
    float *qf = nnz_attn_scratch_q(scratch, d);
    int rc = nnz_attn_prep_launch(ctx, q, k_raw, v_raw, q_norm_scale, k_norm_scale, qf, k_cache,
                                  v_cache, fd.num_query_heads, fd.num_kv_heads, fd.head_dim,
                                  fd.position, nullptr, 1, fd.max_context_length, fd.eps,
                                  fd.rope_theta);
    if (rc) return rc;
    return nnz_attn_launch(ctx, qf, NNZ_F32, k_cache, v_cache, NNZ_F16, true, output, NNZ_F16, scratch,
                           scratch_bytes, -1, fd.rope_theta, d);
}

int nnz_dispatch_gqa_attention_fused_1pass(nnz_ctx *ctx, const void *q, void *k_cache,
                                           void *v_cache, void *output, const void *k_raw,
                                           const void *v_raw, const float *q_norm_scale,
                                           const float *k_norm_scale, void *scratch,
                                           size_t scratch_bytes, const uint32_t *d_seq_len,
                                           nnz_gqa_fused_dims fd) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, fd.num_kv_heads > 0 && fd.seq_len > 0 && fd.seq_len <= fd.max_context_length,
                NNZ_EINVAL, "gqa_fused_1pass: bad seq_len");
    NNZ_REQUIRE(ctx, d_seq_len || fd.seq_len == fd.position + 1, NNZ_EINVAL,
                "gqa_fused_1pass: seq_len must be position + 1");
    NNZ_REQUIRE(ctx, fd.heads_per_kv_group * fd.num_kv_heads == fd.num_query_heads, NNZ_EINVAL,
                "gqa_fused_1pass: heads_per_kv_group mismatch");
    nnz_gqa_dims d{fd.num_query_heads, fd.num_kv_heads, fd.head_dim, fd.seq_len,
                   fd.max_context_length, fd.heads_per_kv_group};
    const size_t need = nnz_gqa_scratch_bytes(d);
    NNZ_REQUIRE(ctx, scratch && scratch_bytes >= need, NNZ_EINVAL,
                "gqa_fused_1pass: scratch of %zu bytes needed", need);
    const uint32_t chunk = nnz_attn_fused_chunk(fd.seq_len, fd.num_kv_heads);
    const uint32_t nch = ceil_div(fd.seq_len, chunk);
    float *base = (float *)(((uintptr_t)scratch + 255) & ~(uintptr_t)255);
    float *part_o = base;
    float *part_ml = base + (size_t)fd.num_query_heads * nch * fd.head_dim;
    return nnz_attn_fused1_launch(ctx, q, k_raw, v_raw, q_norm_scale, k_norm_scale, k_cache, v_cache,
                                  output, part_o, part_ml, d_seq_len, fd.seq_len,
                                  fd.num_query_heads, fd.num_kv_heads, fd.head_dim,
                                  fd.max_context_length, fd.eps, fd.rope_theta, nullptr);
}

uint32_t nnz_gqa_partial_chunks(uint32_t seq_len) { return ceil_div(seq_len, (uint32_t)FCHUNK); }

int nnz_dispatch_gqa_attention_partials(nnz_ctx *ctx, const void *q, void *k_cache, void *v_cache,
                                        const void *k_raw, const void *v_raw,
                                        const float *q_norm_scale, const float *k_norm_scale,
                                        const float *rope_inv_freq, float *part_o, float *part_ml,
                                        const uint32_t *d_seq_len, nnz_gqa_fused_dims fd) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, fd.num_kv_heads > 0 && fd.seq_len > 0 && fd.seq_len <= fd.max_context_length,
                NNZ_EINVAL, "gqa_partials: bad seq_len");
    NNZ_REQUIRE(ctx, d_seq_len || fd.seq_len == fd.position + 1, NNZ_EINVAL,
                "gqa_partials: seq_len must be position + 1");
    NNZ_REQUIRE(ctx, fd.heads_per_kv_group * fd.num_kv_heads == fd.num_query_heads, NNZ_EINVAL,
                "gqa_partials: heads_per_kv_group mismatch");
    NNZ_REQUIRE(ctx, ((uintptr_t)part_o & 15) == 0 && ((uintptr_t)part_ml & 7) == 0, NNZ_EINVAL,
                "gqa_partials: part_o must be 16-byte and part_ml 8-byte aligned");
    return nnz_attn_fused1_launch(ctx, q, k_raw, v_raw, q_norm_scale, k_norm_scale, k_cache, v_cache,
                                  nullptr, part_o, part_ml, d_seq_len, fd.seq_len, fd.num_query_heads,
                                  fd.num_kv_heads, fd.head_dim, fd.max_context_length, fd.eps,
                                  fd.rope_theta, rope_inv_freq, true);
}

int nnz_dispatch_embedding_lookup(nnz_ctx *ctx, const uint32_t *ids, const void *bits,
                                  const void *scales, float *out, nnz_embed_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, ids && bits && scales && out, NNZ_EINVAL, "embedding: null buffer");
    NNZ_REQUIRE(ctx, d.num_tokens > 0 && d.hidden_size > 0 && d.vocab_size > 0 && d.group_size > 0,
                NNZ_EINVAL, "embedding: zero dims");
    const uint32_t n = d.num_tokens * d.hidden_size;
    embed_q1_kernel<<<grid1d(n, 256), 256, 0, ctx->stream>>>(ids, (const uint8_t *)bits,
                                                            (const uint16_t *)scales, out,
                                                            d.hidden_size, d.num_tokens,
                                                            d.group_size, d.vocab_size);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_embedding_lookup_q4(nnz_ctx *ctx, const uint32_t *ids, const void *nibs,
                                     const void *scales, const void *biases, float *out,
                                     nnz_embed_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, ids && nibs && scales && biases && out, NNZ_EINVAL, "embedding_q4: null buffer");
    NNZ_REQUIRE(ctx, d.num_tokens > 0 && d.hidden_size > 0 && d.vocab_size > 0 && d.group_size > 0,
                NNZ_EINVAL, "embedding_q4: zero dims");
    const uint32_t n = d.num_tokens * d.hidden_size;
    embed_q4_kernel<<<grid1d(n, 256), 256, 0, ctx->stream>>>(
        ids, (const uint32_t *)nibs, (const uint16_t *)scales, (const uint16_t *)biases, out,
        d.hidden_size, d.num_tokens, d.group_size, d.vocab_size);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_embedding_lookup_bf16(nnz_ctx *ctx, const uint32_t *ids, const void *table,
                                       float *out, nnz_embed_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, ids && table && out, NNZ_EINVAL, "embedding_bf16: null buffer");
    NNZ_REQUIRE(ctx, d.num_tokens > 0 && d.hidden_size > 0 && d.vocab_size > 0, NNZ_EINVAL,
                "embedding_bf16: zero dims");
    const uint32_t n = d.num_tokens * d.hidden_size;
    embed_bf16_kernel<<<grid1d(n, 256), 256, 0, ctx->stream>>>(ids, (const uint16_t *)table, out,
                                                              d.hidden_size, d.num_tokens,
                                                              d.vocab_size);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_residual_add(nnz_ctx *ctx, float *residual, const float *addition, uint32_t count) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, residual && addition && count > 0, NNZ_EINVAL, "residual_add: bad arguments");
    residual_add_kernel<<<grid1d(count, 256), 256, 0, ctx->stream>>>(residual, addition, count);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int nnz_dispatch_argmax(nnz_ctx *ctx, const float *logits, uint32_t count, uint32_t *out_index,
                        float *out_value) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, logits && out_index && count > 0, NNZ_EINVAL, "argmax: bad arguments");
    return nnz_argmax_launch(ctx, logits, count, out_index, out_value);
}

int nnz_dispatch_dequant(nnz_ctx *ctx, const nnz_qweight *w, float *output, nnz_qmv_dims d) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, w && w->codes && w->scales && output, NNZ_EINVAL, "dequant: null buffer");
    NNZ_REQUIRE(ctx, d.M > 0 && d.K > 0 && d.group_size > 0 && d.K % d.group_size == 0, NNZ_EINVAL,
                "dequant: bad dims");
    NNZ_REQUIRE(ctx, (w->bits == 1 && d.K % 32 == 0) || (w->bits == 4 && d.K % 8 == 0 && w->biases),
                NNZ_EINVAL, "dequant: bad weight");
    NNZ_REQUIRE(ctx, (uint64_t)w->packed_count == (uint64_t)d.M * d.K && w->group_size == d.group_size,
                NNZ_EINVAL, "dequant: descriptor does not match dims");
    const uint64_t n = (uint64_t)d.M * d.K;
    dequant_kernel<<<grid1d(n, 256), 256, 0, ctx->stream>>>(
        (const uint32_t *)w->codes, (const uint16_t *)w->scales, (const uint16_t *)w->biases, output,
        d.M, d.K, d.group_size, (int)w->bits, (int)w->scale_dtype);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

}  // extern "C"

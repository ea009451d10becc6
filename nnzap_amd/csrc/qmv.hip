// Quantised matrix-vector products (batch-1 decode) for gfx950.
//
// One templated kernel covers every QMV variant of the reference:
//   Q1 (1-bit symmetric, +-s):  qmv_specialized.metal (9 kernels) and the
//       generic qmv/qmv_const family of compute.metal:1713-2945;
//   Q4 (4-bit affine, s*n+b):   q4mv_bf16_specialized.metal (9 kernels).
// Variants are template parameters: input dtype, one or two matrices sharing
// the input, an RMSNorm prologue reading the f32 residual, and the epilogue
// (store f32/f16, residual +=, silu(a)*b, BF16-faithful truncation).
//
// Work decomposition (wave64, not the reference's simdgroup-of-32 layout):
//   * A row is split into 32-column "units" (one u32 word for Q1, four u32
//     words = one 16-byte load for Q4).  LPR = lanes per row is the smallest
//     power of two >= units/row, capped at 64; a wave covers 64/LPR rows per
//     step and each lane owns NV units of every row it touches.
//   * Because a lane always owns the same columns, its slice of x (32*NV
//     floats) is loaded once into VGPRs, together with the per-unit sums of x,
//     and reused for every row the wave processes.  No LDS is used: the
//     RMSNorm prologue is a lane-group reduction in registers.
//   * Each lane keeps R row-steps of weight loads in flight.  Lanes of a row
//     read adjacent words, so every load instruction is a contiguous,
//     coalesced segment of the row.
//   * Row sums are reduced across the LPR lanes with cross-lane shuffles.
//
// Q1 arithmetic: sum_c (bit ? +x_c : -x_c) = 2 * sum_{bit=1} x_c - sum_c x_c,
// computed per 32-column unit with a sign-extended bit mask ANDed into x
// (3 VALU ops per weight), then scaled by the unit's group scale.
// Q4 arithmetic: acc += s * sum(n_i x_i) + b * sum(x_i) per unit
// (q4mv_bf16_specialized.metal:14-16), nibbles widened with the byte
// converts after splitting even/odd nibbles.
#include "common.h"

namespace {

enum { EPI_STORE = 0, EPI_RESADD = 1, EPI_SILU = 2 };

struct QmvArgs {
    const uint32_t *codes[2];
    const uint16_t *scales[2];
    const uint16_t *biases[2];
    const void *x;         // input vector (XDT) or f32 residual (NORM)
    const float *norm_w;   // f32 [K], NORM only
    void *out[2];
    uint32_t M, K, gs;
    uint32_t lpr_log2;     // lanes per row = 1 << lpr_log2
    uint32_t sdt;          // scale/bias dtype (NNZ_F16 / NNZ_BF16)
    float eps;
};

template <int BITS, int XDT, int NMAT, bool NORM, int EPI, int ODT, bool FAITH, int NV, int R>
__global__ __launch_bounds__(256) void qmv_kernel(QmvArgs a) {
    constexpr int VEC = (BITS == 1) ? 1 : 4;  // u32 words per 32-column unit
    const int lane = threadIdx.x & 63;
    const int lpr_log2 = (int)a.lpr_log2;
    const int LPR = 1 << lpr_log2;
    const int RPW = 64 >> lpr_log2;
    const int rr = lane >> lpr_log2;       // sub-row within the wave step
    const int ll = lane & (LPR - 1);       // lane within the row group
    const uint32_t K = a.K;
    const uint32_t units = K >> 5;          // 32-column units per row
    const uint32_t G = K / a.gs;            // groups per row
    const uint32_t words_per_row = units * VEC;

    // ---- x slice for the owned units, kept in registers -------------------
    float xr[NV][32];
    float xsum[NV];
    bool uvalid[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t u = (uint32_t)ll + (uint32_t)(LPR * j);
        uvalid[j] = u < units;
    }
    if constexpr (NORM) {
        const float *res = (const float *)a.x;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = (uint32_t)ll + (uint32_t)(LPR * j);
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 v = uvalid[j] ? *(const float4 *)(res + u * 32 + i) : make_float4(0, 0, 0, 0);
                xr[j][i] = v.x; xr[j][i + 1] = v.y; xr[j][i + 2] = v.z; xr[j][i + 3] = v.w;
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        ss = group_sum(ss, LPR);
        const float rms = rsqrtf(ss / (float)K + a.eps);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = (uint32_t)ll + (uint32_t)(LPR * j);
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                float4 w = uvalid[j] ? *(const float4 *)(a.norm_w + u * 32 + i) : make_float4(0, 0, 0, 0);
                float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float v = xr[j][i + t] * rms * wv[t];
                    if constexpr (FAITH) v = bf16_trunc(v);
                    xr[j][i + t] = f16_round(v);
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = (uint32_t)ll + (uint32_t)(LPR * j);
            if constexpr (XDT == NNZ_F32) {
                const float4 *p = (const float4 *)((const float *)a.x + (size_t)u * 32);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float4 v = uvalid[j] ? p[i] : make_float4(0, 0, 0, 0);
                    xr[j][4 * i] = v.x; xr[j][4 * i + 1] = v.y;
                    xr[j][4 * i + 2] = v.z; xr[j][4 * i + 3] = v.w;
                }
            } else {
                const uint4 *p = (const uint4 *)((const uint16_t *)a.x + (size_t)u * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint4 v = uvalid[j] ? p[i] : make_uint4(0, 0, 0, 0);
                    uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint16_t lo = (uint16_t)(wv[t] & 0xFFFFu), hi = (uint16_t)(wv[t] >> 16);
                        if constexpr (XDT == NNZ_F16) {
                            xr[j][8 * i + 2 * t] = (float)__builtin_bit_cast(f16_t, lo);
                            xr[j][8 * i + 2 * t + 1] = (float)__builtin_bit_cast(f16_t, hi);
                        } else {
                            xr[j][8 * i + 2 * t] = bf16_to_f32(lo);
                            xr[j][8 * i + 2 * t + 1] = bf16_to_f32(hi);
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) s += xr[j][i];
        xsum[j] = s;
    }

    // ---- row loop ----------------------------------------------------------
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t rows_per_iter = (uint32_t)(R * RPW);

    for (uint32_t base = wave * rows_per_iter; base < a.M; base += nwaves * rows_per_iter) {
        uint32_t row[R];
        bool rvalid[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            row[r] = base + (uint32_t)(r * RPW + rr);
            rvalid[r] = row[r] < a.M;
        }

        // Issue every weight load of this step before any arithmetic.
        uint32_t cw[NMAT][R][NV][VEC];
        uint16_t sc[NMAT][R][NV];
        uint16_t bi[NMAT][R][NV];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const uint32_t u = (uint32_t)ll + (uint32_t)(LPR * j);
                    const bool ok = rvalid[r] && uvalid[j];
                    const size_t wofs = (size_t)row[r] * words_per_row + (size_t)u * VEC;
                    if constexpr (VEC == 1) {
                        cw[m][r][j][0] = ok ? a.codes[m][wofs] : 0u;
                    } else {
                        uint4 q = ok ? *(const uint4 *)(a.codes[m] + wofs) : make_uint4(0, 0, 0, 0);
                        cw[m][r][j][0] = q.x; cw[m][r][j][1] = q.y;
                        cw[m][r][j][2] = q.z; cw[m][r][j][3] = q.w;
                    }
                    const size_t gidx = (size_t)row[r] * G + (u * 32u) / a.gs;
                    sc[m][r][j] = ok ? a.scales[m][gidx] : (uint16_t)0;
                    if constexpr (BITS == 4) bi[m][r][j] = ok ? a.biases[m][gidx] : (uint16_t)0;
                }

        float acc[NMAT][R];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float accv = 0.f;
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const float s = scale_to_f32(sc[m][r][j], (int)a.sdt);
                    if constexpr (BITS == 1) {
                        const uint32_t w = cw[m][r][j][0];
                        float sb = 0.f;
#pragma unroll
                        for (int i = 0; i < 32; ++i) {
                            const int mask = ((int)(w << (31 - i))) >> 31;  // 0 or -1
                            sb += __int_as_float(mask & __float_as_int(xr[j][i]));
                        }
                        accv = fmaf(s, 2.f * sb - xsum[j], accv);
                    } else {
                        float nd = 0.f;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t w = cw[m][r][j][k];
                            const uint32_t lo = w & 0x0F0F0F0Fu;
                            const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
                            nd = fmaf((float)(lo & 0xFFu), xr[j][8 * k + 0], nd);
                            nd = fmaf((float)(hi & 0xFFu), xr[j][8 * k + 1], nd);
                            nd = fmaf((float)((lo >> 8) & 0xFFu), xr[j][8 * k + 2], nd);
                            nd = fmaf((float)((hi >> 8) & 0xFFu), xr[j][8 * k + 3], nd);
                            nd = fmaf((float)((lo >> 16) & 0xFFu), xr[j][8 * k + 4], nd);
                            nd = fmaf((float)((hi >> 16) & 0xFFu), xr[j][8 * k + 5], nd);
                            nd = fmaf((float)(lo >> 24), xr[j][8 * k + 6], nd);
                            nd = fmaf((float)(hi >> 24), xr[j][8 * k + 7], nd);
                        }
                        const float b = scale_to_f32(bi[m][r][j], (int)a.sdt);
                        accv = fmaf(s, nd, fmaf(b, xsum[j], accv));
                    }
                }
                acc[m][r] = group_sum(accv, LPR);
            }

        if (ll == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (!rvalid[r]) continue;
                if constexpr (EPI == EPI_STORE) {
#pragma unroll
                    for (int m = 0; m < NMAT; ++m) {
                        float v = acc[m][r];
                        if constexpr (FAITH) v = bf16_trunc(v);
                        store_from_f32<ODT>(a.out[m], row[r], v);
                    }
                } else if constexpr (EPI == EPI_RESADD) {
                    float v = acc[0][r];
                    if constexpr (FAITH) v = bf16_trunc(v);
                    ((float *)a.out[0])[row[r]] += v;
                } else {
                    const float g = acc[0][r];
                    float v = g / (1.f + expf(-g)) * acc[NMAT - 1][r];
                    if constexpr (FAITH) v = bf16_trunc(v);
                    store_from_f32<ODT>(a.out[0], row[r], v);
                }
            }
        }
    }
}

int check_weight(nnz_ctx *ctx, const nnz_qweight *w, int bits, const nnz_qmv_dims &d,
                 const char *name) {
    NNZ_REQUIRE(ctx, w != nullptr, NNZ_EINVAL, "%s: null weight descriptor", name);
    NNZ_REQUIRE(ctx, w->codes && w->scales, NNZ_EINVAL, "%s: null codes/scales", name);
    NNZ_REQUIRE(ctx, (int)w->bits == bits, NNZ_EINVAL, "%s: weight has %u bits, kernel needs %d",
                name, w->bits, bits);
    NNZ_REQUIRE(ctx, (uint64_t)w->packed_count == (uint64_t)d.M * d.K, NNZ_EINVAL,
                "%s: packed_count %u != M*K", name, w->packed_count);
    NNZ_REQUIRE(ctx, w->group_size == d.group_size, NNZ_EINVAL,
                "%s: weight group_size %u != dims.group_size %u", name, w->group_size,
                d.group_size);
    if (bits == 1) {
        NNZ_REQUIRE(ctx, w->scale_dtype == NNZ_F16, NNZ_EINVAL, "%s: Q1 scales must be f16", name);
        NNZ_REQUIRE(ctx, ((uintptr_t)w->codes & 3) == 0, NNZ_EINVAL, "%s: codes not 4-byte aligned",
                    name);
    } else {
        NNZ_REQUIRE(ctx, w->biases != nullptr, NNZ_EINVAL, "%s: Q4 needs biases", name);
        NNZ_REQUIRE(ctx, w->scale_dtype == NNZ_F16 || w->scale_dtype == NNZ_BF16, NNZ_EINVAL,
                    "%s: bad scale dtype", name);
        NNZ_REQUIRE(ctx, ((uintptr_t)w->codes & 15) == 0, NNZ_EINVAL,
                    "%s: Q4 codes must be 16-byte aligned", name);
    }
    return NNZ_OK;
}

int check_dims(nnz_ctx *ctx, const nnz_qmv_dims &d, const char *name) {
    NNZ_REQUIRE(ctx, d.M > 0 && d.K > 0 && d.group_size > 0, NNZ_EINVAL, "%s: zero dims", name);
    NNZ_REQUIRE(ctx, d.K % 32 == 0, NNZ_EINVAL, "%s: K=%u not a multiple of 32", name, d.K);
    NNZ_REQUIRE(ctx, d.K % d.group_size == 0, NNZ_EINVAL, "%s: K=%u not a multiple of gs=%u", name,
                d.K, d.group_size);
    NNZ_REQUIRE(ctx, d.group_size % 32 == 0, NNZ_EUNSUPPORTED,
                "%s: group_size %u must be a multiple of 32", name, d.group_size);
    NNZ_REQUIRE(ctx, d.K <= 8192, NNZ_EUNSUPPORTED, "%s: K=%u > 8192 not supported", name, d.K);
    return NNZ_OK;
}

template <int BITS, int XDT, int NMAT, bool NORM, int EPI, int ODT, bool FAITH, int NV>
int launch_nv(nnz_ctx *ctx, const QmvArgs &a, int R, uint32_t blocks) {
    dim3 grid(blocks), block(256);
    switch (R) {
    case 4: qmv_kernel<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, NV, 4><<<grid, block, 0, ctx->stream>>>(a); break;
    case 2: qmv_kernel<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, NV, 2><<<grid, block, 0, ctx->stream>>>(a); break;
    default: qmv_kernel<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, NV, 1><<<grid, block, 0, ctx->stream>>>(a); break;
    }
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

template <int BITS, int XDT, int NMAT, bool NORM, int EPI, int ODT, bool FAITH>
int launch_qmv(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *x,
               const float *norm_w, void *out0, void *out1, nnz_qmv_dims d, const char *name) {
    NNZ_CHECK_CTX(ctx);
    int rc = check_dims(ctx, d, name);
    if (rc) return rc;
    rc = check_weight(ctx, wa, BITS, d, name);
    if (rc) return rc;
    if (NMAT == 2) {
        rc = check_weight(ctx, wb, BITS, d, name);
        if (rc) return rc;
        NNZ_REQUIRE(ctx, wb->scale_dtype == wa->scale_dtype, NNZ_EINVAL,
                    "%s: paired weights differ in scale dtype", name);
    }
    NNZ_REQUIRE(ctx, x && out0, NNZ_EINVAL, "%s: null input/output", name);
    NNZ_REQUIRE(ctx, ((uintptr_t)x & 15) == 0, NNZ_EINVAL, "%s: input must be 16-byte aligned", name);
    NNZ_REQUIRE(ctx, !(NMAT == 2 && EPI == EPI_STORE) || out1, NNZ_EINVAL, "%s: null output_b", name);
    if (NORM) {
        NNZ_REQUIRE(ctx, norm_w != nullptr, NNZ_EINVAL, "%s: null norm_scale", name);
        NNZ_REQUIRE(ctx, (((uintptr_t)x | (uintptr_t)norm_w) & 15) == 0, NNZ_EINVAL,
                    "%s: residual/norm_scale must be 16-byte aligned", name);
    }

    const uint32_t units = d.K / 32;
    uint32_t lpr = 1;
    while (lpr < units && lpr < 64) lpr <<= 1;
    int lpr_log2 = 0;
    while ((1u << lpr_log2) < lpr) ++lpr_log2;
    const uint32_t nv = ceil_div(units, lpr);
    NNZ_REQUIRE(ctx, nv >= 1 && nv <= 4, NNZ_EUNSUPPORTED, "%s: K=%u needs %u units/lane", name, d.K, nv);
    const uint32_t rpw = 64 / lpr;
    const int vec = BITS == 1 ? 1 : 4;
    int R = 4;
    // Keep >= 2 waves of work per CU where the matrix allows, and bound the
    // number of weight words a lane holds in flight.
    while (R > 1 && (ceil_div(d.M, 4u * R * rpw) < 512 || NMAT * R * (int)nv * vec > 32)) R >>= 1;
    uint32_t blocks = ceil_div(d.M, 4u * R * rpw);
    if (blocks > 8192) blocks = 8192;

    QmvArgs a{};
    a.codes[0] = (const uint32_t *)wa->codes;
    a.scales[0] = (const uint16_t *)wa->scales;
    a.biases[0] = (const uint16_t *)wa->biases;
    if (NMAT == 2) {
        a.codes[1] = (const uint32_t *)wb->codes;
        a.scales[1] = (const uint16_t *)wb->scales;
        a.biases[1] = (const uint16_t *)wb->biases;
    }
    a.x = x;
    a.norm_w = norm_w;
    a.out[0] = out0;
    a.out[1] = out1;
    a.M = d.M;
    a.K = d.K;
    a.gs = d.group_size;
    a.lpr_log2 = (uint32_t)lpr_log2;
    a.sdt = wa->scale_dtype;
    a.eps = 1e-6f;
    switch (nv) {
    case 1: return launch_nv<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, 1>(ctx, a, R, blocks);
    case 2: return launch_nv<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, 2>(ctx, a, R, blocks);
    case 3: return launch_nv<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, 3>(ctx, a, R, blocks);
    default: return launch_nv<BITS, XDT, NMAT, NORM, EPI, ODT, FAITH, 4>(ctx, a, R, blocks);
    }
}

}  // namespace

extern "C" {

// ---------------------------- Q1 ------------------------------------------
int nnz_dispatch_qmv(nnz_ctx *ctx, const nnz_qweight *w, const float *input, float *output,
                     nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 1, false, EPI_STORE, NNZ_F32, false>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_qmv");
}
int nnz_dispatch_qmv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const void *input, float *output,
                           nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 1, false, EPI_STORE, NNZ_F32, false>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_qmv_f16in");
}
int nnz_dispatch_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const void *input, void *output,
                           nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 1, false, EPI_STORE, NNZ_F16, false>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_qmv_f16io");
}
int nnz_dispatch_qmv_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                                  float *residual, nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 1, false, EPI_RESADD, NNZ_F32, false>(
        ctx, w, nullptr, input, nullptr, residual, nullptr, dims, "dispatch_qmv_f16io_resadd");
}
int nnz_dispatch_qmv_fused_pair(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                const float *input, float *output_a, float *output_b,
                                nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 2, false, EPI_STORE, NNZ_F32, false>(
        ctx, wa, wb, input, nullptr, output_a, output_b, dims, "dispatch_qmv_fused_pair");
}
int nnz_dispatch_qmv_fused_pair_f16in(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                      const void *input, float *output_a, float *output_b,
                                      nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 2, false, EPI_STORE, NNZ_F32, false>(
        ctx, wa, wb, input, nullptr, output_a, output_b, dims, "dispatch_qmv_fused_pair_f16in");
}
int nnz_dispatch_qmv_fused_pair_f16io(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                      const void *input, void *output_a, void *output_b,
                                      nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 2, false, EPI_STORE, NNZ_F16, false>(
        ctx, wa, wb, input, nullptr, output_a, output_b, dims, "dispatch_qmv_fused_pair_f16io");
}
int nnz_dispatch_qmv_fused_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                           const nnz_qweight *wb, const void *input, void *output,
                                           nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F16, 2, false, EPI_SILU, NNZ_F16, false>(
        ctx, wa, wb, input, nullptr, output, nullptr, dims, "dispatch_qmv_fused_pair_silu_f16io");
}
int nnz_dispatch_qmv_fused_pair_silu(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                     const float *input, float *output, nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 2, false, EPI_SILU, NNZ_F32, false>(
        ctx, wa, wb, input, nullptr, output, nullptr, dims, "dispatch_qmv_fused_pair_silu");
}
int nnz_dispatch_fused_norm_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                            const nnz_qweight *wb, const float *residual,
                                            void *output, const float *norm_scale,
                                            nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 2, true, EPI_SILU, NNZ_F16, false>(
        ctx, wa, wb, residual, norm_scale, output, nullptr, dims,
        "dispatch_fused_norm_pair_silu_f16io");
}
int nnz_dispatch_fused_norm_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                                      void *output, const float *norm_scale, nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 1, true, EPI_STORE, NNZ_F16, false>(
        ctx, w, nullptr, residual, norm_scale, output, nullptr, dims, "dispatch_fused_norm_qmv_f16io");
}
int nnz_dispatch_fused_norm_pair_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                           const nnz_qweight *wb, const float *residual,
                                           void *output_a, void *output_b, const float *norm_scale,
                                           nnz_qmv_dims dims) {
    return launch_qmv<1, NNZ_F32, 2, true, EPI_STORE, NNZ_F16, false>(
        ctx, wa, wb, residual, norm_scale, output_a, output_b, dims,
        "dispatch_fused_norm_pair_qmv_f16io");
}

// ---------------------------- Q4 ------------------------------------------
int nnz_dispatch_q4mv(nnz_ctx *ctx, const nnz_qweight *w, const float *input, float *output,
                      nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F32, 1, false, EPI_STORE, NNZ_F32, false>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_q4mv");
}
int nnz_dispatch_q4mv_f16io(nnz_ctx *ctx, const nnz_qweight *w, const void *input, void *output,
                            nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F16, 1, false, EPI_STORE, NNZ_F16, true>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_q4mv_f16io");
}
int nnz_dispatch_q4mv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const void *input, float *output,
                            nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F16, 1, false, EPI_STORE, NNZ_F32, true>(
        ctx, w, nullptr, input, nullptr, output, nullptr, dims, "dispatch_q4mv_f16in");
}
int nnz_dispatch_q4mv_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const void *input,
                                   float *residual, nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F16, 1, false, EPI_RESADD, NNZ_F32, true>(
        ctx, w, nullptr, input, nullptr, residual, nullptr, dims, "dispatch_q4mv_f16io_resadd");
}
int nnz_dispatch_q4mv_fused_pair_f16io(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                       const void *input, void *output_a, void *output_b,
                                       nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F16, 2, false, EPI_STORE, NNZ_F16, true>(
        ctx, wa, wb, input, nullptr, output_a, output_b, dims, "dispatch_q4mv_fused_pair_f16io");
}
int nnz_dispatch_q4mv_fused_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                            const nnz_qweight *wb, const void *input, void *output,
                                            nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F16, 2, false, EPI_SILU, NNZ_F16, true>(
        ctx, wa, wb, input, nullptr, output, nullptr, dims, "dispatch_q4mv_fused_pair_silu_f16io");
}
int nnz_dispatch_q4_fused_norm_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *w,
                                         const float *residual, void *output,
                                         const float *norm_scale, nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F32, 1, true, EPI_STORE, NNZ_F16, true>(
        ctx, w, nullptr, residual, norm_scale, output, nullptr, dims,
        "dispatch_q4_fused_norm_qmv_f16io");
}
int nnz_dispatch_q4_fused_norm_pair_qmv_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                              const nnz_qweight *wb, const float *residual,
                                              void *output_a, void *output_b,
                                              const float *norm_scale, nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F32, 2, true, EPI_STORE, NNZ_F16, true>(
        ctx, wa, wb, residual, norm_scale, output_a, output_b, dims,
        "dispatch_q4_fused_norm_pair_qmv_f16io");
}
int nnz_dispatch_q4_fused_norm_pair_silu_f16io(nnz_ctx *ctx, const nnz_qweight *wa,
                                               const nnz_qweight *wb, const float *residual,
                                               void *output, const float *norm_scale,
                                               nnz_qmv_dims dims) {
    return launch_qmv<4, NNZ_F32, 2, true, EPI_SILU, NNZ_F16, true>(
        ctx, wa, wb, residual, norm_scale, output, nullptr, dims,
        "dispatch_q4_fused_norm_pair_silu_f16io");
}

}  // extern "C"

// Prefill dequant-GEMM on gfx950 matrix cores.
//
// C[P x M] = A[P x K] . dequant(W[M x K])^T for a prompt of P tokens, where A
// holds the f16 activations of the decode path and W is a Q1 (1-bit, +-s)
// matrix.  The reference has no batched prefill: it runs P sequential decode
// steps (nnmetal/src/transformer.zig:4032-4068), and its only dequant-matmul
// (`qmm`, compute.metal:2975-3083) stores W as [K x N] for the MNIST network.
//
// Design:
//   * 64x64 output tile per 256-thread block, 4 waves in a 2x2 layout, each
//     wave 32x32 = 2x2 MFMA tiles of v_mfma_f32_16x16x32_f16 (fp32 accumulate).
//   * Per 64-wide K step the block stages A (f16, straight copy) and the
//     dequantised W tile (+-s written as f16; exact because s is an f16
//     scale) in LDS, rows padded by 16 bytes to spread LDS banks.
//   * Products of f16 activations and f16 +-s are exact in the MFMA, so the
//     result differs from the decode QMV only in fp32 summation order.
//   * Epilogues match the decode kernels: f16 store (Q/K/V), residual += (O,
//     down), silu(a)*b of a gate/up pair stored as f16.
#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int BM = 64, BN = 64, BK = 64, LDS_STRIDE = BK + 8;  // halfs per LDS row

template <int MODE, int NMAT>
__global__ __launch_bounds__(256) void dq_gemm_kernel(const f16_t *A, const uint32_t *codes0,
                                                      const uint16_t *scales0,
                                                      const uint32_t *codes1,
                                                      const uint16_t *scales1, void *out,
                                                      uint32_t P, uint32_t M, uint32_t K,
                                                      uint32_t gs) {
    __shared__ __attribute__((aligned(16))) f16_t As[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) f16_t Bs[NMAT][BN * LDS_STRIDE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t p0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t words_per_row = K / 32, groups_per_row = K / gs;

    float4v acc[NMAT][2][2];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[m][i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    // Loader roles: A: thread -> (row tid/4, 16 halfs at (tid%4)*16);
    // W: thread -> (row tid/4, 16 columns at (tid%4)*16).
    const int lr = tid >> 2, lc = (tid & 3) * 16;

    for (uint32_t k0 = 0; k0 < K; k0 += BK) {
        {
            const uint32_t p = p0 + lr;
            uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
            if (p < P) {
                const uint4 *src = (const uint4 *)(A + (size_t)p * K + k0 + lc);
                v0 = src[0];
                v1 = src[1];
            }
            uint4 *dst = (uint4 *)(As + lr * LDS_STRIDE + lc);
            dst[0] = v0;
            dst[1] = v1;
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t *codes = m == 0 ? codes0 : codes1;
            const uint16_t *scales = m == 0 ? scales0 : scales1;
            const uint32_t n = n0 + lr;
            const uint32_t col = k0 + lc;
            const uint32_t w = codes[(size_t)n * words_per_row + col / 32];
            const uint32_t bits = (w >> (col & 31)) & 0xFFFFu;
            const f16_t s = __builtin_bit_cast(f16_t, scales[(size_t)n * groups_per_row + col / gs]);
            half8 h0, h1;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                h0[i] = ((bits >> i) & 1) ? s : (f16_t)-s;
                h1[i] = ((bits >> (8 + i)) & 1) ? s : (f16_t)-s;
            }
            half8 *dst = (half8 *)(Bs[m] + lr * LDS_STRIDE + lc);
            dst[0] = h0;
            dst[1] = h1;
        }
        __syncthreads();

#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            const int kofs = kk + 8 * (lane >> 4);
            half8 af[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *(const half8 *)(As + (wm * 32 + i * 16 + (lane & 15)) * LDS_STRIDE + kofs);
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const half8 bf =
                        *(const half8 *)(Bs[m] + (wn * 32 + j * 16 + (lane & 15)) * LDS_STRIDE + kofs);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        acc[m][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[m][i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    // D layout: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t p = p0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                const uint32_t n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (p >= P) continue;
                const size_t o = (size_t)p * M + n;
                const float c = acc[0][i][j][r];
                if constexpr (MODE == NNZ_GEMM_STORE_F16) ((f16_t *)out)[o] = (f16_t)c;
                else if constexpr (MODE == NNZ_GEMM_STORE_F32) ((float *)out)[o] = c;
                else if constexpr (MODE == NNZ_GEMM_RESADD) ((float *)out)[o] += c;
                else {
                    const float u = acc[NMAT - 1][i][j][r];
                    ((f16_t *)out)[o] = (f16_t)(c / (1.f + expf(-c)) * u);
                }
            }
}

}  // namespace

int nnz_gemm_launch(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *a,
                    uint32_t P, void *out, int mode, const nnz_qmv_dims &d) {
    NNZ_REQUIRE(ctx, wa && a && out && P > 0, NNZ_EINVAL, "dequant_gemm: null argument");
    NNZ_REQUIRE(ctx, wa->bits == 1 && wa->codes && wa->scales, NNZ_EUNSUPPORTED,
                "dequant_gemm: Q1 weights only");
    NNZ_REQUIRE(ctx, (uint64_t)wa->packed_count == (uint64_t)d.M * d.K && wa->group_size == d.group_size,
                NNZ_EINVAL, "dequant_gemm: descriptor does not match dims");
    NNZ_REQUIRE(ctx, d.M % BN == 0 && d.K % BK == 0 && d.group_size % BK == 0 && d.K % d.group_size == 0,
                NNZ_EUNSUPPORTED, "dequant_gemm: need M%%64 == K%%64 == gs%%64 == 0");
    NNZ_REQUIRE(ctx, ((uintptr_t)a & 15) == 0, NNZ_EINVAL, "dequant_gemm: A must be 16-byte aligned");
    const bool pair = mode == NNZ_GEMM_SILU_PAIR;
    if (pair) {
        NNZ_REQUIRE(ctx, wb && wb->bits == 1 && wb->codes && wb->scales &&
                             (uint64_t)wb->packed_count == (uint64_t)d.M * d.K &&
                             wb->group_size == d.group_size,
                    NNZ_EINVAL, "dequant_gemm: bad second weight for SILU_PAIR");
    }
    dim3 grid(d.M / BN, ceil_div(P, BM));
    const f16_t *A = (const f16_t *)a;
    const uint32_t *c0 = (const uint32_t *)wa->codes;
    const uint16_t *s0 = (const uint16_t *)wa->scales;
    switch (mode) {
    case NNZ_GEMM_STORE_F16:
        dq_gemm_kernel<NNZ_GEMM_STORE_F16, 1><<<grid, 256, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, d.group_size);
        break;
    case NNZ_GEMM_STORE_F32:
        dq_gemm_kernel<NNZ_GEMM_STORE_F32, 1><<<grid, 256, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, d.group_size);
        break;
    case NNZ_GEMM_RESADD:
        dq_gemm_kernel<NNZ_GEMM_RESADD, 1><<<grid, 256, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, d.group_size);
        break;
    case NNZ_GEMM_SILU_PAIR:
        dq_gemm_kernel<NNZ_GEMM_SILU_PAIR, 2><<<grid, 256, 0, ctx->stream>>>(
            A, c0, s0, (const uint32_t *)wb->codes, (const uint16_t *)wb->scales, out, P, d.M, d.K, d.group_size);
        break;
    default:
        return nnz_fail(ctx, NNZ_EINVAL, "dequant_gemm: unknown mode %d", mode);
    }
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

extern "C" int nnz_dispatch_dequant_gemm(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                         const void *a_f16, uint32_t num_tokens, void *output, int mode,
                                         nnz_qmv_dims dims) {
    NNZ_CHECK_CTX(ctx);
    return nnz_gemm_launch(ctx, wa, wb, a_f16, num_tokens, output, mode, dims);
}

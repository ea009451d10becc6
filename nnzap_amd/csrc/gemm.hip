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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // register arrays of 16-byte pieces

constexpr int BM = 64, BN = 64, BK = 64, LDS_STRIDE = BK + 8;  // halfs per B LDS row
constexpr int GROUP = 4;  // K-steps whose global loads are issued together, one group ahead

// waitcnt immediate for gfx9: lgkmcnt = 0 only (the wave's LDS stores done)
constexpr int LGKM0_IMM = 15 | (3 << 14) | (7 << 4);

// Workgroup barrier for the pipelined loop: the wave's own LDS stores are
// waited for, then s_barrier.  __syncthreads() would add a release fence,
// which also waits for the next group's global loads still in flight.  The
// empty asm statements keep the compiler from moving LDS accesses across.
__device__ __forceinline__ void step_barrier() {
    __builtin_amdgcn_s_waitcnt(LGKM0_IMM);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Rows [0, rows0) of the launch come from matrix 0 (the kernel's codes0 /
// scales0 / out), [rows0, rows0 + rows1) from matrix 1, the rest from
// matrix 2; each writes its own output [P][rows].  n <= 1: one matrix.
struct GemmSegs {
    uint32_t n, rows0, rows1;
    const uint32_t *codes1, *codes2;
    const uint16_t *scales1, *scales2;
    void *out1, *out2;
};

template <int MODE, int NMAT>
__global__ __launch_bounds__(512) void dq_gemm_kernel(const f16_t *A, const uint32_t *codes0,
                                                      const uint16_t *scales0,
                                                      const uint32_t *codes1,
                                                      const uint16_t *scales1, void *out,
                                                      uint32_t P, uint32_t M, uint32_t K,
                                                      uint32_t gs_log2, GemmSegs sg) {
    // A tile of a K-step: 64 rows x 128 bytes, the eight 16-byte pieces of
    // row r stored at slot (piece ^ (r & 7)) so the MFMA fragment reads (16
    // rows, one piece each) spread over the banks.  B: dequantised W rows,
    // padded by 16 bytes.  Both double-buffered by step parity.
    __shared__ __attribute__((aligned(16))) f16_t As[2][BM * BK];
    __shared__ __attribute__((aligned(16))) f16_t Bs[2][NMAT][BN * LDS_STRIDE];
    // sign table: for a byte of weight bits, four words whose halves carry
    // 0x8000 where the bit is clear -- XORed into (s, s) they give +-s
    __shared__ __attribute__((aligned(16))) u32x4 sgn[256];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;   // 8 waves: 2 x 4, each 32 rows x 16 columns
    const uint32_t p0 = blockIdx.y * BM;
    uint32_t n0 = blockIdx.x * BN;
    if (sg.n > 1) {   // row segments of up to three matrices, each with its own output
        if (n0 < sg.rows0) {
            M = sg.rows0;
        } else if (n0 < sg.rows0 + sg.rows1 || sg.n == 2) {
            n0 -= sg.rows0;
            codes0 = sg.codes1;
            scales0 = sg.scales1;
            out = sg.out1;
            M = sg.rows1;
        } else {
            n0 -= sg.rows0 + sg.rows1;
            codes0 = sg.codes2;
            scales0 = sg.scales2;
            out = sg.out2;
            M = M - sg.rows0 - sg.rows1;
        }
    }
    const uint32_t words_per_row = K / 32, groups_per_row = K >> gs_log2;
    const uint32_t nk = K / BK;
    if (tid < 256) {
        const uint32_t b = tid;
        u32x4 e;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            e[q] = (((b >> (2 * q)) & 1u) ? 0u : 0x8000u) | (((b >> (2 * q + 1)) & 1u) ? 0u : 0x80000000u);
        sgn[b] = e;
    }

    float4v acc[NMAT][2];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[m][i] = (float4v){0.f, 0.f, 0.f, 0.f};

    // Loader roles (per step): thread -> row tid/8 and piece tid%8: A's
    // 16-byte piece (rows past P re-read row P-1, discarded at the store),
    // W's 8 columns at 8*(tid%8).
    const int lr = tid >> 3, lq = tid & 7, lc = lq * 8;
    const f16_t *arow = A + (size_t)min(p0 + (uint32_t)lr, P - 1) * K + lc;
    const uint32_t *wrow0 = codes0 + (size_t)(n0 + lr) * words_per_row;
    const uint32_t *wrow1 = NMAT == 2 ? codes1 + (size_t)(n0 + lr) * words_per_row : wrow0;
    const uint16_t *srow0 = scales0 + (size_t)(n0 + lr) * groups_per_row;
    const uint16_t *srow1 = NMAT == 2 ? scales1 + (size_t)(n0 + lr) * groups_per_row : srow0;
    const uint32_t ngroups = ceil_div(nk, (uint32_t)GROUP);

    // One group's registers: A pieces, W words, scales (two sets, used in
    // turn, so no register is copied).
    u32x4 aA[GROUP], aB[GROUP];
    uint32_t wA[GROUP][NMAT], wB[GROUP][NMAT];
    uint32_t sA[GROUP][NMAT], sB[GROUP][NMAT];
    auto issue = [&](u32x4 (&a)[GROUP], uint32_t (&w)[GROUP][NMAT], uint32_t (&sc)[GROUP][NMAT],
                     uint32_t g) __attribute__((always_inline)) {
        // steps past the last one re-read the last step (loads are never
        // branched around; those steps are skipped in run_group)
#pragma unroll
        for (int t = 0; t < GROUP; ++t) a[t] = *(const u32x4 *)(arow + min(g * GROUP + t, nk - 1) * BK);
#pragma unroll
        for (int t = 0; t < GROUP; ++t) {
            const uint32_t col = min(g * GROUP + t, nk - 1) * BK + lc;
            w[t][0] = wrow0[col / 32];
            sc[t][0] = srow0[col >> gs_log2];
            if constexpr (NMAT == 2) {
                w[t][1] = wrow1[col / 32];
                sc[t][1] = srow1[col >> gs_log2];
            }
        }
    };
    // Stage step ks (registers -> LDS buffer ks & 1): the A piece swizzled,
    // the byte of W bits expanded to +-s through the sign table.
    auto stage = [&](const u32x4 &a, const uint32_t (&w)[NMAT], const uint32_t (&sc)[NMAT],
                     uint32_t ks) __attribute__((always_inline)) {
        const int buf = ks & 1;
        ((u32x4 *)(As[buf] + lr * BK))[lq ^ (lr & 7)] = a;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t byte = (w[m] >> (lc & 31)) & 0xFFu;
            const uint32_t s2 = sc[m] | (sc[m] << 16);
            *(u32x4 *)(Bs[buf][m] + lr * LDS_STRIDE + lc) = sgn[byte] ^ s2;
        }
    };
    auto compute = [&](uint32_t ks) __attribute__((always_inline)) {
        const int buf = ks & 1;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            const int piece = kk / 8 + (lane >> 4);
            half8 af[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 32 + i * 16 + (lane & 15);
                af[i] = *(const half8 *)(As[buf] + r * BK + 8 * (piece ^ (r & 7)));
            }
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const half8 bf = *(const half8 *)(Bs[buf][m] + (wn * 16 + (lane & 15)) * LDS_STRIDE +
                                                  kk + 8 * (lane >> 4));
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[m][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[m][i], 0, 0, 0);
            }
        }
    };
    // Steps 4g..4g+3 of group g (registers `cur`): each iteration stages
    // the NEXT step (from `cur`, or for the last one from `nxt`, the next
    // group's set) while the MFMAs of the current step run, then one
    // barrier.  The buffer a step stages into was last read two steps
    // earlier, before the previous barrier.  Steps past the end are skipped
    // (block-uniform).
    auto run_group = [&](const u32x4 (&ca)[GROUP], const uint32_t (&cw)[GROUP][NMAT],
                         const uint32_t (&cs)[GROUP][NMAT], const u32x4 (&na)[GROUP],
                         const uint32_t (&nw)[GROUP][NMAT], const uint32_t (&ns)[GROUP][NMAT],
                         uint32_t g) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < GROUP; ++t) {
            const uint32_t ks = g * GROUP + t;
            if (ks >= nk) break;   // block-uniform
            if (ks + 1 < nk) {
                if (t + 1 < GROUP) stage(ca[t + 1], cw[t + 1], cs[t + 1], ks + 1);
                else stage(na[0], nw[0], ns[0], ks + 1);
            }
            compute(ks);
            step_barrier();
        }
    };

    // Group pipeline: the loads of group g+1 are issued before group g's
    // steps run, so they have a group's worth of compute to arrive.  Two
    // groups per pass, the register sets in turn.
    static_assert(GROUP % 2 == 0, "step parity across groups");
    issue(aA, wA, sA, 0);
    step_barrier();   // the sign table
    stage(aA[0], wA[0], sA[0], 0);
    step_barrier();
    for (uint32_t g = 0; g < ngroups; g += 2) {
        issue(aB, wB, sB, g + 1);
        run_group(aA, wA, sA, aB, wB, sB, g);
        issue(aA, wA, sA, g + 2);
        run_group(aB, wB, sB, aA, wA, sA, g + 1);
    }

    // D layout: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t p = p0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
            const uint32_t n = n0 + wn * 16 + (lane & 15);
            if (p >= P) continue;
            const size_t o = (size_t)p * M + n;
            const float c = acc[0][i][r];
            if constexpr (MODE == NNZ_GEMM_STORE_F16) ((f16_t *)out)[o] = (f16_t)c;
            else if constexpr (MODE == NNZ_GEMM_STORE_F32) ((float *)out)[o] = c;
            else if constexpr (MODE == NNZ_GEMM_RESADD) ((float *)out)[o] += c;
            else {
                const float u = acc[NMAT - 1][i][r];
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
    NNZ_REQUIRE(ctx, d.M % BN == 0 && d.K % BK == 0 && d.group_size % BK == 0 &&
                         d.K % d.group_size == 0,
                NNZ_EUNSUPPORTED, "dequant_gemm: need M %% 64 == 0, K %% 64 == 0, group size %% 64 == 0");
    NNZ_REQUIRE(ctx, ((uintptr_t)a & 15) == 0, NNZ_EINVAL, "dequant_gemm: A must be 16-byte aligned");
    const bool pair = mode == NNZ_GEMM_SILU_PAIR;
    if (pair) {
        NNZ_REQUIRE(ctx, wb && wb->bits == 1 && wb->codes && wb->scales &&
                             (uint64_t)wb->packed_count == (uint64_t)d.M * d.K &&
                             wb->group_size == d.group_size,
                    NNZ_EINVAL, "dequant_gemm: bad second weight for SILU_PAIR");
    }
    NNZ_REQUIRE(ctx, (d.group_size & (d.group_size - 1)) == 0, NNZ_EUNSUPPORTED,
                "dequant_gemm: group size must be a power of two");
    const uint32_t gl = (uint32_t)__builtin_ctz(d.group_size);
    dim3 grid(d.M / BN, ceil_div(P, BM));
    const f16_t *A = (const f16_t *)a;
    const uint32_t *c0 = (const uint32_t *)wa->codes;
    const uint16_t *s0 = (const uint16_t *)wa->scales;
    switch (mode) {
    case NNZ_GEMM_STORE_F16:
        dq_gemm_kernel<NNZ_GEMM_STORE_F16, 1><<<grid, 512, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_STORE_F32:
        dq_gemm_kernel<NNZ_GEMM_STORE_F32, 1><<<grid, 512, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_RESADD:
        dq_gemm_kernel<NNZ_GEMM_RESADD, 1><<<grid, 512, 0, ctx->stream>>>(A, c0, s0, nullptr, nullptr, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_SILU_PAIR:
        dq_gemm_kernel<NNZ_GEMM_SILU_PAIR, 2><<<grid, 512, 0, ctx->stream>>>(
            A, c0, s0, (const uint32_t *)wb->codes, (const uint16_t *)wb->scales, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    default:
        return nnz_fail(ctx, NNZ_EINVAL, "dequant_gemm: unknown mode %d", mode);
    }
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

// One launch for up to three matrices sharing K and the A operand (the
// prefill's Q, K and V projections), f16 outputs of their own.
int nnz_gemm_segments_launch(nnz_ctx *ctx, const nnz_qweight *const *w, void *const *out, int nw,
                             const void *a, uint32_t P, uint32_t K, uint32_t group_size) {
    NNZ_REQUIRE(ctx, nw >= 1 && nw <= 3 && a && P > 0, NNZ_EINVAL, "gemm_segments: bad arguments");
    NNZ_REQUIRE(ctx, K % BK == 0 && group_size % BK == 0 && K % group_size == 0 &&
                         (group_size & (group_size - 1)) == 0,
                NNZ_EUNSUPPORTED, "gemm_segments: need K %% 64 == 0, power-of-two group size %% 64 == 0");
    NNZ_REQUIRE(ctx, ((uintptr_t)a & 15) == 0, NNZ_EINVAL, "gemm_segments: A must be 16-byte aligned");
    uint32_t rows[3] = {0, 0, 0}, M = 0;
    for (int i = 0; i < nw; ++i) {
        NNZ_REQUIRE(ctx, w[i] && out[i] && w[i]->bits == 1 && w[i]->codes && w[i]->scales &&
                             w[i]->group_size == group_size && w[i]->packed_count % K == 0,
                    NNZ_EINVAL, "gemm_segments: bad weight %d", i);
        rows[i] = w[i]->packed_count / K;
        NNZ_REQUIRE(ctx, rows[i] % BN == 0, NNZ_EUNSUPPORTED, "gemm_segments: rows %% 64 != 0");
        M += rows[i];
    }
    GemmSegs sg{(uint32_t)nw, rows[0], rows[1],
                nw > 1 ? (const uint32_t *)w[1]->codes : nullptr,
                nw > 2 ? (const uint32_t *)w[2]->codes : nullptr,
                nw > 1 ? (const uint16_t *)w[1]->scales : nullptr,
                nw > 2 ? (const uint16_t *)w[2]->scales : nullptr,
                nw > 1 ? out[1] : nullptr, nw > 2 ? out[2] : nullptr};
    dim3 grid(M / BN, ceil_div(P, BM));
    dq_gemm_kernel<NNZ_GEMM_STORE_F16, 1><<<grid, 512, 0, ctx->stream>>>(
        (const f16_t *)a, (const uint32_t *)w[0]->codes, (const uint16_t *)w[0]->scales, nullptr,
        nullptr, out[0], P, M, K, (uint32_t)__builtin_ctz(group_size), sg);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

extern "C" int nnz_dispatch_dequant_gemm(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                         const void *a_f16, uint32_t num_tokens, void *output, int mode,
                                         nnz_qmv_dims dims) {
    NNZ_CHECK_CTX(ctx);
    return nnz_gemm_launch(ctx, wa, wb, a_f16, num_tokens, output, mode, dims);
}

// Prefill dequant-GEMM on gfx950 matrix cores.
//
// C[P x M] = A[P x K] . dequant(W[M x K])^T for a prompt of P tokens, where A
// holds the f16 activations of the decode path and W is a Q1 (1-bit, +-s)
// matrix.  The reference has no batched prefill: it runs P sequential decode
// steps (nnmetal/src/transformer.zig:4032-4068), and its only dequant-matmul
// (`qmm`, compute.metal:2975-3083) stores W as [K x N] for the MNIST network.
//
// Design (v_mfma_f32_16x16x32_f16, fp32 accumulate):
//   * One 64 (tokens) x 64 (W rows) output tile per block of 2 KQ waves:
//     2 W-row halves x KQ k-phases (KQ = 8 for single matrices whose grid
//     fits one block per CU, else 4; 2 for the gate/up pair).  Wave (wn, kq) computes a
//     64 x 32 tile over the k-steps (64 k each) with index = kq mod KQ, so a
//     W fragment expanded in registers feeds 4 MFMAs, an A fragment read
//     from LDS feeds 2, and the KQ partial tiles are summed through LDS at
//     the end.
//   * A is staged in LDS KQ k-steps (64 KQ k) at a time, double-buffered, with
//     one barrier per stage, by loads straight into LDS (global_load_lds,
//     no registers); the 16-byte piece p of row r sits at slot p ^ (r & 15),
//     so the 16 rows of an MFMA fragment read hit distinct banks.
//   * W is staged as packed bits (a 16-byte entry per row and k-step: two
//     code words and the group scale); each lane reads the 8 bits of its B
//     fragment and expands them in registers to f16 +-s (two ALU operations
//     per pair of weights).  +-s times an f16
//     activation is exact in the MFMA, so the result differs from the decode
//     QMV only in fp32 summation order.
//   * Blocks are numbered so that those resident on one XCD share their
//     64-token A tile (the XCD's L2 keeps it) when the token tiles divide by 8.
//   * Epilogues match the decode kernels: f16 store (Q/K/V), residual += (O,
//     down), silu(a)*b of a gate/up pair stored as f16.
#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // register arrays of 16-byte pieces
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int V> struct IC { static constexpr int value = V; };   // a compile-time index argument

constexpr int BM = 64, BN = 64, BK = 64;
// KQ k-phases (2 KQ waves, 128 KQ threads); an LDS stage holds KQ k-steps.
template <int KQ> constexpr int SK = BK * KQ;        // k per LDS stage
template <int KQ> constexpr int PIECES = SK<KQ> / 8; // 16-byte pieces per A row and stage
template <int KQ> constexpr int WROW = KQ + 1;       // W entries per LDS row (one of padding)

// One 16-byte global load per lane straight into LDS: lane l's bytes land
// at LDS address lds + 16 l (lds wave-uniform, in M0).  In asm rather than
// the builtin: for the builtin the compiler waits for every such load in
// flight before any LDS read it cannot prove apart (here: the fragment reads
// of the other stage buffer), which would serialise the pipeline.  Its
// completion is waited for explicitly (load_barrier); the compiler's own
// vmcnt waits stay correct, only more conservative, with these loads
// unknown to it (loads complete in order).  The s_nop is the one wait state
// gfx9 requires between an SALU write of M0 and an LDS DMA reading it (the
// compiler's hazard check does not look into asm).
__device__ __forceinline__ void global_load_lds16(const void *g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

// Workgroup barrier for a pipelined loop staging through registers: the
// wave's own LDS stores are waited for, then s_barrier.  __syncthreads()
// would add a release fence, which also waits for the next stage's global
// loads still in flight.  The empty asm statements keep the compiler from
// moving LDS accesses across.
constexpr int LGKM0_IMM = 15 | (3 << 14) | (7 << 4);   // gfx9 waitcnt immediate: lgkmcnt 0 only
__device__ __forceinline__ void step_barrier() {
    __builtin_amdgcn_s_waitcnt(LGKM0_IMM);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Workgroup barrier for a pipelined loop loading A straight into LDS: the
// wave's loads into LDS and its own LDS stores are waited for (vmcnt 0,
// lgkmcnt 0: the data of a global_load_lds is in LDS when it is counted),
// then s_barrier.  The empty asm statements keep the compiler from moving
// LDS accesses across.
constexpr int VM0_LGKM0_IMM = 7 << 4;   // gfx9 waitcnt immediate, expcnt not waited
__device__ __forceinline__ void load_barrier() {
    __builtin_amdgcn_s_waitcnt(VM0_LGKM0_IMM);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Eight weight bits (k ascending from bit 0) -> the B fragment's eight f16
// values: +s where the bit is set, -s where it is clear.  ns2 holds (-s, -s).
// z2 = z | z << 15 carries the byte twice, so one shift by 15 - 2q brings bit
// 2q to position 15 (low half's sign) and bit 2q+1 to position 31.
__device__ __forceinline__ half8 expand_bits(uint32_t z, uint32_t ns2) {
    // z2 is formed in asm so that the compiler does not fold the shifts below
    // into 32-bit multiplies (quarter rate); each dword is then one shift and
    // one three-input bit operation.
    uint32_t z2;
    asm("v_lshl_or_b32 %0, %1, 15, %1" : "=v"(z2) : "v"(z));
    u32x4 e;
    e[0] = ((z2 << 15) & 0x80008000u) ^ ns2;
    e[1] = ((z2 << 13) & 0x80008000u) ^ ns2;
    e[2] = ((z2 << 11) & 0x80008000u) ^ ns2;
    e[3] = ((z2 << 9) & 0x80008000u) ^ ns2;
    return __builtin_bit_cast(half8, e);
}

// silu(c) * u of a gate/up pair, as c / (1 + 2^(-c log2 e)) * u on the
// hardware exponential and reciprocal (each within about one ulp): a few
// float32 ulps from the correctly rounded c / (1 + exp(-c)) * u, well below
// the f16 (or bf16) rounding of the stored result, in 4 instructions where
// expf and the IEEE division take about 20.  c -> -inf: the exponential
// overflows to +inf and the product to -0; c -> +inf: c * u.
__device__ __forceinline__ float silu_mul(float c, float u) {
    const float e = __builtin_amdgcn_exp2f(-c * 1.44269504088896341f);
    return c * __builtin_amdgcn_rcpf(1.f + e) * u;
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

template <int MODE, int NMAT, int KQ, int WN>
__global__ __launch_bounds__(64 * WN * KQ) void dq_gemm_kernel(const f16_t *A, const uint32_t *codes0,
                                                      const uint16_t *scales0,
                                                      const uint32_t *codes1,
                                                      const uint16_t *scales1, void *out,
                                                      uint32_t P, uint32_t M, uint32_t K,
                                                      uint32_t gs_log2, GemmSegs sg) {
    // Two A stages (64 rows x 256 k of f16 each); reused for the k-phase
    // reduction after the main loop.
    constexpr int SK = ::SK<KQ>, PIECES = ::PIECES<KQ>, WROW = ::WROW<KQ>;
    // WN W-row groups x KQ k-phases of waves; a wave's tile is 64 x (64 / WN)
    constexpr int THREADS = 64 * WN * KQ, NJ = 4 / WN, A_LOADS = BM * PIECES / THREADS;
    static_assert(BM * PIECES == A_LOADS * THREADS && 64 * KQ * NMAT <= THREADS, "loader shapes");
    static_assert(PIECES >= 16, "the swizzle p ^ (r & 15) needs 16 pieces per row (KQ >= 2)");
    __shared__ __attribute__((aligned(16))) f16_t As[2][BM * SK];
    // W per stage: for each matrix and row, one 16-byte entry per k-step
    // (code words of its 64 k, scale), rows padded to WROW entries so the 16
    // rows of a fragment read hit distinct banks.
    __shared__ u32x4 Ws[2][NMAT][BN * WROW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave % WN, kq = wave / WN;

    // Block -> (W tile x, token tile y).  Workgroups are dispatched to the 8
    // XCDs round-robin, so block L runs on XCD L % 8; with the token tiles a
    // multiple of 8, XCD j gets token tiles j, j + 8, ... and all W tiles.
    const uint32_t nx = M / BN, ny = ceil_div(P, BM), L = blockIdx.x;
    uint32_t bx, by;
    if ((ny & 7) == 0) {
        const uint32_t slot = L >> 3;
        by = 8 * (slot / nx) + (L & 7);
        bx = slot % nx;
    } else {
        bx = L % nx;
        by = L / nx;
    }
    const uint32_t p0 = by * BM;
    uint32_t n0 = bx * BN;
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
    const uint32_t nk = K / BK, nst = ceil_div(nk, (uint32_t)KQ);

    float4v acc[NMAT][4][NJ];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[m][i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    // A loader: straight into LDS (global_load_lds_dwordx4: the 64 lanes of
    // a wave instruction fill 64 consecutive 16-byte slots, no registers).
    // Thread tid fills slot lp of rows lr + 16 u, u < A_LOADS, which holds
    // piece lp ^ (r & 15) = lp ^ (lr & 15) of the row, so that is the piece
    // it loads (rows past P re-read row P - 1, discarded at the store;
    // k-steps past the end re-read the last one, never used).
    const int lp = tid & (PIECES - 1), lr = tid / PIECES;
    constexpr int A_ROW_STEP = THREADS / PIECES;   // rows between a thread's pieces
    static_assert(A_ROW_STEP % 16 == 0, "a thread's rows share r & 15");
    const int ap = lp ^ (lr & 15);                 // the piece this thread loads
    const f16_t *arow[A_LOADS];
#pragma unroll
    for (int u = 0; u < A_LOADS; ++u)
        arow[u] = A + (size_t)min(p0 + (uint32_t)(lr + A_ROW_STEP * u), P - 1) * K + (ap & 7) * 8;
    // W loader: thread t < 256 NMAT loads k-step t % 4 of the stage for row
    // (t / 4) % 64 of matrix t / 256: the step's two code words and its scale.
    const int wl_m = tid / (64 * KQ), wl_row = (tid / KQ) & 63, wl_q = tid % KQ;
    const bool wl = wl_m < NMAT;
    const uint32_t *wl_codes = (NMAT == 2 && wl_m == 1 ? codes1 : codes0) +
                               (size_t)(n0 + wl_row) * words_per_row;
    const uint16_t *wl_scales = (NMAT == 2 && wl_m == 1 ? scales1 : scales0) +
                                (size_t)(n0 + wl_row) * groups_per_row;
    const int bsh = 8 * (lane >> 4);   // the lane's byte within a 32-k word

    // One stage in flight: the A pieces land in the other LDS buffer and this
    // thread's W entry in registers (loaded first, so waiting for it leaves
    // the A loads in flight), stored to LDS at the stage's end.
    u32x2 wreg = {0u, 0u};
    uint32_t sreg = 0;
    const int wbase = wave * 64;   // the wave's first 16-byte slot of an instruction
    auto issue = [&](uint32_t st) __attribute__((always_inline)) {
        if (wl) {
            const uint32_t ks = min(st * KQ + (uint32_t)wl_q, nk - 1);
            wreg = *(const u32x2 *)(wl_codes + 2 * ks);
            sreg = wl_scales[(ks * BK) >> gs_log2];
        }
        const uint32_t ka = min(st * KQ + (uint32_t)(ap >> 3), nk - 1) * BK;
        const uint32_t lds = __builtin_amdgcn_readfirstlane(
            (uint32_t)(size_t)(__attribute__((address_space(3))) f16_t *)(As[st & 1] + 8 * wbase));
#pragma unroll
        for (int u = 0; u < A_LOADS; ++u) global_load_lds16(arow[u] + ka, lds + 16u * (uint32_t)(u * THREADS));
    };
    auto stage = [&](uint32_t st) __attribute__((always_inline)) {
        if (wl) Ws[st & 1][wl_m][wl_row * WROW + wl_q] = (u32x4){wreg[0], wreg[1], sreg, 0u};
    };
    auto compute = [&](uint32_t st) __attribute__((always_inline)) {
        if (st * KQ + kq >= nk) return;   // wave-uniform
        const f16_t *buf = As[st & 1];
        uint32_t w[NMAT][NJ][2], ns2[NMAT][NJ];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const u32x4 e = Ws[st & 1][m][(16 * NJ * wn + 16 * j + (lane & 15)) * WROW + kq];
                w[m][j][0] = e[0];
                w[m][j][1] = e[1];
                ns2[m][j] = (e[2] | (e[2] << 16)) ^ 0x80008000u;
            }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int piece = kq * 8 + kk * 4 + (lane >> 4);
            half8 af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = i * 16 + (lane & 15);
                af[i] = *(const half8 *)(buf + r * SK + 8 * (piece ^ (r & 15)));
            }
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const half8 bf = expand_bits((w[m][j][kk] >> bsh) & 0xFFu, ns2[m][j]);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[m][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[m][i][j], 0, 0, 0);
                }
        }
    };

    // Stage pipeline: stage st + 1's loads are issued before stage st is
    // computed and stored to the other LDS buffers after it (those were last
    // read in stage st - 1, before the previous barrier).
    issue(0);
    stage(0);
    load_barrier();
    for (uint32_t st = 0; st < nst; ++st) {
        if (st + 1 < nst) issue(st + 1);   // block-uniform
        compute(st);
        if (st + 1 < nst) stage(st + 1);
        load_barrier();
    }

    // k-phase reduction through LDS (the stage buffers are free): phases 2, 3
    // hand their tiles to 0, 1, then phase 1 to phase 0.  Slot layout: one
    // float4 per (fragment, lane), lanes adjacent.
    constexpr int NF = NMAT * 4 * NJ;
    float4v *red = (float4v *)&As[0][0];
    auto put = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) red[(slot * NF + (m * 4 + i) * NJ + j) * 64 + lane] = acc[m][i][j];
    };
    auto add = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[m][i][j] += red[(slot * NF + (m * 4 + i) * NJ + j) * 64 + lane];
    };
    static_assert(KQ / 2 * WN * NF * 64 * 16 <= (int)sizeof(As), "reduction slots fit the stage buffers");
    // tree over the k-phases: phases [h, 2h) hand their tiles to [0, h),
    // down to phases 0 and 1
#pragma unroll
    for (int h = KQ / 2; h >= 2; h /= 2) {
        if (kq >= h && kq < 2 * h) put((kq - h) * WN + wn);
        __syncthreads();
        if (kq < h) add(kq * WN + wn);
        __syncthreads();
    }
    // Phases 0 and 1 swap halves and both finish the block: phase 0 the
    // 16-row tiles i = 0, 1, phase 1 the tiles i = 2, 3.  (With phase 0
    // finishing everything, the waves of phase 0 -- the same SIMDs in every
    // block -- carried the whole epilogue.)  Half slots: NF / 2 float4.
    auto put_half = [&](int slot, auto hh) __attribute__((always_inline)) {
        constexpr int H = decltype(hh)::value;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    red[(slot * (NF / 2) + (m * 2 + ii) * NJ + j) * 64 + lane] = acc[m][2 * H + ii][j];
    };
    auto add_half = [&](int slot, auto hh) __attribute__((always_inline)) {
        constexpr int H = decltype(hh)::value;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[m][2 * H + ii][j] += red[(slot * (NF / 2) + (m * 2 + ii) * NJ + j) * 64 + lane];
    };
    if (kq == 0) put_half(WN + wn, IC<1>{});   // phase 1's tiles
    else if (kq == 1) put_half(wn, IC<0>{});  // phase 0's tiles
    __syncthreads();
    if (kq >= 2) return;   // after the last barrier
    if (kq == 0) add_half(wn, IC<0>{});
    else add_half(WN + wn, IC<1>{});

    // D layout: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile.
    auto epilogue = [&](auto ti) __attribute__((always_inline)) {
        constexpr int i = decltype(ti)::value;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t p = p0 + i * 16 + 4 * (lane >> 4) + r;
            if (p >= P) continue;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t n = n0 + 16 * NJ * wn + 16 * j + (lane & 15);
                const size_t o = (size_t)p * M + n;
                const float c = acc[0][i][j][r];
                if constexpr (MODE == NNZ_GEMM_STORE_F16) ((f16_t *)out)[o] = (f16_t)c;
                else if constexpr (MODE == NNZ_GEMM_STORE_F32) ((float *)out)[o] = c;
                else if constexpr (MODE == NNZ_GEMM_RESADD) ((float *)out)[o] += c;
                else {
                    const float u = acc[NMAT - 1][i][j][r];
                    ((f16_t *)out)[o] = (f16_t)silu_mul(c, u);
                }
            }
        }
    };
    if (kq == 0) {
        epilogue(IC<0>{});
        epilogue(IC<1>{});
    } else {
        epilogue(IC<2>{});
        epilogue(IC<3>{});
    }
}

// ---------------------------------------------------------------------------
// 4-bit (q4_mlx) weights: W = s * n + b per group of >= 64 columns, n a
// nibble, s and b bf16 (or f16).  s * n + b is not exact in f16, so the
// MFMA takes the nibbles themselves, exactly: per 64-k step and W row,
//   sum_k A[p][k] W[r][k] = s_r * (A . n)[p][r] + b_r * (sum_k A[p][k]),
// with (A . n) and the row sums (A against a fragment of ones) on the MFMA
// and the two scalings in fp32 -- the Q4 QMV's arithmetic up to fp32
// summation order.  Nibble pairs become f16 through the exponent trick:
// 0x6400 | n is the f16 value 1024 + n, and subtracting 1024 (v_pk_add_f16)
// leaves n exactly.  Epilogues are the BF16-faithful ones of the Q4 decode
// kernels (q4mv_bf16_specialized.metal:52-57): each result is BF16-truncated
// before the f16 store, the residual += or the SiLU*mul product's store.
// Block: 64 tokens x 64 W rows, 4 waves = 2 W-row halves x 2 k-phases;
// an LDS stage holds 2 k-steps: A (swizzled as above) and, per matrix and
// row, the 16 code words of the two steps plus their (s | b << 16) words,
// rows padded to 20 words so a fragment read of 16 rows hits distinct banks.
// KQ k-phases: 4 KQ waves (2 W-row halves x KQ), LDS stages of KQ k-steps;
// a W row holds 8 code words per step plus one (s | b << 16) word per step,
// padded to a stride of 4 x odd words (20 for KQ = 2, 36 for KQ = 4).
template <int KQ> constexpr int Q4_WROW = KQ == 2 ? 20 : 36;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float q4_param(uint32_t raw16, int sdt) {
    return sdt == NNZ_BF16 ? bf16_to_f32((uint16_t)raw16) : (float)__builtin_bit_cast(f16_t, (uint16_t)raw16);
}

// The 8 nibbles of one code word (k ascending from bit 0) as f16 values.
__device__ __forceinline__ half8 expand_nibbles(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes: n[2q], n[2q+1]
    const half2v k1024 = {(_Float16)1024.f, (_Float16)1024.f};
    half8 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // byte q of lo into byte 0, byte q of hi into byte 2, zeros elsewhere
        const uint32_t sel = (uint32_t)q | (0x0Cu << 8) | ((uint32_t)(4 + q) << 16) | (0x0Cu << 24);
        const uint32_t d = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
        const half2v v = __builtin_bit_cast(half2v, d) - k1024;
        r[2 * q] = v[0];
        r[2 * q + 1] = v[1];
    }
    return r;
}

// At most 256 registers (two waves per SIMD): the pair kernel otherwise
// takes 222 VGPRs + 64 AGPRs, one wave per SIMD, and copies every MFMA
// result out of the AGPRs before its scaling.
template <int MODE, int NMAT, int KQ>
__global__ __launch_bounds__(128 * KQ) __attribute__((amdgpu_waves_per_eu(2))) void dq4_gemm_kernel(const f16_t *A, const uint32_t *codes0,
                                                              const uint16_t *scales0,
                                                              const uint16_t *biases0,
                                                              const uint32_t *codes1,
                                                              const uint16_t *scales1,
                                                              const uint16_t *biases1, void *out,
                                                              uint32_t P, uint32_t M, uint32_t K,
                                                              uint32_t gs_log2, int sdt) {
    constexpr int Q4_KQ = KQ, Q4_SK = BK * KQ, Q4_PIECES = Q4_SK / 8, Q4_THREADS = 128 * KQ;
    constexpr int WR = Q4_WROW<KQ>;
    constexpr int A_LOADS = BM * Q4_PIECES / Q4_THREADS;   // 4
    static_assert(Q4_PIECES >= 16 && 64 * Q4_KQ * NMAT <= Q4_THREADS && WR >= 9 * KQ, "loader shapes");
    __shared__ __attribute__((aligned(16))) f16_t As[2][BM * Q4_SK];
    __shared__ __attribute__((aligned(16))) uint32_t Ws[2][NMAT][BN * WR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, kq = wave >> 1;
    const uint32_t nx = M / BN, ny = ceil_div(P, BM), L = blockIdx.x;
    uint32_t bx, by;
    if ((ny & 7) == 0) {
        const uint32_t slot = L >> 3;
        by = 8 * (slot / nx) + (L & 7);
        bx = slot % nx;
    } else {
        bx = L % nx;
        by = L / nx;
    }
    const uint32_t p0 = by * BM, n0 = bx * BN;
    const uint32_t words_per_row = K / 8, groups_per_row = K >> gs_log2;
    const uint32_t nk = K / BK, nst = ceil_div(nk, (uint32_t)Q4_KQ);

    float4v acc[NMAT][4][2];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[m][i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

    // A through registers (loading it straight into LDS, as dq_gemm_kernel
    // does, measured no faster here: 4-bit down 37.7 -> 38.6 us)
    const int lp = tid & (Q4_PIECES - 1), lr = tid / Q4_PIECES;
    constexpr int A_ROW_STEP = Q4_THREADS / Q4_PIECES;
    const f16_t *arow[A_LOADS];
#pragma unroll
    for (int u = 0; u < A_LOADS; ++u)
        arow[u] = A + (size_t)min(p0 + (uint32_t)(lr + A_ROW_STEP * u), P - 1) * K + (lp & 7) * 8;
    // W loader: thread t < 64 KQ NMAT takes step t % KQ of row (t / KQ) % 64
    // of matrix t / (64 KQ): 8 code words (two 16-byte loads), scale and bias.
    const int wl_m = tid / (64 * KQ), wl_row = (tid / KQ) & 63, wl_q = tid % KQ;
    const bool wl = wl_m < NMAT;
    const uint32_t wrow_g = n0 + wl_row;
    const uint32_t *wl_codes = (NMAT == 2 && wl_m == 1 ? codes1 : codes0) + (size_t)wrow_g * words_per_row;
    const uint16_t *wl_s = (NMAT == 2 && wl_m == 1 ? scales1 : scales0) + (size_t)wrow_g * groups_per_row;
    const uint16_t *wl_b = (NMAT == 2 && wl_m == 1 ? biases1 : biases0) + (size_t)wrow_g * groups_per_row;
    const int gsel = lane >> 4;   // the lane's code word within a 32-k half step

    // scale and bias stay two registers until the stage: joining them at
    // the issue would wait there for their loads, and with them (vmcnt is
    // in order) for the A loads of the stage being prefetched
    u32x4 areg[A_LOADS], wc0 = {0u, 0u, 0u, 0u}, wc1 = {0u, 0u, 0u, 0u};
    uint32_t sreg = 0, breg = 0;
    auto issue = [&](uint32_t st) __attribute__((always_inline)) {
        const uint32_t ka = min(st * Q4_KQ + (uint32_t)(lp >> 3), nk - 1) * BK;
#pragma unroll
        for (int u = 0; u < A_LOADS; ++u) areg[u] = *(const u32x4 *)(arow[u] + ka);
        if (wl) {
            const uint32_t ks = min(st * Q4_KQ + (uint32_t)wl_q, nk - 1);
            wc0 = *(const u32x4 *)(wl_codes + 8 * ks);
            wc1 = *(const u32x4 *)(wl_codes + 8 * ks + 4);
            const uint32_t g = (ks * BK) >> gs_log2;
            sreg = wl_s[g];
            breg = wl_b[g];
        }
    };
    auto stage = [&](uint32_t st) __attribute__((always_inline)) {
        f16_t *buf = As[st & 1];
#pragma unroll
        for (int u = 0; u < A_LOADS; ++u) {
            const int r = lr + A_ROW_STEP * u;
            ((u32x4 *)(buf + r * Q4_SK))[lp ^ (r & 15)] = areg[u];
        }
        if (wl) {
            uint32_t *row = Ws[st & 1][wl_m] + wl_row * WR;
            *(u32x4 *)(row + 8 * wl_q) = wc0;
            *(u32x4 *)(row + 8 * wl_q + 4) = wc1;
            row[8 * KQ + wl_q] = sreg | (breg << 16);
        }
    };
    const half8 ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f,
                        (_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
    auto compute = [&](uint32_t st) __attribute__((always_inline)) {
        if (st * Q4_KQ + kq >= nk) return;   // wave-uniform
        const f16_t *buf = As[st & 1];
        half8 af[2][4];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int piece = kq * 8 + kk * 4 + (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = i * 16 + (lane & 15);
                af[kk][i] = *(const half8 *)(buf + r * Q4_SK + 8 * (piece ^ (r & 15)));
            }
        }
        // row sums of A over the step: every column of the product with ones
        float4v xs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xs[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][i], ones, (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            xs[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[1][i], ones, xs[i], 0, 0, 0);
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t *row = Ws[st & 1][m] + (32 * wn + 16 * j + (lane & 15)) * WR;
                const uint32_t sb = row[8 * KQ + kq];
                const float sc = q4_param(sb & 0xFFFFu, sdt), bi = q4_param(sb >> 16, sdt);
                const half8 b0 = expand_nibbles(row[8 * kq + gsel]);
                const half8 b1 = expand_nibbles(row[8 * kq + 4 + gsel]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4v t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][i], b0, (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[1][i], b1, t, 0, 0, 0);
                    // two multiply-adds per element: + b (row sum), then + s (A . n)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[m][i][j][r] = fmaf(sc, t[r], fmaf(bi, xs[i][r], acc[m][i][j][r]));
                }
            }
    };

    issue(0);
    stage(0);
    step_barrier();
    for (uint32_t st = 0; st < nst; ++st) {
        if (st + 1 < nst) issue(st + 1);   // block-uniform
        compute(st);
        if (st + 1 < nst) stage(st + 1);
        step_barrier();
    }

    // k-phase tree through the (free) A buffers: phases [h, 2h) hand their
    // tiles to [0, h), down to phases 0 and 1
    constexpr int NF = NMAT * 8;
    static_assert(KQ / 2 * 2 * NF * 64 * 16 <= (int)sizeof(As), "reduction slots fit the stage buffers");
    float4v *red = (float4v *)&As[0][0];
#pragma unroll
    for (int h = KQ / 2; h >= 2; h /= 2) {
        if (kq >= h && kq < 2 * h) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        red[(((kq - h) * 2 + wn) * NF + (m * 4 + i) * 2 + j) * 64 + lane] = acc[m][i][j];
        }
        __syncthreads();
        if (kq < h) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[m][i][j] += red[((kq * 2 + wn) * NF + (m * 4 + i) * 2 + j) * 64 + lane];
        }
        __syncthreads();
    }
    // Phases 0 and 1 swap halves and both finish the block: phase 0 the
    // 16-row tiles i = 0, 1, phase 1 the tiles i = 2, 3 (half slots of
    // NF / 2 float4).
    auto put_half = [&](int slot, auto hh) __attribute__((always_inline)) {
        constexpr int H = decltype(hh)::value;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    red[(slot * (NF / 2) + (m * 2 + ii) * 2 + j) * 64 + lane] = acc[m][2 * H + ii][j];
    };
    auto add_half = [&](int slot, auto hh) __attribute__((always_inline)) {
        constexpr int H = decltype(hh)::value;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[m][2 * H + ii][j] += red[(slot * (NF / 2) + (m * 2 + ii) * 2 + j) * 64 + lane];
    };
    if (kq == 0) put_half(2 + wn, IC<1>{});   // phase 1's tiles
    else if (kq == 1) put_half(wn, IC<0>{});  // phase 0's tiles
    __syncthreads();
    if (kq >= 2) return;   // after the last barrier
    if (kq == 0) add_half(wn, IC<0>{});
    else add_half(2 + wn, IC<1>{});

    auto epilogue = [&](auto ti) __attribute__((always_inline)) {
        constexpr int i = decltype(ti)::value;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t p = p0 + i * 16 + 4 * (lane >> 4) + r;
            if (p >= P) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t n = n0 + 32 * wn + 16 * j + (lane & 15);
                const size_t o = (size_t)p * M + n;
                const float c = acc[0][i][j][r];
                if constexpr (MODE == NNZ_GEMM_STORE_F16) ((f16_t *)out)[o] = (f16_t)bf16_trunc(c);
                else if constexpr (MODE == NNZ_GEMM_STORE_F32) ((float *)out)[o] = bf16_trunc(c);
                else if constexpr (MODE == NNZ_GEMM_RESADD) ((float *)out)[o] += bf16_trunc(c);
                else {
                    const float u = acc[NMAT - 1][i][j][r];
                    ((f16_t *)out)[o] = (f16_t)bf16_trunc(silu_mul(c, u));
                }
            }
        }
    };
    if (kq == 0) {
        epilogue(IC<0>{});
        epilogue(IC<1>{});
    } else {
        epilogue(IC<2>{});
        epilogue(IC<3>{});
    }
}

// k-phases and W-row groups of the single-matrix launches.  Measured at P =
// 512: with a grid of at most one block per CU and K > 2048 (the down
// projection), 8 k-phases (16 waves, 149 KB of LDS) are faster than 4
// (23.4 against 23.5-24.3 us); with A loaded straight into LDS, K = 2048
// does better on 4 (O 11.5 -> 11.3, K/V 9.4 -> 8.8 us); larger grids run 4
// (75 KB: two blocks per CU; the fused Q/K/V launch, 512 blocks: 17.1 us
// against 20.6).
// The gate/up pair runs 2 (4-wave blocks, 44 KB, 88 VGPRs: its 768 blocks
// are all resident at once; 48.7 us with 4 k-phases, 39.5 us with 2).  One
// W-row group (64 x 64 wave tiles, half the A reads from LDS, 8 waves) is
// 7-12 % slower than two.
constexpr int WN1 = 2;
constexpr uint32_t ONE_ROUND_BLOCKS = 256;   // CUs of an MI355X

template <int MODE>
void launch_single(nnz_ctx *ctx, uint32_t grid, const f16_t *A, const uint32_t *c0,
                   const uint16_t *s0, void *out, uint32_t P, uint32_t M, uint32_t K, uint32_t gl,
                   const GemmSegs &sg) {
    if (grid <= ONE_ROUND_BLOCKS && K > 2048)
        dq_gemm_kernel<MODE, 1, 8, WN1><<<grid, 64 * WN1 * 8, 0, ctx->stream>>>(
            A, c0, s0, nullptr, nullptr, out, P, M, K, gl, sg);
    else
        dq_gemm_kernel<MODE, 1, 4, WN1><<<grid, 64 * WN1 * 4, 0, ctx->stream>>>(
            A, c0, s0, nullptr, nullptr, out, P, M, K, gl, sg);
}

}  // namespace

namespace {

// 4-bit weights (every mode; results BF16-faithful, see dq4_gemm_kernel).
int gemm4_launch(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *a,
                 uint32_t P, void *out, int mode, const nnz_qmv_dims &d) {
    const bool pair = mode == NNZ_GEMM_SILU_PAIR;
    auto ok = [&](const nnz_qweight *w) {
        return w && w->bits == 4 && w->codes && w->scales && w->biases &&
               (uint64_t)w->packed_count == (uint64_t)d.M * d.K && w->group_size == d.group_size &&
               w->scale_dtype == wa->scale_dtype && ((uintptr_t)w->codes & 15) == 0 &&
               ((uintptr_t)w->scales & 1) == 0 && ((uintptr_t)w->biases & 1) == 0;
    };
    NNZ_REQUIRE(ctx, ok(wa) && (!pair || ok(wb)), NNZ_EINVAL,
                "dequant_gemm: 4-bit weights need codes (16-byte aligned), scales and biases "
                "matching the dims");
    NNZ_REQUIRE(ctx, wa->scale_dtype == NNZ_BF16 || wa->scale_dtype == NNZ_F16, NNZ_EINVAL,
                "dequant_gemm: scale dtype must be bf16 or f16");
    NNZ_REQUIRE(ctx, d.M % BN == 0 && d.K % BK == 0 && d.group_size % BK == 0 &&
                         d.K % d.group_size == 0 && (d.group_size & (d.group_size - 1)) == 0,
                NNZ_EUNSUPPORTED,
                "dequant_gemm: need M %% 64 == 0, K %% 64 == 0, power-of-two group size %% 64 == 0");
    NNZ_REQUIRE(ctx, ((uintptr_t)a & 15) == 0, NNZ_EINVAL, "dequant_gemm: A must be 16-byte aligned");
    const uint32_t gl = (uint32_t)__builtin_ctz(d.group_size);
    const uint32_t grid = d.M / BN * ceil_div(P, BM);
    const f16_t *A = (const f16_t *)a;
    const uint32_t *c0 = (const uint32_t *)wa->codes;
    const uint16_t *s0 = (const uint16_t *)wa->scales, *b0 = (const uint16_t *)wa->biases;
    const int sdt = wa->scale_dtype;
    switch (mode) {
    case NNZ_GEMM_STORE_F16:
        if (grid <= ONE_ROUND_BLOCKS)
            dq4_gemm_kernel<NNZ_GEMM_STORE_F16, 1, 4><<<grid, 512, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        else
            dq4_gemm_kernel<NNZ_GEMM_STORE_F16, 1, 2><<<grid, 256, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        break;
    case NNZ_GEMM_STORE_F32:
        if (grid <= ONE_ROUND_BLOCKS)
            dq4_gemm_kernel<NNZ_GEMM_STORE_F32, 1, 4><<<grid, 512, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        else
            dq4_gemm_kernel<NNZ_GEMM_STORE_F32, 1, 2><<<grid, 256, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        break;
    case NNZ_GEMM_RESADD:
        if (grid <= ONE_ROUND_BLOCKS)
            dq4_gemm_kernel<NNZ_GEMM_RESADD, 1, 4><<<grid, 512, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        else
            dq4_gemm_kernel<NNZ_GEMM_RESADD, 1, 2><<<grid, 256, 0, ctx->stream>>>(
                A, c0, s0, b0, nullptr, nullptr, nullptr, out, P, d.M, d.K, gl, sdt);
        break;
    case NNZ_GEMM_SILU_PAIR:
        dq4_gemm_kernel<NNZ_GEMM_SILU_PAIR, 2, 2><<<grid, 256, 0, ctx->stream>>>(
            A, c0, s0, b0, (const uint32_t *)wb->codes, (const uint16_t *)wb->scales,
            (const uint16_t *)wb->biases, out, P, d.M, d.K, gl, sdt);
        break;
    default:
        return nnz_fail(ctx, NNZ_EINVAL, "dequant_gemm: unknown mode %d", mode);
    }
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

}  // namespace

int nnz_gemm_launch(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *a,
                    uint32_t P, void *out, int mode, const nnz_qmv_dims &d) {
    NNZ_REQUIRE(ctx, wa && a && out && P > 0, NNZ_EINVAL, "dequant_gemm: null argument");
    if (wa->bits == 4) return gemm4_launch(ctx, wa, wb, a, P, out, mode, d);
    NNZ_REQUIRE(ctx, wa->bits == 1 && wa->codes && wa->scales, NNZ_EUNSUPPORTED,
                "dequant_gemm: 1-bit or 4-bit weights");
    NNZ_REQUIRE(ctx, (uint64_t)wa->packed_count == (uint64_t)d.M * d.K && wa->group_size == d.group_size,
                NNZ_EINVAL, "dequant_gemm: descriptor does not match dims");
    NNZ_REQUIRE(ctx, d.M % BN == 0 && d.K % BK == 0 && d.group_size % BK == 0 &&
                         d.K % d.group_size == 0,
                NNZ_EUNSUPPORTED, "dequant_gemm: need M %% 64 == 0, K %% 64 == 0, group size %% 64 == 0");
    NNZ_REQUIRE(ctx, ((uintptr_t)a & 15) == 0, NNZ_EINVAL, "dequant_gemm: A must be 16-byte aligned");
    NNZ_REQUIRE(ctx, ((uintptr_t)wa->codes & 7) == 0 && (!wb || ((uintptr_t)wb->codes & 7) == 0),
                NNZ_EINVAL, "dequant_gemm: codes must be 8-byte aligned");
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
    const uint32_t grid = d.M / BN * ceil_div(P, BM);
    const f16_t *A = (const f16_t *)a;
    const uint32_t *c0 = (const uint32_t *)wa->codes;
    const uint16_t *s0 = (const uint16_t *)wa->scales;
    switch (mode) {
    case NNZ_GEMM_STORE_F16:
        launch_single<NNZ_GEMM_STORE_F16>(ctx, grid, A, c0, s0, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_STORE_F32:
        launch_single<NNZ_GEMM_STORE_F32>(ctx, grid, A, c0, s0, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_RESADD:
        launch_single<NNZ_GEMM_RESADD>(ctx, grid, A, c0, s0, out, P, d.M, d.K, gl, GemmSegs{});
        break;
    case NNZ_GEMM_SILU_PAIR:
        dq_gemm_kernel<NNZ_GEMM_SILU_PAIR, 2, 2, 2><<<grid, 256, 0, ctx->stream>>>(
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
        NNZ_REQUIRE(ctx, ((uintptr_t)w[i]->codes & 7) == 0, NNZ_EINVAL,
                    "gemm_segments: codes must be 8-byte aligned");
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
    const uint32_t grid = M / BN * ceil_div(P, BM);
    launch_single<NNZ_GEMM_STORE_F16>(ctx, grid, (const f16_t *)a, (const uint32_t *)w[0]->codes,
                                      (const uint16_t *)w[0]->scales, out[0], P, M, K,
                                      (uint32_t)__builtin_ctz(group_size), sg);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

extern "C" int nnz_dispatch_dequant_gemm(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb,
                                         const void *a_f16, uint32_t num_tokens, void *output, int mode,
                                         nnz_qmv_dims dims) {
    NNZ_CHECK_CTX(ctx);
    return nnz_gemm_launch(ctx, wa, wb, a_f16, num_tokens, output, mode, dims);
}

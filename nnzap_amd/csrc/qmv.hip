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
//   * Latency: the weight loads of the first row-step are issued before the
//     x / RMSNorm prologue (they do not depend on it), and the row loop is
//     software-pipelined -- the next step's loads are in flight while the
//     current step computes -- so a small matrix costs about one memory round
//     trip instead of two per step.  Lanes of a row read adjacent words, so
//     every load instruction is one contiguous, coalesced segment of a row.
//   * Rows may be split into up to three segments with their own matrix and
//     output (same K): the Q, K and V projections of a layer run as one
//     launch sharing the normalised input.
//
// Q1 arithmetic: sum_c (bit ? +x_c : -x_c) = 2 * sum_{bit=1} x_c - sum_c x_c,
// computed per 32-column unit with a sign-extended bit mask ANDed into x
// (3 VALU ops per weight), then scaled by the unit's group scale.
// Q4 arithmetic: acc += s * sum(n_i x_i) + b * sum(x_i) per unit
// (q4mv_bf16_specialized.metal:14-16), nibbles widened with the byte
// converts after splitting even/odd nibbles.
#include "internal.h"

namespace {

enum { EPI_STORE = 0, EPI_RESADD = 1, EPI_SILU = 2 };

// Input modes: x as given (XDT); RMSNorm of an f32 residual; the merge of
// split-sequence attention partials (x = attention output, f16-rounded).
enum { XIN_X = 0, XIN_NORM = 1, XIN_MERGE = 2 };

// Attention partials read by XIN_MERGE (written by the fused decode
// attention in its unit-major layout): part_o per chunk c the K = Hq * D
// values, column k at c K + ((k >> 2) & 7) K / 8 + (k >> 5) 4 + (k & 3)
// (nibble-major over the 32-column units); part_ml [nchunks][Hq][2]; the
// live chunk count is ceil(seq / chunk), seq = d_seq ? *d_seq : seq_len.
constexpr int MERGE_MAX_CHUNKS = 16;
struct MergeIn {
    const float *part_o, *part_ml;
    const uint32_t *d_seq;
    uint32_t seq_len, nchunks, chunk, head_dim;
};

constexpr int MAX_SEG = 3;

// One matrix (or row segment) and its output.
struct QmvMat {
    const uint32_t *codes;
    const uint16_t *scales;
    const uint16_t *biases;
    void *out;
    uint32_t seg_end;      // NMAT == 1: one past the segment's last row
};

// Stacked launch (gridDim.y > 1): block row y works on matrix y, whose
// codes, scales (and biases), input and output lie these many bytes past
// matrix 0's.  All zero for an ordinary launch.
struct StackArgs {
    uint64_t codes, scales, x, out;
};

struct QmvArgs {
    // NMAT == 2: matrices m0 and m1 share rows [0, M).  NMAT == 1: rows are
    // the concatenation of `nseg` segments, segment s = rows
    // [m(s-1).seg_end, m(s).seg_end) of matrix s, written to its out.
    // Separate fields, not an array: a runtime index into a kernel-argument
    // array makes the compiler copy the arguments to scratch memory.
    QmvMat m0, m1, m2;
    uint32_t nseg;
    const void *x;         // input vector (XDT) or f32 residual (XIN_NORM)
    const float *norm_w;   // f32 [K], XIN_NORM only
    MergeIn mg;            // XIN_MERGE only
    NnzTop2 *top2;         // f32 single-matrix stores: per-block greedy top-2, or null
    uint32_t M, K, gs;
    uint32_t lpr_log2;     // lanes per row = 1 << lpr_log2
    uint32_t sdt;          // scale/bias dtype (NNZ_F16 / NNZ_BF16)
    float eps;
    StackArgs stk;
};

// Pointer `p` of matrix blockIdx.y of a stacked launch (`stride` bytes
// between matrices; 0 for an ordinary launch).  The argument block itself
// is never modified: a modified copy of it would live in scratch memory.
template <bool STK, class T>
__device__ __forceinline__ T *stk(T *p, uint64_t stride) {
    if constexpr (STK) return (T *)((uintptr_t)p + (uint64_t)blockIdx.y * stride);
    else return p;   // ordinary launches carry no stacked-offset arithmetic
}
// Weight registers of one row-step.
template <int NMAT, int R, int NV, int VEC>
struct StepRegs {
    uint32_t cw[NMAT][R][NV][VEC];
    uint16_t sc[NMAT][R][NV];
    uint16_t bi[NMAT][R][NV];
    bool ok[NMAT][R][NV];      // lane holds a real (row, unit)
    float res[R];              // residual-add epilogue: current residual rows
};

// Segment of a wave-uniform step base (steps never straddle segments: the
// host only splits rows at multiples of the rows per step).
__device__ __forceinline__ int step_segment(const QmvArgs &a, uint32_t base, uint32_t &seg_start) {
    int seg = 0;
    seg_start = 0;
    if (a.nseg > 1 && base >= a.m0.seg_end) { seg = 1; seg_start = a.m0.seg_end; }
    if (a.nseg > 2 && base >= a.m1.seg_end) { seg = 2; seg_start = a.m1.seg_end; }
    return seg;   // uniform: a.nseg, the segment ends and `base` are
}

// Matrix `m` of a pair (compile-time index).
template <int m>
__device__ __forceinline__ const QmvMat &mat_of(const QmvArgs &a) {
    static_assert(m >= 0 && m < MAX_SEG, "matrix index");
    if constexpr (m == 0) return a.m0;
    else if constexpr (m == 1) return a.m1;
    else return a.m2;
}

// A wave-uniform pointer as an opaque scalar value.  Selecting between
// argument fields through this keeps the compiler from turning the select
// into a load through a selected field address, which would force a copy of
// the whole argument block to scratch memory.
// The result is typed as a global-memory pointer so loads through it are
// global (not flat) loads.
#if defined(__HIP_DEVICE_COMPILE__)
template <class T>
using gptr = T __attribute__((address_space(1))) *;
#else
template <class T>
using gptr = T *;   // host pass: device bodies are parsed, not generated
#endif
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ gptr<T> uniform_ptr(T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (gptr<T>)(((uint64_t)hi << 32) | lo);
}

template <class T>
__device__ __forceinline__ gptr<T> pick3(int seg, T *p0, T *p1, T *p2) {
    gptr<T> a = uniform_ptr(p0), b = uniform_ptr(p1), c = uniform_ptr(p2);
    return seg == 0 ? a : (seg == 1 ? b : c);
}

// Pointers of segment `seg` (wave-uniform runtime index).
struct SegPtrs {
    gptr<const uint32_t> codes;
    gptr<const uint16_t> scales, biases;
    gptr<void> out;
};

template <bool STK>
__device__ __forceinline__ SegPtrs seg_mat(const QmvArgs &a, int seg) {
    SegPtrs r;
    r.codes = stk<STK>(pick3(seg, a.m0.codes, a.m1.codes, a.m2.codes), a.stk.codes);
    r.scales = stk<STK>(pick3(seg, a.m0.scales, a.m1.scales, a.m2.scales), a.stk.scales);
    r.biases = stk<STK>(pick3(seg, a.m0.biases, a.m1.biases, a.m2.biases), a.stk.scales);
    r.out = stk<STK>(pick3(seg, a.m0.out, a.m1.out, a.m2.out), a.stk.out);
    return r;
}

// Per-lane unit offsets, fixed for the whole kernel: word offset of unit j
// within a row (0 for a unit past the row end, whose scale is zeroed) and
// its group index within the row's scales.
template <int NV>
struct LaneUnits {
    uint32_t uoff[NV];   // units (32-column pieces) from the row start
    uint32_t ugrp[NV];   // byte offset of the unit's scale (and bias) from the row's first
    bool ok[NV];         // the unit exists
};

template <int BITS, int NMAT, int R, int NV, bool RES, bool STK>
__device__ __forceinline__ void load_step(const QmvArgs &a, StepRegs<NMAT, R, NV, (BITS == 1 ? 1 : 4)> &s,
                                          uint32_t base, int RPW, int rr, const LaneUnits<NV> &lu,
                                          uint32_t units, uint32_t G) {
    constexpr int VEC = (BITS == 1) ? 1 : 4;
    const uint32_t words_per_row = units * VEC;
    // Matrix pointers of this step, chosen with a wave-uniform segment index
    // (a per-lane index would turn into a per-lane load of the pointer).
    gptr<const uint32_t> cp[NMAT];
    gptr<const uint16_t> sp[NMAT];
    gptr<const uint16_t> bp[NMAT];
    uint32_t seg_start = 0;
    gptr<void> outp = nullptr;
    if constexpr (NMAT == 1) {
        const SegPtrs sm = seg_mat<STK>(a, step_segment(a, base, seg_start));
        cp[0] = sm.codes; sp[0] = sm.scales; bp[0] = sm.biases;
        outp = sm.out;
    } else {
        cp[0] = stk<STK>(uniform_ptr(a.m0.codes), a.stk.codes); sp[0] = stk<STK>(uniform_ptr(a.m0.scales), a.stk.scales);
        bp[0] = stk<STK>(uniform_ptr(a.m0.biases), a.stk.scales);
        cp[NMAT - 1] = stk<STK>(uniform_ptr(mat_of<NMAT - 1>(a).codes), a.stk.codes);
        sp[NMAT - 1] = stk<STK>(uniform_ptr(mat_of<NMAT - 1>(a).scales), a.stk.scales);
        bp[NMAT - 1] = stk<STK>(uniform_ptr(mat_of<NMAT - 1>(a).biases), a.stk.scales);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // With whole-wave rows (rr == 0) the row and its offsets are
        // wave-uniform: scalar arithmetic, one vector add per address.
        const uint32_t row = base + (uint32_t)(r * RPW + rr);
        const bool rv = row < a.M;
        // Unconditional loads from a clamped address (row 0 stands in for a
        // row past the end, unit 0 for a unit past the row end); the dead
        // lane's scale and bias are zeroed so its weights contribute 0.
        const uint32_t lr = rv ? row - seg_start : 0u;
        if constexpr (RES) {  // residual rows this step will add to, read early
            static_assert(NMAT == 1, "residual add has one matrix");
            s.res[r] = ((gptr<const float>)outp)[lr];
        }
        const size_t rw = (size_t)lr * words_per_row, rg = (size_t)lr * G;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const gptr<const uint32_t> codes = cp[m] + rw;
            const gptr<const uint16_t> scales = sp[m] + rg;
            const gptr<const uint16_t> biases = bp[m] + rg;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                // R == 8 is chosen only for vocabulary-sized matrices (the LM
                // head), read once per token: load those weights
                // non-temporally so they do not evict the layer weights and
                // the KV cache (measured: +0.8% decode tok/s)
                if constexpr (VEC == 1) {
                    if constexpr (R == 8) s.cw[m][r][j][0] = __builtin_nontemporal_load(&codes[lu.uoff[j]]);
                    else s.cw[m][r][j][0] = codes[lu.uoff[j]];
                } else {
                    const u32x4 q = *(gptr<const u32x4>)(codes + (size_t)lu.uoff[j] * VEC);
                    s.cw[m][r][j][0] = q.x; s.cw[m][r][j][1] = q.y;
                    s.cw[m][r][j][2] = q.z; s.cw[m][r][j][3] = q.w;
                }
                // 32-bit byte offsets: scalar base + vector offset addressing
                const gptr<const uint16_t> sj = (gptr<const uint16_t>)((gptr<const char>)scales + lu.ugrp[j]);
                if constexpr (R == 8) s.sc[m][r][j] = __builtin_nontemporal_load(sj);
                else s.sc[m][r][j] = *sj;
                if constexpr (BITS == 4)
                    s.bi[m][r][j] = *(gptr<const uint16_t>)((gptr<const char>)biases + lu.ugrp[j]);
                s.ok[m][r][j] = rv && lu.ok[j];
            }
        }
    }
}

// Whole-wave rows (FULL): per-lane byte offsets of row r's unit j from the
// first row of a step, fixed for the whole kernel, so a step's loads need
// one scalar base per matrix and no per-row address arithmetic.
template <int R, int NV>
struct FullOffsets {
    uint32_t code[R][NV];    // codes
    uint32_t scale[R][NV];   // scales and biases
    uint32_t res;            // the residual of this lane's output row
};

// Raw buffer resource over a weight array: stride 0, no range limit (the
// offsets below are in bounds by construction), gfx9 dword3 (32-bit data
// format).  A load through it adds a 32-bit scalar offset (the step's first
// row) to a 32-bit per-lane offset (fixed for the kernel): no 64-bit
// address arithmetic per row or per step.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)0xFFFFFFFF, 0x00020000);
}

// Loads of one step of R consecutive whole-wave rows starting at `rb`
// (wave-uniform, rb + R <= M: the caller clamps the last step back onto
// valid rows instead of clamping each row).
template <int BITS, int NMAT, int R, int NV, bool RES, bool STK>
__device__ __forceinline__ void load_step_full(const QmvArgs &a, StepRegs<NMAT, R, NV, (BITS == 1 ? 1 : 4)> &s,
                                               uint32_t rb, const FullOffsets<R, NV> &fo,
                                               uint32_t words_per_row, uint32_t G) {
    // Every weight is read once per token: non-temporal loads (measured:
    // decode +0.6% over plain loads for the layer weights, +0.8% for the LM
    // head) leave the caches to the activations and the KV cache.
    constexpr int AUX = 2;
    __amdgpu_buffer_rsrc_t cr[NMAT], sr[NMAT], br[NMAT];
    uint32_t seg_start = 0;
    if constexpr (NMAT == 1) {
        // plain selects of the argument values (already scalar): no
        // per-step moves of the pointers through vector registers
        const int seg = step_segment(a, rb, seg_start);
        auto sel = [&](const void *p0, const void *p1, const void *p2) {
            return seg == 0 ? p0 : (seg == 1 ? p1 : p2);
        };
        cr[0] = weight_rsrc(stk<STK>(sel(a.m0.codes, a.m1.codes, a.m2.codes), a.stk.codes));
        sr[0] = weight_rsrc(stk<STK>(sel(a.m0.scales, a.m1.scales, a.m2.scales), a.stk.scales));
        br[0] = weight_rsrc(stk<STK>(sel(a.m0.biases, a.m1.biases, a.m2.biases), a.stk.scales));
    } else {
        cr[0] = weight_rsrc(stk<STK>(a.m0.codes, a.stk.codes));
        sr[0] = weight_rsrc(stk<STK>(a.m0.scales, a.stk.scales));
        br[0] = weight_rsrc(stk<STK>(a.m0.biases, a.stk.scales));
        cr[NMAT - 1] = weight_rsrc(stk<STK>(mat_of<NMAT - 1>(a).codes, a.stk.codes));
        sr[NMAT - 1] = weight_rsrc(stk<STK>(mat_of<NMAT - 1>(a).scales, a.stk.scales));
        br[NMAT - 1] = weight_rsrc(stk<STK>(mat_of<NMAT - 1>(a).biases, a.stk.scales));
    }
    const uint32_t lr = rb - seg_start;
    const uint32_t co = lr * words_per_row * 4u, so = lr * G * 2u;
    if constexpr (RES) {
        static_assert(NMAT == 1, "residual add has one matrix");
        s.res[0] = *(gptr<const float>)((gptr<const char>)stk<STK>(uniform_ptr(a.m0.out), a.stk.out) + (size_t)rb * 4u + fo.res);
    }
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if constexpr (BITS == 1) {
                    s.cw[m][r][j][0] = __builtin_amdgcn_raw_buffer_load_b32(cr[m], fo.code[r][j], co, AUX);
                } else {
                    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(cr[m], fo.code[r][j], co, AUX);
                    s.cw[m][r][j][0] = q.x; s.cw[m][r][j][1] = q.y;
                    s.cw[m][r][j][2] = q.z; s.cw[m][r][j][3] = q.w;
                    s.bi[m][r][j] = __builtin_amdgcn_raw_buffer_load_b16(br[m], fo.scale[r][j], so, AUX);
                }
                s.sc[m][r][j] = __builtin_amdgcn_raw_buffer_load_b16(sr[m], fo.scale[r][j], so, AUX);
            }
}

// Store / residual-add / SiLU epilogue of one row.  `row` indexes the pair
// outputs and the residual, `lrow` the row within the step's segment.
template <int EPI, int ODT, bool FAITH, int NMAT, bool STK>
__device__ __forceinline__ void qmv_epilogue(const QmvArgs &a, void *out0, uint32_t row,
                                             uint32_t lrow, const float (&tot)[NMAT], float prev) {
    if constexpr (EPI == EPI_STORE) {
        if constexpr (NMAT == 1) {
            float v = tot[0];
            if constexpr (FAITH) v = bf16_trunc(v);
            store_from_f32<ODT>(out0, lrow, v);
        } else {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                float v = tot[m];
                if constexpr (FAITH) v = bf16_trunc(v);
                store_from_f32<ODT>(stk<STK>(m == 0 ? a.m0.out : a.m1.out, a.stk.out), row, v);
            }
        }
    } else if constexpr (EPI == EPI_RESADD) {
        float v = tot[0];
        if constexpr (FAITH) v = bf16_trunc(v);
        ((float *)out0)[row] = prev + v;   // prev: residual[row] read with the weights
    } else {
        const float g = tot[0];
        float v = g / (1.f + expf(-g)) * tot[NMAT - 1];
        if constexpr (FAITH) v = bf16_trunc(v);
        store_from_f32<ODT>(out0, row, v);
    }
}

// FULL: whole-wave rows (LPR == 64, every K >= 2048) fixed at compile time,
// so that row indices, offsets and the row reductions are wave-uniform.
template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH, int NV, int R, bool LUT,
          bool FULL, bool STK>
__global__ __launch_bounds__(256) void qmv_kernel(QmvArgs a) {
    const void *const ax = stk<STK>(a.x, a.stk.x);
    static_assert(!LUT || BITS == 1, "nibble tables are for 1-bit weights");
    static_assert(!LUT || FULL, "nibble tables need whole-wave rows");
    constexpr bool NORM = XIN == XIN_NORM;
    constexpr bool MERGE = XIN == XIN_MERGE;
    constexpr int VEC = (BITS == 1) ? 1 : 4;  // u32 words per 32-column unit
    // greedy top-2 of the stored rows (the LM head's argmax, first pass)
    constexpr bool TOP2 = EPI == EPI_STORE && NMAT == 1 && ODT == NNZ_F32 && FULL && !STK;
    NnzTop2 t2{-INFINITY, -INFINITY, 0xFFFFFFFFu};
    const int lane = threadIdx.x & 63;
    const int lpr_log2 = FULL ? 6 : (int)a.lpr_log2;
    const int LPR = 1 << lpr_log2;
    const int RPW = 64 >> lpr_log2;
    const int rr = lane >> lpr_log2;       // sub-row within the wave step
    const int ll = lane & (LPR - 1);       // lane within the row group
    const uint32_t K = a.K;
    const uint32_t units = K >> 5;          // 32-column units per row
    const uint32_t G = K / a.gs;            // groups per row

    bool uvalid[NV];
    LaneUnits<NV> lu;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        uvalid[j] = (uint32_t)ll + (uint32_t)(LPR * j) < units;
        lu.ok[j] = uvalid[j];
        lu.uoff[j] = uvalid[j] ? (uint32_t)ll + (uint32_t)(LPR * j) : 0u;
        lu.ugrp[j] = (lu.uoff[j] * 32u) / a.gs * 2u;
    }

    const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    const uint32_t rows_per_iter = (uint32_t)(R * RPW);
    uint32_t base = wave * rows_per_iter;

    // ---- load order ----------------------------------------------------------
    // The prologue's own loads (x, or the residual and norm weights, or the
    // attention partials) are issued first and the first row-step's weights
    // right after them: loads complete in issue order, so the prologue then
    // waits only for its own data while the weights are still in flight.
    // The weight loads are never branched around (a branch makes the wait
    // at its join cover every load issued before it): past the end, a step
    // re-reads rows that are valid, and their values go unused.
    StepRegs<NMAT, R, NV, VEC> cur;
    // FULL: a step reads rows [rb, rb + R) with rb = min(base, M - R) (the
    // host keeps M >= R), so every load is in bounds and the last step's
    // rows below `base` are computed but not stored.
    FullOffsets<R, NV> fo;
    if constexpr (FULL) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                fo.code[r][j] = ((uint32_t)r * units * VEC + lu.uoff[j] * VEC) * 4u;
                fo.scale[r][j] = (uint32_t)r * G * 2u + lu.ugrp[j];
            }
        fo.res = (uint32_t)(multi_row_slot<NMAT * R>() / NMAT) * 4u;
    }
    auto step_base = [&](uint32_t b) { return b < a.M - (uint32_t)R ? b : a.M - (uint32_t)R; };
    auto load_rows = [&](StepRegs<NMAT, R, NV, VEC> &dst, uint32_t b) {
        if constexpr (FULL)
            load_step_full<BITS, NMAT, R, NV, EPI == EPI_RESADD, STK>(a, dst, step_base(b), fo, units * VEC, G);
        else
            load_step<BITS, NMAT, R, NV, EPI == EPI_RESADD, STK>(a, dst, b < a.M ? b : 0u, RPW, rr, lu, units, G);
    };
    auto first_weights = [&]() {
        // the prologue's own loads go out first (nothing of the weight
        // addressing may be scheduled ahead of them)
        __builtin_amdgcn_sched_barrier(0);
        load_rows(cur, base);
    };

    // ---- 1-bit signed nibble tables (LUT, full-wave rows only) --------------
    // For each unit j of a lane and nibble n (columns 4n..4n+3 of the unit)
    // the 16 signed sums T[e] = sum_k (bit k of e ? +x : -x)[4n + k], so a
    // row's +-x sum over 32 weights is 8 table reads (no mask-and-add per
    // weight, no separate sum of x).  The tables are built straight from the
    // prologue's own loads: thread (lane l, wave w) loads the float4 of
    // nibbles n = 2w, 2w+1 of units u = l + 64 j, normalises it (RMSNorm
    // input) and writes its 2 x 16 entries at [j][n][e][l] -- the lane that
    // reads a unit's tables is the one that owns it, so the 64 reads (and
    // writes) of a wave hit 64 distinct banks.  One barrier after the norm's
    // sum of squares, one after the tables.
    __shared__ float lut[LUT ? NV * 8 * 16 * 64 : 1];
    float xr[NV][32];
    float xsum[NV];
    if constexpr (LUT && !MERGE) {   // (the merge prologue builds its tables itself)
        const int wid = threadIdx.x >> 6;
        float v[NV][2][4];
        if constexpr (NORM) {
            __shared__ float red[4];
            const float4 *res4 = (const float4 *)ax;
            const float4 *nw4 = (const float4 *)a.norm_w;
            float4 rv[NV][2], wv[NV][2];
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    const uint32_t i4 = uvalid[j] ? (uint32_t)(lane + 64 * j) * 8u + 2u * wid + sb : 0u;
                    rv[j][sb] = res4[i4];
                    wv[j][sb] = nw4[i4];
                }
            first_weights();
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    if (!uvalid[j]) rv[j][sb] = make_float4(0.f, 0.f, 0.f, 0.f);
                    ss = fmaf(rv[j][sb].x, rv[j][sb].x, ss);
                    ss = fmaf(rv[j][sb].y, rv[j][sb].y, ss);
                    ss = fmaf(rv[j][sb].z, rv[j][sb].z, ss);
                    ss = fmaf(rv[j][sb].w, rv[j][sb].w, ss);
                }
            ss = wave_sum(ss);
            if (lane == 0) red[wid] = ss;
            __syncthreads();
            ss = (red[0] + red[1]) + (red[2] + red[3]);
            const float rms = rsqrtf(ss / (float)K + a.eps);
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    float t[4] = {rv[j][sb].x * rms * wv[j][sb].x, rv[j][sb].y * rms * wv[j][sb].y,
                                  rv[j][sb].z * rms * wv[j][sb].z, rv[j][sb].w * rms * wv[j][sb].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (FAITH) t[e] = bf16_trunc(t[e]);
                        v[j][sb][e] = (float)(f16_t)t[e];
                    }
                }
        } else {
            // x as given: 4 columns = one float4 (f32) or 8 bytes (f16 / bf16)
            float4 xf[NV][2];
            uint2 xh[NV][2];
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    const uint32_t i4 = uvalid[j] ? (uint32_t)(lane + 64 * j) * 8u + 2u * wid + sb : 0u;
                    if constexpr (XDT == NNZ_F32) xf[j][sb] = ((const float4 *)ax)[i4];
                    else xh[j][sb] = ((const uint2 *)ax)[i4];
                }
            first_weights();
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    if constexpr (XDT == NNZ_F32) {
                        v[j][sb][0] = xf[j][sb].x; v[j][sb][1] = xf[j][sb].y;
                        v[j][sb][2] = xf[j][sb].z; v[j][sb][3] = xf[j][sb].w;
                    } else {
                        const uint32_t h[4] = {xh[j][sb].x & 0xFFFFu, xh[j][sb].x >> 16,
                                               xh[j][sb].y & 0xFFFFu, xh[j][sb].y >> 16};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            v[j][sb][e] = XDT == NNZ_F16 ? (float)__builtin_bit_cast(f16_t, (uint16_t)h[e])
                                                         : bf16_to_f32((uint16_t)h[e]);
                    }
                    if (!uvalid[j]) v[j][sb][0] = v[j][sb][1] = v[j][sb][2] = v[j][sb][3] = 0.f;
                }
        }
        float *const dst = lut + lane;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                const int n = 2 * wid + sb;
                const float *x4 = v[j][sb];
                // bit 0 of e signs x0, bit 1 x1, bit 2 x2, bit 3 x3
                const float p1 = x4[0] - x4[1], p3 = x4[0] + x4[1];
                const float q1 = x4[2] - x4[3], q3 = x4[2] + x4[3];
                const float p[4] = {-p3, p1, -p1, p3};
                const float q[4] = {-q3, q1, -q1, q3};
#pragma unroll
                for (int e = 0; e < 16; ++e) dst[((j * 8 + n) * 16 + e) * 64] = p[e & 3] + q[e >> 2];
            }
        __syncthreads();
    } else if constexpr (NORM) {
        // The block normalises x once: each thread loads K/256 residual and
        // norm-weight values (K <= 2048*NV, so at most 2*NV float4 each),
        // the sum of squares is reduced through LDS, and the f16-rounded
        // normalised vector is staged in LDS for every wave to read its
        // slice -- one copy of the prologue's loads per block, not per wave.
        constexpr int P4 = 2 * NV;
        __shared__ __align__(16) f16_t xs[2048 * NV];
        __shared__ float red[4];
        const float4 *res4 = (const float4 *)ax;
        const float4 *nw4 = (const float4 *)a.norm_w;
        const uint32_t n4 = K / 4;
        float4 rv[P4], wv[P4];
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t i4 = threadIdx.x + 256u * k;
            const uint32_t ic = i4 < n4 ? i4 : 0u;
            rv[k] = res4[ic];
            wv[k] = nw4[ic];
        }
        first_weights();
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            if (threadIdx.x + 256u * k >= n4) rv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            ss = fmaf(rv[k].x, rv[k].x, ss);
            ss = fmaf(rv[k].y, rv[k].y, ss);
            ss = fmaf(rv[k].z, rv[k].z, ss);
            ss = fmaf(rv[k].w, rv[k].w, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);
        const float rms = rsqrtf(ss / (float)K + a.eps);
#pragma unroll
        for (int k = 0; k < P4; ++k) {
            const uint32_t i4 = threadIdx.x + 256u * k;
            if (i4 < n4) {
                float v[4] = {rv[k].x * rms * wv[k].x, rv[k].y * rms * wv[k].y,
                              rv[k].z * rms * wv[k].z, rv[k].w * rms * wv[k].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (FAITH) v[e] = bf16_trunc(v[e]);
                    xs[4 * i4 + e] = (f16_t)v[e];
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = uvalid[j] ? (uint32_t)ll + (uint32_t)(LPR * j) : 0u;
            const uint4 *p = (const uint4 *)(xs + u * 32);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 q = p[i];
                const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    xr[j][8 * i + 2 * t] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[t] & 0xFFFFu));
                    xr[j][8 * i + 2 * t + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[t] >> 16));
                }
            }
        }
    } else if constexpr (MERGE) {
        // The block merges the attention partials into x once -- the merge
        // that would otherwise be a launch of its own -- and builds the
        // nibble tables from it (LUT), or stages it f16 in LDS for every wave.
        // Thread (lane l, wave w) merges columns 8 w .. 8 w + 7 (nibbles 2 w,
        // 2 w + 1) of units u = l + 64 j, so the table entries it writes sit
        // in its own lane's bank column (no bank conflicts), exactly as the
        // lane that reads them in the row loop.  The partials come in the
        // attention's unit-major layout (chunk c, nibble n, unit u: 4 floats
        // at c K + n K / 8 + 4 u), one 16-byte load per (chunk, nibble): a
        // wave's load is 1 KB contiguous.  Each lane derives its head's
        // softmax weights from the head's (m, l) pairs itself, so no block
        // exchange precedes the merge; one barrier follows the tables.
        // All partials of the allocated chunks (<= MERGE_MAX_CHUNKS) are
        // loaded up front, independently of the live length.
        constexpr int NJ = FULL ? NV : 1;   // units per lane (K < 2048: one, lanes >= units idle)
        __shared__ __align__(16) f16_t xs[LUT ? 8 : 2048 * NV];
        const MergeIn &mg = a.mg;
        const uint32_t D = mg.head_dim;
        const int wid = threadIdx.x >> 6;
        const uint32_t kq = K / 8;          // floats per nibble row of a chunk
        // The device sequence length as a vector load issued ahead of the
        // partials' loads, without a branch: a null d_seq gets an empty range,
        // so the load returns 0 without touching memory and seq_len is used.
        // (A scalar load here is hoisted above the vector loads with its wait,
        // and a flat load's completion is not ordered with them.)
        const uint32_t seq_dev = __builtin_amdgcn_raw_buffer_load_b32(
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t *>(mg.d_seq), (short)0,
                                              mg.d_seq ? 4 : 0, 0x00020000),
            0, 0, 0);
        bool mv[NJ];
        uint32_t mu[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint32_t u = (uint32_t)lane + 64u * j;
            mv[j] = u < units;
            mu[j] = mv[j] ? u : 0u;
        }
        // (m, l) of the unit's head for every allocated chunk, then the
        // partial outputs, then the weights
        float2 mlv[NJ][MERGE_MAX_CHUNKS];
        float4 oa[NJ][MERGE_MAX_CHUNKS], ob[NJ][MERGE_MAX_CHUNKS];
        const uint32_t heads = K / D;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const float2 *ml = (const float2 *)mg.part_ml + (mu[j] * 32u) / D;
#pragma unroll
            for (int c = 0; c < MERGE_MAX_CHUNKS; ++c)
                if ((uint32_t)c < mg.nchunks) mlv[j][c] = ml[(size_t)c * heads];
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const float *po = mg.part_o + (size_t)(2 * wid) * kq + mu[j] * 4u;
#pragma unroll
            for (int c = 0; c < MERGE_MAX_CHUNKS; ++c) {
                if ((uint32_t)c < mg.nchunks) {   // launch bound: uniform
                    oa[j][c] = *(const float4 *)(po + (size_t)c * K);
                    ob[j][c] = *(const float4 *)(po + (size_t)c * K + kq);
                }
            }
        }
        first_weights();
        // the length is used from here on only (an empty asm pins the point:
        // hoisted above the loads, its wait would be theirs too)
        uint32_t seq_v = seq_dev;
        asm volatile("" : "+v"(seq_v));
        const uint32_t seq = mg.d_seq ? __builtin_amdgcn_readfirstlane(seq_v) : mg.seq_len;
        const uint32_t nch = min(mg.nchunks, ceil_div(seq, mg.chunk));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            float M = -INFINITY;
#pragma unroll
            for (int c = 0; c < MERGE_MAX_CHUNKS; ++c)
                if ((uint32_t)c < nch) M = fmaxf(M, mlv[j][c].x);
            // the chunk weights exp(m_c - M) <= 1, all computed before any
            // is used (independent, no branch between them) as 2^((m_c - M)
            // log2 e) on the hardware exponential: 3 instructions each
            // instead of the ~19 of a full-range expf (relative difference
            // <= |m_c - M| 2^-24 plus one ulp)
            float wv[MERGE_MAX_CHUNKS];
#pragma unroll
            for (int c = 0; c < MERGE_MAX_CHUNKS; ++c)
                wv[c] = (uint32_t)c < nch ? __builtin_amdgcn_exp2f((mlv[j][c].x - M) * 1.44269504088896341f)
                                          : 0.f;
            float den = 0.f;
            float num[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < MERGE_MAX_CHUNKS; ++c) {
                if ((uint32_t)c < nch) {
                    const float wgt = wv[c];
                    den = fmaf(wgt, mlv[j][c].y, den);
                    num[0] = fmaf(wgt, oa[j][c].x, num[0]); num[1] = fmaf(wgt, oa[j][c].y, num[1]);
                    num[2] = fmaf(wgt, oa[j][c].z, num[2]); num[3] = fmaf(wgt, oa[j][c].w, num[3]);
                    num[4] = fmaf(wgt, ob[j][c].x, num[4]); num[5] = fmaf(wgt, ob[j][c].y, num[5]);
                    num[6] = fmaf(wgt, ob[j][c].z, num[6]); num[7] = fmaf(wgt, ob[j][c].w, num[7]);
                }
            }
            // one division, then products (the f16 result differs from
            // num / den only where the two straddle an f16 rounding edge);
            // a unit past the row end merges to zeros (its tables then read 0)
            const float rden = mv[j] ? 1.f / den : 0.f;
            float x8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x8[e] = (float)(f16_t)(num[e] * rden);
            if constexpr (LUT) {
                float *const dst = lut + (j * 8 + 2 * wid) * 16 * 64 + lane;
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    const float *x4 = x8 + 4 * sb;
                    const float p1 = x4[0] - x4[1], p3 = x4[0] + x4[1];
                    const float q1 = x4[2] - x4[3], q3 = x4[2] + x4[3];
                    const float pp[4] = {-p3, p1, -p1, p3};
                    const float qq[4] = {-q3, q1, -q1, q3};
#pragma unroll
                    for (int e = 0; e < 16; ++e) dst[(sb * 16 + e) * 64] = pp[e & 3] + qq[e >> 2];
                }
            } else if (mv[j]) {
                uint4 h;
                h.x = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[0]) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[1]) << 16);
                h.y = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[2]) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[3]) << 16);
                h.z = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[4]) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[5]) << 16);
                h.w = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[6]) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, (f16_t)x8[7]) << 16);
                *(uint4 *)(xs + mu[j] * 32u + 8u * (uint32_t)wid) = h;
            }
        }
        __syncthreads();
        if constexpr (!LUT) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const uint32_t u = uvalid[j] ? (uint32_t)ll + (uint32_t)(LPR * j) : 0u;
                const uint4 *p = (const uint4 *)(xs + u * 32);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 q = p[i];
                    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        xr[j][8 * i + 2 * t] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[t] & 0xFFFFu));
                        xr[j][8 * i + 2 * t + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[t] >> 16));
                    }
                }
            }
        }
    } else {
        // unconditional loads (unit 0 stands in past the row end): raw
        // 16-byte vectors first, converted after the weight loads are out
        constexpr int XV = XDT == NNZ_F32 ? 8 : 4;   // 16-byte loads per unit
        uint4 xraw[NV][XV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = uvalid[j] ? (uint32_t)ll + (uint32_t)(LPR * j) : 0u;
            const uint4 *p = XDT == NNZ_F32 ? (const uint4 *)((const float *)ax + (size_t)u * 32)
                                            : (const uint4 *)((const uint16_t *)ax + (size_t)u * 32);
#pragma unroll
            for (int i = 0; i < XV; ++i) xraw[j][i] = p[i];
        }
        first_weights();
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (XDT == NNZ_F32) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint4 v = xraw[j][i];
                    xr[j][4 * i] = __uint_as_float(v.x); xr[j][4 * i + 1] = __uint_as_float(v.y);
                    xr[j][4 * i + 2] = __uint_as_float(v.z); xr[j][4 * i + 3] = __uint_as_float(v.w);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint4 v = xraw[j][i];
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
    if constexpr (!LUT) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) s += xr[j][i];
            xsum[j] = s;
        }
    }

    // ---- software-pipelined row loop ---------------------------------------
    // Two register sets used alternately (the loop body appears twice), so
    // the next step's weights land in the set not being read and nothing is
    // copied at the back edge.  (A third set for the 8-row steps of the LM
    // head, one more step of loads in flight per wave, measured slower:
    // 13.2 -> 15.0 us.)
    const uint32_t stride = nwaves * rows_per_iter;
    // nibble-table addresses: byte 0 = lane * 4, byte 1 = the nibble (the
    // table of one (unit, nibble) pair is 16 entries x 64 lanes x 4 bytes)
    const uint32_t lane4 = (uint32_t)lane * 4u;
    auto row_step = [&](StepRegs<NMAT, R, NV, VEC> &c, StepRegs<NMAT, R, NV, VEC> &n) {
        // Past the last step a wave re-reads its own rows (cache hits): the
        // clamped rows [M - R, M) would be one hot spot for every wave.
        const uint32_t next = base + stride;
        load_rows(n, next < a.M ? next : base);

        float acc[NMAT][R];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float accv = 0.f;
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    if constexpr (BITS == 1 && LUT) {
                        // A unit past the row end has all-zero tables, and a
                        // row past M is never stored: no validity select.
                        // Q1 scales are f16.
                        const float s = (float)__builtin_bit_cast(f16_t, c.sc[m][r][j]);
                        const uint32_t w = c.cw[m][r][j][0];
                        const uint32_t wl = w & 0x0F0F0F0Fu, wh = (w >> 4) & 0x0F0F0F0Fu;
                        const char *tb = (const char *)(lut + (j * 8 * 16) * 64);
                        float t[8];
#pragma unroll
                        for (int n = 0; n < 8; ++n) {
                            // nibble n is byte n/2 of wl (n even) or wh (n odd)
                            const uint32_t sel = 0x0C0C0000u | ((4u + (uint32_t)(n >> 1)) << 8);
                            const uint32_t off = __builtin_amdgcn_perm((n & 1) ? wh : wl, lane4, sel);
                            t[n] = *(const float *)(tb + n * 16 * 64 * 4 + off);
                        }
                        float sb = t[0];
#pragma unroll
                        for (int n = 1; n < 8; ++n) sb += t[n];
                        accv = fmaf(s, sb, accv);
                    } else if constexpr (BITS == 1) {
                        const bool ok = FULL ? lu.ok[j] : c.ok[m][r][j];
                        const float s = ok ? (float)__builtin_bit_cast(f16_t, c.sc[m][r][j]) : 0.f;
                        const uint32_t w = c.cw[m][r][j][0];
                        float sb = 0.f;
#pragma unroll
                        for (int i = 0; i < 32; ++i) {
                            const int mask = ((int)(w << (31 - i))) >> 31;  // 0 or -1
                            sb += __int_as_float(mask & __float_as_int(xr[j][i]));
                        }
                        accv = fmaf(s, 2.f * sb - xsum[j], accv);
                    } else {
                        const bool ok = FULL ? lu.ok[j] : c.ok[m][r][j];
                        const float s = ok ? scale_to_f32(c.sc[m][r][j], (int)a.sdt) : 0.f;
                        float nd = 0.f;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t w = c.cw[m][r][j][k];
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
                        const float b = ok ? scale_to_f32(c.bi[m][r][j], (int)a.sdt) : 0.f;
                        accv = fmaf(s, nd, fmaf(b, xsum[j], accv));
                    }
                }
                acc[m][r] = accv;
            }

        // Row sums: DPP reductions for full-wave rows, lane-group
        // shuffles for narrow ones.
        const uint32_t rb = FULL ? step_base(base) : base;
        uint32_t seg_start = 0;
        int seg = 0;
        if constexpr (NMAT == 1) seg = step_segment(a, rb, seg_start);
        void *out0 = stk<STK>(NMAT == 1 ? (seg == 0 ? a.m0.out : (seg == 1 ? a.m1.out : a.m2.out)) : a.m0.out,
                         a.stk.out);
        if constexpr (FULL) {
            // The NMAT x R row totals in one exchange-halving reduction
            // (slot r * NMAT + m); the lanes heading each slot's lane group
            // store.  A pair's two totals of a row sit in lanes l and l ^ 32.
            constexpr int V = NMAT * R;
            float vals[V];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < NMAT; ++m) vals[r * NMAT + m] = acc[m][r];
            const float t = multi_row_sum<V>(vals);
            const int slot = multi_row_slot<V>();
            const int r = slot / NMAT;
            float tot[NMAT];
            tot[0] = t;
            if constexpr (NMAT == 2) {
                const float2 p = swap32(t, t);   // the partner half's total
                tot[1] = p.y;                    // lanes < 32 hold m = 0 and read m = 1
            }
            const uint32_t row = rb + (uint32_t)r;   // < M
            const bool head = (lane & ((64 / V) - 1)) == 0 && (NMAT == 1 || lane < 32);
            if (head && row >= base)
                qmv_epilogue<EPI, ODT, FAITH, NMAT, STK>(a, out0, row, row - seg_start, tot, c.res[0]);
            if constexpr (TOP2) {
                // the stored value; a lane's rows ascend, so a tie keeps the first
                const float v = FAITH ? bf16_trunc(tot[0]) : tot[0];
                if (a.top2 && head && row >= base) {
                    if (v > t2.best) { t2.second = t2.best; t2.best = v; t2.idx = row; }
                    else if (v > t2.second) t2.second = v;
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float tot[NMAT];
#pragma unroll
                for (int m = 0; m < NMAT; ++m) tot[m] = group_sum(acc[m][r], LPR);
                const uint32_t row = base + (uint32_t)(r * RPW + rr);
                if (ll == 0 && row < a.M)
                    qmv_epilogue<EPI, ODT, FAITH, NMAT, STK>(a, out0, row, row - seg_start, tot, c.res[r]);
            }
        }
    };
    StepRegs<NMAT, R, NV, VEC> nxt;
    while (base < a.M) {
        row_step(cur, nxt);
        base += stride;
        if (base >= a.M) break;
        row_step(nxt, cur);
        base += stride;
    }
    if constexpr (TOP2) {
        // the block's greedy top-2 (merged across the wave, then the waves)
        if (a.top2) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                NnzTop2 o;
                o.best = __shfl_xor(t2.best, off, 64);
                o.second = __shfl_xor(t2.second, off, 64);
                o.idx = (uint32_t)__shfl_xor((int)t2.idx, off, 64);
                t2 = nnz_top2_merge(t2, o);
            }
            __shared__ NnzTop2 t2sh[4];
            if (lane == 0) t2sh[threadIdx.x >> 6] = t2;
            __syncthreads();
            if (threadIdx.x == 0)
                a.top2[blockIdx.x] = nnz_top2_merge(nnz_top2_merge(t2sh[0], t2sh[1]),
                                                    nnz_top2_merge(t2sh[2], t2sh[3]));
        }
    }
}

// ---------------------------------------------------------------------------
// Split-K QMV for long 1-bit rows (64*32*(KS-1) < K <= 64*32*KS, KS = 2..8): the KS waves of
// a block share R rows and wave k takes units [64k, 64k + 64), one per
// lane, so each wave's x slice, bit loop and row reduction are a KS-th of
// the full-row kernel's and a SIMD interleaves several short waves instead
// of running one long one.  The KS row partials meet in LDS (double
// buffered: one barrier per step).
template <int XDT, int EPI, int ODT, int KS, int R, bool STK>
__global__ __launch_bounds__(64 * KS) void qmv1_splitk_kernel(QmvArgs a) {
    static_assert(EPI == EPI_STORE || EPI == EPI_RESADD, "store or residual add");
    const int lane = threadIdx.x & 63, kp = threadIdx.x >> 6;
    const void *const ax = stk<STK>(a.x, a.stk.x);
    const uint32_t K = a.K, units = K >> 5, G = K / a.gs, M = a.M;
    const uint32_t u = (uint32_t)(kp * 64 + lane);
    const bool uv = u < units;
    const uint32_t uc = uv ? u : 0u;
    const gptr<const uint32_t> codes = stk<STK>(uniform_ptr(a.m0.codes), a.stk.codes);
    const gptr<const uint16_t> scales = stk<STK>(uniform_ptr(a.m0.scales), a.stk.scales);
    float *const out = stk<STK>((float *)a.m0.out, a.stk.out);
    __shared__ float part[2][KS][R];

    struct Step { uint32_t cw[R]; uint16_t sc[R]; float prev; };
    auto load = [&](uint32_t base, Step &st) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = base + r;
            const uint32_t lr = row < M ? row : 0u;
            st.cw[r] = codes[(size_t)lr * units + uc];
            st.sc[r] = scales[(size_t)lr * G + (uc * 32u) / a.gs];
        }
        if constexpr (EPI == EPI_RESADD) {   // residual row of lane r (wave 0)
            const uint32_t row = base + (uint32_t)lane;
            st.prev = (kp == 0 && lane < R && row < M) ? out[row] : 0.f;
        }
    };

    uint32_t base = blockIdx.x * R;
    const uint32_t stride = gridDim.x * R;

    // this lane's 32 x values first (unit 0 stands in past the row end; its
    // scale is zeroed below), then the first step's weights: loads complete
    // in issue order, so the x conversion does not wait for the weights
    constexpr int XV = XDT == NNZ_F32 ? 8 : 4;
    uint4 xraw[XV];
    {
        const uint4 *p = XDT == NNZ_F32 ? (const uint4 *)((const float *)ax + (size_t)uc * 32)
                                        : (const uint4 *)((const uint16_t *)ax + (size_t)uc * 32);
#pragma unroll
        for (int i = 0; i < XV; ++i) xraw[i] = p[i];
    }
    Step cur;
    load(base < M ? base : 0u, cur);   // never branched around (see qmv_kernel)
    float xr[32], xsum = 0.f;
    if constexpr (XDT == NNZ_F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xr[4 * i] = __uint_as_float(xraw[i].x); xr[4 * i + 1] = __uint_as_float(xraw[i].y);
            xr[4 * i + 2] = __uint_as_float(xraw[i].z); xr[4 * i + 3] = __uint_as_float(xraw[i].w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t wv[4] = {xraw[i].x, xraw[i].y, xraw[i].z, xraw[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint16_t lo = (uint16_t)(wv[t] & 0xFFFFu), hi = (uint16_t)(wv[t] >> 16);
                if constexpr (XDT == NNZ_F16) {
                    xr[8 * i + 2 * t] = (float)__builtin_bit_cast(f16_t, lo);
                    xr[8 * i + 2 * t + 1] = (float)__builtin_bit_cast(f16_t, hi);
                } else {
                    xr[8 * i + 2 * t] = bf16_to_f32(lo);
                    xr[8 * i + 2 * t + 1] = bf16_to_f32(hi);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) xsum += xr[i];
    uint32_t xw[16];   // f16 x: column pairs (2p, 2p + 1) as loaded
    if constexpr (XDT == NNZ_F16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xw[4 * i] = xraw[i].x; xw[4 * i + 1] = xraw[i].y;
            xw[4 * i + 2] = xraw[i].z; xw[4 * i + 3] = xraw[i].w;
        }
    }

    for (int it = 0; base < M; base += stride, ++it) {
        Step nxt;
        load(base + stride < M ? base + stride : base, nxt);
        const int buf = it & 1;
        float pr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w = cur.cw[r];
            if constexpr (XDT == NNZ_F16) {
                // f16 x: the 32 weights as 16 pairs of f16 +-s (the sign of
                // each half from one bit, as the prefill GEMM expands them)
                // into v_dot2 with the x pairs, f32 accumulation: s * x is
                // exact, so this is the f32 sum of the same products
                const uint32_t s16 = uv ? (uint32_t)cur.sc[r] : 0u;
                const uint32_t ns2 = (s16 | (s16 << 16)) ^ 0x80008000u;   // (-s, -s)
                float acc = 0.f;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t z = (w >> (8 * b)) & 0xFFu;
                    uint32_t z2;   // the byte twice, 15 bits apart (kept from being folded into a multiply)
                    asm("v_lshl_or_b32 %0, %1, 15, %1" : "=v"(z2) : "v"(z));
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t pr2 = ((z2 << (15 - 2 * q)) & 0x80008000u) ^ ns2;
                        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, pr2),
                                                     __builtin_bit_cast(h2v, xw[4 * b + q]), acc, false);
                    }
                }
                pr[r] = acc;
            } else {
                float sb = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int mask = ((int)(w << (31 - i))) >> 31;  // 0 or -1
                    sb += __int_as_float(mask & __float_as_int(xr[i]));
                }
                const float sc = uv ? (float)__builtin_bit_cast(f16_t, cur.sc[r]) : 0.f;
                pr[r] = sc * (2.f * sb - xsum);
            }
        }
        // the R row partials of this wave in one exchange-halving reduction
        const float p = multi_row_sum<R>(pr);
        if ((lane & (64 / R - 1)) == 0) part[buf][kp][multi_row_slot<R>()] = p;
        __syncthreads();
        if (kp == 0 && lane < R) {
            float t = 0.f;
#pragma unroll
            for (int k = 0; k < KS; ++k) t += part[buf][k][lane];
            const uint32_t row = base + (uint32_t)lane;
            if (row < M) {
                if constexpr (EPI == EPI_RESADD) out[row] = cur.prev + t;
                else store_from_f32<ODT>(out, row, t);
            }
        }
        cur = nxt;
    }
}

// Whether a 1-bit QMV of this shape goes to the block-scaled MFMA kernel:
// the context's NNZ_OPT_Q1_MATRIX_CORES, by default for stacked launches
// only, where its per-block set-up (a 64 KB fp4 table, the input's digit
// rows) is amortised over many rows (measured, stacked config-3 pairs: 168
// against 203 us; the 1-bit LM head, ~4.6 tiles per wave: 16.4 against
// 14.5 us, so it stays on the VALU kernel).
bool q1_matrix_cores_wanted(nnz_ctx *ctx, const nnz_qmv_dims &d, bool stacked) {
    if (!nnz_q1_mfma_supported(d.K, d.group_size) || ctx->q1_matrix_cores == 2) return false;
    return ctx->q1_matrix_cores == 1 || stacked;
}

// Blocks per matrix of a stacked launch: the caller's choice, else enough
// for about 8192 blocks in all (measured, 256 config-1 matrices: 32 blocks
// each 0.70 of 8 TB/s, 8 each 0.62), never more than a single launch of the
// shape would use.
uint32_t stack_blocks(const nnz_qmv_stack *stk, uint32_t single) {
    uint32_t b = stk->blocks_per_matrix ? stk->blocks_per_matrix : ceil_div(8192u, stk->count);
    return b < 1 ? 1 : (b > single ? single : b);
}

int check_weight(nnz_ctx *ctx, const nnz_qweight *w, int bits, uint32_t M, const nnz_qmv_dims &d,
                 const char *name) {
    NNZ_REQUIRE(ctx, w != nullptr, NNZ_EINVAL, "%s: null weight descriptor", name);
    NNZ_REQUIRE(ctx, w->codes && w->scales, NNZ_EINVAL, "%s: null codes/scales", name);
    NNZ_REQUIRE(ctx, (int)w->bits == bits, NNZ_EINVAL, "%s: weight has %u bits, kernel needs %d",
                name, w->bits, bits);
    NNZ_REQUIRE(ctx, (uint64_t)w->packed_count == (uint64_t)M * d.K, NNZ_EINVAL,
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
    NNZ_REQUIRE(ctx, d.K <= 16384, NNZ_EUNSUPPORTED, "%s: K=%u > 16384 not supported", name, d.K);
    return NNZ_OK;
}

// The variants the stacked entry points launch (f32 in and out): Q1 and Q4
// single matrices, the Q1 pair with SiLU.
template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH>
constexpr bool stackable() {
    return XIN == XIN_X && !FAITH && XDT == NNZ_F32 && ODT == NNZ_F32 &&
           ((NMAT == 1 && EPI == EPI_STORE) || (BITS == 1 && NMAT == 2 && EPI == EPI_SILU));
}

// Nibble tables take NV * 32 KB of LDS per block.
constexpr int LUT_MAX_NV = 3;

// Weight words a lane holds for one row-step; the host keeps it <= 32.
constexpr int step_words(int BITS, int NMAT, int NV, int R) { return NMAT * R * NV * (BITS == 1 ? 1 : 4); }

template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH, int NV, bool LUT, bool FULL>
void launch_r(nnz_ctx *ctx, const QmvArgs &a, int R, uint32_t blocks, uint32_t gy) {
    dim3 grid(blocks, gy), block(256);
    // stacked launches (gy > 1) of the stackable variants take the kernel
    // with per-matrix offsets; every other launch the one without
    constexpr bool STACKABLE = stackable<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH>();
#define QK(RR)                                                                                           \
    do {                                                                                                 \
        if constexpr (STACKABLE) {                                                                       \
            if (gy > 1) {                                                                                \
                qmv_kernel<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, RR, LUT, FULL, true>               \
                    <<<grid, block, 0, ctx->stream>>>(a);                                                \
                break;                                                                                   \
            }                                                                                            \
        }                                                                                                \
        qmv_kernel<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, RR, LUT, FULL, false><<<grid, block, 0, ctx->stream>>>(a); \
    } while (0)
    if (R == 8) {
        // long matrices only (the 1-bit LM head): more rows in flight per wave
        if constexpr (LUT && NMAT == 1 && step_words(BITS, NMAT, NV, 8) <= 32) QK(8);
        else R = 4;
    }
    if (R == 4) {
        if constexpr (step_words(BITS, NMAT, NV, 4) <= 32) QK(4);
        else R = 1;
    } else if (R == 2) {
        if constexpr (step_words(BITS, NMAT, NV, 2) <= 32) QK(2);
        else R = 1;
    }
    if (R == 1) QK(1);
#undef QK
}

template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH, int NV>
int launch_nv(nnz_ctx *ctx, const QmvArgs &a, int R, uint32_t blocks, bool lut, uint32_t gy) {
    if constexpr (XIN == XIN_MERGE && NV > 2) {
        // the merge prologue keeps every chunk's partials in registers
        return nnz_fail(ctx, NNZ_EUNSUPPORTED, "merge_o_resadd: K > 4096");
    } else {
        // rows narrower than a wave (K < 2048) occur only with one unit per lane
        const bool full = a.lpr_log2 == 6;
        if constexpr (BITS == 1 && NV <= LUT_MAX_NV) {
            if (lut) launch_r<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, true, true>(ctx, a, R, blocks, gy);
            else if (full) launch_r<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, false, true>(ctx, a, R, blocks, gy);
            else if constexpr (NV == 1) launch_r<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, false, false>(ctx, a, R, blocks, gy);
        } else if (full) {
            launch_r<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, false, true>(ctx, a, R, blocks, gy);
        } else if constexpr (NV == 1) {
            launch_r<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, NV, false, false>(ctx, a, R, blocks, gy);
        }
        NNZ_LAUNCHED(ctx);
        return NNZ_OK;
    }
}

// `w[0..nw)` are either a pair sharing rows (NMAT == 2) or row segments of
// one concatenated matrix (NMAT == 1, seg_rows[s] rows each).
template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH>
int launch_qmv_ex(nnz_ctx *ctx, const nnz_qweight *const *w, const uint32_t *seg_rows, int nw,
                  const void *x, const float *norm_w, void *const *out, nnz_qmv_dims d,
                  const char *name, const MergeIn *merge = nullptr, float eps = 1e-6f,
                  const nnz_qmv_stack *stk = nullptr, NnzTop2 *top2 = nullptr) {
    constexpr bool NORM = XIN == XIN_NORM;
    constexpr bool MERGE = XIN == XIN_MERGE;
    constexpr bool STACKABLE = stackable<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH>();
    NNZ_CHECK_CTX(ctx);
    int rc = check_dims(ctx, d, name);
    if (rc) return rc;
    NNZ_REQUIRE(ctx, !stk || STACKABLE, NNZ_EUNSUPPORTED, "%s: no stacked form", name);
    // Stacked launch: `count` matrices of this shape at fixed byte strides,
    // one block row each (x and the outputs advance by their own strides).
    const uint32_t gy = stk ? stk->count : 1u;
    if (stk) {
        NNZ_REQUIRE(ctx, !MERGE && !NORM && nw == 1 + (NMAT == 2), NNZ_EUNSUPPORTED,
                    "%s: stacking takes one matrix or a pair with a plain input", name);
        NNZ_REQUIRE(ctx, stk->count >= 1 && stk->count <= 65535, NNZ_EINVAL,
                    "%s: stack count %u (1..65535)", name, stk->count);
        NNZ_REQUIRE(ctx, stk->codes_stride % 16 == 0 && stk->scales_stride % 4 == 0 &&
                             stk->input_stride % 16 == 0 && stk->output_stride % 4 == 0,
                    NNZ_EINVAL, "%s: stack strides must keep the 16/4/16/4-byte alignments", name);
    }
    uint32_t total = 0;
    for (int i = 0; i < nw; ++i) {
        const uint32_t rows = NMAT == 1 ? seg_rows[i] : d.M;
        rc = check_weight(ctx, w[i], BITS, rows, d, name);
        if (rc) return rc;
        NNZ_REQUIRE(ctx, w[i]->scale_dtype == w[0]->scale_dtype, NNZ_EINVAL,
                    "%s: weights differ in scale dtype", name);
        NNZ_REQUIRE(ctx, out[i] != nullptr || (EPI != EPI_STORE && i > 0), NNZ_EINVAL,
                    "%s: null output", name);
        total += rows;
    }
    if (NMAT == 1) NNZ_REQUIRE(ctx, total == d.M, NNZ_EINVAL, "%s: segments do not add up to M", name);
    // whole-row steps address a matrix through 32-bit byte offsets
    NNZ_REQUIRE(ctx, (uint64_t)d.M * d.K * BITS / 8 < (1ull << 32), NNZ_EUNSUPPORTED,
                "%s: matrix of %llu bytes (4 GiB at most)", name,
                (unsigned long long)((uint64_t)d.M * d.K * BITS / 8));
    NNZ_REQUIRE(ctx, EPI != EPI_RESADD || nw == 1, NNZ_EINVAL, "%s: residual add takes one matrix", name);
    if (MERGE) {
        NNZ_REQUIRE(ctx, merge && merge->part_o && merge->part_ml, NNZ_EINVAL, "%s: null partials", name);
        NNZ_REQUIRE(ctx, merge->nchunks >= 1 && merge->nchunks <= (uint32_t)MERGE_MAX_CHUNKS &&
                             merge->chunk > 0 && merge->head_dim % 8 == 0 && d.K % merge->head_dim == 0 &&
                             ((uintptr_t)merge->part_o & 15) == 0 && ((uintptr_t)merge->part_ml & 7) == 0,
                    NNZ_EUNSUPPORTED, "%s: bad attention partials", name);
    } else {
        NNZ_REQUIRE(ctx, x != nullptr, NNZ_EINVAL, "%s: null input", name);
        NNZ_REQUIRE(ctx, ((uintptr_t)x & 15) == 0, NNZ_EINVAL, "%s: input must be 16-byte aligned", name);
    }
    if (NORM) {
        NNZ_REQUIRE(ctx, norm_w != nullptr, NNZ_EINVAL, "%s: null norm_scale", name);
        NNZ_REQUIRE(ctx, ((uintptr_t)norm_w & 15) == 0, NNZ_EINVAL,
                    "%s: norm_scale must be 16-byte aligned", name);
    }

    // 1-bit rows of K = 2048, group size 128: the block-scaled MFMA kernel
    // (qmv_mfma.hip) where the context's policy picks it.
    NNZ_REQUIRE(ctx, !top2 || (EPI == EPI_STORE && NMAT == 1 && ODT == NNZ_F32 && nw == 1 && !stk),
                NNZ_EUNSUPPORTED, "%s: top-2 partials need one f32-output matrix", name);
    if constexpr (BITS == 1 && !FAITH && !MERGE) {
        if (!top2 && q1_matrix_cores_wanted(ctx, d, stk != nullptr) && (NMAT == 2 || nw == 1)) {
            NnzQ1Mfma c;
            for (int i = 0; i < NMAT; ++i) {
                c.codes[i] = w[i]->codes;
                c.scales[i] = w[i]->scales;
            }
            c.x = x;
            c.norm_w = norm_w;
            c.out = out[0];
            c.M = d.M;
            c.K = d.K;
            c.group_size = d.group_size;
            c.nmat = NMAT;
            c.xdt = XDT;
            c.xin = NORM ? 1 : 0;
            c.epi = EPI == EPI_STORE ? 0 : (EPI == EPI_RESADD ? 1 : 2);
            c.odt = ODT;
            c.eps = eps;
            if (stk) {
                c.stack_count = stk->count;
                c.blocks_per_matrix = stk->blocks_per_matrix;
                c.cs = stk->codes_stride;
                c.ss = stk->scales_stride;
                c.xs = stk->input_stride;
                c.os = stk->output_stride;
            }
            if (nnz_q1_mfma_has_variant(c)) return nnz_q1_mfma_launch(ctx, c);
        }
    }
    const uint32_t units = d.K / 32;
    uint32_t lpr = 1;
    while (lpr < units && lpr < 64) lpr <<= 1;
    int lpr_log2 = 0;
    while ((1u << lpr_log2) < lpr) ++lpr_log2;
    const uint32_t nv = ceil_div(units, lpr);
    NNZ_REQUIRE(ctx, nv >= 1 && nv <= 8, NNZ_EUNSUPPORTED, "%s: K=%u needs %u units/lane", name, d.K, nv);
    const uint32_t rpw = 64 / lpr;
    const int vec = BITS == 1 ? 1 : 4;
    if constexpr (BITS == 1 && XIN == XIN_X && NMAT == 1 && !FAITH &&
                  (EPI == EPI_STORE || EPI == EPI_RESADD)) {
        // long single-segment rows: split K over the waves of a block (the
        // last wave may be partly idle: K = 9728 is 4 full waves + 48 units)
        if (nw == 1 && lpr == 64 && nv >= 2 && nv <= 8) {
            constexpr int SR = 4;
            QmvArgs a{};
            a.m0.codes = (const uint32_t *)w[0]->codes;
            a.m0.scales = (const uint16_t *)w[0]->scales;
            a.m0.out = out[0];
            a.m0.seg_end = d.M;
            a.nseg = 1;
            a.x = x;
            a.M = d.M;
            a.K = d.K;
            a.gs = d.group_size;
            a.sdt = w[0]->scale_dtype;
            uint32_t blocks = ceil_div(d.M, (uint32_t)SR);
            if (blocks > 4096) blocks = 4096;
            if (stk) {
                a.stk = {stk->codes_stride, stk->scales_stride, stk->input_stride, stk->output_stride};
                blocks = stack_blocks(stk, blocks);
            }
            const dim3 grid(blocks, gy);
            // the stacked form only for the stackable shape (config 2's)
#define SPLITK(KS_, TH_)                                                                          \
    do {                                                                                          \
        if constexpr (STACKABLE) {                                                                \
            if (gy > 1) {                                                                         \
                qmv1_splitk_kernel<XDT, EPI, ODT, KS_, SR, true><<<grid, TH_, 0, ctx->stream>>>(a); \
                break;                                                                            \
            }                                                                                     \
        }                                                                                         \
        qmv1_splitk_kernel<XDT, EPI, ODT, KS_, SR, false><<<grid, TH_, 0, ctx->stream>>>(a);      \
    } while (0)
            switch (nv) {
            case 2: SPLITK(2, 128); break;
            case 3: SPLITK(3, 192); break;
            case 4: SPLITK(4, 256); break;
            case 5: SPLITK(5, 320); break;
            case 6: SPLITK(6, 384); break;
            case 7: SPLITK(7, 448); break;
            default: SPLITK(8, 512); break;
            }
#undef SPLITK
            NNZ_LAUNCHED(ctx);
            return NNZ_OK;
        }
    }
    // the full-row kernel holds up to 4 units per lane (K <= 8192)
    NNZ_REQUIRE(ctx, nv <= 4, NNZ_EUNSUPPORTED, "%s: K=%u needs %u units/lane (this form: K <= 8192)",
                name, d.K, nv);
    int R = 4;
    // Rows per wave-step: as many as keep about one block per CU (pairs and
    // 4-bit matrices: two; config 1 5.55 -> 5.34 us, 4-bit decode +2 %) --
    // measured best for the decode shapes -- bounded by the weight words a
    // lane holds in flight (two steps are live).
    const uint32_t min_blocks = NMAT == 2 || BITS == 4 ? 512u : 256u;
    while (R > 1 && (ceil_div(d.M, 4u * R * rpw) < min_blocks || NMAT * R * (int)nv * vec > 32)) R >>= 1;
    // a stacked launch has blocks enough: four rows per step, twice the
    // bytes in flight per wave (stacked 4-bit config-1 matrices: 0.68-0.70 ->
    // 0.71-0.73 of 8 TB/s; eight rows: 0.67-0.71)
    if (stk && NMAT * 4 * (int)nv * vec <= 32) R = 4;
    // 1-bit full-wave rows may use the nibble tables.  Building them is a
    // fixed cost per block that pays off from about four matrix rows per
    // wave: pairs take two rows per wave.
    bool lut = BITS == 1 && lpr == 64 && nv <= (uint32_t)LUT_MAX_NV;
    if (lut && NMAT == 2 && R < 2 && 2 * 2 * (int)nv * vec <= 32) R = 2;
    if (lut && NMAT == 1 && d.M >= 4u * 2048u * 8u) R = 8;   // e.g. a vocabulary-sized LM head
    if (NMAT == 1 && nw > 1) {  // a step must not straddle two segments
        auto aligned = [&](uint32_t step) {
            for (int i = 0; i < nw; ++i)
                if (seg_rows[i] % step) return false;
            return true;
        };
        while (R > 1 && !aligned((uint32_t)R * rpw)) R >>= 1;
        NNZ_REQUIRE(ctx, aligned(rpw), NNZ_EUNSUPPORTED,
                    "%s: segment rows must be multiples of %u", name, rpw);
    }
    uint32_t blocks = ceil_div(d.M, 4u * R * rpw);
    // Every wave re-reads its x slice (and, with the norm prologue, the
    // residual and norm weights): cap the grid so large matrices amortise
    // that over several row-steps per wave (measured: the normalised gate/up
    // pair at 512 blocks instead of 768, 4.37 -> 3.81 us; the plain pair and
    // single matrices do best uncapped up to 2048 / 1024).
    const uint32_t max_blocks = NORM ? (NMAT == 2 ? 512u : 1024u) : 2048u;
    if (blocks > max_blocks) blocks = max_blocks;
    if (MERGE) {
        // every block re-reads all partials: fewer, fuller blocks
        while (R < 4 && NMAT * 2 * R * (int)nv * vec <= 32 && ceil_div(d.M, 4u * R * rpw) > 256) R <<= 1;
        blocks = ceil_div(d.M, 4u * R * rpw);
    }
    if (lpr == 64 && d.M < (uint32_t)R) {
        // whole-wave rows: a step's R rows must exist (the last step is
        // clamped back onto rows [M - R, M))
        while (R > 1 && d.M < (uint32_t)R) R >>= 1;
        blocks = ceil_div(d.M, 4u * R * rpw);
    }
    if (stk) blocks = stack_blocks(stk, blocks);
    // measured: tables pay off from 4 row-units per wave (fused Q/K/V, 4
    // rows per wave: 3.55 us without, 3.16 us with)
    // (the merge keeps its tables at any row count: built from the merged
    // values, they measured 0.2-0.5 us faster than the f16 staging)
    if (lut && ceil_div(d.M, blocks * 4u) * NMAT < 4u && !MERGE) lut = false;

    QmvArgs a{};
    for (int i = 0; i < nw; ++i) {
        QmvMat &mm = i == 0 ? a.m0 : (i == 1 ? a.m1 : a.m2);
        mm.codes = (const uint32_t *)w[i]->codes;
        mm.scales = (const uint16_t *)w[i]->scales;
        mm.biases = (const uint16_t *)w[i]->biases;
        mm.out = out[i];
    }
    a.nseg = NMAT == 1 ? (uint32_t)nw : 1;
    uint32_t acc = 0;
    for (int i = 0; i < MAX_SEG; ++i) {
        if (NMAT == 1 && i < nw) acc += seg_rows[i];
        (i == 0 ? a.m0 : (i == 1 ? a.m1 : a.m2)).seg_end = NMAT == 1 ? acc : d.M;
    }
    a.x = x;
    a.norm_w = norm_w;
    if (MERGE) a.mg = *merge;
    if (top2) {
        // whole-wave rows only (the partial is built from the row heads)
        NNZ_REQUIRE(ctx, lpr == 64 && blocks <= NNZ_TOP2_MAX, NNZ_EUNSUPPORTED,
                    "%s: top-2 partials need K >= 2048 and at most %u blocks", name, NNZ_TOP2_MAX);
        a.top2 = top2;
    }
    a.M = d.M;
    a.K = d.K;
    a.gs = d.group_size;
    a.lpr_log2 = (uint32_t)lpr_log2;
    a.sdt = w[0]->scale_dtype;
    a.eps = eps;
    if (stk) a.stk = {stk->codes_stride, stk->scales_stride, stk->input_stride, stk->output_stride};
    switch (nv) {
    case 1: return launch_nv<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, 1>(ctx, a, R, blocks, lut, gy);
    case 2: return launch_nv<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, 2>(ctx, a, R, blocks, lut, gy);
    case 3: return launch_nv<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, 3>(ctx, a, R, blocks, lut, gy);
    default: return launch_nv<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH, 4>(ctx, a, R, blocks, lut, gy);
    }
}

template <int BITS, int XDT, int NMAT, int XIN, int EPI, int ODT, bool FAITH>
int launch_qmv(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *x,
               const float *norm_w, void *out0, void *out1, nnz_qmv_dims d, const char *name,
               float eps = 1e-6f, NnzTop2 *top2 = nullptr) {
    const nnz_qweight *w[2] = {wa, wb};
    void *out[2] = {out0, out1};
    const uint32_t rows[1] = {d.M};
    if (NMAT == 2) NNZ_REQUIRE(ctx, wb != nullptr, NNZ_EINVAL, "%s: null second weight", name);
    return launch_qmv_ex<BITS, XDT, NMAT, XIN, EPI, ODT, FAITH>(ctx, w, rows, NMAT, x, norm_w, out, d,
                                                                  name, nullptr, eps, nullptr, top2);
}

}  // namespace

// ---------------------------------------------------------------------------
// Internal fused launches used by the decoder (csrc/model.hip).
// ---------------------------------------------------------------------------

// The decoder's fused launches take the form of the weights: 1-bit (Q1) or
// 4-bit with the reference's BF16-faithful rounding (Q4: fused-norm input
// BF16-truncated before f16, results BF16-truncated before the store or +=,
// q4mv_bf16_specialized.metal:52-57, :806).

// RMSNorm prologue + Q, K and V projections in one launch (f16 outputs).
// `eps` is the model's RMSNorm epsilon (the reference's fused kernels use
// 1e-6, qmv_specialized.metal:1158; the public dispatchers keep that value).
int nnz_qmv_norm_qkv_launch(nnz_ctx *ctx, const nnz_qweight *wq, const nnz_qweight *wk,
                            const nnz_qweight *wv, const float *residual, const float *norm_w,
                            void *q, void *k, void *v, uint32_t qrows, uint32_t kvrows, uint32_t K,
                            uint32_t gs, float eps) {
    const nnz_qweight *w[3] = {wq, wk, wv};
    void *out[3] = {q, k, v};
    const uint32_t rows[3] = {qrows, kvrows, kvrows};
    NNZ_REQUIRE(ctx, wq != nullptr, NNZ_EINVAL, "norm_qkv: null weight");
    if (wq->bits == 4)
        return launch_qmv_ex<4, NNZ_F32, 1, true, EPI_STORE, NNZ_F16, true>(
            ctx, w, rows, 3, residual, norm_w, out, {qrows + 2 * kvrows, K, gs}, "q4_norm_qkv",
            nullptr, eps);
    return launch_qmv_ex<1, NNZ_F32, 1, true, EPI_STORE, NNZ_F16, false>(
        ctx, w, rows, 3, residual, norm_w, out, {qrows + 2 * kvrows, K, gs}, "norm_qkv", nullptr,
        eps);
}

// RMSNorm prologue + gate/up pair + SiLU*mul (f16 output) with the model's
// epsilon: the reference's qmv_spec_fused_norm_pair_silu_f16io /
// q4mv_spec_fused_norm_pair_silu_f16io (qmv_specialized.metal:1083-1279,
// q4mv_bf16_specialized.metal:716-865).
int nnz_qmv_norm_pair_silu_launch(nnz_ctx *ctx, const nnz_qweight *wg, const nnz_qweight *wu,
                                  const float *residual, const float *norm_w, void *out,
                                  nnz_qmv_dims d, float eps) {
    NNZ_REQUIRE(ctx, wg != nullptr, NNZ_EINVAL, "norm_pair_silu: null weight");
    if (wg->bits == 4)
        return launch_qmv<4, NNZ_F32, 2, true, EPI_SILU, NNZ_F16, true>(
            ctx, wg, wu, residual, norm_w, out, nullptr, d, "q4_norm_pair_silu", eps);
    return launch_qmv<1, NNZ_F32, 2, true, EPI_SILU, NNZ_F16, false>(
        ctx, wg, wu, residual, norm_w, out, nullptr, d, "norm_pair_silu", eps);
}

// RMSNorm prologue (x rounded to f16 like rms_norm_f16out, or BF16-truncated
// first like rms_norm_bf16_f16out for Q4) + LM head, f32 logits: the
// reference's final norm + qmv_spec_f16in / q4mv_spec_f16in pair
// (transformer.zig:2730-2785) in one launch.
int nnz_qmv_norm_f32out_launch(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                               const float *norm_w, float *out, nnz_qmv_dims d, float eps,
                               NnzTop2 *top2) {
    NNZ_REQUIRE(ctx, w != nullptr, NNZ_EINVAL, "norm_lm_head: null weight");
    if (w->bits == 4)
        return launch_qmv<4, NNZ_F32, 1, true, EPI_STORE, NNZ_F32, true>(
            ctx, w, nullptr, residual, norm_w, out, nullptr, d, "q4_norm_lm_head", eps, top2);
    return launch_qmv<1, NNZ_F32, 1, true, EPI_STORE, NNZ_F32, false>(ctx, w, nullptr, residual,
                                                                       norm_w, out, nullptr, d,
                                                                       "norm_lm_head", eps, top2);
}

// O-projection with residual += whose input is merged from split-sequence
// attention partials inside the kernel (f16-rounded, as the separate merge
// would store it).
int nnz_qmv_merge_resadd_launch(nnz_ctx *ctx, const nnz_qweight *w, const float *part_o,
                                const float *part_ml, const uint32_t *d_seq, uint32_t seq_len,
                                uint32_t nchunks, uint32_t chunk, uint32_t head_dim,
                                float *residual, nnz_qmv_dims d) {
    MergeIn mg{part_o, part_ml, d_seq, seq_len, nchunks, chunk, head_dim};
    const nnz_qweight *ws[1] = {w};
    void *out[1] = {residual};
    const uint32_t rows[1] = {d.M};
    NNZ_REQUIRE(ctx, w != nullptr, NNZ_EINVAL, "merge_o_resadd: null weight");
    if (w->bits == 4)
        return launch_qmv_ex<4, NNZ_F16, 1, XIN_MERGE, EPI_RESADD, NNZ_F32, true>(
            ctx, ws, rows, 1, nullptr, nullptr, out, d, "q4_merge_o_resadd", &mg);
    return launch_qmv_ex<1, NNZ_F16, 1, XIN_MERGE, EPI_RESADD, NNZ_F32, false>(
        ctx, ws, rows, 1, nullptr, nullptr, out, d, "merge_o_resadd", &mg);
}

extern "C" {

int nnz_dispatch_qmv_merge_f16io_resadd(nnz_ctx *ctx, const nnz_qweight *w, const float *part_o,
                                        const float *part_ml, const uint32_t *d_seq_len,
                                        uint32_t seq_len, uint32_t head_dim, float *residual,
                                        nnz_qmv_dims dims) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, seq_len > 0 && head_dim > 0, NNZ_EINVAL, "merge_o_resadd: zero dims");
    NNZ_REQUIRE(ctx, w && w->bits == 1, NNZ_EINVAL, "merge_o_resadd: 1-bit weights");
    const uint32_t chunk = nnz_attn_fused_chunk(seq_len, 1);
    return nnz_qmv_merge_resadd_launch(ctx, w, part_o, part_ml, d_seq_len, seq_len,
                                       ceil_div(seq_len, chunk), chunk, head_dim, residual, dims);
}

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

int nnz_dispatch_fused_norm_qkv_f16io(nnz_ctx *ctx, const nnz_qweight *wq, const nnz_qweight *wk,
                                      const nnz_qweight *wv, const float *residual, void *out_q,
                                      void *out_k, void *out_v, const float *norm_scale,
                                      nnz_qmv_dims q_dims, uint32_t kv_rows) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, kv_rows > 0, NNZ_EINVAL, "fused_norm_qkv: kv_rows == 0");
    NNZ_REQUIRE(ctx, wq && wq->bits == 1, NNZ_EINVAL, "fused_norm_qkv: 1-bit weights");
    return nnz_qmv_norm_qkv_launch(ctx, wq, wk, wv, residual, norm_scale, out_q, out_k, out_v,
                                   q_dims.M, kv_rows, q_dims.K, q_dims.group_size, 1e-6f);
}
int nnz_dispatch_fused_norm_qmv_f16in(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                                      float *output, const float *norm_scale, nnz_qmv_dims dims) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, w && w->bits == 1, NNZ_EINVAL, "fused_norm_qmv_f16in: 1-bit weights");
    return nnz_qmv_norm_f32out_launch(ctx, w, residual, norm_scale, output, dims, 1e-6f);
}

// ---------------------------- stacked (one launch, many matrices) --------
int nnz_dispatch_qmv_stacked(nnz_ctx *ctx, const nnz_qweight *w, const float *input,
                             float *output, nnz_qmv_dims dims, const nnz_qmv_stack *stack) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, stack != nullptr, NNZ_EINVAL, "qmv_stacked: null stack");
    const nnz_qweight *ws[1] = {w};
    void *out[1] = {output};
    const uint32_t rows[1] = {dims.M};
    return launch_qmv_ex<1, NNZ_F32, 1, XIN_X, EPI_STORE, NNZ_F32, false>(
        ctx, ws, rows, 1, input, nullptr, out, dims, "qmv_stacked", nullptr, 1e-6f, stack);
}
int nnz_dispatch_q4mv_stacked(nnz_ctx *ctx, const nnz_qweight *w, const float *input,
                              float *output, nnz_qmv_dims dims, const nnz_qmv_stack *stack) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, stack != nullptr, NNZ_EINVAL, "q4mv_stacked: null stack");
    const nnz_qweight *ws[1] = {w};
    void *out[1] = {output};
    const uint32_t rows[1] = {dims.M};
    return launch_qmv_ex<4, NNZ_F32, 1, XIN_X, EPI_STORE, NNZ_F32, false>(
        ctx, ws, rows, 1, input, nullptr, out, dims, "q4mv_stacked", nullptr, 1e-6f, stack);
}
int nnz_dispatch_qmv_fused_pair_silu_stacked(nnz_ctx *ctx, const nnz_qweight *wa,
                                             const nnz_qweight *wb, const float *input,
                                             float *output, nnz_qmv_dims dims,
                                             const nnz_qmv_stack *stack) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, stack != nullptr, NNZ_EINVAL, "pair_silu_stacked: null stack");
    NNZ_REQUIRE(ctx, wb != nullptr, NNZ_EINVAL, "pair_silu_stacked: null second weight");
    const nnz_qweight *ws[2] = {wa, wb};
    void *out[2] = {output, nullptr};
    const uint32_t rows[1] = {dims.M};
    return launch_qmv_ex<1, NNZ_F32, 2, XIN_X, EPI_SILU, NNZ_F32, false>(
        ctx, ws, rows, 2, input, nullptr, out, dims, "pair_silu_stacked", nullptr, 1e-6f, stack);
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

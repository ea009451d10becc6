// 1-bit QMV on the block-scaled matrix cores of gfx950.
//
// Same arithmetic as the 1-bit kernels of qmv.hip (qmv_specialized.metal's
// family: y[r] = sum_g s[r,g] * sum_{c in g} (bit ? +x_c : -x_c), f32
// accumulation), for rows of K = 2048 with group size 128, computed with one
// v_mfma_scale_f32_16x16x128_f8f6f4 per (16 rows, 128-column group):
//
//   B (fp4 e2m1, 128 k x 16 columns = 16 weight rows): the group's bits, bit 1
//     widened to the fp4 code of +1 (0x2) and bit 0 to that of -1 (0xA)
//     through a byte table in LDS -- one lookup turns 8 weights into the 8
//     nibbles of one B register.  The table holds one copy per lane (entry
//     byte * 64 + lane), so a lookup's 64 reads hit 64 distinct banks, and its
//     address is one v_perm of the code word with the lane offset.
//   A (fp4 e2m1, 16 rows): x split into NDIG rows of signed integer digits
//     (|d| <= 4, exact in e2m1) with one power-of-two scale per row and
//     group (the MFMA's E8M0 block scales, equal for the group's four
//     32-column blocks): x_c = sum_s d_s,c 2^e_s + rest; each row gains at
//     least two bits, |rest| <= 2^-25 of the group's largest |x|; rows
//     NDIG..15 are zero.
//   C row s = the group's signed sum of digit row s, exact (an integer of
//     at most 4 * 128 times 2^e_s: the matrix core adds such sums exactly,
//     whereas rows of general fp8 values spanning several binades lose bits
//     in its adder, measured 2^-14 of the largest product).  The rows'
//     total times the group's f16 scale accumulates in f32.
//
// A wave owns whole 16-row tiles (4 KB of codes, contiguous): each of its
// four load instructions reads one contiguous KB (4 rows), the tile goes
// through a per-wave LDS staging area with a 272-byte row pitch, and lane
// (n, g) reads word g of each group of row n from it -- the B layout, with no
// bank conflicts.  (Reading 16 rows x 64 B per instruction instead, which
// needs no staging, streams at 5.1-5.7 TB/s on MI355X against 6.5-7.0 for
// contiguous KB instructions, measured without any arithmetic.)  The digit
// rows (A) stay in registers for the whole kernel (16 groups x 4 VGPRs).
// One block per CU shares the table: 12 waves for a single matrix, 8 for a
// pair; each wave keeps three tiles in flight.
// The MFMA operand layouts used here (fp4 A and B: lane row g holds k =
// 32 g .. 32 g + 31 of row / column lane % 16, nibble j = k 32 g + j; A's
// scale lane m + 16 b covers k = 32 b .. 32 b + 31; C[m][n] at lane n +
// 16 (m / 4), element m % 4) were established by one-hot probes on MI355X.
#include <type_traits>
#include <utility>

#include "internal.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NDIG = 12;       // digit rows of x (A rows; C rows 0-11 in lane rows 0-2)
constexpr int KG = 16;         // 128-column groups per row (K = 2048)
constexpr int KC = KG * 128;   // columns
constexpr int NS = KG / 4;     // 512-column pieces per row
// Threads per block: one block per CU.  A single matrix: 12 waves of <= 168
// VGPRs; a pair: 8 waves of <= 256 (its loop needs ~210: at 168 it spills,
// even with two units in flight).
template <int NMAT>
constexpr int threads_of() { return NMAT == 2 ? 512 : 768; }
constexpr int PREP = KC / 8;   // threads preparing x (8 columns each)

enum { EPI_STORE = 0, EPI_RESADD = 1, EPI_SILU = 2 };
enum { XIN_X = 0, XIN_NORM = 1 };

struct MqArgs {
    const uint32_t *codes0, *codes1;   // [M][K/32] words, LSB first
    const uint16_t *scales0, *scales1; // f16 [M][K/128] (symmetric half-scales)
    const void *x;                     // input (XDT) or the f32 residual (XIN_NORM)
    const float *norm_w;               // f32 [K] (XIN_NORM)
    void *out;                         // output (ODT) or the f32 residual (EPI_RESADD)
    uint32_t M;
    float eps;
    uint64_t cs, ss, xs, os;           // stacked launch: bytes between matrices (blockIdx.y)
};

template <class T>
__device__ __forceinline__ T *stk(T *p, uint64_t stride) {
    return (T *)((uintptr_t)p + (uint64_t)blockIdx.y * stride);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)0xFFFFFFFF, 0x00020000);
}

// Bit i of a 4-bit value at bit 4 i.
__host__ __device__ constexpr uint32_t spread4(uint32_t v) {
    return (v & 1u) | ((v & 2u) << 3) | ((v & 4u) << 6) | ((v & 8u) << 9);
}

// Weights of one 16-row tile of one matrix: lane l holds group l % 16 of row
// 4S + l / 16 for each S (16 bytes), the 16 f16 scales of row l % 16, and the
// residual entry of that row (EPI_RESADD).
struct Tile {
    u32x4 code[NS];
    u32x4 scl[2];
    float res;
};

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), unrolled.
template <class F, int... I>
__device__ __forceinline__ void static_for_seq(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// One group's product: A (fp4, format 4) x B (fp4, format 4), A's scale in
// byte `SEL` of `sa` (B's scale 1.0).
template <int SEL>
__device__ __forceinline__ v4f mfma_sel(const v8i &A, const v8i &B, int sa) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, v4f{0.f, 0.f, 0.f, 0.f}, 4, 4, SEL, sa,
                                                            0, 0x7F);
}
__device__ __forceinline__ v4f mfma_group(int sel, const v8i &A, const v8i &B, int sa) {
    switch (sel) {   // a constant after unrolling
    case 0: return mfma_sel<0>(A, B, sa);
    case 1: return mfma_sel<1>(A, B, sa);
    case 2: return mfma_sel<2>(A, B, sa);
    default: return mfma_sel<3>(A, B, sa);
    }
}

template <int XDT, int NMAT, int XIN, int EPI, int ODT>
__global__ __launch_bounds__(threads_of<NMAT>()) __attribute__((amdgpu_waves_per_eu(NMAT == 2 ? 2 : 3)))
void qmv1_mfma_kernel(MqArgs a) {
    constexpr int THREADS = threads_of<NMAT>();
    constexpr int WAVES = THREADS / 64;
    static_assert(NMAT == 1 || EPI == EPI_SILU, "pairs take the SiLU epilogue");
    static_assert(NMAT == 2 || EPI != EPI_SILU, "SiLU takes a pair");
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int n = lane & 15, q = lane >> 4;
    const uint32_t M = a.M;
    const uint32_t T = ceil_div(M, 16u);

    // Lane-private fp4 tables: entry b (byte value) at [b][lane].
    __shared__ __align__(16) uint32_t tab[256 * 64];
    // digit rows: row s, columns 8 w .. 8 w + 7 in dword xs4[s * XP + w]
    // (nibble j = column 8 w + j); scales sc8[s * KG + G] (E8M0).
    // (rows NDIG..15 are zero, so every lane loads its A row unconditionally)
    // The row pitch XP = PREP + 4 dwords puts row n's A reads 4 n banks
    // apart: the 16 lane rows of a 16-byte read cover the 64 banks once (a
    // pitch of PREP, a multiple of 64 banks, made that read 16-way
    // conflicted).
    constexpr int XP = PREP + 4;
    __shared__ __align__(16) uint32_t xs4[16 * XP];
    __shared__ __align__(16) uint8_t sc8[16 * KG];
    __shared__ float red[16];
    // per-wave staging of one tile's codes: 16 rows at a 272-byte pitch
    constexpr int STG_PITCH = KC / 8 + 16;
    __shared__ __align__(16) char stage[WAVES * 16 * STG_PITCH];
    char *const stg = stage + wid * 16 * STG_PITCH;

    const uint32_t *c0 = stk(a.codes0, a.cs), *c1 = stk(a.codes1, a.cs);
    const uint16_t *s0 = stk(a.scales0, a.ss), *s1 = stk(a.scales1, a.ss);
    const void *xp = stk(a.x, a.xs);
    void *op = stk(a.out, a.os);
    const __amdgpu_buffer_rsrc_t cr[2] = {rsrc(c0), rsrc(NMAT == 2 ? c1 : c0)};
    const __amdgpu_buffer_rsrc_t sr[2] = {rsrc(s0), rsrc(NMAT == 2 ? s1 : s0)};

    // This wave's units: (tile, matrix) pairs, tiles gw, gw + nw, ...
    const uint32_t gw = __builtin_amdgcn_readfirstlane(blockIdx.x * WAVES + wid);
    const uint32_t nw = gridDim.x * WAVES;
    const uint32_t ntile = gw < T ? ceil_div(T - gw, nw) : 0u;
    const uint32_t nunit = ntile * NMAT;

    // Loads of unit k (clamped rows: the last tile re-reads row M - 1).
    // Output resource sized to the M outputs: a store at an offset past
    // them is dropped, so lanes without a row to write store "nowhere" and
    // every step issues the same store (no branch around it).
    constexpr uint32_t OB = ODT == NNZ_F32 ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t orc =
        __builtin_amdgcn_make_buffer_rsrc(op, (short)0, (int)(M * (EPI == EPI_RESADD ? 4u : OB)), 0x00020000);
    // Codes: instruction S reads rows 4S..4S+3 of the tile, one contiguous KB
    // (lane l: row 4S + l / 16, bytes 16 (l % 16) .. of it -- the whole
    // group l % 16); measured on MI355X, a read stream of contiguous KB
    // instructions runs at 6.5-7.0 TB/s, one of 16 rows x 64 B at 5.1-5.7.
    auto load = [&](Tile &t, uint32_t k, int mat) {
        const uint32_t tile = gw + (k / NMAT) * nw;
        const uint32_t row0 = tile * 16u;
        const uint32_t row = min(row0 + (uint32_t)n, M - 1u);
        const uint32_t so = row * (uint32_t)(KG * 2);
#pragma unroll
        for (int S = 0; S < NS; ++S) {
            const uint32_t crow = min(row0 + 4u * S + ((uint32_t)lane >> 4), M - 1u);
            t.code[S] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      cr[mat], crow * (uint32_t)(KC / 8) + ((uint32_t)lane & 15u) * 16u, 0, 2));
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
            t.scl[h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     sr[mat], so + (uint32_t)h * 16u, 0, 2));
        if constexpr (EPI == EPI_RESADD)
            t.res = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(orc, row * 4u, 0, 0));
    };

    // ---- prologue loads (x, or the residual and norm weights) go out first,
    // the first unit's weights right after them: loads complete in order, so
    // the prologue waits for its own data only.
    // threads >= PREP (waves 4..11) read x at column 0 (in bounds, unused)
    const uint32_t xt = tid < PREP ? (uint32_t)tid : 0u;
    float4 xa[2], wn[2];
    uint4 xh;
    if constexpr (XIN == XIN_NORM) {
        xa[0] = ((const float4 *)xp)[2 * xt]; xa[1] = ((const float4 *)xp)[2 * xt + 1];
        wn[0] = ((const float4 *)a.norm_w)[2 * xt]; wn[1] = ((const float4 *)a.norm_w)[2 * xt + 1];
    } else if constexpr (XDT == NNZ_F32) {
        xa[0] = ((const float4 *)xp)[2 * xt]; xa[1] = ((const float4 *)xp)[2 * xt + 1];
    } else {
        xh = ((const uint4 *)xp)[xt];
    }
    __builtin_amdgcn_sched_barrier(0);
    Tile ta, tb;
    if (nunit) load(ta, 0, 0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- x (8 columns per thread), optionally normalised ---------------------
    float r[8];
    if constexpr (XIN == XIN_NORM) {
        const float rv[8] = {xa[0].x, xa[0].y, xa[0].z, xa[0].w, xa[1].x, xa[1].y, xa[1].z, xa[1].w};
        const float wv[8] = {wn[0].x, wn[0].y, wn[0].z, wn[0].w, wn[1].x, wn[1].y, wn[1].z, wn[1].w};
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(rv[i], rv[i], ss);
        ss = wave_sum(ss);
        if (lane == 0) red[wid] = ss;
        __syncthreads();
        ss = (red[0] + red[1]) + (red[2] + red[3]);   // waves 0-3 hold the columns
        const float rms = rsqrtf(ss / (float)KC + a.eps);
        // the normalised input is stored as f16 (rms_norm_f16out)
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = (float)(f16_t)(rv[i] * rms * wv[i]);
    } else if constexpr (XDT == NNZ_F32) {
        r[0] = xa[0].x; r[1] = xa[0].y; r[2] = xa[0].z; r[3] = xa[0].w;
        r[4] = xa[1].x; r[5] = xa[1].y; r[6] = xa[1].z; r[7] = xa[1].w;
    } else {
        const uint32_t hw[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t lo = (uint16_t)(hw[i] & 0xFFFFu), hi = (uint16_t)(hw[i] >> 16);
            if constexpr (XDT == NNZ_F16) {
                r[2 * i] = (float)__builtin_bit_cast(f16_t, lo);
                r[2 * i + 1] = (float)__builtin_bit_cast(f16_t, hi);
            } else {
                r[2 * i] = bf16_to_f32(lo);
                r[2 * i + 1] = bf16_to_f32(hi);
            }
        }
    }

    // ---- fp4 tables: the 16-byte piece i (dwords 4 i .. 4 i + 3) holds entry
    // b = i / 16 for lanes 4 (i % 16) .. +3
    for (uint32_t i = (uint32_t)tid; i < 256u * 16u; i += THREADS) {
        const uint32_t b = i >> 4;
        const uint32_t v = 0xAAAAAAAAu ^ ((spread4(b & 15u) | (spread4(b >> 4) << 16)) << 3);
        *(u32x4 *)&tab[4 * i] = u32x4{v, v, v, v};
    }

    // ---- digit rows: NDIG signed digits per column, one scale per group ----
    // Row s of group G: d = rint(r / 2^e) with 2^e set by the group's largest
    // |r| (max |r| / 2^e in [2, 4), so |d| <= 4, every such integer exact in
    // e2m1), then r -= d 2^e (exact): |r| drops at least fourfold per row.
    // Thread t < PREP holds columns 8t..8t+7; a group's 16 threads are one
    // 16-lane row (the maximum by DPP).
    if (tid < PREP) {
        const uint32_t G = (uint32_t)tid >> 4;
#pragma unroll
        for (int s = 0; s < NDIG; ++s) {
            float mx = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(r[i]));
            mx = fmaxf(mx, dpp_move<DPP_XOR1>(mx, 0.f));
            mx = fmaxf(mx, dpp_move<DPP_XOR2>(mx, 0.f));
            mx = fmaxf(mx, dpp_move<DPP_ROW_HALF_MIRROR>(mx, 0.f));
            mx = fmaxf(mx, dpp_move<DPP_ROW_MIRROR>(mx, 0.f));
            int e = 0;
            if (mx > 0.f) e = max(-126, min(126, __builtin_amdgcn_frexp_expf(mx) - 2));
            const float inv = __int_as_float((127 - e) << 23), pw = __int_as_float((127 + e) << 23);
            float d[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                d[i] = rintf(r[i] * inv);
                r[i] = fmaf(-d[i], pw, r[i]);
            }
            // digits are exact in e2m1; the first operand lands in the low nibble
            uint32_t q = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, d[0], d[1], 1.f, 0);
            q = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(q, d[2], d[3], 1.f, 1);
            q = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(q, d[4], d[5], 1.f, 2);
            q = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(q, d[6], d[7], 1.f, 3);
            xs4[s * XP + tid] = q;
            if ((tid & 15) == 0) sc8[s * KG + G] = (uint8_t)(127 + e);
        }
#pragma unroll
        for (int s = NDIG; s < 16; ++s) {
            xs4[s * XP + tid] = 0u;
            if ((tid & 15) == 0) sc8[s * KG + G] = 127;   // 1.0: finite, the row is zero
        }
    }
    __syncthreads();

    // ---- A operands (digit rows) and their scales, kept for the whole kernel
    v4i A[KG];
    uint32_t sa[KG / 4];
#pragma unroll
    for (int G = 0; G < KG; ++G) A[G] = __builtin_bit_cast(v4i, *(const u32x4 *)&xs4[n * XP + G * 16 + 4 * q]);
    {
        const u32x4 sv = *(const u32x4 *)&sc8[n * KG];
        sa[0] = sv.x; sa[1] = sv.y; sa[2] = sv.z; sa[3] = sv.w;
    }

    // ---- main loop -----------------------------------------------------------
    const uint32_t lane4 = (uint32_t)lane * 4u;
    const char *tb8 = (const char *)tab;
    float gate = 0.f;   // EPI_SILU: the gate row total until the up total is known
    // The last store's value and offset stay live until the next loads are
    // issued: were their registers reused as load destinations, the loads
    // would first wait for the store (and everything before it) to finish.
    float st_v = 0.f;
    uint32_t st_off = 0x80000000u;
    auto compute = [&](const Tile &t, uint32_t k, auto mat_c) {
        constexpr int MAT = decltype(mat_c)::value;
        float acc = 0.f;
        // the tile's codes into this wave's staging rows (272-byte pitch),
        // then lane (n, g) reads word g of each group of row n: banks
        // 4n + 4G + g, all distinct for a read (LDS keeps a wave's order)
#pragma unroll
        for (int S = 0; S < NS; ++S)
            *(u32x4 *)(stg + (4 * S + (lane >> 4)) * STG_PITCH + 16 * (lane & 15)) = t.code[S];
#pragma unroll
        for (int S = 0; S < NS; ++S) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = *(const uint32_t *)(stg + n * STG_PITCH + 16 * (4 * S + i) + 4 * q);
            // the piece's 16 table reads first (one LDS round trip for four
            // groups), then its four independent MFMAs, then their sums
            uint32_t b4[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    // address = byte bb of the word * 256 + lane * 4
                    const uint32_t off = __builtin_amdgcn_perm(w[i], lane4, 0x0C0C0000u | ((4u + bb) << 8));
                    b4[i][bb] = *(const uint32_t *)(tb8 + off);
                }
            v4f c[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int G = 4 * S + i;
                const v8i B = v8i{(int)b4[i][0], (int)b4[i][1], (int)b4[i][2], (int)b4[i][3], 0, 0, 0, 0};
                const v8i A8 = v8i{A[G][0], A[G][1], A[G][2], A[G][3], 0, 0, 0, 0};
                c[i] = mfma_group(i, A8, B, (int)sa[G >> 2]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int G = 4 * S + i;
                const float tsum = (c[i][0] + c[i][1]) + (c[i][2] + c[i][3]);
                const uint32_t sw = t.scl[G >> 3][(G >> 1) & 3];
                const float sc = (float)__builtin_bit_cast(f16_t, (uint16_t)((G & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
                acc = fmaf(sc, tsum, acc);
            }
        }
        // digit rows 4r..4r+3 sit in lane row r: sum the four lane rows
        const float t1 = acc + __int_as_float((int)__builtin_amdgcn_permlane32_swap(
                                   __float_as_int(acc), __float_as_int(acc), false, false)[1]);
        const float tot = t1 + __int_as_float((int)__builtin_amdgcn_permlane16_swap(
                                   __float_as_int(t1), __float_as_int(t1), false, false)[1]);
        const uint32_t tile = gw + (k / NMAT) * nw;
        const uint32_t row = tile * 16u + (uint32_t)n;
        if constexpr (EPI == EPI_SILU && MAT == 0) {
            gate = tot;   // the up matrix's unit comes next
        } else {
            float v = tot;
            if constexpr (EPI == EPI_RESADD) v = t.res + tot;
            if constexpr (EPI == EPI_SILU) v = gate / (1.f + expf(-gate)) * tot;
            const uint32_t off = (q == 0 && row < M) ? row * (EPI == EPI_RESADD ? 4u : OB) : 0x80000000u;
            st_v = v;
            st_off = off;
            if constexpr (ODT == NNZ_F32 || EPI == EPI_RESADD)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), orc, off, 0, 0);
            else if constexpr (ODT == NNZ_F16)
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16_t)v), orc, off, 0, 0);
            else
                __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(v), orc, off, 0, 0);
        }
    };
    // DEPTH units in flight per wave: unit k + DEPTH - 1's loads are issued
    // before anything of unit k's arithmetic (a scheduling fence: hoisted
    // above them, the transposes would make the loads wait for unit k's
    // data).  The loop body covers one period of the ring; a pair's units
    // alternate gate, up and its period is even, so each position's matrix
    // is a compile-time constant.  The units left at the end run the same
    // positions with a (wave-uniform) guard.
    constexpr int DEPTH = 3;
    constexpr int PERIOD = NMAT == 2 ? 6 : 3;
    Tile tc, td;
    if (nunit > 1) load(tb, 1, 1 % NMAT);
    if constexpr (DEPTH > 3)
        if (nunit > 2) load(tc, 2, 2 % NMAT);
    __builtin_amdgcn_sched_barrier(0);
    auto slot = [&](auto sc) -> Tile & {
        constexpr int S = decltype(sc)::value % DEPTH;
        if constexpr (S == 0) return ta;
        else if constexpr (S == 1) return tb;
        else if constexpr (S == 2) return tc;
        else return td;
    };
    uint32_t k = 0;
    auto body = [&](auto jc, bool guard) {
        constexpr int J = decltype(jc)::value;
        const uint32_t u = k + J;
        if (guard && u >= nunit) return;
        load(slot(std::integral_constant<int, J + DEPTH - 1>{}), min(u + DEPTH - 1, nunit - 1),
             (J + DEPTH - 1) % NMAT);
        asm volatile("" ::"v"(st_v), "v"(st_off));
        __builtin_amdgcn_sched_barrier(0);
        compute(slot(jc), u, std::integral_constant<int, J % NMAT>{});
        __builtin_amdgcn_sched_barrier(0);
    };
    for (; k + PERIOD <= nunit; k += PERIOD)
        static_for<PERIOD>([&](auto jc) { body(jc, false); });
    // the rest (fewer than PERIOD units; a pair's count is even, so position
    // J still takes matrix J % NMAT)
    static_for<PERIOD - 1>([&](auto jc) { body(jc, true); });
}

template <int XDT, int NMAT, int XIN, int EPI, int ODT>
void launch(nnz_ctx *ctx, const MqArgs &a, uint32_t blocks, uint32_t gy) {
    qmv1_mfma_kernel<XDT, NMAT, XIN, EPI, ODT><<<dim3(blocks, gy), threads_of<NMAT>(), 0, ctx->stream>>>(a);
}

}  // namespace

bool nnz_q1_mfma_supported(uint32_t K, uint32_t group_size) {
    return K == (uint32_t)KC && group_size == 128;
}

// The variants built below (x dtype, pair, input mode, epilogue, output dtype).
bool nnz_q1_mfma_has_variant(const NnzQ1Mfma &c) {
    const int k[5] = {c.xdt, (int)c.nmat, c.xin, c.epi, c.odt};
    static const int built[][5] = {
        {NNZ_F32, 1, XIN_X, EPI_STORE, NNZ_F32},     {NNZ_F16, 1, XIN_X, EPI_STORE, NNZ_F32},
        {NNZ_F32, 1, XIN_NORM, EPI_STORE, NNZ_F32},  {NNZ_F32, 2, XIN_X, EPI_SILU, NNZ_F32},
        {NNZ_F32, 2, XIN_NORM, EPI_SILU, NNZ_F16},   {NNZ_F16, 1, XIN_X, EPI_RESADD, NNZ_F32}};
    for (const auto &b : built)
        if (b[0] == k[0] && b[1] == k[1] && b[2] == k[2] && b[3] == k[3] && b[4] == k[4]) return true;
    return false;
}

int nnz_q1_mfma_launch(nnz_ctx *ctx, const NnzQ1Mfma &c) {
    NNZ_REQUIRE(ctx, nnz_q1_mfma_supported(c.K, c.group_size), NNZ_EUNSUPPORTED,
                "q1_mfma: K=%u gs=%u (needs K=%d, gs=128)", c.K, c.group_size, KC);
    NNZ_REQUIRE(ctx, c.M >= 1 && (c.nmat == 1 || c.nmat == 2), NNZ_EINVAL, "q1_mfma: bad shape");
    NNZ_REQUIRE(ctx, (uint64_t)c.M * (KC / 8) < (1ull << 32), NNZ_EUNSUPPORTED,
                "q1_mfma: matrix of 4 GiB or more");
    MqArgs a{};
    a.codes0 = (const uint32_t *)c.codes[0];
    a.codes1 = (const uint32_t *)(c.nmat == 2 ? c.codes[1] : c.codes[0]);
    a.scales0 = (const uint16_t *)c.scales[0];
    a.scales1 = (const uint16_t *)(c.nmat == 2 ? c.scales[1] : c.scales[0]);
    a.x = c.x;
    a.norm_w = c.norm_w;
    a.out = c.out;
    a.M = c.M;
    a.eps = c.eps;
    a.cs = c.cs; a.ss = c.ss; a.xs = c.xs; a.os = c.os;
    const uint32_t tiles = ceil_div(c.M, 16u);
    // one 12-wave block per CU (the table's 64 KB of LDS and <= 168 VGPRs
    // per lane), about 256 blocks in all, never more than one wave per tile
    const uint32_t gy = c.stack_count ? c.stack_count : 1u;
    uint32_t blocks = c.blocks_per_matrix ? c.blocks_per_matrix : ceil_div(256u, gy);
    blocks = min(blocks, ceil_div(tiles, (uint32_t)(c.nmat == 2 ? threads_of<2>() : threads_of<1>()) / 64u));
    blocks = max(blocks, 1u);
#define MQ(XDT, NMAT, XIN, EPI, ODT)                                                           \
    if (c.xdt == XDT && c.nmat == NMAT && c.xin == XIN && c.epi == EPI && c.odt == ODT) {     \
        launch<XDT, NMAT, XIN, EPI, ODT>(ctx, a, blocks, gy);                                 \
        NNZ_LAUNCHED(ctx);                                                                    \
        return NNZ_OK;                                                                        \
    }
    MQ(NNZ_F32, 1, XIN_X, EPI_STORE, NNZ_F32)       // dispatchQMV form
    MQ(NNZ_F16, 1, XIN_X, EPI_STORE, NNZ_F32)       // f16in (LM head)
    MQ(NNZ_F32, 1, XIN_NORM, EPI_STORE, NNZ_F32)    // final norm + LM head
    MQ(NNZ_F32, 2, XIN_X, EPI_SILU, NNZ_F32)        // fused gate/up + SiLU, f32 I/O
    MQ(NNZ_F32, 2, XIN_NORM, EPI_SILU, NNZ_F16)     // fused norm + gate/up + SiLU
    MQ(NNZ_F16, 1, XIN_X, EPI_RESADD, NNZ_F32)      // f16io residual add
#undef MQ
    return nnz_fail(ctx, NNZ_EUNSUPPORTED, "q1_mfma: variant not built");
}

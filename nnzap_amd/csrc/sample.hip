// Device-side sampling: sampleToken (nnmetal/src/transformer.zig:3860-3894)
// with the reference's filters -- temperature (:3709-3719), top-k
// (:3743-3766), top-p (:3768-3816) -- the final softmax (:3721-3741) and the
// inverse-CDF draw (:3896-3908), fed by generate's random stream
// (:3969-3972, Zig std.Random.DefaultPrng).
//
// The reference copies the 151k logits to the host and sorts them there.
// Here the logits never leave HBM; two launches per draw:
//   * selection kernel: one 256-thread block per 1024 logits writes its
//     maximum scaled logit and its sum of exp(x - max) and, when a filter
//     needs candidates, every element >= its k-th largest (8-bit radix select
//     in LDS), ties included, in index order.  Every element of the global
//     top-k set is in its block's list: a block's k-th largest exceeds the
//     global k-th largest only if that block alone holds k larger elements.
//   * finishing kernel (one 1024-thread block):
//       - temperature only: the draw walks the blocks' masses in index order,
//         then the 1024 logits of the block it lands in;
//       - top-k (+ top-p): the lists (<= 8192 candidates: each block keeps at
//         most 8192 / blocks) sit in registers, 8 per thread in index order;
//         the global k-th largest comes from a radix select.  When the lists
//         were cut shorter than k, the result stands only if the k-th largest
//         is >= every cut list's threshold (then every element of the top-k
//         set is in a list).  With <= 64 survivors one wave finishes with the
//         reference's sequential sums; otherwise top-p is a radix select
//         weighted by fixed-point probability mass and the walk a block scan;
//       - top-p alone: the same over each block's largest (up to 96), when
//         the nucleus provably ends above every list's threshold (checked
//         with the total mass from the block sums);
//       - otherwise (ties overflowing the registers, nucleus or top-k set
//         beyond the lists) the same filters run from global memory.
//
// Rounding: sums are tree sums rather than the reference's sequential f32
// sums, and exp is the device's expf, so a draw can differ from the
// reference's only when r (or the top-p cut) lies within float32 summation
// rounding of a boundary of the cumulative distribution.
#include "internal.h"

namespace {

constexpr uint32_t SB = 1024;          // logits per selection block (256 threads x 4)
constexpr uint32_t FT = 1024;          // threads of the finishing block
constexpr uint32_t PER = 8;            // candidates per finishing thread held in registers
constexpr uint32_t RCAP = FT * PER;    // candidates the registers hold
constexpr uint32_t KB_TOPP = 96;       // per-block list length when top-p filters alone
constexpr uint32_t MAX_BLOCKS = 4096;  // selection blocks: count <= 4,194,304
constexpr int SEL_W = 11;              // radix digit bits: selection kernel
constexpr int FIN_W = 12;              // ... finishing kernel, k-th largest
constexpr int MASS_W = 11;             // ... finishing kernel, nucleus cut
constexpr double MASS_ONE = 1099511627776.0;  // 2^40: fixed-point probability unit

// Order-preserving map float -> uint32 (larger float, larger key); -0 and +0
// share a key, as they compare equal.
__device__ __forceinline__ uint32_t fkey(float x) {
    uint32_t b = __float_as_uint(x);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t clz64(uint64_t v) { return v ? (uint32_t)__builtin_clzll(v) : 64u; }

// Zig std.Random.Xoshiro256.next (xoshiro256++, Blackman & Vigna).
__device__ __forceinline__ uint64_t xoshiro_next(uint64_t *s) {
    const uint64_t a = s[0] + s[3];
    const uint64_t r = ((a << 23) | (a >> 41)) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = (s[3] << 45) | (s[3] >> 19);
    return r;
}

// Zig std.Random.float(f32): 23 random mantissa bits, the exponent from the
// leading zeros of the remaining bits (every float in [0, 1) reachable).
__device__ __forceinline__ float zig_float32(uint64_t *s) {
    const uint64_t rnd = xoshiro_next(s);
    uint32_t lz = clz64(rnd);
    if (lz >= 41) {
        lz = 41 + clz64(xoshiro_next(s));
        if (lz == 41 + 64) lz += (uint32_t)__builtin_clz((uint32_t)xoshiro_next(s) | 0x7FFu);
    }
    return __uint_as_float(((126u - lz) << 23) | ((uint32_t)rnd & 0x7FFFFFu));
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float *sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < NT / 64; ++i) r = fmaxf(r, sh[i]);
    __syncthreads();
    return r;
}

template <int NT>
__device__ __forceinline__ float block_sum(float v, float *sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
    for (int i = 0; i < NT / 64; ++i) r += sh[i];
    __syncthreads();
    return r;
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const T t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

// Exclusive prefix over the block in thread order; *total = block sum.
template <int NT, typename T>
__device__ __forceinline__ T block_excl_scan(T v, T *sh, T *total) {
    const T inc = wave_incl_scan(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) sh[w] = inc;
    __syncthreads();
    T base = 0, tot = 0;
    for (int i = 0; i < NT / 64; ++i) {
        const T s = sh[i];
        if (i < w) base += s;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return base + inc - v;
}

// LDS scratch of the radix selections.
struct RadixSh {
    uint32_t red[32];
    uint32_t scan[16];
    unsigned long long lscan[16];
    uint32_t sel[4];
    unsigned long long msel[2];
};

// Common leading bits of the keys `visit` hands out: returns their number
// (32 when all keys are equal or there are none) and the shared bits.
template <int NT, class Visit>
__device__ __forceinline__ uint32_t common_prefix(Visit visit, RadixSh &R, uint32_t *bits) {
    uint32_t kand = 0xFFFFFFFFu, kor = 0u;
    visit([&](uint32_t key) {
        kand &= key;
        kor |= key;
    });
    for (int o = 32; o > 0; o >>= 1) {
        kand &= __shfl_xor(kand, o);
        kor |= __shfl_xor(kor, o);
    }
    if ((threadIdx.x & 63) == 0) {
        R.red[threadIdx.x >> 6] = kand;
        R.red[16 + (threadIdx.x >> 6)] = kor;
    }
    __syncthreads();
    kand = 0xFFFFFFFFu;
    kor = 0u;
    for (int i = 0; i < NT / 64; ++i) {
        kand &= R.red[i];
        kor |= R.red[16 + i];
    }
    __syncthreads();
    if (kor == 0u && kand == 0xFFFFFFFFu) {  // nothing visited
        *bits = 0;
        return 32;
    }
    const uint32_t diff = kand ^ kor;
    const uint32_t L = diff ? (uint32_t)__builtin_clz(diff) : 32u;
    *bits = L ? (kand & (0xFFFFFFFFu << (32 - L))) : 0u;
    return L;
}

// Key of the kr-th largest (1-based, ties counted) among the keys that
// `visit` hands to its callback; requires 1 <= kr <= their number.  Digits
// of up to W bits below the keys' common prefix (so that close values do not
// all land in one bin); histogram hist[2^W] in LDS; each thread owns 2^W/NT
// consecutive bins (highest first) and a block scan finds the bin.
template <int NT, int W, class Visit>
__device__ __forceinline__ uint32_t radix_kth_largest(Visit visit, uint32_t kr, uint32_t *hist, RadixSh &R) {
    constexpr int NBINS = 1 << W, BPT = NBINS / NT;
    static_assert(BPT >= 1, "at least one bin per thread");
    uint32_t prefix;
    const uint32_t L = common_prefix<NT>(visit, R, &prefix);
    uint32_t mask = L ? 0xFFFFFFFFu << (32 - L) : 0u;
    for (int hi = 32 - (int)L; hi > 0;) {
        const int sh = hi > W ? hi - W : 0, width = hi - sh;
        const uint32_t dmask = (1u << width) - 1u;
        for (uint32_t i = threadIdx.x; i < (uint32_t)NBINS; i += NT) hist[i] = 0;
        __syncthreads();
        visit([&](uint32_t key) {
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> sh) & dmask], 1u);
        });
        __syncthreads();
        uint32_t h[BPT], s = 0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            h[j] = hist[NBINS - 1 - ((int)threadIdx.x * BPT + j)];
            s += h[j];
        }
        uint32_t tot;
        uint32_t above = block_excl_scan<NT>(s, R.scan, &tot);  // elements in higher bins
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            if (above < kr && kr <= above + h[j]) {
                R.sel[0] = NBINS - 1 - ((int)threadIdx.x * BPT + j);
                R.sel[1] = kr - above;
            }
            above += h[j];
        }
        __syncthreads();
        prefix |= R.sel[0] << sh;
        mask |= dmask << sh;
        kr = R.sel[1];
        hi = sh;
    }
    return prefix;
}

// Nucleus cut: the largest key tau with mass(key > tau) < need <=
// mass(key >= tau), masses in units of 2^-40.  On return: tau, the mass
// still needed from elements equal to tau, one such element's mass and
// their number; all = true when the whole set holds less than `need`.
struct MassCut {
    uint32_t tau, n_eq;
    unsigned long long rem, q_eq;
    bool all;
};

template <int NT, int W, class Visit>
__device__ __forceinline__ MassCut radix_mass_cut(Visit visit, unsigned long long need, uint32_t *hcnt,
                                  unsigned long long *hmass, RadixSh &R) {
    constexpr int NBINS = 1 << W, BPT = NBINS / NT;
    static_assert(BPT >= 1, "at least one bin per thread");
    uint32_t prefix;
    const uint32_t L = common_prefix<NT>(
        [&](auto f) { visit([&](uint32_t key, unsigned long long) { f(key); }); }, R, &prefix);
    uint32_t mask = L ? 0xFFFFFFFFu << (32 - L) : 0u;
    MassCut r{0, 0, 0, 0, false};
    // with all keys equal there is no digit left: one pass over a 0-bit digit
    int hi = 32 - (int)L;
    bool first = true;
    while (hi > 0 || first) {
        first = false;
        const int sh = hi > W ? hi - W : 0, width = hi - sh;
        const uint32_t dmask = width ? (1u << width) - 1u : 0u;
        for (uint32_t i = threadIdx.x; i < (uint32_t)NBINS; i += NT) {
            hcnt[i] = 0;
            hmass[i] = 0;
        }
        if (threadIdx.x == 0) R.sel[2] = 0;
        __syncthreads();
        visit([&](uint32_t key, unsigned long long m) {
            if ((key & mask) == prefix) {
                const uint32_t b = (key >> sh) & dmask;
                atomicAdd(&hcnt[b], 1u);
                atomicAdd(&hmass[b], m);
            }
        });
        __syncthreads();
        unsigned long long h[BPT], s = 0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            h[j] = hmass[NBINS - 1 - ((int)threadIdx.x * BPT + j)];
            s += h[j];
        }
        unsigned long long tot;
        unsigned long long above = block_excl_scan<NT>(s, R.lscan, &tot);
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            if (above < need && need <= above + h[j]) {
                const int b = NBINS - 1 - ((int)threadIdx.x * BPT + j);
                R.sel[0] = b;
                R.sel[1] = hcnt[b];
                R.sel[2] = 1;
                R.msel[0] = need - above;
                R.msel[1] = h[j];
            }
            above += h[j];
        }
        __syncthreads();
        if (!R.sel[2]) {  // the set holds less mass than asked: keep everything
            r.all = true;
            __syncthreads();
            return r;
        }
        prefix |= R.sel[0] << sh;
        mask |= dmask << sh;
        need = R.msel[0];
        r.n_eq = R.sel[1];
        r.q_eq = r.n_eq ? R.msel[1] / r.n_eq : 0;
        __syncthreads();
        hi = sh;
    }
    r.tau = prefix;
    r.rem = need;
    return r;
}

// Selection kernel: one 256-thread block per SB logits.  Writes the block's
// maximum scaled logit, its sum of exp(x - max), and -- with kc > 0 -- every
// element >= the block's kc-th largest (ties included), in index order, with
// that threshold's key (0 when the whole block is kept).
__global__ __launch_bounds__(256) void sample_select_kernel(const float *logits, uint32_t n,
                                                            float inv_t, uint32_t kc,
                                                            float *blk_max, float *blk_sum,
                                                            uint32_t *blk_cnt, uint32_t *blk_kth,
                                                            float *cx, uint32_t *ci) {
    __shared__ uint32_t hist[1 << SEL_W];
    __shared__ RadixSh R;
    __shared__ float fsh[4];
    __shared__ uint32_t ush[4];
    const uint32_t base = blockIdx.x * SB, t = threadIdx.x;
    float x[4];
    bool ok[4];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = base + 4 * t + j;
        ok[j] = i < n;
        x[j] = ok[j] ? logits[i] * inv_t : -INFINITY;
        m = fmaxf(m, x[j]);
    }
    m = block_max<256>(m, fsh);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ok[j]) s += expf(x[j] - m);
    s = block_sum<256>(s, fsh);
    if (t == 0) {
        blk_max[blockIdx.x] = m;
        blk_sum[blockIdx.x] = s;
    }
    if (kc == 0) return;
    const uint32_t nvalid = n - base < SB ? n - base : SB;
    uint32_t tk = 0;  // keep keys >= tk; 0 keeps every element
    if (kc < nvalid)
        tk = radix_kth_largest<256, SEL_W>(
            [&](auto f) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (ok[j]) f(fkey(x[j]));
            },
            kc, hist, R);
    bool keep[4];
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        keep[j] = ok[j] && fkey(x[j]) >= tk;
        c += keep[j];
    }
    uint32_t tot;
    uint32_t off = block_excl_scan<256>(c, ush, &tot);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (keep[j]) {
            cx[base + off] = x[j];
            ci[base + off] = base + 4 * t + j;
            ++off;
        }
    if (t == 0) {
        blk_cnt[blockIdx.x] = tot;
        blk_kth[blockIdx.x] = tk;
    }
}

enum { MODE_TEMP = 0, MODE_TOPK = 1, MODE_TOPP = 2 };

struct FinishArgs {
    const float *logits;
    uint32_t n;
    float inv_t;
    uint32_t k;      // top-k (MODE_TOPK)
    uint32_t kc;     // list length asked of each selection block
    float top_p;     // >= 1: off
    int mode;
    uint32_t nb;     // selection blocks
    const float *blk_max;
    const float *blk_sum;
    const uint32_t *blk_cnt;
    const uint32_t *blk_kth;
    const float *cx;
    const uint32_t *ci;
    float *kx;
    uint32_t *ki;
    unsigned long long *rng;  // xoshiro256 state, 4 words
    uint32_t *out_index;
    float *out_prob;
    NnzPick pick;             // pick.state != nullptr: record into a decode state block
};

struct FinSh {
    float fsh[16];
    uint32_t ush[16];
    unsigned long long lsh[16];
    RadixSh R;
    uint32_t hist[1 << FIN_W];
    unsigned long long hmass[1 << MASS_W];
    uint32_t koff[MAX_BLOCKS + 1];
    float wx[64];       // survivors of top-k for the one-wave finish
    uint32_t wi[64];
    float r, prob, cum0;
    uint32_t tok, aux, fallback;
};

__device__ __forceinline__ unsigned long long mass_of(float q) {
    return (unsigned long long)((double)q * MASS_ONE);
}

__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long v, unsigned long long *sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long r = 0;
    for (int i = 0; i < (int)(FT / 64); ++i) r += sh[i];
    __syncthreads();
    return r;
}

// Largest list threshold key over the selection blocks: every logit whose
// key is >= it is in some list (blocks kept whole report 0).
__device__ __forceinline__ uint32_t lists_floor(const FinishArgs &a, FinSh &S) {
    uint32_t t = 0;
    for (uint32_t b = threadIdx.x; b < a.nb; b += FT) t = max(t, a.blk_kth[b]);
    for (int o = 32; o > 0; o >>= 1) t = max(t, (uint32_t)__shfl_xor(t, o));
    if ((threadIdx.x & 63) == 0) S.ush[threadIdx.x >> 6] = t;
    __syncthreads();
    uint32_t mx = 0;
    for (int i = 0; i < (int)(FT / 64); ++i) mx = max(mx, S.ush[i]);
    __syncthreads();
    return mx;
}

// Total of exp(x - M) over all n logits from the per-block statistics;
// *M_out = the global maximum.  Thread t reads blocks t, t + FT, ...
__device__ __forceinline__ float total_from_blocks(const FinishArgs &a, FinSh &S, float *M_out) {
    float M = -INFINITY;
    for (uint32_t b = threadIdx.x; b < a.nb; b += FT) M = fmaxf(M, a.blk_max[b]);
    M = block_max<FT>(M, S.fsh);
    float s = 0.f;
    for (uint32_t b = threadIdx.x; b < a.nb; b += FT) s += a.blk_sum[b] * expf(a.blk_max[b] - M);
    *M_out = M;
    return block_sum<FT>(s, S.fsh);
}

// Temperature only: softmax over all logits, the inverse-CDF walk first over
// the blocks' masses (index order), then inside the block it crosses.
__device__ __forceinline__ void finish_temperature(const FinishArgs &a, FinSh &S) {
    const uint32_t tid = threadIdx.x;
    // thread t owns blocks [4t, 4t + 4) (nb <= 4 * FT): one round of loads
    float bm[4], bs[4], M = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t b = 4 * tid + j;
        bm[j] = b < a.nb ? a.blk_max[b] : -INFINITY;
        bs[j] = b < a.nb ? a.blk_sum[b] : 0.f;
        M = fmaxf(M, bm[j]);
    }
    M = block_max<FT>(M, S.fsh);
    float w[4], cs = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        w[j] = 4 * tid + j < a.nb ? bs[j] * expf(bm[j] - M) : 0.f;
        cs += w[j];
    }
    float tot;
    const float before = block_excl_scan<FT>(cs, S.fsh, &tot);
    const float inv = 1.0f / tot, r = S.r;
    float cum = before * inv, cum_at = 0.f;
    uint32_t bstar = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t b = 4 * tid + j;
        if (b >= a.nb || bstar != 0xFFFFFFFFu) continue;
        const float c2 = cum + w[j] * inv;
        if (c2 > r) {
            bstar = b;
            cum_at = cum;
        }
        cum = c2;
    }
    if (bstar != 0xFFFFFFFFu) atomicMin(&S.aux, bstar);
    __syncthreads();
    const uint32_t B = S.aux;
    if (bstar != 0xFFFFFFFFu && bstar == B) S.cum0 = cum_at;  // one owner per block
    __syncthreads();
    if (B == 0xFFFFFFFFu) return;  // rounding tail: no block reaches r
    const uint32_t i = B * SB + tid;
    const bool ok = i < a.n;
    const float x = ok ? a.logits[i] * a.inv_t : -INFINITY;
    const float p = ok ? expf(x - M) * inv : 0.f;
    float ptot;
    const float pb = block_excl_scan<FT>(p, S.fsh, &ptot);
    const float c = S.cum0 + pb + p;
    if (ok && p > 0.f && c > r) atomicMin(&S.tok, i);
    if (ok && p > 0.f) atomicMax(&S.fallback, i + 1);  // last element with mass, if none crosses
    __syncthreads();
    if (S.tok == 0xFFFFFFFFu && S.fallback) {
        if (tid == 0) S.tok = S.fallback - 1;
        __syncthreads();
    }
    if (ok && i == S.tok) S.prob = p;
    __syncthreads();
}

__device__ __forceinline__ float lane_f(float v, uint32_t j) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)j));
}
__device__ __forceinline__ uint32_t lane_u(uint32_t v, uint32_t j) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)j);
}

// At most 64 survivors (index order) in S.wx / S.wi, finished by one wave
// (threads 0..63) with the reference's sequential float32 sums: the top-p
// softmax (over the survivors, or s_topp > 0: the sum over every logit) and
// its cumulative walk in descending-probability order (ties by index), the
// final softmax and the inverse-CDF walk in index order.  Sequential steps
// read lanes with v_readlane (uniform lane index).
__device__ __forceinline__ void finish_wave(const FinishArgs &a, FinSh &S, uint32_t nk, float M,
                                            float s_topp) {
    const uint32_t l = threadIdx.x;
    const bool v = l < nk;
    const float e = v ? expf(S.wx[l] - M) : 0.f;
    unsigned long long keep = nk >= 64 ? ~0ull : ((1ull << nk) - 1ull);
    if (a.top_p < 1.0f) {
        float s = s_topp;
        if (s <= 0.f) {
            s = 0.f;
            for (uint32_t j = 0; j < nk; ++j) s += lane_f(e, j);
        }
        const float q = e * (1.0f / s);
        // bitonic sort, ascending on (~q bits, lane): q descending, ties by index
        unsigned long long key =
            v ? ((unsigned long long)(~__float_as_uint(q)) << 32) | l : ~0ull;
        for (uint32_t k = 2; k <= 64; k <<= 1)
            for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                const unsigned long long o = __shfl_xor(key, (int)j);
                const bool take_min = ((l & j) == 0) == ((l & k) == 0);
                key = take_min ? (key < o ? key : o) : (key > o ? key : o);
            }
        const uint32_t src = (uint32_t)(key & 0xFFFFFFFFull) & 63u;  // lane holding the r-th
        const float qs = __shfl(q, (int)src);
        float c = 0.f;
        uint32_t cut = nk - 1;
        for (uint32_t r = 0; r < nk; ++r) {
            c += lane_f(qs, r);
            if (c >= a.top_p) {
                cut = r;
                break;
            }
        }
        keep = 0;
        for (uint32_t r = 0; r <= cut; ++r) keep |= 1ull << lane_u(src, r);
    }
    float s1 = 0.f;
    for (uint32_t j = 0; j < nk; ++j)
        if ((keep >> j) & 1ull) s1 += lane_f(e, j);
    const float p = ((keep >> l) & 1ull) ? e * (1.0f / s1) : 0.f;
    float c = 0.f;
    uint32_t tok = 0xFFFFFFFFu;
    float tp = 0.f;
    const float r = S.r;
    for (uint32_t j = 0; j < nk; ++j) {
        const float pj = lane_f(p, j);
        c += pj;
        if (c > r) {
            tok = j;
            tp = pj;
            break;
        }
    }
    if (l == 0 && tok != 0xFFFFFFFFu) {
        S.tok = S.wi[tok];
        S.prob = tp;
    }
}

// Survivors of a key threshold (key >= kmin) in index order into S.wx / S.wi
// when there are at most 64 of them; returns their number (> 64: not copied).
template <class Kept>
__device__ __forceinline__ uint32_t gather_survivors(FinSh &S, const float *x, const uint32_t *id, Kept kept) {
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < (int)PER; ++j) c += kept(j);
    uint32_t n;
    uint32_t pos = block_excl_scan<FT>(c, S.ush, &n);
    if (n <= 64) {
#pragma unroll
        for (int j = 0; j < (int)PER; ++j)
            if (kept(j)) {
                S.wx[pos] = x[j];
                S.wi[pos] = id[j];
                ++pos;
            }
    }
    __syncthreads();
    return n;
}

// Candidates (the selection lists, in index order) held in registers, PER
// per thread in contiguous runs; every filter runs on chip.  Returns false
// (uniformly) when top-p alone is asked and the lists cannot be shown to
// hold the whole nucleus.
__device__ __forceinline__ bool finish_registers(const FinishArgs &a, FinSh &S, uint32_t nc) {
    const uint32_t tid = threadIdx.x;
    const uint32_t i0 = tid * PER;
    float x[PER];
    uint32_t id[PER];
    {
        // list holding element i0: the last b with koff[b] <= i0
        uint32_t lo = 0, hi = a.nb;  // koff[a.nb] = nc
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (S.koff[mid] <= i0) lo = mid;
            else hi = mid;
        }
        uint32_t b = lo, src[PER];
#pragma unroll
        for (int j = 0; j < (int)PER; ++j) {  // addresses first (LDS only) ...
            const uint32_t i = i0 + j;
            src[j] = 0;
            if (i < nc) {
                while (i >= S.koff[b + 1]) ++b;
                src[j] = b * SB + (i - S.koff[b]);
            }
        }
#pragma unroll
        for (int j = 0; j < (int)PER; ++j) {  // ... then every load in flight at once
            const bool v = i0 + j < nc;
            x[j] = v ? a.cx[src[j]] : -INFINITY;
            id[j] = v ? a.ci[src[j]] : 0xFFFFFFFFu;
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < (int)PER; ++j) M = fmaxf(M, x[j]);
    M = block_max<FT>(M, S.fsh);
    // top-k: keep x >= the k-th largest (applyTopK)
    uint32_t kmin = 0;  // kept: valid and key >= kmin
    if (a.mode == MODE_TOPK)
        kmin = radix_kth_largest<FT, FIN_W>(
            [&](auto f) {
#pragma unroll
                for (int j = 0; j < (int)PER; ++j)
                    if (id[j] != 0xFFFFFFFFu) f(fkey(x[j]));
            },
            a.k, S.hist, S.R);
    auto kept1 = [&](int j) { return id[j] != 0xFFFFFFFFu && fkey(x[j]) >= kmin; };
    // lists shorter than k: exact only if the k-th largest is inside them
    if (a.mode == MODE_TOPK && a.kc < a.k && a.kc < SB && kmin < lists_floor(a, S)) return false;
    if (a.mode == MODE_TOPK) {
        const uint32_t n1 = gather_survivors(S, x, id, kept1);
        if (n1 <= 64) {
            if (tid < 64) finish_wave(a, S, n1, M, 0.f);
            __syncthreads();
            return true;
        }
    }
    // top-p: the nucleus (applyTopP)
    MassCut cut{0, 0, 0, 0, true};
    if (a.top_p < 1.0f) {
        float s;
        if (a.mode == MODE_TOPK) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < (int)PER; ++j)
                if (kept1(j)) v += expf(x[j] - M);
            s = block_sum<FT>(v, S.fsh);
        } else {
            float Mg;
            s = total_from_blocks(a, S, &Mg);  // every logit counts; Mg == M
        }
        const float inv_s = 1.0f / s;
        const double needd = ceil((double)a.top_p * MASS_ONE);
        const unsigned long long need = needd < 1.0 ? 1ull : (unsigned long long)needd;
        if (a.mode == MODE_TOPP) {
            // every logit >= the largest list threshold is in the lists; the
            // nucleus must end above it
            unsigned long long cov = 0;
            const uint32_t tcmax = lists_floor(a, S);
#pragma unroll
            for (int j = 0; j < (int)PER; ++j)
                if (kept1(j) && fkey(x[j]) >= tcmax) cov += mass_of(expf(x[j] - M) * inv_s);
            cov = block_sum_u64(cov, S.lsh);
            if (cov < need) return false;
            // the nucleus usually lies within the 64 largest: one wave then
            const uint32_t k64 = nc < 64 ? nc : 64;
            const uint32_t t64 = radix_kth_largest<FT, FIN_W>(
                [&](auto f) {
#pragma unroll
                    for (int j = 0; j < (int)PER; ++j)
                        if (id[j] != 0xFFFFFFFFu) f(fkey(x[j]));
                },
                k64, S.hist, S.R);
            if (t64 >= tcmax) {
                unsigned long long m64 = 0;
#pragma unroll
                for (int j = 0; j < (int)PER; ++j)
                    if (kept1(j) && fkey(x[j]) >= t64) m64 += mass_of(expf(x[j] - M) * inv_s);
                m64 = block_sum_u64(m64, S.lsh);
                if (m64 >= need) {
                    const uint32_t n1 = gather_survivors(
                        S, x, id, [&](int j) { return kept1(j) && fkey(x[j]) >= t64; });
                    if (n1 <= 64) {
                        if (tid < 64) finish_wave(a, S, n1, M, s);
                        __syncthreads();
                        return true;
                    }
                }
            }
        }
        cut = radix_mass_cut<FT, MASS_W>(
            [&](auto f) {
#pragma unroll
                for (int j = 0; j < (int)PER; ++j)
                    if (kept1(j)) f(fkey(x[j]), mass_of(expf(x[j] - M) * inv_s));
            },
            need, S.hist, S.hmass, S.R);
    }
    uint32_t j_eq = 0xFFFFFFFFu;
    if (!cut.all) {
        unsigned long long j = cut.q_eq ? (cut.rem + cut.q_eq - 1) / cut.q_eq : cut.n_eq;
        if (j < 1) j = 1;
        if (j > cut.n_eq) j = cut.n_eq;
        j_eq = (uint32_t)j;
    }
    uint32_t c_eq = 0;
    if (!cut.all) {
#pragma unroll
        for (int j = 0; j < (int)PER; ++j) c_eq += kept1(j) && fkey(x[j]) == cut.tau;
    }
    uint32_t eq_tot;
    const uint32_t eq_before = block_excl_scan<FT>(c_eq, S.ush, &eq_tot);
    bool k2[PER];
    {
        uint32_t rank = eq_before;
#pragma unroll
        for (int j = 0; j < (int)PER; ++j) {
            bool k = kept1(j);
            if (k && !cut.all) {
                const uint32_t key = fkey(x[j]);
                if (key < cut.tau) k = false;
                else if (key == cut.tau) k = rank++ < j_eq;
            }
            k2[j] = k;
        }
    }
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < (int)PER; ++j)
        if (k2[j]) v += expf(x[j] - M);
    const float inv1 = 1.0f / block_sum<FT>(v, S.fsh);
    float cp = 0.f;
#pragma unroll
    for (int j = 0; j < (int)PER; ++j)
        if (k2[j]) cp += expf(x[j] - M) * inv1;
    float ptot;
    float cum = block_excl_scan<FT>(cp, S.fsh, &ptot);
    const float r = S.r;
    uint32_t found = 0xFFFFFFFFu;
    float fp = 0.f;
#pragma unroll
    for (int j = 0; j < (int)PER; ++j) {
        if (!k2[j] || found != 0xFFFFFFFFu) continue;
        const float p = expf(x[j] - M) * inv1;
        cum += p;
        if (cum > r) {
            found = id[j];
            fp = p;
        }
    }
    if (found != 0xFFFFFFFFu) atomicMin(&S.tok, found);
    __syncthreads();
    if (found != 0xFFFFFFFFu && found == S.tok) S.prob = fp;
    __syncthreads();
    return true;
}

// Element loops of the general path: 4 loads in flight per thread.
template <class Get, class F>
__device__ __forceinline__ void each_strided(uint32_t nk, Get get, F f) {
    uint32_t i = threadIdx.x;
    for (; i + 3 * FT < nk; i += 4 * FT) {
        float x[4];
        uint32_t id[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) get(i + j * FT, x[j], id[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) f(x[j], id[j]);
    }
    for (; i < nk; i += FT) {
        float x;
        uint32_t id;
        get(i, x, id);
        f(x, id);
    }
}

// In index order over [lo, hi); f returns true to stop.
template <class Get, class F>
__device__ __forceinline__ void each_run(uint32_t lo, uint32_t hi, Get get, F f) {
    uint32_t i = lo;
    for (; i + 4 <= hi; i += 4) {
        float x[4];
        uint32_t id[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) get(i + j, x[j], id[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (f(x[j], id[j])) return;
    }
    for (; i < hi; ++i) {
        float x;
        uint32_t id;
        get(i, x, id);
        if (f(x, id)) return;
    }
}

// General case in global memory (more candidates than the registers hold,
// or top-p alone over a flat distribution): the same filters over elements
// get(i), i < nk, each thread owning a contiguous run for the ordered steps.
template <class Get>
__device__ __forceinline__ void finish_general(const FinishArgs &a, FinSh &S, uint32_t nk, Get get, bool topk,
                               float s_all) {
    const uint32_t tid = threadIdx.x;
    float M = -INFINITY;
    each_strided(nk, get, [&](float x, uint32_t) { M = fmaxf(M, x); });
    M = block_max<FT>(M, S.fsh);
    uint32_t kmin = 0;
    if (topk)
        kmin = radix_kth_largest<FT, FIN_W>(
            [&](auto f) { each_strided(nk, get, [&](float x, uint32_t) { f(fkey(x)); }); }, a.k,
            S.hist, S.R);
    MassCut cut{0, 0, 0, 0, true};
    if (a.top_p < 1.0f) {
        float s = s_all;
        if (topk) {
            float v = 0.f;
            each_strided(nk, get, [&](float x, uint32_t) {
                if (fkey(x) >= kmin) v += expf(x - M);
            });
            s = block_sum<FT>(v, S.fsh);
        }
        const float inv_s = 1.0f / s;
        const double needd = ceil((double)a.top_p * MASS_ONE);
        const unsigned long long need = needd < 1.0 ? 1ull : (unsigned long long)needd;
        cut = radix_mass_cut<FT, MASS_W>(
            [&](auto f) {
                each_strided(nk, get, [&](float x, uint32_t) {
                    if (fkey(x) >= kmin) f(fkey(x), mass_of(expf(x - M) * inv_s));
                });
            },
            need, S.hist, S.hmass, S.R);
    }
    uint32_t j_eq = 0xFFFFFFFFu;
    if (!cut.all) {
        unsigned long long j = cut.q_eq ? (cut.rem + cut.q_eq - 1) / cut.q_eq : cut.n_eq;
        if (j < 1) j = 1;
        if (j > cut.n_eq) j = cut.n_eq;
        j_eq = (uint32_t)j;
    }
    const uint32_t cs = (nk + FT - 1) / FT;
    const uint32_t lo = tid * cs < nk ? tid * cs : nk, hi = lo + cs < nk ? lo + cs : nk;
    uint32_t c_eq = 0;
    if (!cut.all)
        each_run(lo, hi, get, [&](float x, uint32_t) {
            c_eq += fkey(x) >= kmin && fkey(x) == cut.tau;
            return false;
        });
    uint32_t eq_tot;
    const uint32_t eq_before = block_excl_scan<FT>(c_eq, S.ush, &eq_tot);
    auto kept = [&](float x, uint32_t &rank) {
        const uint32_t key = fkey(x);
        if (key < kmin) return false;
        if (cut.all) return true;
        if (key < cut.tau) return false;
        if (key == cut.tau) return rank++ < j_eq;
        return true;
    };
    float v = 0.f;
    {
        uint32_t rank = eq_before;
        each_run(lo, hi, get, [&](float x, uint32_t) {
            if (kept(x, rank)) v += expf(x - M);
            return false;
        });
    }
    const float inv1 = 1.0f / block_sum<FT>(v, S.fsh);
    float cp = 0.f;
    {
        uint32_t rank = eq_before;
        each_run(lo, hi, get, [&](float x, uint32_t) {
            if (kept(x, rank)) cp += expf(x - M) * inv1;
            return false;
        });
    }
    float ptot;
    float cum = block_excl_scan<FT>(cp, S.fsh, &ptot);
    const float r = S.r;
    uint32_t found = 0xFFFFFFFFu;
    float fp = 0.f;
    {
        uint32_t rank = eq_before;
        each_run(lo, hi, get, [&](float x, uint32_t idx) {
            if (!kept(x, rank)) return false;
            const float p = expf(x - M) * inv1;
            cum += p;
            if (cum > r) {
                found = idx;
                fp = p;
                return true;
            }
            return false;
        });
    }
    if (found != 0xFFFFFFFFu) atomicMin(&S.tok, found);
    __syncthreads();
    if (found != 0xFFFFFFFFu && found == S.tok) S.prob = fp;
    __syncthreads();
}

__global__ __launch_bounds__(1024) void sample_finish_kernel(FinishArgs a) {
    __shared__ FinSh S;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) {
        uint64_t st[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) st[j] = a.rng[j];
        S.r = zig_float32(st);
#pragma unroll
        for (int j = 0; j < 4; ++j) a.rng[j] = st[j];
        S.tok = 0xFFFFFFFFu;
        S.aux = 0xFFFFFFFFu;
        S.fallback = 0;
        S.prob = 0.f;
    }
    __syncthreads();
    if (a.mode == MODE_TEMP) {
        finish_temperature(a, S);
    } else {
        // list offsets (exclusive prefix of the list lengths), koff[nb] = total
        uint32_t carry = 0;
        for (uint32_t b0 = 0; b0 < a.nb; b0 += FT) {
            const uint32_t b = b0 + tid;
            const uint32_t v = b < a.nb ? a.blk_cnt[b] : 0u;
            uint32_t tot;
            const uint32_t ex = block_excl_scan<FT>(v, S.ush, &tot);
            if (b < a.nb) S.koff[b] = carry + ex;
            carry += tot;
        }
        if (tid == 0) S.koff[a.nb] = carry;
        __syncthreads();
        const uint32_t nc = carry;
        bool done = false;
        if (nc <= RCAP) done = finish_registers(a, S, nc);
        if (!done) {
            if (a.mode == MODE_TOPK && (a.kc >= a.k || a.kc >= SB)) {
                // complete lists: gather them densely, then work from global memory
                for (uint32_t e = tid; e < nc; e += FT) {
                    uint32_t lo = 0, hi = a.nb;
                    while (hi - lo > 1) {
                        const uint32_t mid = (lo + hi) >> 1;
                        if (S.koff[mid] <= e) lo = mid;
                        else hi = mid;
                    }
                    while (e >= S.koff[lo + 1]) ++lo;
                    const size_t src = (size_t)lo * SB + (e - S.koff[lo]);
                    a.kx[e] = a.cx[src];
                    a.ki[e] = a.ci[src];
                }
                __syncthreads();
                finish_general(
                    a, S, nc,
                    [&](uint32_t i, float &x, uint32_t &idx) {
                        x = a.kx[i];
                        idx = a.ki[i];
                    },
                    true, 0.f);
            } else {
                // truncated lists that miss part of the top-k set, or top-p
                // alone with the nucleus beyond the lists: every logit
                float Mg;
                const float s_all = total_from_blocks(a, S, &Mg);
                finish_general(
                    a, S, a.n,
                    [&](uint32_t i, float &x, uint32_t &idx) {
                        x = a.logits[i] * a.inv_t;
                        idx = i;
                    },
                    a.mode == MODE_TOPK, s_all);
            }
        }
    }
    if (tid == 0) {
        // rounding tail: the reference returns the last index (probs.len - 1)
        const uint32_t tok = S.tok;
        const uint32_t out = tok == 0xFFFFFFFFu ? a.n - 1 : tok;
        const float pr = tok == 0xFFFFFFFFu ? 0.f : S.prob;
        if (a.out_index) a.out_index[0] = out;
        if (a.out_prob) a.out_prob[0] = pr;
        if (a.pick.state) nnz_pick_advance(a.pick, out, pr);
    }
}

// Zig std.Random.SplitMix64.next, used by Xoshiro256.init to expand the seed.
uint64_t splitmix64_next(uint64_t &s) {
    s += 0x9e3779b97f4a7c15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct WsLayout {
    size_t blk_max, blk_sum, blk_cnt, blk_kth, cx, ci, kx, ki, total;
};

WsLayout ws_layout(uint32_t n) {
    const size_t nb = ceil_div(n, SB);
    WsLayout L{};
    size_t o = 0;
    L.blk_max = o; o += align256(nb * 4);
    L.blk_sum = o; o += align256(nb * 4);
    L.blk_cnt = o; o += align256(nb * 4);
    L.blk_kth = o; o += align256(nb * 4);
    L.cx = o; o += align256(nb * SB * 4);
    L.ci = o; o += align256(nb * SB * 4);
    L.kx = o; o += align256((size_t)n * 4);
    L.ki = o; o += align256((size_t)n * 4);
    L.total = o;
    return L;
}

}  // namespace

void nnz_rng_seed_words(uint64_t seed, uint64_t out[4]) {
    uint64_t s = seed;
    for (int i = 0; i < 4; ++i) out[i] = splitmix64_next(s);
}

size_t nnz_sample_ws_bytes(uint32_t n) { return ws_layout(n).total; }

int nnz_sample_launch(nnz_ctx *ctx, const float *logits, uint32_t n, const nnz_sampling_params &p,
                      uint64_t *rng, void *ws, uint32_t *out_index, float *out_prob,
                      const NnzPick *pick) {
    NNZ_REQUIRE(ctx, n > 0 && n <= MAX_BLOCKS * SB, NNZ_EUNSUPPORTED,
                "sample: count %u outside 1..%u", n, MAX_BLOCKS * SB);
    NNZ_REQUIRE(ctx, p.temperature > 0.f && p.temperature <= 3.0e38f, NNZ_EINVAL,
                "sample: temperature must be > 0 (0 selects argmax)");
    // applyTopP asserts 0 < p <= 1 (transformer.zig:3781-3790); p >= 1 is
    // "off" at the call site (:3878).  NaN and p <= 0 are refused.
    NNZ_REQUIRE(ctx, p.top_p > 0.f, NNZ_EINVAL, "sample: top_p must be > 0 (>= 1 disables it)");
    // applyTemperature: inv_t = 1/T in f32, then logit * inv_t (transformer.zig:3713-3718)
    const float inv_t = 1.0f / p.temperature;
    const WsLayout L = ws_layout(n);
    char *w = (char *)ws;
    const uint32_t nb = ceil_div(n, SB);
    FinishArgs a{};
    a.logits = logits;
    a.n = n;
    a.inv_t = inv_t;
    a.top_p = p.top_p;
    a.nb = nb;
    a.blk_max = (const float *)(w + L.blk_max);
    a.blk_sum = (const float *)(w + L.blk_sum);
    a.blk_cnt = (const uint32_t *)(w + L.blk_cnt);
    a.blk_kth = (const uint32_t *)(w + L.blk_kth);
    a.cx = (const float *)(w + L.cx);
    a.ci = (const uint32_t *)(w + L.ci);
    a.kx = (float *)(w + L.kx);
    a.ki = (uint32_t *)(w + L.ki);
    a.rng = (unsigned long long *)rng;
    a.out_index = out_index;
    a.out_prob = out_prob;
    if (pick) a.pick = *pick;
    // per-block list length: what the finishing registers hold over nb lists
    const uint32_t fit = RCAP / nb > 1 ? RCAP / nb : 1;
    uint32_t kc = 0;
    if (p.top_k > 0 && p.top_k < n) {  // applyTopK returns early when k >= len
        a.mode = MODE_TOPK;
        a.k = p.top_k;
        kc = p.top_k < SB ? p.top_k : SB;
        if (kc > fit) kc = fit;
    } else if (p.top_p < 1.0f) {
        a.mode = MODE_TOPP;
        kc = KB_TOPP < fit ? KB_TOPP : fit;
    } else {
        a.mode = MODE_TEMP;
    }
    a.kc = kc;
    sample_select_kernel<<<nb, 256, 0, ctx->stream>>>(
        logits, n, inv_t, kc, (float *)(w + L.blk_max), (float *)(w + L.blk_sum),
        (uint32_t *)(w + L.blk_cnt), (uint32_t *)(w + L.blk_kth), (float *)(w + L.cx),
        (uint32_t *)(w + L.ci));
    NNZ_LAUNCHED(ctx);
    sample_finish_kernel<<<1, FT, 0, ctx->stream>>>(a);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

extern "C" {

size_t nnz_sample_workspace_bytes(uint32_t count) { return nnz_sample_ws_bytes(count); }

int nnz_rng_seed(nnz_ctx *ctx, uint64_t seed, uint64_t *d_state) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, d_state, NNZ_EINVAL, "rng_seed: null state");
    uint64_t s[4];
    nnz_rng_seed_words(seed, s);
    NNZ_HIP(ctx, hipMemcpyAsync(d_state, s, sizeof(s), hipMemcpyHostToDevice, ctx->stream));
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return NNZ_OK;
}

int nnz_dispatch_sample(nnz_ctx *ctx, const float *logits, uint32_t count,
                        const nnz_sampling_params *params, uint64_t *d_rng, void *workspace,
                        size_t workspace_bytes, uint32_t *out_index, float *out_prob) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, logits && params && out_index && count > 0, NNZ_EINVAL,
                "sample: bad arguments");
    if (params->temperature == 0.f)  // sampleToken: greedy returns argmax
        return nnz_argmax_launch(ctx, logits, count, out_index, nullptr);
    NNZ_REQUIRE(ctx, d_rng && workspace, NNZ_EINVAL, "sample: null rng state or workspace");
    NNZ_REQUIRE(ctx, workspace_bytes >= nnz_sample_ws_bytes(count), NNZ_EINVAL,
                "sample: workspace %zu bytes, %zu needed", workspace_bytes,
                nnz_sample_ws_bytes(count));
    return nnz_sample_launch(ctx, logits, count, *params, d_rng, workspace, out_index, out_prob,
                             nullptr);
}

}  // extern "C"

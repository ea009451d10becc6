// Causal GQA attention of a prefill batch on the matrix cores.
//
// Replaces, for the batched prefill, the reference's token-by-token
// attention (gqa_attention_fused_f16io_tg per prompt token,
// transformer.metal:1438-1695, driven by chunkedPrefill,
// transformer.zig:4032-4068) with one flash-attention launch per layer:
// queries n tokens at positions start.., keys/values from the layer's f16
// KV cache (K [Hkv][max_ctx][D], V transposed [Hkv][D][max_ctx]) after the
// prep kernel appended the batch's own keys and values.
//
// Layout on the MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulate):
//   * a wave owns 16 queries of one query head; a block holds the G query
//     heads of one KV head, so the K/V tiles staged in LDS serve all of them
//     (and, for G = 2, four key splits of each head: S consecutive tiles are
//     staged per step, wave split s takes tile s, and the partial softmax
//     states are merged through LDS at the end);
//   * scores are computed transposed, S^T[key][q] = K . Q^T: A = 16 keys x
//     32 dims of K from LDS, B = Q^T from registers.  The accumulator puts
//     keys 4g..4g+3 of a 16-key block in lane group g's four registers, all
//     for the lane's own query q = lane % 16;
//   * O^T[d][q] += V^T . P^T takes B = P^T straight from those registers:
//     for a 32-key step, B slot 8g + 4s + r is key 16(2k+s) + 4g + r, and
//     the A operand (V^T from LDS) reads V in the same key order, so no
//     data moves between lanes;
//   * the online softmax of query q runs in its own lanes (max/sum over the
//     lane's 16 keys, then over the 4 lane groups).
// Precision: the queries are kept unrounded (float32, as the reference
// keeps q), so each MFMA operand that is not already f16 is split into an
// f16 high part and an f16 remainder -- q and the probabilities p -- and
// both products are accumulated: the scores carry ~2^-22 and P.V ~2^-20
// relative error, float32-level arithmetic on these f16 keys and values.
// The prep kernel writes q pre-scaled by log2(e)/sqrt(D) and already split
// (hi = f16(x), lo = f16(x - hi)), so the scores come out in log2 units and
// the softmax runs in base 2 (v_exp_f32) with the same probabilities.
#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
// 16-byte staging pieces as a native vector (a struct type is copied by
// memcpy, which can keep the staging arrays in scratch memory)
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int KT = 64;  // keys per LDS tile
// Key splits of the G = 2 blocks (8 waves; measured per layer at P = 512:
// 24.5 us unsplit, 18.6 us with 2 splits, 16.5 us with 4).  G = 4 and 8
// blocks already hold 4 and 8 waves.
constexpr int S_G2 = 4;

struct PrefillArgs {
    const f16_t *q;      // [n][hq][2][D]: hi and lo f16 rows of q log2(e)/sqrt(D)
    const f16_t *kc;     // [hkv][max_ctx][D]
    const f16_t *vc;     // [hkv][D][max_ctx]
    f16_t *out;          // [n][hq][D]
    uint32_t start, n, hq, max_ctx;
};

// S key splits: the block holds S x G waves; wave (ws, w) walks the key
// tiles ws, ws + S, ... of query head w and the S partial softmax states
// (running max, sum, O) of each head are merged through LDS at the end.
template <int D, int G, int S>
__global__ __launch_bounds__(64 * G * S) void attn_prefill_kernel(PrefillArgs a) {
    constexpr int NT = 64 * G * S;
    constexpr int NKS = D / 32;  // 32-dim steps of the score MFMAs
    constexpr int NDT = D / 16;  // 16-dim tiles of O^T
    constexpr int KP = D + 8;    // LDS pitch (halves) of a K row
    constexpr int VP = KT + 8;   // LDS pitch (halves) of a V^T row
    constexpr int KTILE = KT * KP, VTILE = D * VP;          // halves per staged tile
    constexpr int MSLOT = (NDT * 4 + 2) * 64;               // floats per merge slot
    constexpr int SMEM = S * (KTILE + VTILE) * 2 > (S - 1) * G * MSLOT * 4
                             ? S * (KTILE + VTILE) * 2 : (S - 1) * G * MSLOT * 4;
    __shared__ __align__(16) unsigned char smem[SMEM];
    _Float16 *Ks = (_Float16 *)smem;              // [S][KT][KP]
    _Float16 *Vs = (_Float16 *)smem + S * KTILE;  // [S][D][VP]
    // the queries of the block with key splits: [G][16][QP], row pitch
    // 2D + 8 halves (the 16 rows of a fragment read hit distinct banks)
    constexpr int QP = 2 * D + 8;
    __shared__ __align__(16) _Float16 Qs[S > 1 ? G * 16 * QP : 8];

    const int tid = threadIdx.x, lane = tid & 63, w = (tid >> 6) % G, ws = (tid >> 6) / G;
    const int g = lane >> 4, c = lane & 15;
    const uint32_t hkv = blockIdx.y;
    const uint32_t h = hkv * G + (uint32_t)w;
    const uint32_t q0 = blockIdx.x * 16u;
    const uint32_t qi = q0 + (uint32_t)c;
    const bool qvalid = qi < a.n;
    const uint32_t qpos = a.start + qi;
    const uint32_t seq_end = a.start + a.n;
    const uint32_t qlast = (q0 + 15u < a.n ? q0 + 15u : a.n - 1u) + a.start;
    const uint32_t ntiles = qlast / KT + 1u, nsteps = (ntiles + S - 1) / S;

    // Q^T fragments: lane (g, c) holds dims 32 ks + 8 g .. +8 of query c,
    // the f16 hi and lo parts the prep kernel wrote (zero past the batch).
    // With key splits the S waves of a head share one copy: the block loads
    // its 16 queries x G heads once into Qs and each wave reads its
    // fragments from there.  The query loads are issued first and the first
    // tile's right after them; both are used only at the first stage, so
    // their latencies overlap.
    constexpr int QROW = G * 2 * D / 8;   // Q staging: 16-byte pieces per query
    constexpr int QPT = S > 1 ? 16 * QROW / NT : 1;
    static_assert(S == 1 || 16 * QROW % NT == 0, "Q staging layout");
    v4u qr[QPT];
    half8 qh[NKS], ql[NKS];
    if constexpr (S > 1) {
#pragma unroll
        for (int i = 0; i < QPT; ++i) {
            const uint32_t p = (uint32_t)(tid + i * NT), qc = p / QROW, e = p % QROW;
            const uint32_t qq = q0 + qc < a.n ? q0 + qc : 0u;
            qr[i] = *(const v4u *)(a.q + ((size_t)qq * a.hq + hkv * G) * (2 * D) + e * 8);
        }
    } else {
        const f16_t *qp = a.q + ((size_t)(qvalid ? qi : 0u) * a.hq + h) * (2 * D);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            qh[ks] = *(const half8 *)(qp + 32 * ks + 8 * g);
            ql[ks] = *(const half8 *)(qp + D + 32 * ks + 8 * g);
        }
    }
    float4v o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = (float4v){0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    const f16_t *kbase = a.kc + (size_t)hkv * a.max_ctx * D;
    const f16_t *vbase = a.vc + (size_t)hkv * D * a.max_ctx;
    // Tiles are staged through registers, one ahead: the next tile's loads
    // are in flight while the current one is computed.  A step stages S
    // consecutive tiles, tile j of the step in LDS slot j (8-key V pieces
    // never cross max_ctx: max_ctx % 8 == 0).  Lane offsets: staging piece i of lane tid is K row krow + i NT/(D/8)
    // of the step, dims kcol..+8, and V^T row vrow + (i NT mod D KT/8)/(KT/8)
    // of tile (i NT)/(D KT/8), keys vcol..+8.
    constexpr int KPT = S * KT * D / 8 / NT, VPT = S * D * KT / 8 / NT;
    constexpr int RPI = NT / (D / 8);   // K rows per staging piece index
    static_assert(NT % (D / 8) == 0 && (D * KT / 8) % NT == 0, "staging layout");
    static_assert(KT % RPI == 0 || RPI % KT == 0, "a K piece lies in one tile");
    const uint32_t krow = (uint32_t)tid / (D / 8), kcol = ((uint32_t)tid % (D / 8)) * 8u;
    const uint32_t vrow = (uint32_t)tid / (KT / 8), vcol = ((uint32_t)tid % (KT / 8)) * 8u;
    v4u kr[KPT], vr[VPT];
    // live = false: nothing to stage (the loop's look-ahead past the last
    // step).  Nothing uses the loaded data before the stage (an early use
    // would wait there for every older load, the query loads' wait for the
    // first tile's).  Pieces of tiles no query of the block reaches are not
    // loaded (block-uniform branches; their LDS slots are never read);
    // pieces of keys past the batch read the head's key 0 instead (in
    // bounds for any max_ctx): such K rows are finite and their scores
    // masked, and V pieces past the batch are zeroed at the stage, since
    // p = 0 must not meet a non-finite value.
    auto load_tile = [&](uint32_t k0, bool live) __attribute__((always_inline)) {
        if (!live) return;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            if (k0 + (uint32_t)((i * RPI) / KT * KT) > qlast) continue;
            const uint32_t key = k0 + (uint32_t)(i * RPI) + krow;
            kr[i] = *(const v4u *)(kbase + (key < seq_end ? key * D + kcol : kcol));
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            constexpr uint32_t TS = D * KT / 8;
            const uint32_t j = (uint32_t)(i * NT) / TS, dr = ((uint32_t)(i * NT) % TS) / (KT / 8);
            if (k0 + j * KT > qlast) continue;
            const uint32_t key = k0 + j * KT + vcol;
            vr[i] = *(const v4u *)(vbase + (vrow + dr) * a.max_ctx + (key < seq_end ? key : 0u));
        }
    };
    auto store_tile = [&](uint32_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int p = tid + i * NT;
            *(v4u *)(Ks + (p / (D / 8)) * KP + (p % (D / 8)) * 8) = kr[i];
        }
        if (k0 + (uint32_t)(S * KT) > seq_end) {   // block-uniform: the step crosses the batch end
#pragma unroll
            for (int i = 0; i < VPT; ++i) {   // halves e with key + e >= seq_end become 0
                const uint32_t key = k0 + (uint32_t)((i * NT) / (D * KT / 8) * KT) + vcol;
                const int keep = key >= seq_end ? 0 : (int)(seq_end - key < 8u ? seq_end - key : 8u);
                vr[i].x &= keep >= 2 ? ~0u : (keep >= 1 ? 0xFFFFu : 0u);
                vr[i].y &= keep >= 4 ? ~0u : (keep >= 3 ? 0xFFFFu : 0u);
                vr[i].z &= keep >= 6 ? ~0u : (keep >= 5 ? 0xFFFFu : 0u);
                vr[i].w &= keep >= 8 ? ~0u : (keep >= 7 ? 0xFFFFu : 0u);
            }
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int p = tid + i * NT;
            const int j = p / (D * KT / 8), pp = p % (D * KT / 8);
            *(v4u *)(Vs + j * VTILE + (pp / (KT / 8)) * VP + (pp % (KT / 8)) * 8) = vr[i];
        }
    };
    load_tile(0, true);

    // The first stage also stages the queries (zeros past the batch): with
    // key splits into their own LDS rows, read back after its barrier.
    store_tile(0u);
    if constexpr (S > 1) {
#pragma unroll
        for (int i = 0; i < QPT; ++i) {
            const uint32_t p = (uint32_t)(tid + i * NT), qc = p / QROW, e = p % QROW;
            const uint32_t hw = e / (2 * D / 8), col = e % (2 * D / 8);
            *(v4u *)(Qs + (hw * 16 + qc) * QP + col * 8) = q0 + qc < a.n ? qr[i] : (v4u){0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();
    if constexpr (S > 1) {
        const _Float16 *qrow = Qs + (w * 16 + c) * QP;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            qh[ks] = *(const half8 *)(qrow + 32 * ks + 8 * g);
            ql[ks] = *(const half8 *)(qrow + D + 32 * ks + 8 * g);
        }
    } else {
        const half8 zero = {};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            qh[ks] = qvalid ? qh[ks] : zero;
            ql[ks] = qvalid ? ql[ks] : zero;
        }
    }
    for (uint32_t step = 0; step < nsteps; ++step) {
        if (step > 0) {   // block-uniform
            store_tile(step * (S * KT));
            __syncthreads();
        }
        load_tile((step + 1) * (S * KT), step + 1 < nsteps);
        const uint32_t t = step * S + (uint32_t)ws;   // this wave's tile
        if (t < ntiles) {   // wave-uniform
        const uint32_t k0 = t * KT;
        const _Float16 *Kt = Ks + ws * KTILE, *Vt = Vs + ws * VTILE;

        // S^T = K . Q^T, 4 blocks of 16 keys
        float4v s[KT / 16];
#pragma unroll
        for (int st = 0; st < KT / 16; ++st) {
            s[st] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const half8 ka = *(const half8 *)(Kt + (st * 16 + c) * KP + 32 * ks + 8 * g);
                s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[ks], s[st], 0, 0, 0);
                s[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[ks], s[st], 0, 0, 0);
            }
        }
        // causal mask (tiles that end before the block's first query need
        // none; keys past the batch end are masked there too), online
        // softmax of query c in log2 units: p = 2^(s - m)
        if (k0 + (uint32_t)(KT - 1) > a.start + q0) {   // wave-uniform
#pragma unroll
            for (int st = 0; st < KT / 16; ++st)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t key = k0 + (uint32_t)(st * 16 + 4 * g + r);
                    s[st][r] = key <= qpos ? s[st][r] : -INFINITY;
                }
        }
        float mx = s[0][0];
#pragma unroll
        for (int st = 0; st < KT / 16; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[st][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        // a query with every key so far masked keeps p = 0 (2^-inf)
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float ls = 0.f;
#pragma unroll
        for (int st = 0; st < KT / 16; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = __builtin_amdgcn_exp2f(s[st][r] - m_use);
                s[st][r] = p;
                ls += p;
            }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        m_run = m_new;
        if (step == 0) {   // wave-uniform: nothing accumulated yet
            l_run = ls;
        } else {
            l_run = l_run * alpha + ls;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
        }

        // P^T as B operands: slot 8g + 4 sb + r = key 16 (2 kk + sb) + 4 g + r,
        // p = hi + lo with both halves rounded toward zero (|p - hi - lo| <
        // 2^-20 p)
        half8 ph[KT / 32], pl[KT / 32];
#pragma unroll
        for (int kk = 0; kk < KT / 32; ++kk)
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    const float p0 = s[2 * kk + sb][r], p1 = s[2 * kk + sb][r + 1];
                    const auto hi = __builtin_amdgcn_cvt_pkrtz(p0, p1);
                    const auto lo = __builtin_amdgcn_cvt_pkrtz(p0 - (float)hi[0], p1 - (float)hi[1]);
                    ph[kk][4 * sb + r] = hi[0];
                    ph[kk][4 * sb + r + 1] = hi[1];
                    pl[kk][4 * sb + r] = lo[0];
                    pl[kk][4 * sb + r + 1] = lo[1];
                }
        // O^T += V^T . P^T
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const _Float16 *vrow = Vt + (16 * dt + c) * VP + 4 * g;
#pragma unroll
            for (int kk = 0; kk < KT / 32; ++kk) {
                const uint2 lo4 = *(const uint2 *)(vrow + (2 * kk) * 16);
                const uint2 hi4 = *(const uint2 *)(vrow + (2 * kk + 1) * 16);
                const uint4 u = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
                const half8 va = __builtin_bit_cast(half8, u);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph[kk], o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[kk], o[dt], 0, 0, 0);
            }
        }
        }   // t < ntiles
        __syncthreads();
    }

    if constexpr (S > 1) {
        // merge the S partial states of head w into split 0 (the tile
        // buffers are free: the loop ended with a barrier)
        float *mrg = (float *)smem;
        if (ws > 0) {
            float *slot = mrg + ((ws - 1) * G + w) * MSLOT + lane;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) slot[(dt * 4 + r) * 64] = o[dt][r];
            slot[(NDT * 4) * 64] = m_run;
            slot[(NDT * 4 + 1) * 64] = l_run;
        }
        __syncthreads();
        if (ws != 0) return;   // after the last barrier
        float m = m_run;
#pragma unroll
        for (int s2 = 1; s2 < S; ++s2) m = fmaxf(m, mrg[((s2 - 1) * G + w) * MSLOT + (NDT * 4) * 64 + lane]);
        const float c0 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m);
        l_run *= c0;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] *= c0;
#pragma unroll
        for (int s2 = 1; s2 < S; ++s2) {
            const float *slot = mrg + ((s2 - 1) * G + w) * MSLOT + lane;
            const float ms = slot[(NDT * 4) * 64];
            const float cs = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - m);
            l_run += slot[(NDT * 4 + 1) * 64] * cs;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dt][r] += slot[(dt * 4 + r) * 64] * cs;
        }
    }
    if (qvalid) {
        const float inv = 1.0f / l_run;
        f16_t *op = a.out + ((size_t)qi * a.hq + h) * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const uint32_t d = 16u * dt + 4u * g;
            const uint32_t p0 = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)(o[dt][0] * inv)) |
                                (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)(o[dt][1] * inv)) << 16;
            const uint32_t p1 = (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)(o[dt][2] * inv)) |
                                (uint32_t)__builtin_bit_cast(uint16_t, (f16_t)(o[dt][3] * inv)) << 16;
            *(uint2 *)(op + d) = make_uint2(p0, p1);
        }
    }
}

template <int D>
int launch_d(nnz_ctx *ctx, const PrefillArgs &a, uint32_t hkv, uint32_t G) {
    const dim3 grid((a.n + 15) / 16, hkv);
    switch (G) {
    case 2: attn_prefill_kernel<D, 2, S_G2><<<grid, 128 * S_G2, 0, ctx->stream>>>(a); break;
    case 4: attn_prefill_kernel<D, 4, 1><<<grid, 256, 0, ctx->stream>>>(a); break;
    default: attn_prefill_kernel<D, 8, 1><<<grid, 512, 0, ctx->stream>>>(a); break;
    }
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

}  // namespace

bool nnz_attn_prefill_supported(uint32_t head_dim, uint32_t hq, uint32_t hkv, uint32_t max_ctx) {
    if (head_dim != 64 && head_dim != 128) return false;
    if (hkv == 0 || hq % hkv) return false;
    const uint32_t G = hq / hkv;   // blocks of G waves stage the tiles: G >= 2
    return (G == 2 || G == 4 || G == 8) && max_ctx % 8 == 0;
}

float nnz_attn_prefill_qscale(uint32_t head_dim) {
    return 1.44269504088896341f / sqrtf((float)head_dim);
}

int nnz_attn_prefill_launch(nnz_ctx *ctx, const void *q, const void *kc, const void *vc, void *out,
                            uint32_t start, uint32_t n, uint32_t hq, uint32_t hkv,
                            uint32_t head_dim, uint32_t max_ctx) {
    NNZ_REQUIRE(ctx, q && kc && vc && out && n > 0, NNZ_EINVAL, "attn_prefill: bad arguments");
    NNZ_REQUIRE(ctx, nnz_attn_prefill_supported(head_dim, hq, hkv, max_ctx), NNZ_EUNSUPPORTED,
                "attn_prefill: head_dim %u, %u/%u heads, max_ctx %u not supported", head_dim, hq,
                hkv, max_ctx);
    NNZ_REQUIRE(ctx, (uint64_t)start + n <= max_ctx, NNZ_EINVAL,
                "attn_prefill: positions %u..%u beyond max_ctx %u", start, start + n - 1, max_ctx);
    NNZ_REQUIRE(ctx, (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc | (uintptr_t)out) & 15) == 0,
                NNZ_EINVAL, "attn_prefill: buffers must be 16-byte aligned");
    PrefillArgs a{(const f16_t *)q, (const f16_t *)kc, (const f16_t *)vc, (f16_t *)out,
                  start, n, hq, max_ctx};
    return head_dim == 128 ? launch_d<128>(ctx, a, hkv, hq / hkv) : launch_d<64>(ctx, a, hkv, hq / hkv);
}

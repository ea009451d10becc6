// Decoder model: Model(Config) state, forwardDecode, batched prefill and the
// greedy generate loop on one MI355X.
//
// Replaces nnmetal/src/model.zig:38-777 (Model: weights, KV caches and
// activation scratch allocated once), transformer.zig:2389-3646 (the decode
// graph: embed -> 28 x (attention half, MLP half) -> final norm -> LM head)
// and transformer.zig:3942-4123 (generate / decodeOneToken).
//
// MI355X-first differences:
//   * Every buffer lives in HBM (hipMalloc), uploaded once; nothing is shared
//     with the host on the hot path.
//   * The decode step reads token id, position and sequence length from a
//     small device state block, so the whole step is captured once as a HIP
//     graph and replayed for every token.  Greedy argmax runs on the device
//     and writes the next token into that state block, so consecutive steps
//     are queued back to back with no host round trip (the reference reads
//     607 KB of logits to the CPU and spin-waits on a flag per token,
//     transformer.zig:4072-4122, metal.zig:1325-1352).
//   * Prefill runs the prompt as one batch through the MFMA dequant-GEMM and a
//     causal batched attention instead of P sequential decode steps
//     (transformer.zig:4032-4068).  Storage rounding points are the same as
//     the decode step: f16 activations and KV cache, f32 residual stream.
#include "internal.h"

#include <algorithm>
#include <vector>

// Public launchers implemented in qmv.hip / transformer.hip.
extern "C" {
int nnz_dispatch_fused_norm_qmv_f16io(nnz_ctx *, const nnz_qweight *, const float *, void *,
                                      const float *, nnz_qmv_dims);
int nnz_dispatch_fused_norm_pair_qmv_f16io(nnz_ctx *, const nnz_qweight *, const nnz_qweight *,
                                           const float *, void *, void *, const float *,
                                           nnz_qmv_dims);
int nnz_dispatch_fused_norm_pair_silu_f16io(nnz_ctx *, const nnz_qweight *, const nnz_qweight *,
                                            const float *, void *, const float *, nnz_qmv_dims);
int nnz_dispatch_qmv_f16io_resadd(nnz_ctx *, const nnz_qweight *, const void *, float *,
                                  nnz_qmv_dims);
int nnz_dispatch_qmv_f16in(nnz_ctx *, const nnz_qweight *, const void *, float *, nnz_qmv_dims);
}

namespace {

// Device state block: token id, position, visible sequence length, emitted
// count, stopped flag.
enum { ST_TOKEN = NNZ_ST_TOKEN, ST_POS = NNZ_ST_POS, ST_SEQ = NNZ_ST_SEQ, ST_STEP = NNZ_ST_STEP,
       ST_DONE = NNZ_ST_DONE, ST_WORDS = 5 };

__global__ void embed_state_q1_kernel(const uint32_t *state, const uint8_t *bits,
                                      const uint16_t *scales, float *out, uint32_t hidden,
                                      uint32_t gs, uint32_t vocab) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= hidden) return;
    uint32_t row = state[ST_TOKEN];
    if (row >= vocab) row = vocab - 1;
    const uint64_t flat = (uint64_t)row * hidden + d;
    const bool bit = (bits[flat >> 3] >> (flat & 7)) & 1;
    const float s = (float)__builtin_bit_cast(f16_t, scales[flat / gs]);
    out[d] = bit ? s : -s;
}

__global__ void embed_state_bf16_kernel(const uint32_t *state, const uint16_t *table, float *out,
                                        uint32_t hidden, uint32_t vocab) {
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= hidden) return;
    uint32_t row = state[ST_TOKEN];
    if (row >= vocab) row = vocab - 1;
    out[d] = bf16_to_f32(table[(size_t)row * hidden + d]);
}

__global__ void embed_ids_q1_kernel(const uint32_t *ids, const uint8_t *bits, const uint16_t *scales,
                                    float *out, uint32_t hidden, uint32_t ntok, uint32_t gs,
                                    uint32_t vocab) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= ntok * hidden) return;
    const uint32_t t = gid / hidden, d = gid % hidden;
    uint32_t row = ids[t];
    if (row >= vocab) row = vocab - 1;
    const uint64_t flat = (uint64_t)row * hidden + d;
    const bool bit = (bits[flat >> 3] >> (flat & 7)) & 1;
    const float s = (float)__builtin_bit_cast(f16_t, scales[flat / gs]);
    out[gid] = bit ? s : -s;
}

__global__ void embed_ids_bf16_kernel(const uint32_t *ids, const uint16_t *table, float *out,
                                      uint32_t hidden, uint32_t ntok, uint32_t vocab) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= ntok * hidden) return;
    const uint32_t t = gid / hidden, d = gid % hidden;
    uint32_t row = ids[t];
    if (row >= vocab) row = vocab - 1;
    out[gid] = bf16_to_f32(table[(size_t)row * hidden + d]);
}

// Dense bf16 LM head (tied embedding table): y[v] = sum_k E[v][k] x[k], x f16.
// Same lane layout as the QMV kernels: a lane owns 32-column units of the
// row (64 bytes = four 16-byte loads), x slice in registers, rows reduced
// across the lane group.
template <int NV>
__global__ __launch_bounds__(256) void dense_bf16_gemv_kernel(const uint16_t *E, const f16_t *x,
                                                              float *y, uint32_t M, uint32_t K,
                                                              uint32_t lpr_log2) {
    const int lane = threadIdx.x & 63;
    const int LPR = 1 << lpr_log2, RPW = 64 >> lpr_log2;
    const int rr = lane >> lpr_log2, ll = lane & (LPR - 1);
    const uint32_t units = K / 32;
    float xr[NV][32];
    bool uv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t u = ll + LPR * j;
        uv[j] = u < units;
#pragma unroll
        for (int i = 0; i < 32; ++i) xr[j][i] = uv[j] ? (float)x[u * 32 + i] : 0.f;
    }
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6), nw = gridDim.x * 4;
    for (uint32_t row = wave * RPW + rr; row < M + rr; row += nw * RPW) {
        const bool ok = row < M;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t u = ll + LPR * j;
            if (!(ok && uv[j])) continue;
            const uint4 *p = (const uint4 *)(E + (size_t)row * K + u * 32);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint4 w = p[v];
                const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc = fmaf(bf16_to_f32((uint16_t)(wv[e] & 0xFFFFu)), xr[j][8 * v + 2 * e], acc);
                    acc = fmaf(bf16_to_f32((uint16_t)(wv[e] >> 16)), xr[j][8 * v + 2 * e + 1], acc);
                }
            }
        }
        acc = group_sum(acc, LPR);
        if (ok && ll == 0) y[row] = acc;
    }
}

// Tied bf16 LM head for hidden = 512 * NU: a row is NU segments of 512
// columns (1 KB); lane l owns the 16-byte piece l of every segment, so each
// load instruction of a wave reads one contiguous kilobyte.  The lane's x
// slice (8 * NU values) stays in registers, and a wave takes R rows per
// step.  Two register sets alternate: the next step's rows are loading
// while the current step computes.  The table is read once per token and
// streams past the caches (non-temporal loads), leaving the Infinity Cache
// to the layer weights and the KV cache.
template <int NU, int R>
__global__ __launch_bounds__(256) void lm_head_bf16_kernel(const uint16_t *__restrict__ E,
                                                           const f16_t *__restrict__ x,
                                                           float *__restrict__ y, uint32_t M) {
    constexpr uint32_t K = 512 * NU;
    const int lane = threadIdx.x & 63;
    float xr[NU][8];
#pragma unroll
    for (int v = 0; v < NU; ++v) {
        const uint4 q = ((const uint4 *)x)[v * 64 + lane];
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xr[v][2 * e] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[e] & 0xFFFFu));
            xr[v][2 * e + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w4[e] >> 16));
        }
    }
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t stride = gridDim.x * 4 * R;
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    typedef v4u Rows[R][NU];
    auto load = [&](uint32_t b, Rows &dst) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = b + r < M ? b + r : M - 1;
            const v4u *p = (const v4u *)(E + (size_t)row * K) + lane;
#pragma unroll
            for (int v = 0; v < NU; ++v) dst[r][v] = __builtin_nontemporal_load(p + v * 64);
        }
    };
    auto consume = [&](const Rows &src, uint32_t b) {
        float rt[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int v = 0; v < NU; ++v) {
                const uint32_t w4[4] = {src[r][v].x, src[r][v].y, src[r][v].z, src[r][v].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc = fmaf(__uint_as_float(w4[e] << 16), xr[v][2 * e], acc);
                    acc = fmaf(__uint_as_float(w4[e] & 0xFFFF0000u), xr[v][2 * e + 1], acc);
                }
            }
            rt[r] = lane63(wave_sum_to_last(acc));
        }
        float t = rt[0];
#pragma unroll
        for (int k = 1; k < R; ++k) t = lane == k ? rt[k] : t;
        if (lane < R && b + (uint32_t)lane < M) y[b + lane] = t;
    };
    uint32_t base = wave * R;
    Rows ra, rb;
    load(base < M ? base : 0u, ra);
    while (base < M) {
        uint32_t nb = base + stride;
        load(nb < M ? nb : base, rb);
        consume(ra, base);
        base = nb;
        if (base >= M) break;
        nb = base + stride;
        load(nb < M ? nb : base, ra);
        consume(rb, base);
        base = nb;
    }
}

// Greedy sampling (argmax: first maximum wins, NaN never wins,
// transformer.zig:3694-3707) from top-2 partials (best, index, runner-up).
// The 1-bit and 4-bit LM heads write one partial per block themselves (the
// qmv kernel's top-2 epilogue), so a decode step needs only the final pass;
// other logits (the tied bf16 head, the prefill) take the first pass below,
// ARGMAX_BLOCKS blocks over strided slices.  The final pass, one block,
// merges n partials, records the token and its top-2 margin, and advances
// the state.
constexpr int ARGMAX_BLOCKS = 256;
typedef NnzTop2 Top2;

__device__ __forceinline__ Top2 block_top2_256(Top2 t, Top2 *sh) {
    sh[threadIdx.x] = t;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) sh[threadIdx.x] = nnz_top2_merge(sh[threadIdx.x], sh[threadIdx.x + s]);
        __syncthreads();
    }
    return sh[0];
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *x, uint32_t n, Top2 *part) {
    __shared__ Top2 sh[256];
    Top2 t{-INFINITY, -INFINITY, 0xFFFFFFFFu};
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += ARGMAX_BLOCKS * 256) {
        const float v = x[i];
        if (v > t.best) { t.second = t.best; t.best = v; t.idx = i; }
        else if (v > t.second) t.second = v;
    }
    const Top2 r = block_top2_256(t, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = r;
}

__global__ __launch_bounds__(256) void argmax_final_advance_kernel(const Top2 *part, uint32_t n,
                                                                   NnzPick pick) {
    __shared__ Top2 sh[256];
    Top2 t{-INFINITY, -INFINITY, 0xFFFFFFFFu};
    for (uint32_t i = threadIdx.x; i < n; i += 256) t = nnz_top2_merge(t, part[i]);
    const Top2 r = block_top2_256(t, sh);
    if (threadIdx.x == 0) nnz_pick_advance(pick, r.idx == 0xFFFFFFFFu ? 0u : r.idx, r.best - r.second);
}

struct Proj {
    void *codes = nullptr, *scales = nullptr, *biases = nullptr;
    uint32_t M = 0, K = 0;
    nnz_qweight w{};
};

struct Layer {
    Proj q, k, v, o, gate, up, down;
    float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    void *kc = nullptr, *vc = nullptr;
};

// The decode steps of one plan as a few captured graphs.  Step i attends
// over first + i keys; the graph serving it sizes the attention grid and the
// O projection's merge for the longest sequence of its bucket (top), so the
// partials of attention chunks past the live length are neither launched
// for nor read.  Buckets are whole attention chunks, at most
// MAX_STEP_GRAPHS graphs per plan.
constexpr uint32_t MAX_STEP_GRAPHS = 8;
struct StepGraphs {
    std::vector<nnz_graph *> g;
    std::vector<uint32_t> top;
    uint32_t first = 0;
    bool empty() const { return g.empty(); }
    nnz_graph *for_seq(uint32_t seq) const {
        size_t b = 0;
        while (b + 1 < g.size() && seq > top[b]) ++b;
        return g[b];
    }
    void destroy() {
        for (nnz_graph *x : g) nnz_graph_destroy(x);
        g.clear();
        top.clear();
    }
};

}  // namespace

struct nnz_model {
    nnz_ctx *ctx = nullptr;
    nnz_model_config c{};
    uint32_t qdim = 0, kvdim = 0, G = 0;
    std::vector<Layer> L;
    void *emb = nullptr, *emb_scales = nullptr, *emb_biases = nullptr;
    Proj lm;
    float *final_norm = nullptr;
    // decode activations
    float *residual = nullptr, *logits = nullptr, *qf = nullptr;
    f16_t *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *h = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;
    uint32_t part_chunks = 0;  // capacity in chunks per query head
    float *rope_inv = nullptr;     // [head_dim/2] RoPE frequencies
    Top2 *top2 = nullptr;          // [NNZ_TOP2_MAX + ARGMAX_BLOCKS] argmax partials
    uint32_t *state = nullptr;
    uint32_t *tokens_out = nullptr;
    float *margins_out = nullptr;
    uint32_t out_cap = 0;
    // token choice of the decode loop: greedy unless sp.temperature != 0
    nnz_sampling_params sp{};
    uint64_t *rng = nullptr;        // xoshiro256 state [4]
    void *sample_ws = nullptr;
    uint32_t n_eos = 0, eos[NNZ_MAX_EOS] = {};
    // prefill activations (allocated on first use, sized for max_prefill_length)
    float *p_res = nullptr, *p_qf = nullptr, *p_part_o = nullptr, *p_part_ml = nullptr;
    size_t p_part_floats = 0;
    f16_t *p_xn = nullptr, *p_q = nullptr, *p_k = nullptr, *p_v = nullptr, *p_att = nullptr,
          *p_h = nullptr;
    uint32_t *p_ids = nullptr;
    std::vector<void *> allocs;
    // streaming decode (decode_begin / steps / read / end)
    StepGraphs steps;
    uint32_t stream_steps_left = 0;
    uint32_t stream_step = 0;       // steps queued so far
};

namespace {

int model_alloc(nnz_model *m, size_t bytes, void **out) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess)
        return nnz_fail(m->ctx, NNZ_ENOMEM, "model: hipMalloc(%zu) failed", bytes);
    m->allocs.push_back(p);
    if (hipMemsetAsync(p, 0, bytes, m->ctx->stream) != hipSuccess)
        return nnz_fail(m->ctx, NNZ_EHIP, "model: memset failed");
    *out = p;
    return NNZ_OK;
}

#define MALLOC(ptr, bytes)                                                   \
    do {                                                                     \
        void *p_;                                                            \
        int rc_ = model_alloc(m, (bytes), &p_);                              \
        if (rc_) return rc_;                                                 \
        (ptr) = (decltype(ptr))p_;                                           \
    } while (0)

bool is_q4(const nnz_model *m) { return m->c.quant_format == NNZ_QUANT_Q4; }

// Q1: bits + f16 scales.  Q4 (MLX affine): nibbles + raw bf16 scales and
// biases (model.zig:962-1026 loadQ4Projection keeps them as BF16).
size_t codes_bytes(const nnz_model *m, size_t n) { return is_q4(m) ? n / 2 : n / 8; }

int alloc_proj(nnz_model *m, Proj &p, uint32_t M, uint32_t K) {
    p.M = M;
    p.K = K;
    const size_t groups = (size_t)M * K / m->c.group_size;
    MALLOC(p.codes, codes_bytes(m, (size_t)M * K));
    MALLOC(p.scales, groups * 2);
    if (is_q4(m)) MALLOC(p.biases, groups * 2);
    p.w.codes = p.codes;
    p.w.scales = p.scales;
    p.w.biases = p.biases;
    p.w.packed_count = M * K;
    p.w.group_size = m->c.group_size;
    p.w.bits = is_q4(m) ? 4 : 1;
    p.w.scale_dtype = is_q4(m) ? NNZ_BF16 : NNZ_F16;
    return NNZ_OK;
}

nnz_qmv_dims dims_of(const nnz_model *m, const Proj &p) { return {p.M, p.K, m->c.group_size}; }

nnz_gqa_dims gqa_dims(const nnz_model *m, uint32_t seq) {
    return {m->c.num_query_heads, m->c.num_kv_heads, m->c.head_dim, seq, m->c.max_context_length,
            m->G};
}

// Rows per wave step and blocks of the tied bf16 LM head (measured).
constexpr int LMH_R = 2;
constexpr uint32_t LMH_BLOCKS = 256;

// Dense bf16 LM head: the pipelined kernel for hidden 2048 / 4096, the
// lane-group kernel otherwise.
int lm_head_bf16_launch(nnz_ctx *ctx, const uint16_t *E, const f16_t *x, float *logits, uint32_t V,
                        uint32_t K) {
    if (K == 2048 || K == 4096) {
        const uint32_t blocks = std::min<uint32_t>(LMH_BLOCKS, ceil_div(V, 4u * LMH_R));
        if (K == 2048) lm_head_bf16_kernel<4, LMH_R><<<blocks, 256, 0, ctx->stream>>>(E, x, logits, V);
        else lm_head_bf16_kernel<8, LMH_R><<<blocks, 256, 0, ctx->stream>>>(E, x, logits, V);
        NNZ_LAUNCHED(ctx);
        return NNZ_OK;
    }
    const uint32_t units = K / 32;
    uint32_t lpr = 1;
    while (lpr < units && lpr < 64) lpr <<= 1;
    int lg = 0;
    while ((1u << lg) < lpr) ++lg;
    const uint32_t nv = ceil_div(units, lpr);
    const uint32_t rows_per_block = 4 * (64 / lpr);
    uint32_t blocks = ceil_div(V, rows_per_block);
    if (blocks > 4096) blocks = 4096;
    if (nv == 1)
        dense_bf16_gemv_kernel<1><<<blocks, 256, 0, ctx->stream>>>(E, x, logits, V, K, lg);
    else if (nv == 2)
        dense_bf16_gemv_kernel<2><<<blocks, 256, 0, ctx->stream>>>(E, x, logits, V, K, lg);
    else
        return nnz_fail(ctx, NNZ_EUNSUPPORTED, "bf16 LM head: hidden %u > 4096", K);
    NNZ_LAUNCHED(ctx);
    return NNZ_OK;
}

int lm_head(nnz_model *m, const f16_t *x, float *logits) {
    if (m->c.lm_head_kind == NNZ_LMHEAD_Q4)
        return nnz_dispatch_q4mv_f16in(m->ctx, &m->lm.w, x, logits, dims_of(m, m->lm));
    if (m->c.lm_head_kind == NNZ_LMHEAD_Q1)
        return nnz_dispatch_qmv_f16in(m->ctx, &m->lm.w, x, logits, dims_of(m, m->lm));
    return lm_head_bf16_launch(m->ctx, (const uint16_t *)m->emb, x, logits, m->c.vocab_size,
                               m->c.hidden_size);
}

#define RC(x)                  \
    do {                       \
        int rc_ = (x);         \
        if (rc_) return rc_;   \
    } while (0)

// One decode step for the token/position held in the device state block:
// per layer 5 launches (norm+QKV, fused attention, O +=, norm+gate/up+SiLU,
// down +=), then norm+LM head.  `max_seq` sizes the attention grid for every
// position this step may be replayed at.
int enqueue_decode_step(nnz_model *m, uint32_t max_seq, bool top2 = false) {
    nnz_ctx *ctx = m->ctx;
    const nnz_model_config &c = m->c;
    const uint32_t H = c.hidden_size;
    if (c.embed_kind == NNZ_EMBED_Q4) {
        // transformer.zig:2646-2668 (Q4 branch): embedding_lookup_q4
        RC(nnz_dispatch_embedding_lookup_q4(ctx, m->state + ST_TOKEN, m->emb, m->emb_scales,
                                            m->emb_biases, m->residual,
                                            {c.vocab_size, H, 1, c.group_size}));
    } else {
        if (c.embed_kind == NNZ_EMBED_Q1)
            embed_state_q1_kernel<<<ceil_div(H, 256), 256, 0, ctx->stream>>>(
                m->state, (const uint8_t *)m->emb, (const uint16_t *)m->emb_scales, m->residual, H,
                c.group_size, c.vocab_size);
        else
            embed_state_bf16_kernel<<<ceil_div(H, 256), 256, 0, ctx->stream>>>(
                m->state, (const uint16_t *)m->emb, m->residual, H, c.vocab_size);
        NNZ_LAUNCHED(ctx);
    }

    for (uint32_t l = 0; l < c.num_layers; ++l) {
        Layer &Ly = m->L[l];
        // transformer.zig:3024-3083 encodeAttnProjFusedNorm: the Q and the K/V
        // dispatches share one normalised input -> one launch here.
        RC(nnz_qmv_norm_qkv_launch(ctx, &Ly.q.w, &Ly.k.w, &Ly.v.w, m->residual, Ly.attn_norm, m->q,
                                   m->k, m->v, m->qdim, m->kvdim, H, c.group_size, c.rms_eps));
        // transformer.zig:3244-3370 encodeAttentionGather: Q/K norm, RoPE, KV
        // append and attention in one launch, then O-proj with residual +=.
        // Up to MERGE chunks of partials, the O-projection merges them itself.
        const uint32_t nch = ceil_div(max_seq, nnz_attn_fused_chunk(max_seq, c.num_kv_heads));
        const bool merge_in_o = nch <= NNZ_O_MERGE_MAX_CHUNKS;
        RC(nnz_attn_fused1_launch(ctx, m->q, m->k, m->v, Ly.q_norm, Ly.k_norm, Ly.kc, Ly.vc, m->att,
                                  m->part_o, m->part_ml, m->state + ST_SEQ, max_seq,
                                  c.num_query_heads, c.num_kv_heads, c.head_dim,
                                  c.max_context_length, c.rms_eps, c.rope_theta, m->rope_inv,
                                  merge_in_o));
        if (merge_in_o)
            RC(nnz_qmv_merge_resadd_launch(ctx, &Ly.o.w, m->part_o, m->part_ml, m->state + ST_SEQ,
                                           max_seq, nch, nnz_attn_fused_chunk(max_seq, c.num_kv_heads),
                                           c.head_dim, m->residual, dims_of(m, Ly.o)));
        else if (is_q4(m))
            RC(nnz_dispatch_q4mv_f16io_resadd(ctx, &Ly.o.w, m->att, m->residual, dims_of(m, Ly.o)));
        else
            RC(nnz_dispatch_qmv_f16io_resadd(ctx, &Ly.o.w, m->att, m->residual, dims_of(m, Ly.o)));
        // transformer.zig:3372-3646 encodeMLPHalf (fused norm + gate/up + SiLU, down += )
        RC(nnz_qmv_norm_pair_silu_launch(ctx, &Ly.gate.w, &Ly.up.w, m->residual, Ly.ffn_norm, m->h,
                                         dims_of(m, Ly.gate), c.rms_eps));
        if (is_q4(m))
            RC(nnz_dispatch_q4mv_f16io_resadd(ctx, &Ly.down.w, m->h, m->residual, dims_of(m, Ly.down)));
        else
            RC(nnz_dispatch_qmv_f16io_resadd(ctx, &Ly.down.w, m->h, m->residual, dims_of(m, Ly.down)));
    }
    // transformer.zig:2730-2785 encodeFinalNormAndLMHead (norm fused into the
    // 1-bit LM head; the tied bf16 head keeps a separate norm)
    if (c.lm_head_kind == NNZ_LMHEAD_Q1 || c.lm_head_kind == NNZ_LMHEAD_Q4)
        return nnz_qmv_norm_f32out_launch(ctx, &m->lm.w, m->residual, m->final_norm, m->logits,
                                          dims_of(m, m->lm), c.rms_eps, top2 ? m->top2 : nullptr);
    RC(nnz_dispatch_rms_norm(ctx, m->residual, m->final_norm, m->xn, NNZ_F16, 0,
                             {H, 1, c.rms_eps}));
    return lm_head(m, m->xn, m->logits);
}

NnzPick pick_of(const nnz_model *m) {
    NnzPick p;
    p.state = m->state;
    p.tokens = m->tokens_out;
    p.values = m->margins_out;
    p.cap = m->out_cap;
    p.n_eos = m->n_eos;
    for (uint32_t i = 0; i < m->n_eos; ++i) p.eos[i] = m->eos[i];
    return p;
}

// Pick the next token from the logits into the state block: argmax or the
// sampler (sampleToken, transformer.zig:3860-3894).  `partials`: the LM head
// has written its per-block top-2 partials (NNZ_TOP2_MAX entries, the ones
// past its block count neutral), so only the final pass runs.
int enqueue_argmax_advance(nnz_model *m, bool partials = false) {
    const NnzPick pick = pick_of(m);
    if (m->sp.temperature != 0.f)
        return nnz_sample_launch(m->ctx, m->logits, m->c.vocab_size, m->sp, m->rng, m->sample_ws,
                                 nullptr, nullptr, &pick);
    Top2 *part = m->top2;
    uint32_t n = NNZ_TOP2_MAX;
    if (!partials) {
        // the first pass writes its own slots, apart from the LM head's
        part = m->top2 + NNZ_TOP2_MAX;
        n = ARGMAX_BLOCKS;
        argmax_partial_kernel<<<ARGMAX_BLOCKS, 256, 0, m->ctx->stream>>>(m->logits, m->c.vocab_size,
                                                                         part);
        NNZ_LAUNCHED(m->ctx);
    }
    argmax_final_advance_kernel<<<1, 256, 0, m->ctx->stream>>>(part, n, pick);
    NNZ_LAUNCHED(m->ctx);
    return NNZ_OK;
}

// Whether the decode step's LM head writes the greedy top-2 partials (the
// 1-bit and 4-bit heads with whole-wave rows, hidden >= 2048; greedy
// decoding).
bool lm_head_top2(const nnz_model *m) {
    return m->sp.temperature == 0.f && m->c.hidden_size >= 2048 &&
           (m->c.lm_head_kind == NNZ_LMHEAD_Q1 || m->c.lm_head_kind == NNZ_LMHEAD_Q4);
}

void decode_plan(const nnz_model *m, uint32_t max_seq, uint32_t *chunk, uint32_t *nch) {
    *chunk = nnz_attn_fused_chunk(max_seq, m->c.num_kv_heads);
    *nch = ceil_div(max_seq, *chunk);
}

int ensure_prefill_buffers(nnz_model *m, uint32_t n, uint32_t start) {
    const nnz_model_config &c = m->c;
    const uint32_t P = c.max_prefill_length;
    if (!m->p_res) {
        MALLOC(m->p_res, (size_t)P * c.hidden_size * 4);
        MALLOC(m->p_xn, (size_t)P * c.hidden_size * 2);
        MALLOC(m->p_q, (size_t)P * m->qdim * 2);
        MALLOC(m->p_k, (size_t)P * m->kvdim * 2);
        MALLOC(m->p_v, (size_t)P * m->kvdim * 2);
        MALLOC(m->p_att, (size_t)P * m->qdim * 2);
        MALLOC(m->p_h, (size_t)P * c.intermediate_size * 2);
        MALLOC(m->p_qf, (size_t)P * m->qdim * 4);
        MALLOC(m->p_ids, (size_t)P * 4);
    }
    const uint32_t nch = ceil_div(start + n, 512);
    const size_t need = (size_t)n * c.num_query_heads * nch * (c.head_dim + 2) + 64;
    if (need > m->p_part_floats) {
        float *p;
        MALLOC(p, need * 4);
        m->p_part_o = p;
        m->p_part_ml = p + (size_t)n * c.num_query_heads * nch * c.head_dim;
        m->p_part_floats = need;
    }
    return NNZ_OK;
}

}  // namespace

extern "C" {

int nnz_dispatch_lm_head_bf16(nnz_ctx *ctx, const void *table, const void *x, float *logits,
                              uint32_t vocab, uint32_t hidden) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, table && x && logits, NNZ_EINVAL, "lm_head_bf16: null buffer");
    NNZ_REQUIRE(ctx, vocab > 0 && hidden > 0 && hidden % 32 == 0, NNZ_EINVAL,
                "lm_head_bf16: vocab > 0 and hidden a multiple of 32 required");
    NNZ_REQUIRE(ctx, ((uintptr_t)table & 15) == 0 && ((uintptr_t)x & 15) == 0, NNZ_EINVAL,
                "lm_head_bf16: table and x must be 16-byte aligned");
    return lm_head_bf16_launch(ctx, (const uint16_t *)table, (const f16_t *)x, logits, vocab, hidden);
}

int nnz_model_create(nnz_ctx *ctx, const nnz_model_config *cfg, nnz_model **out) {
    NNZ_CHECK_CTX(ctx);
    NNZ_REQUIRE(ctx, cfg && out, NNZ_EINVAL, "model_create: null argument");
    NNZ_REQUIRE(ctx, !ctx->capturing, NNZ_ESTATE, "model_create: not allowed during capture");
    const nnz_model_config &c = *cfg;
    NNZ_REQUIRE(ctx, c.vocab_size && c.hidden_size && c.intermediate_size && c.num_layers &&
                         c.num_query_heads && c.num_kv_heads && c.head_dim && c.max_context_length &&
                         c.max_prefill_length && c.group_size,
                NNZ_EINVAL, "model_create: zero field in config");
    NNZ_REQUIRE(ctx, c.num_query_heads % c.num_kv_heads == 0, NNZ_EINVAL,
                "model_create: query heads not a multiple of KV heads");
    NNZ_REQUIRE(ctx, c.max_prefill_length <= c.max_context_length, NNZ_EINVAL,
                "model_create: max_prefill_length > max_context_length");
    NNZ_REQUIRE(ctx, c.hidden_size % 64 == 0 && c.intermediate_size % 64 == 0 &&
                         (c.num_query_heads * c.head_dim) % 64 == 0 &&
                         (c.num_kv_heads * c.head_dim) % 64 == 0 && c.group_size % 64 == 0 &&
                         c.hidden_size % c.group_size == 0 &&
                         c.intermediate_size % c.group_size == 0 &&
                         (c.num_query_heads * c.head_dim) % c.group_size == 0,
                NNZ_EUNSUPPORTED, "model_create: dims must be multiples of 64 and of group_size");
    NNZ_REQUIRE(ctx, c.max_context_length % 8 == 0, NNZ_EUNSUPPORTED,
                "model_create: max_context_length must be a multiple of 8");
    NNZ_REQUIRE(ctx, (uint64_t)c.vocab_size * c.hidden_size < (1ull << 32), NNZ_EUNSUPPORTED,
                "model_create: vocab*hidden must fit in 32 bits");
    if (c.quant_format == NNZ_QUANT_Q4)
        NNZ_REQUIRE(ctx, c.embed_kind == NNZ_EMBED_Q4 && c.lm_head_kind == NNZ_LMHEAD_Q4, NNZ_EINVAL,
                    "model_create: Q4 models take NNZ_EMBED_Q4 and NNZ_LMHEAD_Q4");
    else
        NNZ_REQUIRE(ctx, c.quant_format == NNZ_QUANT_Q1 && c.embed_kind <= NNZ_EMBED_BF16 &&
                             c.lm_head_kind <= NNZ_LMHEAD_TIED_BF16 &&
                             !(c.lm_head_kind == NNZ_LMHEAD_TIED_BF16 && c.embed_kind != NNZ_EMBED_BF16),
                    NNZ_EINVAL, "model_create: bad quant format or embed/lm_head kind");

    nnz_model *m = new nnz_model();
    m->ctx = ctx;
    m->c = c;
    m->qdim = c.num_query_heads * c.head_dim;
    m->kvdim = c.num_kv_heads * c.head_dim;
    m->G = c.num_query_heads / c.num_kv_heads;
    auto fail = [&](int rc) {
        nnz_model_destroy(m);
        return rc;
    };
    auto body = [&]() -> int {
        const size_t VH = (size_t)c.vocab_size * c.hidden_size;
        if (c.embed_kind == NNZ_EMBED_Q1 || c.embed_kind == NNZ_EMBED_Q4) {
            MALLOC(m->emb, codes_bytes(m, VH) + 4);
            MALLOC(m->emb_scales, ceil_div((uint32_t)VH, c.group_size) * 2);
            if (c.embed_kind == NNZ_EMBED_Q4) MALLOC(m->emb_biases, ceil_div((uint32_t)VH, c.group_size) * 2);
        } else {
            MALLOC(m->emb, VH * 2);
        }
        if (c.lm_head_kind == NNZ_LMHEAD_Q1 || c.lm_head_kind == NNZ_LMHEAD_Q4)
            RC(alloc_proj(m, m->lm, c.vocab_size, c.hidden_size));
        MALLOC(m->final_norm, c.hidden_size * 4);
        m->L.resize(c.num_layers);
        const size_t kv_bytes = (size_t)c.num_kv_heads * c.max_context_length * c.head_dim * 2;
        for (auto &Ly : m->L) {
            RC(alloc_proj(m, Ly.q, m->qdim, c.hidden_size));
            RC(alloc_proj(m, Ly.k, m->kvdim, c.hidden_size));
            RC(alloc_proj(m, Ly.v, m->kvdim, c.hidden_size));
            RC(alloc_proj(m, Ly.o, c.hidden_size, m->qdim));
            RC(alloc_proj(m, Ly.gate, c.intermediate_size, c.hidden_size));
            RC(alloc_proj(m, Ly.up, c.intermediate_size, c.hidden_size));
            RC(alloc_proj(m, Ly.down, c.hidden_size, c.intermediate_size));
            MALLOC(Ly.attn_norm, c.hidden_size * 4);
            MALLOC(Ly.ffn_norm, c.hidden_size * 4);
            MALLOC(Ly.q_norm, c.head_dim * 4);
            MALLOC(Ly.k_norm, c.head_dim * 4);
            MALLOC(Ly.kc, kv_bytes);
            MALLOC(Ly.vc, kv_bytes);
        }
        MALLOC(m->residual, c.hidden_size * 4);
        MALLOC(m->logits, (size_t)c.vocab_size * 4);
        MALLOC(m->qf, m->qdim * 4);
        MALLOC(m->xn, c.hidden_size * 2);
        MALLOC(m->q, m->qdim * 2);
        MALLOC(m->k, m->kvdim * 2);
        MALLOC(m->v, m->kvdim * 2);
        MALLOC(m->att, m->qdim * 2);
        MALLOC(m->h, c.intermediate_size * 2);
        // Worst-case attention partials: chunk >= 64 tokens at any length.
        m->part_chunks = ceil_div(c.max_context_length, 64);
        float *parts;
        MALLOC(parts, (size_t)c.num_query_heads * m->part_chunks * (c.head_dim + 2) * 4);
        m->part_o = parts;
        m->part_ml = parts + (size_t)c.num_query_heads * m->part_chunks * c.head_dim;
        // the LM head's partials (neutral past its block count: they are
        // never written), then the first argmax pass's ARGMAX_BLOCKS
        MALLOC(m->top2, ((size_t)NNZ_TOP2_MAX + ARGMAX_BLOCKS) * sizeof(Top2));
        {
            std::vector<Top2> neutral(NNZ_TOP2_MAX + ARGMAX_BLOCKS, Top2{-INFINITY, -INFINITY, 0xFFFFFFFFu});
            NNZ_HIP(ctx, hipMemcpy(m->top2, neutral.data(), neutral.size() * sizeof(Top2),
                                   hipMemcpyHostToDevice));
        }
        MALLOC(m->state, 64);
        MALLOC(m->rng, 32);
        MALLOC(m->sample_ws, nnz_sample_ws_bytes(c.vocab_size));
        MALLOC(m->rope_inv, (size_t)c.head_dim / 2 * 4);
        RC(nnz_rope_table_launch(ctx, m->rope_inv, c.head_dim, c.rope_theta));
        m->out_cap = c.max_context_length + 1;
        MALLOC(m->tokens_out, (size_t)m->out_cap * 4);
        MALLOC(m->margins_out, (size_t)m->out_cap * 4);
        NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return NNZ_OK;
    };
    int rc = body();
    if (rc) return fail(rc);
    *out = m;
    return NNZ_OK;
}

int nnz_model_destroy(nnz_model *m) {
    if (!m) return NNZ_EINVAL;
    hipStreamSynchronize(m->ctx->stream);
    m->steps.destroy();
    for (void *p : m->allocs) hipFree(p);
    delete m;
    return NNZ_OK;
}

int nnz_model_tensor(nnz_model *m, int id, uint32_t layer, void **ptr, size_t *bytes) {
    if (!m || !ptr || !bytes) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    const nnz_model_config &c = m->c;
    const size_t VH = (size_t)c.vocab_size * c.hidden_size;
    auto set = [&](void *p, size_t b) {
        *ptr = p;
        *bytes = b;
        return p ? NNZ_OK : nnz_fail(ctx, NNZ_ESTATE, "tensor %d not present in this config", id);
    };
    const bool per_layer = (id >= 10 && id < 40) || (id >= NNZ_T_Q_BIASES && id <= NNZ_T_DOWN_BIASES);
    if (!per_layer) {
        const bool qemb = c.embed_kind == NNZ_EMBED_Q1 || c.embed_kind == NNZ_EMBED_Q4;
        switch (id) {
        case NNZ_T_EMBED_CODES:
            return set(m->emb, qemb ? codes_bytes(m, VH) : VH * 2);
        case NNZ_T_EMBED_SCALES:
            return set(m->emb_scales, qemb ? ceil_div((uint32_t)VH, c.group_size) * 2 : 0);
        case NNZ_T_EMBED_BIASES:
            return set(m->emb_biases, ceil_div((uint32_t)VH, c.group_size) * 2);
        case NNZ_T_LM_CODES: return set(m->lm.codes, codes_bytes(m, VH));
        case NNZ_T_LM_SCALES: return set(m->lm.scales, VH / c.group_size * 2);
        case NNZ_T_LM_BIASES: return set(m->lm.biases, VH / c.group_size * 2);
        case NNZ_T_FINAL_NORM: return set(m->final_norm, c.hidden_size * 4);
        case NNZ_T_LOGITS: return set(m->logits, (size_t)c.vocab_size * 4);
        case NNZ_T_RESIDUAL: return set(m->residual, c.hidden_size * 4);
        default: return nnz_fail(ctx, NNZ_EINVAL, "unknown tensor id %d", id);
        }
    }
    NNZ_REQUIRE(ctx, layer < c.num_layers, NNZ_EINVAL, "layer %u out of range", layer);
    Layer &Ly = m->L[layer];
    const size_t kv_bytes = (size_t)c.num_kv_heads * c.max_context_length * c.head_dim * 2;
    auto codes = [&](Proj &p) { return set(p.codes, codes_bytes(m, (size_t)p.M * p.K)); };
    auto scales = [&](Proj &p) { return set(p.scales, (size_t)p.M * p.K / c.group_size * 2); };
    auto biases = [&](Proj &p) { return set(p.biases, (size_t)p.M * p.K / c.group_size * 2); };
    switch (id) {
    case NNZ_T_Q_CODES: return codes(Ly.q);
    case NNZ_T_Q_SCALES: return scales(Ly.q);
    case NNZ_T_K_CODES: return codes(Ly.k);
    case NNZ_T_K_SCALES: return scales(Ly.k);
    case NNZ_T_V_CODES: return codes(Ly.v);
    case NNZ_T_V_SCALES: return scales(Ly.v);
    case NNZ_T_O_CODES: return codes(Ly.o);
    case NNZ_T_O_SCALES: return scales(Ly.o);
    case NNZ_T_GATE_CODES: return codes(Ly.gate);
    case NNZ_T_GATE_SCALES: return scales(Ly.gate);
    case NNZ_T_UP_CODES: return codes(Ly.up);
    case NNZ_T_UP_SCALES: return scales(Ly.up);
    case NNZ_T_DOWN_CODES: return codes(Ly.down);
    case NNZ_T_DOWN_SCALES: return scales(Ly.down);
    case NNZ_T_Q_BIASES: return biases(Ly.q);
    case NNZ_T_K_BIASES: return biases(Ly.k);
    case NNZ_T_V_BIASES: return biases(Ly.v);
    case NNZ_T_O_BIASES: return biases(Ly.o);
    case NNZ_T_GATE_BIASES: return biases(Ly.gate);
    case NNZ_T_UP_BIASES: return biases(Ly.up);
    case NNZ_T_DOWN_BIASES: return biases(Ly.down);
    case NNZ_T_ATTN_NORM: return set(Ly.attn_norm, c.hidden_size * 4);
    case NNZ_T_FFN_NORM: return set(Ly.ffn_norm, c.hidden_size * 4);
    case NNZ_T_Q_NORM: return set(Ly.q_norm, c.head_dim * 4);
    case NNZ_T_K_NORM: return set(Ly.k_norm, c.head_dim * 4);
    case NNZ_T_K_CACHE: return set(Ly.kc, kv_bytes);
    case NNZ_T_V_CACHE: return set(Ly.vc, kv_bytes);
    default: return nnz_fail(ctx, NNZ_EINVAL, "unknown tensor id %d", id);
    }
}

int nnz_model_forward_decode(nnz_model *m, uint32_t token_id, uint32_t position) {
    if (!m) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    NNZ_REQUIRE(ctx, position < m->c.max_context_length, NNZ_EINVAL,
                "forward_decode: position %u >= max_context_length", position);
    NNZ_REQUIRE(ctx, token_id < m->c.vocab_size, NNZ_EINVAL, "forward_decode: token id out of range");
    NNZ_REQUIRE(ctx, !ctx->capturing, NNZ_ESTATE, "forward_decode: use generate() for graphs");
    NNZ_REQUIRE(ctx, m->steps.empty(), NNZ_ESTATE,
                "forward_decode: a decode stream is active (call decode_end first)");
    const uint32_t st[ST_WORDS] = {token_id, position, position + 1, 0, 0};
    NNZ_HIP(ctx, hipMemcpyAsync(m->state, st, sizeof(st), hipMemcpyHostToDevice, ctx->stream));
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return enqueue_decode_step(m, position + 1);
}

int nnz_model_prefill(nnz_model *m, const uint32_t *tokens_host, uint32_t n, uint32_t start) {
    if (!m) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    const nnz_model_config &c = m->c;
    NNZ_REQUIRE(ctx, tokens_host && n > 0 && n <= c.max_prefill_length, NNZ_EINVAL,
                "prefill: need 1 <= n <= max_prefill_length");
    NNZ_REQUIRE(ctx, (uint64_t)start + n <= c.max_context_length, NNZ_EINVAL,
                "prefill: positions exceed max_context_length");
    NNZ_REQUIRE(ctx, !ctx->capturing, NNZ_ESTATE, "prefill: not capturable");
    // A captured decode stream replays an attention plan sized for its own
    // sequence; rewriting the KV cache or the state block under it would
    // make its later steps silently wrong.
    NNZ_REQUIRE(ctx, m->steps.empty(), NNZ_ESTATE,
                "prefill: a decode stream is active (call decode_end first)");
    for (uint32_t i = 0; i < n; ++i)
        NNZ_REQUIRE(ctx, tokens_host[i] < c.vocab_size, NNZ_EINVAL, "prefill: token id out of range");
    RC(ensure_prefill_buffers(m, n, start));
    NNZ_HIP(ctx, hipMemcpyAsync(m->p_ids, tokens_host, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    const uint32_t H = c.hidden_size;
    // q4_mlx models take the Q4 rounding points (transformer.zig:2646, :2977,
    // :3100): BF16-truncated embedding rows and norm outputs; the 4-bit GEMMs
    // truncate their results like the Q4 decode kernels.
    const int tr = is_q4(m) ? 1 : 0;
    if (c.embed_kind == NNZ_EMBED_Q4) {
        RC(nnz_dispatch_embedding_lookup_q4(ctx, m->p_ids, m->emb, m->emb_scales, m->emb_biases,
                                            m->p_res, {c.vocab_size, H, n, c.group_size}));
    } else {
        if (c.embed_kind == NNZ_EMBED_Q1)
            embed_ids_q1_kernel<<<ceil_div(n * H, 256), 256, 0, ctx->stream>>>(
                m->p_ids, (const uint8_t *)m->emb, (const uint16_t *)m->emb_scales, m->p_res, H, n,
                c.group_size, c.vocab_size);
        else
            embed_ids_bf16_kernel<<<ceil_div(n * H, 256), 256, 0, ctx->stream>>>(
                m->p_ids, (const uint16_t *)m->emb, m->p_res, H, n, c.vocab_size);
        NNZ_LAUNCHED(ctx);
    }
    const uint32_t nch = ceil_div(start + n, 512);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        Layer &Ly = m->L[l];
        RC(nnz_dispatch_rms_norm(ctx, m->p_res, Ly.attn_norm, m->p_xn, NNZ_F16, tr, {H, n, c.rms_eps}));
        if (is_q4(m)) {
            RC(nnz_gemm_launch(ctx, &Ly.q.w, nullptr, m->p_xn, n, m->p_q, NNZ_GEMM_STORE_F16, dims_of(m, Ly.q)));
            RC(nnz_gemm_launch(ctx, &Ly.k.w, nullptr, m->p_xn, n, m->p_k, NNZ_GEMM_STORE_F16, dims_of(m, Ly.k)));
            RC(nnz_gemm_launch(ctx, &Ly.v.w, nullptr, m->p_xn, n, m->p_v, NNZ_GEMM_STORE_F16, dims_of(m, Ly.v)));
        } else {   // Q, K and V in one launch (row segments of one grid)
            const nnz_qweight *ws[3] = {&Ly.q.w, &Ly.k.w, &Ly.v.w};
            void *outs[3] = {m->p_q, m->p_k, m->p_v};
            RC(nnz_gemm_segments_launch(ctx, ws, outs, 3, m->p_xn, n, H, c.group_size));
        }
        const bool mfma_attn = nnz_attn_prefill_supported(c.head_dim, c.num_query_heads,
                                                          c.num_kv_heads, c.max_context_length);
        RC(nnz_attn_prep_waves_launch(ctx, m->p_q, m->p_k, m->p_v, Ly.q_norm, Ly.k_norm, m->p_qf,
                                      Ly.kc, Ly.vc, m->rope_inv, c.num_query_heads, c.num_kv_heads,
                                      c.head_dim, start, n, c.max_context_length, c.rms_eps,
                                      mfma_attn ? nnz_attn_prefill_qscale(c.head_dim) : 0.f));
        if (mfma_attn) {
            RC(nnz_attn_prefill_launch(ctx, m->p_qf, Ly.kc, Ly.vc, m->p_att, start, n,
                                       c.num_query_heads, c.num_kv_heads, c.head_dim,
                                       c.max_context_length));
        } else {
        NnzAttnCall ac{};
        ac.q = m->p_qf;
        ac.qdt = NNZ_F32;
        ac.kc = Ly.kc;
        ac.vc = Ly.vc;
        ac.kvdt = NNZ_F16;
        ac.vt = true;
        ac.out = m->p_att;
        ac.odt = NNZ_F16;
        ac.part_o = m->p_part_o;
        ac.part_ml = m->p_part_ml;
        ac.chunk = 512;
        ac.nchunks = nch;
        ac.nq = n;
        ac.dims = gqa_dims(m, start + 1);
        RC(nnz_attn_launch_ex(ctx, ac));
        }
        RC(nnz_gemm_launch(ctx, &Ly.o.w, nullptr, m->p_att, n, m->p_res, NNZ_GEMM_RESADD, dims_of(m, Ly.o)));
        RC(nnz_dispatch_rms_norm(ctx, m->p_res, Ly.ffn_norm, m->p_xn, NNZ_F16, tr, {H, n, c.rms_eps}));
        RC(nnz_gemm_launch(ctx, &Ly.gate.w, &Ly.up.w, m->p_xn, n, m->p_h, NNZ_GEMM_SILU_PAIR,
                           dims_of(m, Ly.gate)));
        RC(nnz_gemm_launch(ctx, &Ly.down.w, nullptr, m->p_h, n, m->p_res, NNZ_GEMM_RESADD,
                           dims_of(m, Ly.down)));
    }
    RC(nnz_dispatch_rms_norm(ctx, m->p_res + (size_t)(n - 1) * H, m->final_norm, m->xn, NNZ_F16, tr,
                             {H, 1, c.rms_eps}));
    NNZ_HIP(ctx, hipMemcpyAsync(m->residual, m->p_res + (size_t)(n - 1) * H, (size_t)H * 4,
                                hipMemcpyDeviceToDevice, ctx->stream));
    return lm_head(m, m->xn, m->logits);
}

}  // extern "C"

namespace {

// Prefill the prompt (in max_prefill_length batches), take the greedy first
// token into the state block; *max_seq = longest sequence of the plan.
int begin_decode(nnz_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                 uint32_t *max_seq) {
    nnz_ctx *ctx = m->ctx;
    const nnz_model_config &c = m->c;
    NNZ_REQUIRE(ctx, prompt && n_prompt > 0 && max_new > 0, NNZ_EINVAL, "decode: bad arguments");
    NNZ_REQUIRE(ctx, (uint64_t)n_prompt + max_new <= c.max_context_length, NNZ_EINVAL,
                "decode: prompt + new tokens exceed max_context_length");
    NNZ_REQUIRE(ctx, max_new + 1 <= m->out_cap, NNZ_EINVAL, "decode: too many tokens");
    for (uint32_t s = 0; s < n_prompt; s += c.max_prefill_length) {
        const uint32_t n = n_prompt - s < c.max_prefill_length ? n_prompt - s : c.max_prefill_length;
        RC(nnz_model_prefill(m, prompt + s, n, s));
    }
    // state = (-, n_prompt - 1, n_prompt, 0, 0); the advance kernel stores t0
    // and moves to (t0, n_prompt, n_prompt + 1, 1, 0).
    const uint32_t st[ST_WORDS] = {0, n_prompt - 1, n_prompt, 0, 0};
    NNZ_HIP(ctx, hipMemcpyAsync(m->state, st, sizeof(st), hipMemcpyHostToDevice, ctx->stream));
    if (m->sp.temperature != 0.f) {  // generate: DefaultPrng.init(params.seed)
        uint64_t rs[4];
        nnz_rng_seed_words(m->sp.seed, rs);
        NNZ_HIP(ctx, hipMemcpyAsync(m->rng, rs, sizeof(rs), hipMemcpyHostToDevice, ctx->stream));
    }
    // st and rs live on this stack frame: wait for the uploads before
    // returning (as forward_decode does) rather than rely on the runtime
    // staging pageable copies.
    NNZ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    RC(enqueue_argmax_advance(m));
    *max_seq = n_prompt + max_new;
    uint32_t chunk, nch;
    decode_plan(m, *max_seq, &chunk, &nch);
    NNZ_REQUIRE(ctx, nch <= m->part_chunks, NNZ_EINVAL, "decode: attention plan exceeds scratch");
    return NNZ_OK;
}

// One decode step: forwardDecode of the state's token, then the token pick
// and state advance.  Graph-capturable (no host data, no allocation).
int pick_step(nnz_model *m, uint32_t max_seq) {
    const bool t2 = lm_head_top2(m);
    RC(enqueue_decode_step(m, max_seq, t2));
    return enqueue_argmax_advance(m, t2);
}

int capture_step(nnz_model *m, uint32_t max_seq, nnz_graph **g) {
    RC(nnz_graph_begin(m->ctx));
    const int brc = pick_step(m, max_seq);
    const int erc = nnz_graph_end(m->ctx, g);
    return brc ? brc : erc;
}

// The step graphs of a plan whose steps attend over first .. last keys: one
// per run of `per` attention-chunk counts, `per` the smallest that keeps the
// plan within MAX_STEP_GRAPHS graphs.
int capture_steps(nnz_model *m, uint32_t first, uint32_t last, StepGraphs &s) {
    const uint32_t chunk = nnz_attn_fused_chunk(last, m->c.num_kv_heads);
    const uint32_t c0 = ceil_div(first, chunk), c1 = ceil_div(last, chunk);
    const uint32_t per = ceil_div(c1 - c0 + 1, MAX_STEP_GRAPHS);
    s.first = first;
    for (uint32_t c = c0; c <= c1; c += per) {
        const uint32_t top = std::min(last, (c + per - 1) * chunk);
        nnz_graph *g = nullptr;
        const int rc = capture_step(m, top, &g);
        if (rc) {
            s.destroy();
            return rc;
        }
        s.g.push_back(g);
        s.top.push_back(top);
    }
    return NNZ_OK;
}

}  // namespace

extern "C" {

int nnz_model_generate(nnz_model *m, const uint32_t *prompt, uint32_t n_prompt, uint32_t n_new,
                       uint32_t *out_tokens, float *out_margins, float *out_step_ms, int use_graph,
                       uint32_t *out_count) {
    if (!m) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    NNZ_REQUIRE(ctx, out_tokens, NNZ_EINVAL, "generate: null output");
    NNZ_REQUIRE(ctx, m->steps.empty(), NNZ_ESTATE,
                "generate: a decode stream is active (call decode_end first)");
    uint32_t max_seq;
    RC(begin_decode(m, prompt, n_prompt, n_new, &max_seq));
    std::vector<hipEvent_t> ev;
    int rc = NNZ_OK;
    if (out_step_ms) {
        ev.resize(n_new + 1);
        for (auto &e : ev)
            if (!rc && hipEventCreate(&e) != hipSuccess) rc = NNZ_EHIP;
    }
    // The reference decodes every emitted token (transformer.zig:3982-4016):
    // n_new forward passes for n_new output tokens.  With stop tokens the
    // host looks at the state block every POLL steps and stops queueing
    // once the stream has ended.
    constexpr uint32_t POLL = 8;
    StepGraphs sg;
    if (!rc && use_graph) rc = capture_steps(m, n_prompt + 1, max_seq, sg);
    if (!rc && out_step_ms && hipEventRecord(ev[0], ctx->stream) != hipSuccess) rc = NNZ_EHIP;
    uint32_t done_steps = 0;
    for (uint32_t i = 0; i < n_new && !rc; ++i) {
        if (m->n_eos && i % POLL == 0) {
            uint32_t st[ST_WORDS];
            rc = nnz_stream_sync(ctx, 600000);
            if (!rc && hipMemcpy(st, m->state, sizeof(st), hipMemcpyDeviceToHost) != hipSuccess)
                rc = NNZ_EHIP;
            if (rc || st[ST_DONE]) break;
        }
        // step i attends over n_prompt + 1 + i keys (fewer once a stop token ended the stream)
        rc = use_graph ? nnz_graph_replay(ctx, sg.for_seq(n_prompt + 1 + i)) : pick_step(m, n_prompt + 1 + i);
        if (!rc && out_step_ms && hipEventRecord(ev[i + 1], ctx->stream) != hipSuccess) rc = NNZ_EHIP;
        done_steps = i + 1;
    }
    if (!rc) rc = nnz_stream_sync(ctx, 600000);
    if (!rc && out_step_ms)
        for (uint32_t i = 0; i < n_new; ++i)
            if (i < done_steps) hipEventElapsedTime(&out_step_ms[i], ev[i], ev[i + 1]);
            else out_step_ms[i] = 0.f;
    for (auto &e : ev)
        if (e) hipEventDestroy(e);
    sg.destroy();
    if (rc) return rc;
    uint32_t emitted;
    int stopped;
    RC(nnz_model_decode_status(m, &emitted, &stopped));
    if (emitted > n_new) emitted = n_new;
    if (out_count) *out_count = emitted;
    return nnz_model_decode_read(m, emitted, out_tokens, out_margins);
}

int nnz_model_set_sampling(nnz_model *m, const nnz_sampling_params *p) {
    if (!m) return NNZ_EINVAL;
    NNZ_REQUIRE(m->ctx, p, NNZ_EINVAL, "set_sampling: null params");
    NNZ_REQUIRE(m->ctx, p->temperature >= 0.f && p->temperature <= 3.0e38f, NNZ_EINVAL,
                "set_sampling: temperature must be >= 0");
    NNZ_REQUIRE(m->ctx, p->top_p > 0.f, NNZ_EINVAL,
                "set_sampling: top_p must be > 0 (>= 1 disables it)");
    NNZ_REQUIRE(m->ctx, m->steps.empty(), NNZ_ESTATE, "set_sampling: a decode stream is active");
    m->sp = *p;
    return NNZ_OK;
}

int nnz_model_set_eos(nnz_model *m, const uint32_t *ids, uint32_t n) {
    if (!m) return NNZ_EINVAL;
    NNZ_REQUIRE(m->ctx, n <= NNZ_MAX_EOS && (n == 0 || ids), NNZ_EINVAL,
                "set_eos: at most %u stop tokens", NNZ_MAX_EOS);
    NNZ_REQUIRE(m->ctx, m->steps.empty(), NNZ_ESTATE, "set_eos: a decode stream is active");
    m->n_eos = n;
    for (uint32_t i = 0; i < n; ++i) m->eos[i] = ids[i];
    return NNZ_OK;
}

int nnz_model_decode_status(nnz_model *m, uint32_t *emitted, int *stopped) {
    if (!m) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    RC(nnz_stream_sync(ctx, 600000));
    uint32_t st[ST_WORDS];
    NNZ_HIP(ctx, hipMemcpy(st, m->state, sizeof(st), hipMemcpyDeviceToHost));
    if (emitted) *emitted = st[ST_STEP];
    if (stopped) *stopped = (int)st[ST_DONE];
    return NNZ_OK;
}

int nnz_model_decode_begin(nnz_model *m, const uint32_t *prompt, uint32_t n_prompt,
                           uint32_t max_new) {
    if (!m) return NNZ_EINVAL;
    NNZ_REQUIRE(m->ctx, m->steps.empty(), NNZ_ESTATE, "decode_begin: a decode stream is active");
    uint32_t max_seq;
    RC(begin_decode(m, prompt, n_prompt, max_new, &max_seq));
    RC(capture_steps(m, n_prompt + 1, max_seq, m->steps));
    m->stream_steps_left = max_new;
    m->stream_step = 0;
    return NNZ_OK;
}

int nnz_model_decode_steps(nnz_model *m, uint32_t n) {
    if (!m) return NNZ_EINVAL;
    NNZ_REQUIRE(m->ctx, !m->steps.empty(), NNZ_ESTATE, "decode_steps: call decode_begin first");
    NNZ_REQUIRE(m->ctx, n <= m->stream_steps_left, NNZ_EINVAL,
                "decode_steps: %u steps requested, %u left in the plan", n, m->stream_steps_left);
    for (uint32_t i = 0; i < n; ++i) {
        RC(nnz_graph_replay(m->ctx, m->steps.for_seq(m->steps.first + m->stream_step)));
        ++m->stream_step;
        --m->stream_steps_left;
    }
    return NNZ_OK;
}

int nnz_model_decode_read(nnz_model *m, uint32_t n, uint32_t *out_tokens, float *out_margins) {
    if (!m) return NNZ_EINVAL;
    nnz_ctx *ctx = m->ctx;
    NNZ_REQUIRE(ctx, out_tokens && n <= m->out_cap, NNZ_EINVAL, "decode_read: bad arguments");
    RC(nnz_stream_sync(ctx, 600000));
    NNZ_HIP(ctx, hipMemcpy(out_tokens, m->tokens_out, (size_t)n * 4, hipMemcpyDeviceToHost));
    if (out_margins)
        NNZ_HIP(ctx, hipMemcpy(out_margins, m->margins_out, (size_t)n * 4, hipMemcpyDeviceToHost));
    return NNZ_OK;
}

int nnz_model_decode_end(nnz_model *m) {
    if (!m) return NNZ_EINVAL;
    if (!m->steps.empty()) {
        RC(nnz_stream_sync(m->ctx, 600000));
        m->steps.destroy();
    }
    m->stream_steps_left = 0;
    m->stream_step = 0;
    return NNZ_OK;
}

}  // extern "C"

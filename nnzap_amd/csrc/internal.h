// Internal (non-exported) entry points shared between the library's sources.
#pragma once

#include "common.h"

// Greedy token choice (transformer.zig:3694-3707: first maximum wins, NaN
// never wins): the best value, its index and the runner-up value of a set
// of logits.  Partials of disjoint index ranges merge in any order.
struct NnzTop2 {
    float best, second;
    uint32_t idx;
};
// Capacity of a model's top-2 partials (one per block of the pass that
// writes them; unwritten entries stay neutral).
constexpr uint32_t NNZ_TOP2_MAX = 2048;

__device__ __forceinline__ NnzTop2 nnz_top2_merge(NnzTop2 a, NnzTop2 b) {
    const bool take_b = (b.best > a.best) || (b.best == a.best && b.idx < a.idx);
    NnzTop2 r;
    r.best = take_b ? b.best : a.best;
    r.idx = take_b ? b.idx : a.idx;
    r.second = fmaxf(fmaxf(a.second, b.second), take_b ? a.best : b.best);
    return r;
}

// One attention launch with full control over chunking and batching.
struct NnzAttnCall {
    const void *q = nullptr;
    int qdt = NNZ_F32;
    uint32_t q_stride = 0;       // elements between queries (0: Hq*D)
    const void *kc = nullptr;
    const void *vc = nullptr;
    int kvdt = NNZ_F16;
    bool vt = true;              // V stored [Hkv][D][max_ctx]
    void *out = nullptr;
    int odt = NNZ_F16;
    uint32_t o_stride = 0;       // elements between outputs (0: Hq*D)
    float *part_o = nullptr;     // [nq][Hq][nchunks][D]
    float *part_ml = nullptr;    // [nq][Hq][nchunks][2]
    const uint32_t *d_seq = nullptr;  // device seq_len of query 0 (overrides dims.seq_len)
    uint32_t chunk = 0, nchunks = 0, nq = 1;
    int32_t rope_pos = -1;
    float rope_theta = 0.f;
    nnz_gqa_dims dims{};
};

uint32_t nnz_attn_chunk(uint32_t seq_len, uint32_t hkv);
uint32_t nnz_attn_fused_chunk(uint32_t max_seq, uint32_t hkv);
int nnz_rope_table_launch(nnz_ctx *ctx, float *out, uint32_t head_dim, float theta);
int nnz_attn_launch_ex(nnz_ctx *ctx, const NnzAttnCall &c);
// Single-query attention with the partials carved out of `scratch`
// (nnz_dispatch_gqa_attention's body).
int nnz_attn_launch(nnz_ctx *ctx, const void *q, int qdt, const void *kc, const void *vc, int kvdt,
                    bool vt, void *out, int odt, void *scratch, size_t scratch_bytes,
                    int32_t rope_pos, float theta, const nnz_gqa_dims &d);
// Fixed partials buffer of nnz_dispatch_gqa_attention_noalloc (noalloc.hip):
// looks up its device address for ctx->device (called by nnz_ctx_create).
constexpr size_t NNZ_NOALLOC_SCRATCH_BYTES = NNZ_GQA_NOALLOC_MAX_BYTES;
int nnz_noalloc_init(nnz_ctx *ctx);
int nnz_attn_prep_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                         const float *qn, const float *kn, float *qout, void *kc, void *vc,
                         uint32_t hq, uint32_t hkv, uint32_t head_dim, uint32_t pos,
                         const uint32_t *d_pos, uint32_t nq, uint32_t max_ctx, float eps,
                         float theta);
int nnz_argmax_launch(nnz_ctx *ctx, const float *x, uint32_t n, uint32_t *oi, float *ov);
int nnz_attn_fused1_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                           const float *qn, const float *kn, void *kc, void *vc, void *out,
                           float *part_o, float *part_ml, const uint32_t *d_seq, uint32_t max_seq,
                           uint32_t hq, uint32_t hkv, uint32_t head_dim, uint32_t max_ctx,
                           float eps, float theta, const float *inv_freq,
                           bool partials_only = false);
int nnz_qmv_norm_qkv_launch(nnz_ctx *ctx, const nnz_qweight *wq, const nnz_qweight *wk,
                            const nnz_qweight *wv, const float *residual, const float *norm_w,
                            void *q, void *k, void *v, uint32_t qrows, uint32_t kvrows, uint32_t K,
                            uint32_t gs, float eps);
int nnz_qmv_norm_pair_silu_launch(nnz_ctx *ctx, const nnz_qweight *wg, const nnz_qweight *wu,
                                  const float *residual, const float *norm_w, void *out,
                                  nnz_qmv_dims d, float eps);
// Largest attention chunk count the merge-in-O-projection path accepts.
constexpr uint32_t NNZ_O_MERGE_MAX_CHUNKS = 16;
int nnz_qmv_merge_resadd_launch(nnz_ctx *ctx, const nnz_qweight *w, const float *part_o,
                                const float *part_ml, const uint32_t *d_seq, uint32_t seq_len,
                                uint32_t nchunks, uint32_t chunk, uint32_t head_dim,
                                float *residual, nnz_qmv_dims d);
// top2: when set, every block also writes the greedy top-2 partial of the
// rows it stored to top2[block] (at most NNZ_TOP2_MAX blocks).
int nnz_qmv_norm_f32out_launch(nnz_ctx *ctx, const nnz_qweight *w, const float *residual,
                               const float *norm_w, float *out, nnz_qmv_dims d, float eps,
                               NnzTop2 *top2 = nullptr);
int nnz_gemm_launch(nnz_ctx *ctx, const nnz_qweight *wa, const nnz_qweight *wb, const void *a,
                    uint32_t P, void *out, int mode, const nnz_qmv_dims &d);

// Decode state block of the model's device-resident loop: {token, position,
// sequence length, emitted count, done}.
enum { NNZ_ST_TOKEN = 0, NNZ_ST_POS = 1, NNZ_ST_SEQ = 2, NNZ_ST_STEP = 3, NNZ_ST_DONE = 4 };
constexpr uint32_t NNZ_MAX_EOS = 8;

// Where a picked token goes: the state block, the emitted-token and
// per-token value arrays (capacity `cap`) and the stop tokens.
struct NnzPick {
    uint32_t *state = nullptr;
    uint32_t *tokens = nullptr;
    float *values = nullptr;
    uint32_t cap = 0;
    uint32_t n_eos = 0;
    uint32_t eos[NNZ_MAX_EOS] = {};
};

// Record token `tok` (one thread): an EOS id ends the stream without being
// emitted, and after that nothing is emitted or advanced (generate,
// transformer.zig:3992, isEosToken :4126).
__device__ __forceinline__ void nnz_pick_advance(const NnzPick &p, uint32_t tok, float value) {
    uint32_t *st = p.state;
    if (st[NNZ_ST_DONE]) return;
    for (uint32_t i = 0; i < p.n_eos; ++i)
        if (tok == p.eos[i]) {
            st[NNZ_ST_DONE] = 1;
            return;
        }
    const uint32_t step = st[NNZ_ST_STEP];
    if (step < p.cap) {
        p.tokens[step] = tok;
        p.values[step] = value;
    }
    st[NNZ_ST_TOKEN] = tok;
    st[NNZ_ST_POS] += 1;
    st[NNZ_ST_SEQ] += 1;
    st[NNZ_ST_STEP] = step + 1;
}

// Device sampling (sample.hip).
void nnz_rng_seed_words(uint64_t seed, uint64_t out[4]);
size_t nnz_sample_ws_bytes(uint32_t n);
int nnz_sample_launch(nnz_ctx *ctx, const float *logits, uint32_t n, const nnz_sampling_params &p,
                      uint64_t *rng, void *ws, uint32_t *out_index, float *out_prob,
                      const NnzPick *pick);

// Causal GQA attention of a prefill batch on MFMA (attn_prefill.hip):
// queries as the prep kernel writes them with qsplit = nnz_attn_prefill_qscale
// (f16 hi/lo rows [n][hq][2][D]), f16 KV cache (V transposed), f16 output
// [n][hq][D].
bool nnz_attn_prefill_supported(uint32_t head_dim, uint32_t hq, uint32_t hkv, uint32_t max_ctx);
float nnz_attn_prefill_qscale(uint32_t head_dim);
int nnz_attn_prefill_launch(nnz_ctx *ctx, const void *q, const void *kc, const void *vc, void *out,
                            uint32_t start, uint32_t n, uint32_t hq, uint32_t hkv,
                            uint32_t head_dim, uint32_t max_ctx);

// Per-head q/k RMSNorm + RoPE and the KV append of a prefill batch, one wave
// per (head, token) (transformer.hip); frequencies from a [head_dim/2] table.
// q out: float32 [nq][hq][D] (qsplit 0), or pre-scaled by qsplit and split
// into f16 hi/lo rows [nq][hq][2][D] (the MFMA prefill attention's operands).
int nnz_attn_prep_waves_launch(nnz_ctx *ctx, const void *q, const void *kr, const void *vr,
                               const float *qn, const float *kn, void *qout, void *kc, void *vc,
                               const float *inv_freq, uint32_t hq, uint32_t hkv, uint32_t head_dim,
                               uint32_t pos0, uint32_t nq, uint32_t max_ctx, float eps,
                               float qsplit = 0.f);

// One prefill GEMM launch over up to three 1-bit matrices that share K and
// the f16 A operand, each written to its own f16 output [P][rows] (gemm.hip).
int nnz_gemm_segments_launch(nnz_ctx *ctx, const nnz_qweight *const *w, void *const *out, int nw,
                             const void *a, uint32_t P, uint32_t K, uint32_t group_size);

// 1-bit QMV on the block-scaled matrix cores (qmv_mfma.hip): K = 2048, group
// size 128.  nmat 2 = a pair sharing the input with the SiLU epilogue.
// xdt / odt: NNZ_F32 / NNZ_F16 / NNZ_BF16; xin 0 = x as given, 1 = RMSNorm
// of the f32 residual `x` with `norm_w` (f16-rounded); epi 0 = store,
// 1 = residual +=, 2 = silu(a) * b.  Stacked launch: stack_count matrices at
// the byte strides cs (codes), ss (scales), xs (inputs), os (outputs).
struct NnzQ1Mfma {
    const void *codes[2] = {nullptr, nullptr};
    const void *scales[2] = {nullptr, nullptr};
    const void *x = nullptr;
    const float *norm_w = nullptr;
    void *out = nullptr;
    uint32_t M = 0, K = 0, group_size = 0, nmat = 1;
    int xdt = NNZ_F32, xin = 0, epi = 0, odt = NNZ_F32;
    float eps = 1e-6f;
    uint32_t stack_count = 1, blocks_per_matrix = 0;
    uint64_t cs = 0, ss = 0, xs = 0, os = 0;
};
bool nnz_q1_mfma_supported(uint32_t K, uint32_t group_size);
bool nnz_q1_mfma_has_variant(const NnzQ1Mfma &c);
int nnz_q1_mfma_launch(nnz_ctx *ctx, const NnzQ1Mfma &c);

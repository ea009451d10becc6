"""Scalar restatement of the CPU references in nnmetal's transformer tests --
TEST INFRASTRUCTURE ONLY (pins the oracle's whole-step composition).

Follows nnmetal/src/transformer_test.zig line by line, one scalar operation
at a time, independently of ``oracle/``:

* cpuRMSNorm :72-103, cpuSiLUElementwiseMul :114-126, cpuRoPE :128-157,
  cpuSoftmax :159-177, cpuAttentionHead :179-227, cpuGQAAttention :229-263,
  cpuEmbeddingDequant :265-297, cpuQMV :299-334;
* cpuForwardBlock :364-388 = cpuForwardBlockAttention :390-423
  (cpuAttentionProjections :428-487, cpuRoPEAndKVCache :490-533,
  cpuProjectQKV :536-577, cpuKVCacheWrite :580-602, cpuAttentionGather
  :605-650) + cpuForwardBlockMLP :653-716;
* the fixtures createTestPackedBuffer :886-923 and populateTestKVCache
  :850-881, and the two composed-path tests "single-block forward matches CPU
  reference" :1697-1997 and "forwardDecode full path matches CPU reference"
  :2086-2489 (TinyBlock config :53-65).

Two arithmetic modes:

* ``ft=np.float32``: the reference's own CPU precision -- every operation
  rounded to float32 in the reference's order, activations unrounded except
  the float16 KV cache;
* ``ft=float`` (float64) with ``r16`` rounding hooks at the GPU path's
  storage points (normalised inputs, q/k/v projections, attention output,
  SiLU*mul, final norm -> float16) and the float32 residual: the same
  composition evaluated with the rounding points of the decode kernels, which
  pins the oracle's op order and rounding points to ~1e-12.

The RoPE frequency follows the reference's ``1 / pow(theta, 2p/d)`` in
float32, or (``rope="build"``) this build's convention: theta^(-2p/d) in
double rounded once to float32, angle = one float32 multiply.
"""
from __future__ import annotations

import math

import numpy as np

F32, F16 = np.float32, np.float16


# ---------------------------------------------------------------------------
# TinyBlock fixtures (transformer_test.zig:53-65, :850-923)
# ---------------------------------------------------------------------------

TINY_BLOCK = dict(vocab_size=32, hidden_size=128, intermediate_size=256, num_layers=1,
                  num_query_heads=2, num_kv_heads=2, head_dim=64, max_context_length=8,
                  max_prefill_length=4, rope_theta=10000.0, group_size=128)


def packed_buffer_fixture(num_weights: int, seed: int, gs: int = 128):
    """createTestPackedBuffer: (packed bytes, f16 scales).  Byte i =
    seed +% (i % 37); scale i = f16(0.1 + (seed % 10) * 0.01 + i * 0.005)
    evaluated in float32."""
    nbytes = num_weights // 8
    raw = bytes(((seed + (i % 37)) & 0xFF) for i in range(nbytes))
    scales = []
    for i in range(num_weights // gs):
        val = F32(F32(0.1) + F32(F32(seed % 10) * F32(0.01))) + F32(F32(i) * F32(0.005))
        scales.append(F16(val))
    return raw, scales


def linear_f32(n: int, base: float, step: float):
    """``base + f32(i) * step`` in float32 (the tests' norm-scale fills)."""
    return [F32(F32(base) + F32(F32(i) * F32(step))) for i in range(n)]


def populate_kv(num_kvh: int, seq_len: int, hd: int, max_ctx: int):
    """populateTestKVCache: K and V [h][t][d] float16 caches (zeros beyond
    seq_len); value seed = h*seq_len*hd + t*hd + d + 1, K = seed*0.05,
    V = seed*0.025 (float32 products narrowed to float16)."""
    n = num_kvh * max_ctx * hd
    k, v = [F16(0)] * n, [F16(0)] * n
    for h in range(num_kvh):
        for t in range(seq_len):
            for d in range(hd):
                idx = h * max_ctx * hd + t * hd + d
                seed = F32(h * seq_len * hd + t * hd + d + 1)
                k[idx] = F16(F32(seed * F32(0.05)))
                v[idx] = F16(F32(seed * F32(0.025)))
    return k, v


# ---------------------------------------------------------------------------
# CPU kernels (transformer_test.zig:67-334)
# ---------------------------------------------------------------------------

class Ref:
    """One arithmetic mode of the reference's CPU functions."""

    def __init__(self, ft=F32, r16=None, rope: str = "reference"):
        self.ft = ft
        self.r16 = r16 or (lambda xs: list(xs))
        self.rope_mode = rope

    def f(self, x):
        return self.ft(x)

    def rmsnorm(self, inp, scale, h: int, ntok: int, eps: float):
        f = self.f
        out = [None] * (h * ntok)
        for t in range(ntok):
            off = t * h
            sum_sq = f(0.0)
            for i in range(h):
                val = f(inp[off + i])
                sum_sq = f(sum_sq + f(val * val))
            rms = f(f(1.0) / f(self._sqrt(f(f(sum_sq / f(h)) + f(eps)))))
            for i in range(h):
                out[off + i] = f(f(f(inp[off + i]) * rms) * f(scale[i]))
        return out

    def _sqrt(self, x):
        return np.sqrt(x) if self.ft is F32 else math.sqrt(x)

    def _exp(self, x):
        return np.exp(x) if self.ft is F32 else math.exp(x)

    def silu_mul(self, gate, up):
        f = self.f
        out = []
        for g, u in zip(gate, up):
            sig = f(f(1.0) / f(f(1.0) + f(self._exp(f(-g)))))
            out.append(f(f(f(g) * sig) * f(u)))
        return out

    def rope(self, data, num_heads: int, head_dim: int, position: int, theta: float):
        f = self.f
        out = list(data)
        half = head_dim // 2
        for h in range(num_heads):
            for p in range(half):
                if self.rope_mode == "reference":
                    exponent = F32(F32(2 * p) / F32(head_dim))
                    theta_i = F32(F32(1.0) / np.power(F32(theta), exponent))
                    angle = F32(F32(position) * theta_i)
                else:
                    inv = F32(2.0 ** (-(2.0 * p / head_dim) * math.log2(theta)))
                    angle = F32(F32(position) * inv)
                if self.ft is F32:
                    c, s = np.cos(angle), np.sin(angle)
                else:
                    c, s = math.cos(float(angle)), math.sin(float(angle))
                base = h * head_dim + 2 * p
                x0, x1 = f(out[base]), f(out[base + 1])
                out[base] = f(f(x0 * c) - f(x1 * s))
                out[base + 1] = f(f(x0 * s) + f(x1 * c))
        return out

    def softmax(self, scores):
        f = self.f
        m = scores[0]
        for s in scores[1:]:
            if s > m:
                m = s
        e = [f(self._exp(f(s - m))) for s in scores]
        tot = f(0.0)
        for x in e:
            tot = f(tot + x)
        return [f(x / tot) for x in e]

    def attention_head(self, q_head, k_cache, v_cache, kv_head: int, hd: int, seq_len: int,
                       max_ctx: int):
        f = self.f
        inv_sqrt_d = f(f(1.0) / f(self._sqrt(f(hd))))
        stride = max_ctx * hd
        scores = []
        for t in range(seq_len):
            dot = f(0.0)
            for d in range(hd):
                kv = f(k_cache[kv_head * stride + t * hd + d])
                dot = f(dot + f(f(q_head[d]) * kv))
            scores.append(f(dot * inv_sqrt_d))
        p = self.softmax(scores)
        out = []
        for d in range(hd):
            acc = f(0.0)
            for t in range(seq_len):
                vv = f(v_cache[kv_head * stride + t * hd + d])
                acc = f(acc + f(p[t] * vv))
            out.append(acc)
        return out

    def gqa(self, q, k_cache, v_cache, nqh: int, hd: int, seq_len: int, max_ctx: int,
            group: int):
        out = []
        for h in range(nqh):
            out += self.attention_head(q[h * hd:(h + 1) * hd], k_cache, v_cache, h // group, hd,
                                       seq_len, max_ctx)
        return out

    def embedding(self, token_ids, packed: bytes, scales, hidden: int, gs: int):
        out = []
        for row in token_ids:
            for d in range(hidden):
                flat = row * hidden + d
                bit = (packed[flat // 8] >> (flat % 8)) & 1
                s = self.f(scales[flat // gs])
                out.append(s if bit == 1 else self.f(-s))
        return out

    def qmv(self, packed: bytes, scales, inp, M: int, K: int, gs: int):
        f = self.f
        out = []
        for row in range(M):
            acc = f(0.0)
            for col in range(K):
                flat = row * K + col
                bit = (packed[flat // 8] >> (flat % 8)) & 1
                s = f(scales[flat // gs])
                w = s if bit == 1 else f(-s)
                acc = f(acc + f(w * f(inp[col])))
            out.append(acc)
        return out

    # -- composed block (transformer_test.zig:364-716) ------------------------
    def _res_add(self, residual, add):
        # the residual buffer is float32 in every mode (model.zig:87-102)
        return [F32(self.f(r) + self.f(a)) for r, a in zip(residual, add)]

    def forward_block(self, cfg, residual, w, k_cache, v_cache, position: int, seq_len: int,
                      eps: float = 1e-6):
        """cpuForwardBlock: returns the new residual; writes the caches."""
        H, HD = cfg["hidden_size"], cfg["head_dim"]
        NQH, NKVH = cfg["num_query_heads"], cfg["num_kv_heads"]
        QD, KVD, I = NQH * HD, NKVH * HD, cfg["intermediate_size"]
        GS, MAXC = cfg["group_size"], cfg["max_context_length"]
        r16 = self.r16
        # cpuAttentionProjections
        norm_out = r16(self.rmsnorm(residual, w["attn_norm"], H, 1, eps))
        q = r16(self.qmv(*w["q"], norm_out, QD, H, GS))
        k = r16(self.qmv(*w["k"], norm_out, KVD, H, GS))
        v = r16(self.qmv(*w["v"], norm_out, KVD, H, GS))
        q = self.rmsnorm(q, w["q_norm"], HD, NQH, eps)
        k = self.rmsnorm(k, w["k_norm"], HD, NKVH, eps)
        # cpuRoPEAndKVCache + cpuKVCacheWrite (f32 -> f16)
        q = self.rope(q, NQH, HD, position, cfg["rope_theta"])
        k = self.rope(k, NKVH, HD, position, cfg["rope_theta"])
        for h in range(NKVH):
            for d in range(HD):
                idx = h * MAXC * HD + position * HD + d
                k_cache[idx] = F16(k[h * HD + d])
                v_cache[idx] = F16(v[h * HD + d])
        # cpuAttentionGather
        attn = r16(self.gqa(q, k_cache, v_cache, NQH, HD, seq_len, MAXC, NQH // NKVH))
        o = self.qmv(*w["o"], attn, H, QD, GS)
        residual = self._res_add(residual, o)
        # cpuForwardBlockMLP
        norm_out = r16(self.rmsnorm(residual, w["ffn_norm"], H, 1, eps))
        gate = self.qmv(*w["gate"], norm_out, I, H, GS)
        up = self.qmv(*w["up"], norm_out, I, H, GS)
        hidden = r16(self.silu_mul(gate, up))
        down = self.qmv(*w["down"], hidden, H, I, GS)
        return self._res_add(residual, down)

    def forward_decode(self, cfg, emb, layers, final_norm, token: int, position: int,
                       k_caches, v_caches, eps: float = 1e-6):
        """The forwardDecode test's CPU path (:2413-2474): embedding lookup,
        the blocks, final RMSNorm, LM head with the (tied) embedding matrix."""
        H, V, GS = cfg["hidden_size"], cfg["vocab_size"], cfg["group_size"]
        res = [F32(x) for x in self.embedding([token], *emb, H, GS)]
        for l, w in enumerate(layers):
            res = self.forward_block(cfg, res, w, k_caches[l], v_caches[l], position,
                                     position + 1, eps)
        norm_out = self.r16(self.rmsnorm(res, final_norm, H, 1, eps))
        return [F32(x) for x in self.qmv(*emb, norm_out, V, H, GS)]


def round16(xs):
    """float16 storage rounding of a list of values (RNE from the exact value)."""
    return [float(F16(x)) for x in xs]


# ---------------------------------------------------------------------------
# The two composed-path fixtures
# ---------------------------------------------------------------------------

BLOCK_SEEDS = dict(q=0xA5, k=0x5A, v=0x33, o=0xCC, gate=0x55, up=0xAA, down=0x69)
EMBED_SEED = 0xB7


def block_weights(cfg, q_norm=(0.9, 0.003), k_norm=(0.85, 0.004)):
    """The block weights both tests build (transformer_test.zig:1741-1807 and
    :2124-2240): seven createTestPackedBuffer matrices and the norm fills."""
    H, HD = cfg["hidden_size"], cfg["head_dim"]
    QD, KVD = cfg["num_query_heads"] * HD, cfg["num_kv_heads"] * HD
    I, GS = cfg["intermediate_size"], cfg["group_size"]
    sizes = dict(q=QD * H, k=KVD * H, v=KVD * H, o=H * QD, gate=I * H, up=I * H, down=H * I)
    w = {n: packed_buffer_fixture(sizes[n], BLOCK_SEEDS[n], GS) for n in BLOCK_SEEDS}
    w["attn_norm"] = linear_f32(H, 0.5, 0.01)
    w["ffn_norm"] = linear_f32(H, 0.8, 0.005)
    w["q_norm"] = linear_f32(HD, *q_norm)
    w["k_norm"] = linear_f32(HD, *k_norm)
    return w


def single_block_case():
    """:1697-1997 -- TinyBlock, KV pre-filled for 3 positions, residual
    (i+1)*0.05, token at position 3 (seq_len 4).  Returns (cfg, weights,
    residual, k_cache, v_cache, position)."""
    cfg = TINY_BLOCK
    w = block_weights(cfg)
    k, v = populate_kv(cfg["num_kv_heads"], 3, cfg["head_dim"], cfg["max_context_length"])
    res = [F32(F32(i + 1) * F32(0.05)) for i in range(cfg["hidden_size"])]
    return cfg, w, res, k, v, 3


def forward_decode_case():
    """:2086-2489 -- TinyBlock, tied 1-bit embedding (seed 0xB7), token 1 at
    position 0, zeroed KV caches, norms q 0.6+0.01i, k 0.7+0.01i, final
    1.0+0.002i.  Returns (cfg, emb, [block weights], final_norm, token,
    position)."""
    cfg = TINY_BLOCK
    emb = packed_buffer_fixture(cfg["vocab_size"] * cfg["hidden_size"], EMBED_SEED,
                             cfg["group_size"])
    w = block_weights(cfg, q_norm=(0.6, 0.01), k_norm=(0.7, 0.01))
    final_norm = linear_f32(cfg["hidden_size"], 1.0, 0.002)
    return cfg, emb, [w], final_norm, 1, 0


# ---------------------------------------------------------------------------
# The fixtures in the build's own weight format
# ---------------------------------------------------------------------------

def _qweight(packed_scales, M: int, K: int, gs: int):
    from nnzap_amd import formats as fm
    raw, scales = packed_scales
    codes = np.frombuffer(raw, dtype="<u4").reshape(M, K // 32).copy()
    sc = np.array(scales, dtype=np.float16).view(np.uint16).reshape(M, K // gs)
    return fm.QWeight(1, M, K, gs, codes, sc, None, fm.DT_F16)


def decoder_config(cfg):
    """TinyBlock as the build's DecoderConfig: 1-bit embedding table and a
    1-bit LM head holding the same matrix (tie_word_embeddings)."""
    from nnzap_amd.configs import DecoderConfig
    return DecoderConfig(vocab_size=cfg["vocab_size"], hidden_size=cfg["hidden_size"],
                         intermediate_size=cfg["intermediate_size"],
                         num_layers=cfg["num_layers"], num_query_heads=cfg["num_query_heads"],
                         num_kv_heads=cfg["num_kv_heads"], head_dim=cfg["head_dim"],
                         max_context_length=cfg["max_context_length"],
                         max_prefill_length=cfg["max_prefill_length"],
                         group_size=cfg["group_size"], rope_theta=cfg["rope_theta"],
                         rms_eps=1e-6, embed_kind=0, lm_head_kind=0)


def decoder_weights(cfg, layers, emb=None, final_norm=None):
    """DecoderWeights of the fixture (layers: block_weights dicts)."""
    from nnzap_amd.configs import DecoderWeights
    H, HD, GS = cfg["hidden_size"], cfg["head_dim"], cfg["group_size"]
    QD, KVD = cfg["num_query_heads"] * HD, cfg["num_kv_heads"] * HD
    I = cfg["intermediate_size"]
    shapes = dict(q=(QD, H), k=(KVD, H), v=(KVD, H), o=(H, QD), gate=(I, H), up=(I, H),
                  down=(H, I))
    dw = DecoderWeights(decoder_config(cfg))
    for w in layers:
        layer = {n: _qweight(w[n], *shapes[n], GS) for n in shapes}
        for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            layer[n] = np.array(w[n], dtype=np.float32)
        dw.layers.append(layer)
    if emb is not None:
        dw.embed_q1 = _qweight(emb, cfg["vocab_size"], H, GS)
        dw.lm_head = dw.embed_q1
    dw.final_norm = (np.array(final_norm, dtype=np.float32) if final_norm is not None
                     else np.ones(H, dtype=np.float32))
    return dw


def kv_as_array(cache, cfg):
    """A flat [h][t][d] cache list as a float64 array [Hkv, max_ctx, D]."""
    return np.array([float(x) for x in cache]).reshape(cfg["num_kv_heads"],
                                                        cfg["max_context_length"],
                                                        cfg["head_dim"])


def from_qweight(q):
    """A 1-bit QWeight as the restatement's (packed bytes, f16 scales)."""
    return (np.ascontiguousarray(q.codes).tobytes(),
            list(np.ascontiguousarray(q.scales).view(np.float16).reshape(-1)))


def soft_case(num_layers: int = 2):
    """A second fixture for what the reference's deterministic ones leave
    open: their pre-filled keys (up to ~19 in every dimension) make each
    softmax one-hot, so a positive rescaling of q or k (a missing q_norm or
    k_norm) cannot show.  Seeded random 1-bit weights at a TINY-like shape
    (hidden 256, MLP 512, 4 query / 2 KV heads x 64, vocab 512), norm scales
    1 + N(0, 0.02), tied 1-bit embedding; returns (cfg dict, emb, layers,
    final_norm, DecoderWeights)."""
    from nnzap_amd import configs as cf
    cfg = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=num_layers,
               num_query_heads=4, num_kv_heads=2, head_dim=64, max_context_length=16,
               max_prefill_length=8, rope_theta=10000.0, group_size=128)
    dc = decoder_config(cfg)
    w = cf.decoder_weights(dc, norm_mode="unit", host_embed=False)
    w.embed_q1 = w.lm_head
    emb = from_qweight(w.lm_head)
    layers = []
    for L in w.layers:
        d = {n: from_qweight(L[n]) for n in BLOCK_SEEDS}
        for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            d[n] = [F32(x) for x in L[n]]
        layers.append(d)
    fnorm = [F32(x) for x in w.final_norm]
    return cfg, emb, layers, fnorm, w

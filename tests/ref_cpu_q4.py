"""Scalar restatement of nnmetal's q4_mlx decode step -- TEST INFRASTRUCTURE
ONLY (pins the oracle's 4-bit whole-step composition).

Written from the reference's Metal kernels, independently of ``oracle/``
(the attention half reuses ``ref_cpu.Ref``, the restatement of the
reference's CPU test functions, which the Q1 composition tests pin):

* BF16 rounding = truncation of the float32 value to its high 16 bits
  (``bf16_round``, q4mv_bf16_specialized.metal:52-57);
* ``embedding_lookup_q4`` (transformer.metal:505-549): row value
  ``bf16_round(scale * nibble + bias)``, scale/bias raw BF16 (zero-extended,
  :534-539);
* the Q4 matrix-vector product, per 8-column word (q4mv_bf16_specialized.metal
  :138-160): ``nd = sum n_i x_i``, ``gs = sum x_i``, ``acc += s nd + b gs``;
* its epilogues: ``half(bf16_round(acc))`` for the fused-norm Q and K/V
  projections (:1022-1025, :1178-1179), ``residual += bf16_round(acc)`` for
  the O and down projections (:288-289, :619-620), ``half(bf16_round(silu(g)
  u))`` for gate/up (:863), ``bf16_round(acc)`` in float32 for the LM head
  (q4mv_spec_f16in :495-498);
* the normalised input of every fused-norm projection, and the final norm
  (``rms_norm_bf16_f16out``, transformer.metal:610-677):
  ``half(bf16_round(x rms w))`` (q4mv_bf16_specialized.metal:806, :956, :1120);
* the decode flow (transformer.zig:2646-2668 Q4 embedding, :2743-2785 final
  norm + LM head, the blocks :2452-3646).

Arithmetic: float64, with the storage rounding points above applied as
float32 rounding (RNE) followed by the BF16 truncation, float16 (RNE) at the
half stores, and the float32 residual -- the same convention the Q1
restatement's float64 mode uses for its hooks.  ``drop`` names rounding
points to leave out, for the planted-mistake tests.
"""
from __future__ import annotations

import math

import numpy as np

import ref_cpu as R

POINTS = ("embed", "norm", "qkv", "o_add", "silu", "down_add", "final_norm", "logits")


def f32(x) -> float:
    return float(np.float32(x))


def f16(x) -> float:
    return float(np.float16(x))


def bf16_round(x) -> float:
    """Zero the low 16 bits of the float32 value (truncation toward zero)."""
    b = np.array([x], dtype=np.float32).view(np.uint32)[0] & np.uint32(0xFFFF0000)
    return float(np.array([b], dtype=np.uint32).view(np.float32)[0])


def raw16(raw: int, bf16: bool) -> float:
    """A raw 16-bit scale or bias: BF16 zero-extended into a float32, or f16."""
    if bf16:
        return float(np.array([int(raw) << 16], dtype=np.uint32).view(np.float32)[0])
    return float(np.array([int(raw)], dtype=np.uint16).view(np.float16)[0])


class RefQ4:
    """The q4_mlx decode step of one model (nnzap_amd.configs.DecoderWeights
    of a ``quant_format == 1`` config) as scalar per-row loops."""

    def __init__(self, w, drop=()):
        self.w, self.cfg = w, w.cfg
        self.drop = set(drop)
        assert self.drop <= set(POINTS), self.drop
        self.att = R.Ref(ft=float, r16=R.round16, rope="build")

    # -- storage rounding points ----------------------------------------------
    def _bf(self, point, x):
        """float32 then BF16 truncation, unless ``point`` is dropped (then
        the float32 value)."""
        return f32(x) if point in self.drop else bf16_round(f32(x))

    def _half_bf(self, point, xs):
        return [f16(self._bf(point, x)) for x in xs]

    # -- kernels ----------------------------------------------------------------
    @staticmethod
    def _row_words(q, r):
        return [int(v) for v in np.asarray(q.codes)[r]]

    def q4mv(self, q, x):
        """y[r] = sum over words of s nd + b gs (float64)."""
        bf = q.scale_dtype == 2
        gs = q.group_size
        S, B = np.asarray(q.scales), np.asarray(q.biases)
        out = []
        for r in range(q.M):
            acc = 0.0
            for wi, word in enumerate(self._row_words(q, r)):
                c0 = wi * 8
                nd = gsum = 0.0
                for i in range(8):
                    xv = x[c0 + i]
                    nd += float((word >> (4 * i)) & 0xF) * xv
                    gsum += xv
                g = c0 // gs
                acc += raw16(S[r, g], bf) * nd + raw16(B[r, g], bf) * gsum
            out.append(acc)
        return out

    def embedding(self, token: int):
        q = self.w.embed_q1
        bf = q.scale_dtype == 2
        H, gs = self.cfg.hidden_size, q.group_size
        S, B = np.asarray(q.scales).reshape(-1), np.asarray(q.biases).reshape(-1)
        words = np.asarray(q.codes).reshape(-1)
        out = []
        for d in range(H):
            flat = token * H + d
            n = (int(words[flat // 8]) >> (4 * (flat % 8))) & 0xF
            g = flat // gs
            out.append(self._bf("embed", raw16(S[g], bf) * n + raw16(B[g], bf)))
        return out

    def _rms(self, x, w):
        eps = self.cfg.rms_eps
        ss = 0.0
        for v in x:
            ss += v * v
        r = 1.0 / math.sqrt(ss / len(x) + eps)
        return [v * r * float(s) for v, s in zip(x, w)]

    def _norm16(self, point, x, w):
        return self._half_bf(point, self._rms(x, w))

    # -- one block, one token (forwardBlock for the Q4 kernels) -----------------
    def block(self, l, res, kc, vc, pos):
        cfg, L = self.cfg, self.w.layers[l]
        H, D = cfg.hidden_size, cfg.head_dim
        Hq, Hkv, T = cfg.num_query_heads, cfg.num_kv_heads, cfg.max_context_length
        xn = self._norm16("norm", res, L["attn_norm"])
        q = self._half_bf("qkv", self.q4mv(L["q"], xn))
        k = self._half_bf("qkv", self.q4mv(L["k"], xn))
        v = self._half_bf("qkv", self.q4mv(L["v"], xn))
        a = self.att
        eps = cfg.rms_eps
        q = a.rmsnorm(q, [float(s) for s in L["q_norm"]], D, Hq, eps)
        k = a.rmsnorm(k, [float(s) for s in L["k_norm"]], D, Hkv, eps)
        q = a.rope(q, Hq, D, pos, cfg.rope_theta)
        k = a.rope(k, Hkv, D, pos, cfg.rope_theta)
        for h in range(Hkv):
            for d in range(D):
                idx = h * T * D + pos * D + d
                kc[idx] = np.float16(k[h * D + d])
                vc[idx] = np.float16(v[h * D + d])
        att = R.round16(a.gqa(q, kc, vc, Hq, D, pos + 1, T, Hq // Hkv))
        o = self.q4mv(L["o"], att)
        res = [f32(r + self._bf("o_add", t)) for r, t in zip(res, o)]
        xn2 = self._norm16("norm", res, L["ffn_norm"])
        g = self.q4mv(L["gate"], xn2)
        u = self.q4mv(L["up"], xn2)
        hmid = self._half_bf("silu", [gv / (1.0 + math.exp(-gv)) * uv for gv, uv in zip(g, u)])
        dn = self.q4mv(L["down"], hmid)
        assert len(res) == H
        return [f32(r + self._bf("down_add", t)) for r, t in zip(res, dn)]

    def new_caches(self):
        cfg = self.cfg
        n = cfg.num_kv_heads * cfg.max_context_length * cfg.head_dim
        return ([[np.float16(0)] * n for _ in range(cfg.num_layers)],
                [[np.float16(0)] * n for _ in range(cfg.num_layers)])

    def decode(self, token: int, pos: int, kcs, vcs):
        """forwardDecode for one token: returns the float32 logits."""
        res = [f32(x) for x in self.embedding(token)]
        for l in range(self.cfg.num_layers):
            res = self.block(l, res, kcs[l], vcs[l], pos)
        xf = self._norm16("final_norm", res, self.w.final_norm)
        return [self._bf("logits", t) for t in self.q4mv(self.w.lm_head, xf)]

"""CPU oracle of the whole decode step -- TEST INFRASTRUCTURE ONLY.

Restates nnmetal's forwardDecode (nnmetal/src/transformer.zig:2566-2785,
blocks :2452-3646) and generate (:3942-4030) in numpy, float64 arithmetic,
with the reference's storage rounding points:

* residual stream: float32, rounded after every ``+=`` (model.zig:87-102);
* fused-norm prologue output, Q/K/V projections, attention output, the
  SiLU*mul activation and the final-norm output: float16
  (qmv_specialized.metal:1137-1177, :1432, :1617, :1276; transformer.metal:1689);
* normalised/rotated q kept unrounded (transformer.metal:1529-1557), the
  normalised/rotated k and v stored as float16 in the KV cache (:1583-1592);
* logits: float32 (qmv_spec_f16in, qmv_specialized.metal:735).

A q4_mlx model (``cfg.quant_format == 1``) takes the Q4 path's extra
rounding points (transformer.zig:2646, :2743, :2977, :3100): the embedding
row, every norm output before it is narrowed to float16, and every
projection result (stored, added to the residual, or the SiLU*mul product,
and the logits) are BF16-truncated (q4mv_bf16_specialized.metal:52-57, :806;
transformer.metal:505-549, :610-677).

Prefill is evaluated as a batch (all prompt tokens at once, causal mask):
mathematically identical to the reference's token-by-token prefill
(transformer.zig:4032-4068) because every token's computation only reads
keys/values of earlier positions.
"""
from __future__ import annotations

import numpy as np

from nnzap_amd.configs import PROJS, DecoderConfig, DecoderWeights
from nnzap_amd import synth as S

from . import oracle as O


def _f32(x):
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


class OracleDecoder:
    def __init__(self, w: DecoderWeights, max_ctx: int | None = None, round16: bool = True,
                 matmul_dtype=np.float64):
        """``round16=False`` drops the float16 storage roundings of the
        activations (normalised inputs, q/k/v, attention output, SiLU*mul,
        final norm) and keeps the float16 KV cache and the float32 residual:
        the precision of the reference's own CPU test references
        (transformer_test.zig:364-716), against which the composition is
        pinned.

        ``matmul_dtype=np.float32`` evaluates every weight product in float32
        (the precision of the GPU's accumulators) with the same rounding
        points: the spread between that and the float64 oracle is the
        rounding noise any float32 implementation carries, which sets the
        end-to-end bar at full size."""
        cfg = w.cfg
        self.cfg, self.w = cfg, w
        self.mdt = matmul_dtype
        self.r16 = O.f16 if round16 else (lambda x: np.asarray(x, dtype=np.float64))
        self.q4 = getattr(cfg, "quant_format", 0) == 1
        self.W = [{n: O.dequant(layer[n]).astype(matmul_dtype) for n in PROJS}
                  for layer in w.layers]
        self.lm = O.dequant(w.lm_head).astype(matmul_dtype) if w.lm_head is not None else None
        T = max_ctx or cfg.max_context_length
        self.kc = np.zeros((cfg.num_layers, cfg.num_kv_heads, T, cfg.head_dim))
        self.vc = np.zeros((cfg.num_layers, cfg.num_kv_heads, T, cfg.head_dim))
        self._emb_cache = {}

    # -- embedding (bf16 table, widened to f32) -------------------------------
    def embed_rows(self, ids) -> np.ndarray:
        cfg = self.cfg
        ids = [int(i) for i in ids]
        e = self.w.embed_q1
        if e is not None and e.bits == 4:
            # embedding_lookup_q4 (transformer.metal:505-549)
            return O.embed_q4(ids, e.codes, e.scales, e.biases, cfg.hidden_size, e.group_size,
                              e.scale_dtype)
        if e is not None:
            # embedding_lookup (transformer.metal:428-481): +-s of row `id`
            return O.embed_q1(ids, e.codes.view(np.uint8).reshape(-1),
                              e.scales.view(np.float16).reshape(-1), cfg.hidden_size,
                              e.group_size)
        if self.w.embed_bf16 is not None:
            return S.bf16_bits_to_f32(self.w.embed_bf16[ids]).astype(np.float64)
        out = []
        for t in ids:
            if t not in self._emb_cache:
                idx = np.arange(t * cfg.hidden_size, (t + 1) * cfg.hidden_size, dtype=np.uint64)
                z = 0.02 * S.normal_at(S.SEED_MODEL_BASE + 0, idx)
                self._emb_cache[t] = S.bf16_bits_to_f32(S.f64_to_bf16_bits(z)).astype(np.float64)
            out.append(self._emb_cache[t])
        return np.stack(out)

    def _t(self, x):
        """The Q4 path's BF16 truncation of a float32 result (identity for Q1)."""
        return O.bf16_trunc(_f32(x)) if self.q4 else x

    def _norm16(self, x, w):
        return self.r16(self._t(O.rmsnorm(x, w, self.cfg.rms_eps)))

    def lm_head(self, xf: np.ndarray) -> np.ndarray:
        if self.lm is not None:
            return _f32(self._t((xf.astype(self.mdt) @ self.lm.T).astype(np.float64)))
        table = S.bf16_bits_to_f32(self.w.embed_bf16).astype(np.float64)
        return _f32(xf @ table.T)

    # -- one batch of consecutive tokens (P >= 1) -------------------------------
    def forward(self, ids, start: int) -> np.ndarray:
        """Run tokens ``ids`` at positions start..start+P-1; returns the logits
        of every token [P, vocab] (float32 values as float64)."""
        res = _f32(self.embed_rows(ids))
        for l in range(self.cfg.num_layers):
            res = self.layer(l, res, start)
        xf = self._norm16(res, self.w.final_norm)
        return self.lm_head(xf)

    def layer(self, l: int, res: np.ndarray, start: int) -> np.ndarray:
        """One decoder block (forwardBlock, transformer.zig:2452-2564) for the
        residual rows ``res`` [P, H] of tokens at positions start..start+P-1:
        attention half then MLP half; appends the block's K/V rows to its
        cache.  Returns the new residual (float32 values)."""
        cfg = self.cfg
        P = res.shape[0]
        D, Hq, Hkv = cfg.head_dim, cfg.num_query_heads, cfg.num_kv_heads
        g = Hq // Hkv
        positions = np.arange(start, start + P)
        layer, W, r16 = self.w.layers[l], self.W[l], self.r16
        mm = lambda a, b: (a.astype(self.mdt) @ b.T).astype(np.float64)  # noqa: E731
        xn = self._norm16(res, layer["attn_norm"])
        q = r16(self._t(mm(xn, W["q"])))
        k = r16(self._t(mm(xn, W["k"])))
        v = r16(self._t(mm(xn, W["v"])))
        qn = np.stack([O.head_norm_rope(q[p].reshape(Hq, D), layer["q_norm"], int(positions[p]),
                                        cfg.rope_theta, cfg.rms_eps) for p in range(P)])
        kn = np.stack([O.f16(O.head_norm_rope(k[p].reshape(Hkv, D), layer["k_norm"],
                                              int(positions[p]), cfg.rope_theta, cfg.rms_eps))
                       for p in range(P)])
        self.kc[l, :, start:start + P, :] = kn.transpose(1, 0, 2)
        self.vc[l, :, start:start + P, :] = O.f16(v).reshape(P, Hkv, D).transpose(1, 0, 2)
        att = np.empty((P, Hq, D))
        scale = 1.0 / np.sqrt(D)
        T = start + P
        K = self.kc[l, :, :T, :]
        V = self.vc[l, :, :T, :]
        mask = np.arange(T)[None, :] <= positions[:, None]  # [P, T]
        for h in range(Hq):
            s = qn[:, h, :] @ K[h // g].T * scale  # [P, T]
            s = np.where(mask, s, -np.inf)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            s /= s.sum(axis=1, keepdims=True)
            att[:, h, :] = s @ V[h // g]
        att = r16(att.reshape(P, Hq * D))
        res = _f32(res + self._t(mm(att, W["o"])))
        xn2 = self._norm16(res, layer["ffn_norm"])
        hmid = r16(self._t(O.silu(mm(xn2, W["gate"])) * mm(xn2, W["up"])))
        return _f32(res + self._t(mm(hmid, W["down"])))

    def generate(self, prompt, n_new: int, eos=()):
        """Greedy generate with the reference's loop (transformer.zig:3942-4030):
        returns (tokens, top-2 margins) -- up to n_new tokens, one decode pass
        per emitted token; a stop token in ``eos`` ends it unemitted (:3992)."""
        logits = self.forward(list(prompt), 0)[-1]
        pos = len(prompt)
        toks, margins = [], []
        for _ in range(n_new):
            t = O.argmax_first(logits)
            if t in eos:
                break
            srt = np.sort(logits)
            toks.append(t)
            margins.append(float(srt[-1] - srt[-2]))
            logits = self.forward([t], pos)[0]
            pos += 1
        return np.array(toks, dtype=np.uint32), np.array(margins)

    def generate_sampled(self, prompt, n_new: int, temperature: float, top_k: int, top_p: float,
                         seed: int, eos=()):
        """generate with SamplingParams (transformer.zig:3969-4016): returns
        (tokens, sampled probabilities, per-step decision margins)."""
        from .sampling import ZigPrng, sample_token
        prng = ZigPrng(seed)
        logits = self.forward(list(prompt), 0)[-1]
        pos = len(prompt)
        toks, probs, margins = [], [], []
        for _ in range(n_new):
            t, pr, mg = sample_token(logits.astype(np.float32), temperature, top_k, top_p, prng)
            mg = min(mg, 1.0)
            if t in eos:
                break
            toks.append(t)
            probs.append(pr)
            margins.append(mg)
            logits = self.forward([t], pos)[0]
            pos += 1
        return np.array(toks, dtype=np.uint32), np.array(probs), np.array(margins)

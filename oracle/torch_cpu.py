"""PyTorch-CPU float32 restatement of the decode hot path -- the timed CPU
baseline of bench.py (TEST / BENCH INFRASTRUCTURE ONLY; nothing in the
product imports it).

The reference has no PyTorch path for this workload (its PyTorch scripts are
MNIST), so the CPU baseline is this build's own dequant + matmul in float32,
written from the same formulas as the oracle:

* 1-bit: bit i of byte b is column 8b + i (LSB first), +1 / -1 from a
  byte -> 8 signs table, times the group scale (transformer.metal:469-480;
  the stored scale is already halved, model.zig:1058-1070);
* 4-bit: ``(word >> 4*arange(8)) & 15`` -> s*n + b (q4mv_bf16_specialized
  .metal:14-27);
* one decode step of the config-5 decoder (transformer.zig:2440-3646): per
  layer RMSNorm, Q/K/V, per-head q/k RMSNorm + consecutive-pair RoPE, KV
  append, GQA softmax attention, O += , RMSNorm, silu(gate)*up, down +=; final
  RMSNorm and the LM head.  Activations stay float32 (the reference's CPU
  test precision, transformer_test.zig:364-716);
* the prompt as one batch (``prefill``): the same layer arithmetic with
  [P x K] products and causal attention -- the reference itself prefills
  token by token (chunkedPrefill, transformer.zig:4032-4068), which on this
  CPU would be P decode steps.

Two variants are timed: weights dequantised once up front (float32 GEMVs on
resident matrices), and dequantised from the packed codes on every call.
"""
from __future__ import annotations

import numpy as np
import torch


_SIGNS = None


def _sign_table() -> torch.Tensor:
    """[256, 8] float32: bit i of byte b as +1 / -1 (LSB = lowest column)."""
    global _SIGNS
    if _SIGNS is None:
        b = torch.arange(256, dtype=torch.int32)
        _SIGNS = ((b[:, None] >> torch.arange(8, dtype=torch.int32)) & 1).float() * 2.0 - 1.0
    return _SIGNS


def dequant_q1(codes: np.ndarray, scales_f16: np.ndarray, M: int, K: int, gs: int) -> torch.Tensor:
    """[M, K] float32 +-s from uint32 words [M, K/32] (LSB-first bytes) and
    f16 scales [M, K/gs]: a byte -> 8 signs table lookup, times the scale."""
    by = torch.from_numpy(np.ascontiguousarray(codes).view(np.uint8).reshape(M, K // 8))
    signs = torch.nn.functional.embedding(by.to(torch.int32), _sign_table())   # [M, K/8, 8]
    s = torch.from_numpy(np.ascontiguousarray(scales_f16).view(np.float16)).reshape(M, K // gs)
    return (signs.reshape(M, K // gs, gs) * s.float().unsqueeze(-1)).reshape(M, K)


def dequant_q4(codes: np.ndarray, scales: np.ndarray, biases: np.ndarray, M: int, K: int,
               gs: int, bf16: bool) -> torch.Tensor:
    """[M, K] float32 s*n + b from uint32 words [M, K/8] and 16-bit s, b."""
    w = torch.from_numpy(np.ascontiguousarray(codes).view(np.int32)).reshape(M, K // 8)
    n = ((w.unsqueeze(-1) >> (4 * torch.arange(8, dtype=torch.int32))) & 15).reshape(M, K).float()

    def widen(raw):
        r = torch.from_numpy(np.ascontiguousarray(raw).view(np.int16)).reshape(M, K // gs)
        if bf16:
            return (r.to(torch.int32) << 16).view(torch.float32)
        return r.view(torch.float16).float()
    return widen(scales).repeat_interleave(gs, dim=1) * n + widen(biases).repeat_interleave(gs, dim=1)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * w


def rope(x: torch.Tensor, pos: int, inv_freq: torch.Tensor) -> torch.Tensor:
    """Consecutive pairs (x[2p], x[2p+1]) rotated by pos * inv_freq[p]."""
    ang = pos * inv_freq
    c, s = torch.cos(ang), torch.sin(ang)
    a, b = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


class TorchDecoder:
    """A 1-bit config-5-shaped decoder on the CPU, float32."""

    PROJS = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, w, max_ctx: int, predequantise: bool = True):
        cfg = w.cfg
        self.cfg, self.w, self.pre = cfg, w, predequantise
        self.norms = [{n: torch.from_numpy(np.asarray(L[n], dtype=np.float32))
                       for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")} for L in w.layers]
        self.final_norm = torch.from_numpy(np.asarray(w.final_norm, dtype=np.float32))
        self.W = [{n: self._deq(L[n]) for n in self.PROJS} for L in w.layers] if predequantise \
            else None
        self.lm = self._deq(w.lm_head) if predequantise else None
        p = torch.arange(cfg.head_dim // 2, dtype=torch.float64)
        self.inv_freq = torch.exp2(-(2.0 * p / cfg.head_dim) * np.log2(cfg.rope_theta)).float()
        shape = (cfg.num_layers, cfg.num_kv_heads, max_ctx, cfg.head_dim)
        self.kc = torch.zeros(shape)
        self.vc = torch.zeros(shape)

    @staticmethod
    def _deq(q) -> torch.Tensor:
        return dequant_q1(q.codes, q.scales, q.M, q.K, q.group_size)

    def _weight(self, l: int, name: str) -> torch.Tensor:
        return self.W[l][name] if self.pre else self._deq(self.w.layers[l][name])

    def fill_cache(self, upto: int, seed: int = 0) -> None:
        """Random float16-valued keys/values at positions < upto (timing
        runs: the work of a step does not depend on the cached values)."""
        g = torch.Generator().manual_seed(seed)
        self.kc[:, :, :upto] = torch.randn(self.kc[:, :, :upto].shape, generator=g).half().float()
        self.vc[:, :, :upto] = torch.randn(self.vc[:, :, :upto].shape, generator=g).half().float()

    @torch.no_grad()
    def prefill(self, xs: torch.Tensor, start: int = 0) -> torch.Tensor:
        """The prompt as one batch: residual rows ``xs`` [P, H] at positions
        start.. (every projection one [P x K] . W^T product, causal GQA
        attention over the cache); fills the KV cache and returns the float32
        logits of the last row [V] -- the same arithmetic as P ``step``
        calls up to float32 summation order."""
        cfg = self.cfg
        D, Hq, Hkv = cfg.head_dim, cfg.num_query_heads, cfg.num_kv_heads
        g, eps = Hq // Hkv, cfg.rms_eps
        P = xs.shape[0]
        pos = torch.arange(start, start + P, dtype=torch.float32)
        ang = pos[:, None] * self.inv_freq[None, :]                      # [P, D/2]
        c, s_ = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]

        def rope_rows(x):                                                # [P, heads, D]
            a, b = x[..., 0::2], x[..., 1::2]
            out = torch.empty_like(x)
            out[..., 0::2] = a * c - b * s_
            out[..., 1::2] = a * s_ + b * c
            return out

        # query i sees keys 0 .. start + i
        mask = torch.arange(start + P)[None, :] > (start + torch.arange(P))[:, None]
        res = xs.clone()
        for l in range(cfg.num_layers):
            nm = self.norms[l]
            xn = rmsnorm(res, nm["attn_norm"], eps)
            q = xn @ self._weight(l, "q").T
            k = xn @ self._weight(l, "k").T
            v = xn @ self._weight(l, "v").T
            q = rope_rows(rmsnorm(q.view(P, Hq, D), nm["q_norm"], eps))
            k = rope_rows(rmsnorm(k.view(P, Hkv, D), nm["k_norm"], eps))
            self.kc[l, :, start:start + P] = k.transpose(0, 1).half().float()
            self.vc[l, :, start:start + P] = v.view(P, Hkv, D).transpose(0, 1).half().float()
            K, V = self.kc[l, :, :start + P], self.vc[l, :, :start + P]   # [Hkv, T, D]
            qh = q.view(P, Hkv, g, D).permute(1, 2, 0, 3)                 # [Hkv, g, P, D]
            sc = torch.matmul(qh, K.transpose(1, 2)[:, None]) / np.sqrt(D)  # [Hkv, g, P, T]
            sc = sc.masked_fill(mask, float("-inf"))
            att = torch.matmul(torch.softmax(sc, dim=-1), V[:, None])       # [Hkv, g, P, D]
            att = att.permute(2, 0, 1, 3).reshape(P, Hq * D)
            res = res + att @ self._weight(l, "o").T
            xn2 = rmsnorm(res, nm["ffn_norm"], eps)
            h = torch.nn.functional.silu(xn2 @ self._weight(l, "gate").T) * (xn2 @ self._weight(l, "up").T)
            res = res + h @ self._weight(l, "down").T
        xf = rmsnorm(res[-1], self.final_norm, eps)
        lm = self.lm if self.pre else self._deq(self.w.lm_head)
        return lm @ xf

    @torch.no_grad()
    def step(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """One decode step for the residual row ``x`` [H] at ``pos``; returns
        the float32 logits [V]."""
        cfg = self.cfg
        D, Hq, Hkv = cfg.head_dim, cfg.num_query_heads, cfg.num_kv_heads
        g, eps = Hq // Hkv, cfg.rms_eps
        res = x.clone()
        for l in range(cfg.num_layers):
            nm = self.norms[l]
            xn = rmsnorm(res, nm["attn_norm"], eps)
            q = self._weight(l, "q") @ xn
            k = self._weight(l, "k") @ xn
            v = self._weight(l, "v") @ xn
            q = rope(rmsnorm(q.view(Hq, D), nm["q_norm"], eps), pos, self.inv_freq)
            k = rope(rmsnorm(k.view(Hkv, D), nm["k_norm"], eps), pos, self.inv_freq)
            self.kc[l, :, pos] = k.half().float()
            self.vc[l, :, pos] = v.view(Hkv, D).half().float()
            K, V = self.kc[l, :, :pos + 1], self.vc[l, :, :pos + 1]       # [Hkv, T, D]
            s = torch.matmul(q.view(Hkv, g, D), K.transpose(1, 2)) / np.sqrt(D)
            att = torch.matmul(torch.softmax(s, dim=-1), V).reshape(Hq * D)
            res = res + self._weight(l, "o") @ att
            xn2 = rmsnorm(res, nm["ffn_norm"], eps)
            h = torch.nn.functional.silu(self._weight(l, "gate") @ xn2) * (self._weight(l, "up") @ xn2)
            res = res + self._weight(l, "down") @ h
        xf = rmsnorm(res, self.final_norm, eps)
        lm = self.lm if self.pre else self._deq(self.w.lm_head)
        return lm @ xf

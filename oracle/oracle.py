"""CPU oracle for the Bonsai/Qwen3 decode hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of duanebester/nnzap's
``nnmetal`` decode path (Zig host + Metal shaders).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker / the timed CPU baseline -- never as a code path of
the product.  The product (``nnzap_amd``) must not import anything from here.

Conventions
-----------
* Every sum is accumulated in float64 (``acc`` dtype) unless a function says
  otherwise; the GPU accumulates in float32, so results are compared with a
  relative tolerance, never bit-for-bit.
* Storage rounding points are reproduced exactly where the reference stores a
  narrower type: ``f16(...)`` for half activations and the KV cache,
  ``bf16_trunc`` for the Q4 "BF16-faithful" outputs.
* Integer/byte work (unpacking, dequantised values, argmax) is exact and is
  compared bit-for-bit.

Pinning status of each function (how a plausible mistake is caught):
see ``tests/test_oracle.py`` -- every public function below is checked against
the reference's known-answer tests / fixtures and closed-form invariants.
"""
from __future__ import annotations

import numpy as np

import nnzap_amd.formats as fm  # pure-numpy packing helpers (no GPU code)

F16 = np.float16


# ---------------------------------------------------------------------------
# Scalar helpers
# ---------------------------------------------------------------------------

def f16(x) -> np.ndarray:
    """Round to IEEE half (RNE), return float64 holding the half value.
    numpy's float64->float16 cast rounds once, so there is no double rounding
    through float32."""
    return np.asarray(x, dtype=np.float64).astype(F16).astype(np.float64)


def bf16_trunc(x) -> np.ndarray:
    """q4mv_bf16_specialized.metal:52-57 ``bf16_round``: zero the low 16 bits
    of the float32 value (truncation toward zero, not RNE)."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    return (f.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)


def raw16_to_f64(raw: np.ndarray, dtype: int) -> np.ndarray:
    raw = np.asarray(raw, dtype=np.uint16)
    if dtype == fm.DT_F16:
        return raw.view(F16).astype(np.float64)
    if dtype == fm.DT_BF16:
        # q4mv_bf16_specialized.metal:48-50: zero-extend into the high half.
        return (raw.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# Dequantisation (a1, a2)
# ---------------------------------------------------------------------------

def dequant_q1(w: fm.QWeight) -> np.ndarray:
    """``bit ? +s : -s`` per element, transformer.metal:469-480 and
    transformer_test.zig:303-330 (cpuQMV).  Exact (values are f16 scales)."""
    assert w.bits == 1
    bits = fm.unpack_q1(w.codes, w.K).astype(bool)
    s = raw16_to_f64(w.scales, fm.DT_F16).reshape(w.M, w.K // w.group_size)
    s_full = np.repeat(s, w.group_size, axis=1)
    return np.where(bits, s_full, -s_full)


def dequant_q4(w: fm.QWeight) -> np.ndarray:
    """``s * nibble + b`` (q4mv_bf16_specialized.metal:14-16,
    transformer.metal:537-545), evaluated exactly in float64 and rounded once
    to float32 -- the value ``fmaf(s, n, b)`` produces on the GPU."""
    assert w.bits == 4
    n = fm.unpack_q4(w.codes, w.K).astype(np.float64)
    G = w.K // w.group_size
    s = np.repeat(raw16_to_f64(w.scales, w.scale_dtype).reshape(w.M, G), w.group_size, axis=1)
    b = np.repeat(raw16_to_f64(w.biases, w.scale_dtype).reshape(w.M, G), w.group_size, axis=1)
    return (s * n + b).astype(np.float32).astype(np.float64)


def dequant(w: fm.QWeight) -> np.ndarray:
    return dequant_q1(w) if w.bits == 1 else dequant_q4(w)


def dequant_q1_affine(w_codes, scale_f16, bias_f16, M, K, gs) -> np.ndarray:
    """The BASELINE definition ``scale * bit + bias`` before the symmetric
    load transform (used to show the transform is lossless)."""
    bits = fm.unpack_q1(w_codes, K).astype(np.float64)
    s = np.repeat(np.asarray(scale_f16, F16).astype(np.float64).reshape(M, K // gs), gs, axis=1)
    b = np.repeat(np.asarray(bias_f16, F16).astype(np.float64).reshape(M, K // gs), gs, axis=1)
    return s * bits + b


# ---------------------------------------------------------------------------
# QMV family (a3-a9)
# ---------------------------------------------------------------------------

def qmv(w: fm.QWeight, x: np.ndarray, Wd: np.ndarray | None = None) -> np.ndarray:
    """y[r] = sum_c W[r,c] x[c] with W dequantised (cpuQMV,
    transformer_test.zig:303-330; kernel math compute.metal:2321-2478,
    qmv_specialized.metal:44-205, q4mv_bf16_specialized.metal:83-174)."""
    if Wd is None:
        Wd = dequant(w)
    return Wd @ np.asarray(x, dtype=np.float64)


def silu(g):
    """g / (1 + exp(-g)), qmv_specialized.metal:1077-1078."""
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g))


def qmv_pair_silu(wg: fm.QWeight, wu: fm.QWeight, x: np.ndarray) -> np.ndarray:
    """silu(Wg x) * (Wu x), qmv_specialized.metal:941-1081."""
    return silu(qmv(wg, x)) * qmv(wu, x)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * w per row (cpuRMSNorm,
    transformer_test.zig:72-103; transformer.metal:49-104)."""
    x = np.asarray(x, dtype=np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * np.asarray(w, dtype=np.float64)


def norm_to_half(residual: np.ndarray, w: np.ndarray, q4_faithful: bool = False,
                 eps: float = 1e-6) -> np.ndarray:
    """Fused-norm prologue: half(rmsnorm(residual) * w), with the Q4 path's
    extra BF16 truncation before narrowing (qmv_specialized.metal:1137-1177,
    q4mv_bf16_specialized.metal:800-807)."""
    v = rmsnorm(residual, w, eps)
    if q4_faithful:
        v = bf16_trunc(v)
    return f16(v)


# ---------------------------------------------------------------------------
# RoPE (a12)
# ---------------------------------------------------------------------------

def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """theta^(-2p/d) for each pair p, computed in double and rounded once to
    float32 (the GPU computes the same double expression on device)."""
    p = np.arange(head_dim // 2, dtype=np.float64)
    return np.exp2(-(2.0 * p / head_dim) * np.log2(np.float64(theta))).astype(np.float32)


def rope_angles(position: int, head_dim: int, theta: float) -> np.ndarray:
    """angle_p = f32(f32(pos) * inv_freq_p) -- one IEEE float32 multiply."""
    return (np.float32(position) * rope_inv_freq(head_dim, theta)).astype(np.float32)


def rope(x: np.ndarray, position: int, theta: float) -> np.ndarray:
    """Rotate consecutive pairs (x[2p], x[2p+1]) by angle_p (cpuRoPE,
    transformer_test.zig:128-156; transformer.metal:154-202).  ``x`` is
    [..., head_dim]."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1]
    ang = rope_angles(position, d, theta).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


# ---------------------------------------------------------------------------
# Attention (a10, a11)
# ---------------------------------------------------------------------------

def attention_decode(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     seq_len: int, v_transposed: bool) -> np.ndarray:
    """GQA decode attention for one query token (cpuAttentionHead,
    transformer_test.zig:179-226; transformer.metal:1597-1694).

    q: [Hq, D] (already normed/roped); k_cache: [Hkv, T, D];
    v_cache: [Hkv, D, T] if ``v_transposed`` (the reference's layout,
    transformer.metal:1092-1112) else [Hkv, T, D].  Returns [Hq, D] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    Hq, D = q.shape
    Hkv = k_cache.shape[0]
    g = Hq // Hkv
    out = np.empty((Hq, D))
    scale = 1.0 / np.sqrt(D)
    for h in range(Hq):
        kvh = h // g
        K = np.asarray(k_cache[kvh, :seq_len, :], dtype=np.float64)
        V = (np.asarray(v_cache[kvh, :, :seq_len], dtype=np.float64).T if v_transposed
             else np.asarray(v_cache[kvh, :seq_len, :], dtype=np.float64))
        s = K @ q[h] * scale
        s = np.exp(s - s.max())
        s /= s.sum()
        out[h] = s @ V
    return out


def head_norm_rope(x: np.ndarray, w: np.ndarray, position: int, theta: float,
                   eps: float = 1e-6) -> np.ndarray:
    """Per-head RMSNorm then RoPE (transformer.metal:1506-1572)."""
    return rope(rmsnorm(x, w, eps), position, theta)


def gqa_fused_step(q_raw, k_raw, v_raw, k_cache, v_cache, q_norm, k_norm,
                   position: int, theta: float, v_transposed: bool = True,
                   eps: float = 1e-6, kv_round=None):
    """gqa_attention_fused_f16io_tg (transformer.metal:1467-1695): q/k norm +
    RoPE, append k,v at ``position`` (stored with ``kv_round``), attend over
    positions 0..position.  Mutates the caches; returns [Hq, D] float64."""
    kv_round = kv_round or f16
    qn = head_norm_rope(q_raw, q_norm, position, theta, eps)
    kn = kv_round(head_norm_rope(k_raw, k_norm, position, theta, eps))
    k_cache[:, position, :] = kn
    if v_transposed:
        v_cache[:, :, position] = kv_round(v_raw)
    else:
        v_cache[:, position, :] = kv_round(v_raw)
    return attention_decode(qn, k_cache, v_cache, position + 1, v_transposed)


# ---------------------------------------------------------------------------
# Embedding (a14) and sampling (a17)
# ---------------------------------------------------------------------------

def embed_q1(token_ids, codes_bytes: np.ndarray, scales_f16: np.ndarray,
             hidden: int, gs: int) -> np.ndarray:
    """cpuEmbeddingDequant (transformer_test.zig:232-266): flat bit index
    row*hidden + d, scale group flat_bit / gs."""
    by = np.asarray(codes_bytes, dtype=np.uint8)
    sc = np.asarray(scales_f16, dtype=F16).astype(np.float64)
    out = np.empty((len(token_ids), hidden))
    for t, row in enumerate(token_ids):
        flat = row * hidden + np.arange(hidden)
        bit = (by[flat // 8] >> (flat % 8)) & 1
        s = sc[flat // gs]
        out[t] = np.where(bit == 1, s, -s)
    return out


def embed_q4(token_ids, codes_words: np.ndarray, scales_raw, biases_raw, hidden: int,
             gs: int, scale_dtype: int = fm.DT_BF16) -> np.ndarray:
    """embedding_lookup_q4 (transformer.metal:505-549): s*n+b, BF16-truncated."""
    wds = np.asarray(codes_words, dtype=np.uint32).reshape(-1)
    s_all = raw16_to_f64(np.asarray(scales_raw).reshape(-1), scale_dtype)
    b_all = raw16_to_f64(np.asarray(biases_raw).reshape(-1), scale_dtype)
    out = np.empty((len(token_ids), hidden))
    for t, row in enumerate(token_ids):
        flat = row * hidden + np.arange(hidden)
        n = ((wds[flat // 8] >> ((flat % 8) * 4).astype(np.uint32)) & 0xF).astype(np.float64)
        g = flat // gs
        out[t] = bf16_trunc((s_all[g] * n + b_all[g]).astype(np.float32))
    return out


def argmax_first(logits: np.ndarray) -> int:
    """First maximum wins (transformer.zig:3694-3707)."""
    return int(np.argmax(np.asarray(logits)))

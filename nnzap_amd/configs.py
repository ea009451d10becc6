"""The BASELINE.json workloads, built from the seeded generator in synth.py.

Config 1: 4-bit QMV   W[6144 x 2048] gs64, f16 scale U(0.005,0.02), f16 bias U(-0.1,0.1)
Config 2: 1-bit QMV   W[2048 x 6144] gs128, f16 scale U(0.01,0.05), bias = -scale/2
Config 3: fused gate/up + SiLU*mul, two [6144 x 2048] 1-bit matrices as config 2
Config 4: GQA decode attention, 16 q heads / 8 KV heads x 128, bf16 q/K/V ~N(0,1)
Config 5: Qwen3-1.7B-shaped decoder, all linears 1-bit gs128, bf16 embeddings/norms
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import synth as S
from .formats import (DT_BF16, DT_F16, QWeight, f16_bits, pack_q1, q1_affine_to_symmetric)


def q1_matrix(M: int, K: int, gs: int, code_seed: int, scale_seed: int,
              scale_lo: float = 0.01, scale_hi: float = 0.05,
              return_affine: bool = False):
    """1-bit matrix in MLX affine form (scale, bias = -scale/2), converted to
    the symmetric on-device form by the reference's load transform."""
    words = S.words(code_seed, M * K // 32).reshape(M, K // 32)
    scale = S.uniform(scale_seed, M * K // gs, scale_lo, scale_hi).astype(np.float16)
    bias = (-(scale.astype(np.float32) / np.float32(2.0))).astype(np.float16)
    sym = q1_affine_to_symmetric(scale, bias, check=True).reshape(M, K // gs)
    w = QWeight(1, M, K, gs, words, sym, None, DT_F16)
    if return_affine:
        return w, scale.reshape(M, K // gs), bias.reshape(M, K // gs)
    return w


def q4_matrix(M: int, K: int, gs: int, code_seed: int, scale_seed: int, bias_seed: int,
              scale_lo=0.005, scale_hi=0.02, bias_lo=-0.1, bias_hi=0.1,
              scale_dtype: int = DT_F16) -> QWeight:
    words = S.words(code_seed, M * K // 8).reshape(M, K // 8)  # 8 uniform nibbles per word
    G = M * K // gs
    s = S.uniform(scale_seed, G, scale_lo, scale_hi)
    b = S.uniform(bias_seed, G, bias_lo, bias_hi)
    if scale_dtype == DT_F16:
        sr, br = f16_bits(s), f16_bits(b)
    else:
        sr, br = S.f64_to_bf16_bits(s), S.f64_to_bf16_bits(b)
    return QWeight(4, M, K, gs, words, sr.reshape(M, K // gs), br.reshape(M, K // gs), scale_dtype)


def config1():
    x = S.normal(S.SEED_X, 2048).astype(np.float32)
    w = q4_matrix(6144, 2048, 64, S.SEED_CODES, S.SEED_SCALES, S.SEED_BIASES)
    return w, x


def config2(return_affine: bool = False):
    x = S.normal(S.SEED_X, 6144).astype(np.float32)
    w = q1_matrix(2048, 6144, 128, S.SEED_CODES, S.SEED_SCALES, return_affine=return_affine)
    return (w, x) if not return_affine else (w[0], x, w[1], w[2])


def config3():
    """Gate uses seeds (2, 3); up uses (12, 13)."""
    x = S.normal(S.SEED_X, 2048).astype(np.float32)
    wg = q1_matrix(6144, 2048, 128, S.SEED_CODES, S.SEED_SCALES)
    wu = q1_matrix(6144, 2048, 128, S.SEED_CODES + 10, S.SEED_SCALES + 10)
    return wg, wu, x


def config4(L: int, hq: int = 16, hkv: int = 8, d: int = 128):
    """q [hq, d], K and V [hkv, L, d] as raw bf16 bits (uint16)."""
    q = S.f64_to_bf16_bits(S.normal(S.SEED_Q, hq * d)).reshape(hq, d)
    k = S.f64_to_bf16_bits(S.normal(S.SEED_K, hkv * L * d)).reshape(hkv, L, d)
    v = S.f64_to_bf16_bits(S.normal(S.SEED_V, hkv * L * d)).reshape(hkv, L, d)
    return q, k, v


# ---------------------------------------------------------------------------
# Config 5: decoder
# ---------------------------------------------------------------------------

@dataclass
class DecoderConfig:
    vocab_size: int = 151936
    hidden_size: int = 2048
    intermediate_size: int = 6144
    num_layers: int = 28
    num_query_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    max_context_length: int = 1024
    max_prefill_length: int = 512
    group_size: int = 128
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6
    embed_kind: int = 1      # EMBED_BF16; 0 = EMBED_Q1, 2 = EMBED_Q4
    lm_head_kind: int = 0    # LMHEAD_Q1 (own 1-bit matrix); 1 = tied bf16 table; 2 = LMHEAD_Q4
    quant_format: int = 0    # 0 = q1_0 (1-bit), 1 = q4_mlx (4-bit affine, bf16 scales/biases)

    @property
    def qdim(self):
        return self.num_query_heads * self.head_dim

    @property
    def kvdim(self):
        return self.num_kv_heads * self.head_dim


BONSAI_1_7B = DecoderConfig()

# Tiny shape for CPU-oracle checks (every dim a multiple of 64 / group_size).
TINY = DecoderConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2,
                     num_query_heads=4, num_kv_heads=2, head_dim=64, max_context_length=256,
                     max_prefill_length=64, group_size=128, rope_theta=10000.0)

# The same tiny shape as a q4_mlx model (Bonsai*_Q4 presets,
# transformer.zig:336-382: group size 64, Q4 embedding tied to the LM head).
TINY_Q4 = DecoderConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2,
                        num_query_heads=4, num_kv_heads=2, head_dim=64, max_context_length=256,
                        max_prefill_length=64, group_size=64, rope_theta=10000.0,
                        embed_kind=2, lm_head_kind=2, quant_format=1)

PROJS = ("q", "k", "v", "o", "gate", "up", "down")


def proj_shape(cfg: DecoderConfig, name: str):
    H, I = cfg.hidden_size, cfg.intermediate_size
    return {"q": (cfg.qdim, H), "k": (cfg.kvdim, H), "v": (cfg.kvdim, H), "o": (H, cfg.qdim),
            "gate": (I, H), "up": (I, H), "down": (H, I)}[name]


def tensor_seed(layer: int, slot: int) -> int:
    """Seed of tensor ``slot`` of ``layer`` (model weights = 100 + tensor index)."""
    return S.SEED_MODEL_BASE + 64 * (layer + 1) + slot


@dataclass
class DecoderWeights:
    cfg: DecoderConfig
    embed_bf16: np.ndarray | None = None      # uint16 [V, H]
    embed_q1: QWeight | None = None           # quantised table (1-bit, or 4-bit for q4_mlx)
    lm_head: QWeight | None = None
    final_norm: np.ndarray | None = None      # f32 [H]
    layers: list = field(default_factory=list)  # dicts: q..down (QWeight), norms (f32)


def norm_weights(seed: int, n: int, mode: str) -> np.ndarray:
    """bf16 norm weights, widened to f32 at load (lossless, model.zig:1103-1167).
    mode "small": ~N(0, 0.02) literally; "unit": 1 + N(0, 0.02)."""
    z = 0.02 * S.normal(seed, n)
    if mode == "unit":
        z = 1.0 + z
    return S.bf16_bits_to_f32(S.f64_to_bf16_bits(z)).astype(np.float32)


def decoder_weights(cfg: DecoderConfig, norm_mode: str = "small",
                    host_embed: bool = True) -> DecoderWeights:
    """All weights of the synthetic decoder.  With ``host_embed=False`` the
    bf16 embedding table is left out (the GPU generates it from the same
    stream, nnz_synth_normal_bf16; the oracle regenerates single rows)."""
    dw = DecoderWeights(cfg)
    V, H = cfg.vocab_size, cfg.hidden_size
    if cfg.quant_format == 1:
        return _decoder_weights_q4(cfg, norm_mode)
    if host_embed or cfg.lm_head_kind == 1:
        dw.embed_bf16 = S.f64_to_bf16_bits(0.02 * S.normal(S.SEED_MODEL_BASE + 0, V * H)).reshape(V, H)
    if cfg.lm_head_kind == 0:
        dw.lm_head = q1_matrix(V, H, cfg.group_size, S.SEED_MODEL_BASE + 1, S.SEED_MODEL_BASE + 2)
    dw.final_norm = norm_weights(S.SEED_MODEL_BASE + 3, H, norm_mode)
    for l in range(cfg.num_layers):
        layer = {}
        for i, name in enumerate(PROJS):
            M, K = proj_shape(cfg, name)
            layer[name] = q1_matrix(M, K, cfg.group_size, tensor_seed(l, 2 * i),
                                    tensor_seed(l, 2 * i + 1))
        layer.update(layer_norm_weights(cfg, l, norm_mode))
        dw.layers.append(layer)
    return dw


def layer_norm_weights(cfg: DecoderConfig, l: int, norm_mode: str) -> dict:
    """The four norm vectors of 1-bit decoder layer ``l`` (the final norm
    is norm_weights(SEED_MODEL_BASE + 3, hidden, mode)).  Only these differ
    between the norm modes, so a loaded model switches mode by uploading
    them again."""
    H = cfg.hidden_size
    return {"attn_norm": norm_weights(tensor_seed(l, 20), H, norm_mode),
            "ffn_norm": norm_weights(tensor_seed(l, 21), H, norm_mode),
            "q_norm": norm_weights(tensor_seed(l, 22), cfg.head_dim, norm_mode),
            "k_norm": norm_weights(tensor_seed(l, 23), cfg.head_dim, norm_mode)}


def _decoder_weights_q4(cfg: DecoderConfig, norm_mode: str) -> DecoderWeights:
    """Synthetic q4_mlx decoder: every projection and the (tied) embedding a
    4-bit affine matrix with raw bf16 scales and biases."""
    dw = DecoderWeights(cfg)
    V, H, gs = cfg.vocab_size, cfg.hidden_size, cfg.group_size
    dw.embed_q1 = q4_matrix(V, H, gs, S.SEED_MODEL_BASE + 0, S.SEED_MODEL_BASE + 1,
                            S.SEED_MODEL_BASE + 2, scale_dtype=DT_BF16)
    dw.lm_head = dw.embed_q1
    dw.final_norm = norm_weights(S.SEED_MODEL_BASE + 3, H, norm_mode)
    for l in range(cfg.num_layers):
        layer = {}
        for i, name in enumerate(PROJS):
            M, K = proj_shape(cfg, name)
            layer[name] = q4_matrix(M, K, gs, tensor_seed(l, 3 * i), tensor_seed(l, 3 * i + 1),
                                    tensor_seed(l, 3 * i + 2), scale_dtype=DT_BF16)
        layer["attn_norm"] = norm_weights(tensor_seed(l, 40), H, norm_mode)
        layer["ffn_norm"] = norm_weights(tensor_seed(l, 41), H, norm_mode)
        layer["q_norm"] = norm_weights(tensor_seed(l, 42), cfg.head_dim, norm_mode)
        layer["k_norm"] = norm_weights(tensor_seed(l, 43), cfg.head_dim, norm_mode)
        dw.layers.append(layer)
    return dw


def prompt_ids(cfg: DecoderConfig, n: int) -> np.ndarray:
    return (S.u64(S.SEED_PROMPT, n) % np.uint64(cfg.vocab_size)).astype(np.uint32)

"""Synthetic MLX-format checkpoints for the loader tests.

Writes the tensors an MLX-quantised Qwen3 / Bonsai model directory holds
(names as nnmetal/src/model.zig:566-812 reads them), split over several
shards so every lookup has to search across files.  The affine pairs are
returned too, so tests can check the load transforms against the affine
definition ``w = scale * q + bias`` itself.
"""
import os

import numpy as np

from nnzap_amd import synth as S
from nnzap_amd.checkpoint import LAYER_NORM_NAMES, LAYER_PROJ_NAMES, layer_tensor_name
from nnzap_amd.configs import PROJS, proj_shape
from nnzap_amd.safetensors import save

SEED = 7000


def _affine(M, K, gs, bits, seed, bias_rule="exact"):
    n_words = M * K * bits // 32
    codes = S.words(seed, n_words).reshape(M, K * bits // 32)
    scale = S.uniform(seed + 1, M * K // gs, 0.01, 0.05).astype(np.float16).reshape(M, K // gs)
    if bits == 1:
        bias = (-(scale.astype(np.float32) / np.float32(2))).astype(np.float16)
        if bias_rule == "off":
            bias = bias.copy()
            bias.reshape(-1)[3] = np.float16(bias.reshape(-1)[3] * np.float16(1.5))
    else:
        bias = S.uniform(seed + 2, M * K // gs, -0.4, -0.1).astype(np.float16).reshape(M, K // gs)
    return codes, scale, bias


def _norm(seed, n, dtype):
    z = (1.0 + 0.02 * S.normal(seed, n))
    if dtype == "F32":
        return z.astype(np.float32)
    if dtype == "F16":
        return z.astype(np.float16)
    return ("BF16", S.f64_to_bf16_bits(z))


def write_mlx_checkpoint(dirpath, cfg, bits=1, tie=True, nshards=3, scale_dtype="F16",
                         bias_rule="exact"):
    """Write ``nshards`` files model-0000i-of-0000n.safetensors; returns a
    dict name -> (codes, scale, bias) of every quantised matrix and
    name -> raw norm value of every norm."""
    os.makedirs(dirpath, exist_ok=True)
    tensors, src = {}, {}
    seed = [SEED]

    def quant(prefix, M, K, codes_as_u8=False):
        codes, scale, bias = _affine(M, K, cfg.group_size, bits, seed[0], bias_rule)
        seed[0] += 4
        src[prefix] = (codes, scale, bias)
        w = codes.view(np.uint8).reshape(M, -1) if codes_as_u8 else codes
        tensors[prefix + ".weight"] = w
        if scale_dtype == "BF16":
            tensors[prefix + ".scales"] = ("BF16", S.f32_to_bf16_bits(scale.astype(np.float32)))
            tensors[prefix + ".biases"] = ("BF16", S.f32_to_bf16_bits(bias.astype(np.float32)))
        else:
            tensors[prefix + ".scales"] = scale
            tensors[prefix + ".biases"] = bias

    def norm(name, n, dtype):
        v = _norm(seed[0], n, dtype)
        seed[0] += 1
        src[name] = v
        tensors[name] = v

    V, H = cfg.vocab_size, cfg.hidden_size
    quant("model.embed_tokens", V, H)
    norm("model.norm.weight", H, "F16")
    if not tie:
        quant("lm_head", V, H)
    norm_dtypes = ("BF16", "F16", "F32")
    for l in range(cfg.num_layers):
        for i, name in enumerate(PROJS):
            M, K = proj_shape(cfg, name)
            quant(layer_tensor_name(l, LAYER_PROJ_NAMES[name], ""), M, K, codes_as_u8=(i == 2))
        for j, (key, comp) in enumerate(LAYER_NORM_NAMES.items()):
            n = cfg.head_dim if key in ("q_norm", "k_norm") else H
            norm(layer_tensor_name(l, comp, ".weight"), n, norm_dtypes[(l + j) % 3])
    names = list(tensors)
    for s in range(nshards):
        part = {n: tensors[n] for n in names[s::nshards]}
        save(os.path.join(dirpath, f"model-{s + 1:05d}-of-{nshards:05d}.safetensors"), part,
             metadata={"format": "mlx"})
    return src

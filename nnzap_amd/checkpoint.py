"""MLX-format Bonsai / Qwen3 checkpoints: safetensors shards -> DecoderWeights.

Mirrors nnmetal/src/model.zig:

* loadWeights (:196-242): every shard is opened first, each tensor is then
  found in whichever shard holds it (findTensorInFiles, :786-798);
* tensor names (:566-785, :799-812): ``model.embed_tokens.*``,
  ``model.norm.weight``, ``lm_head.*`` (untied models only) and
  ``model.layers.{i}.{component}{suffix}`` with components
  ``self_attn.{q,k,v,o}_proj``, ``mlp.{gate,up,down}_proj`` (suffixes
  ``.weight``, ``.scales``, ``.biases``) and the norms ``input_layernorm``,
  ``post_attention_layernorm``, ``self_attn.{q,k}_norm`` (``.weight``);
* 1-bit projections (loadPackedProjection, :911-960): the bit matrix is
  taken as stored (U8 or U32, LSB first), F16 scales become the symmetric
  half scale ``f16(f32(s) / 2)`` (convertScalesAffineToSymmetric,
  :1058-1070) and the MLX bias is not read;
* 4-bit projections (loadQ4Projection, :962-1026): nibbles as stored, F16 or
  BF16 scales and biases kept as raw BF16, F16 values truncated to BF16
  (copyRawBF16, :1169-1220);
* norms (loadNormScale, :1030-1056): F32 copied, F16/BF16 widened to F32.

Differences from the reference, all of them checks it does not make:
shapes and byte sizes must match the configuration exactly (the reference
asserts ``data.len >= needed`` and reads a prefix); with ``strict`` (the
default) a 1-bit group whose MLX bias is not exactly ``-scale/2`` is an
error, since dropping the bias is lossless only then -- ``strict=False``
drops it anyway, as the reference does.
"""
from __future__ import annotations

import json
import os
from contextlib import ExitStack

import numpy as np

from . import formats as fm
from .configs import PROJS, DecoderConfig, DecoderWeights, proj_shape
from .safetensors import SafetensorsError, SafetensorsFile, TensorDescriptor, find_tensor

QUANT_Q1 = "q1"
QUANT_Q4 = "q4_mlx"

LAYER_PROJ_NAMES = {"q": "self_attn.q_proj", "k": "self_attn.k_proj",
                    "v": "self_attn.v_proj", "o": "self_attn.o_proj",
                    "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
LAYER_NORM_NAMES = {"attn_norm": "input_layernorm", "ffn_norm": "post_attention_layernorm",
                    "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm"}

MAX_SHARDS = 16


def layer_tensor_name(layer: int, component: str, suffix: str) -> str:
    """formatLayerTensorName (model.zig:799-812)."""
    return f"model.layers.{layer}.{component}{suffix}"


def find_shards(model_dir: str | os.PathLike) -> list[str]:
    """Every ``*.safetensors`` file of ``model_dir``, sorted by name
    (findSafetensorShards, nnmetal/examples/bonsai_bench.zig:557-630)."""
    names = sorted(n for n in os.listdir(model_dir) if n.endswith(".safetensors"))
    if not names:
        raise SafetensorsError("NoSafetensorFiles", f"no .safetensors files in {model_dir}")
    if len(names) > MAX_SHARDS:
        raise SafetensorsError("TooManyShards", f"too many shards (max {MAX_SHARDS})")
    return [os.path.join(model_dir, n) for n in names]


def _bytes_of(desc: TensorDescriptor, what: str, nbytes: int, dtypes) -> np.ndarray:
    if desc.dtype not in dtypes:
        raise SafetensorsError("UnsupportedDtype",
                               f"{desc.name}: {desc.dtype} (want one of {sorted(dtypes)}) for {what}")
    if desc.size_bytes() != nbytes or len(desc.data) != nbytes:
        raise SafetensorsError("ShapeMismatch",
                               f"{desc.name}: {len(desc.data)} bytes, shape {desc.shape}; "
                               f"{nbytes} bytes expected for {what}")
    return np.frombuffer(desc.data, dtype=np.uint8)


def _raw16(desc: TensorDescriptor, n: int, what: str, dtypes) -> np.ndarray:
    return _bytes_of(desc, what, 2 * n, dtypes).view("<u2")


def q1_projection(weight: TensorDescriptor, scales: TensorDescriptor,
                  biases: TensorDescriptor | None, M: int, K: int, gs: int,
                  strict: bool = True) -> fm.QWeight:
    """loadPackedProjection: bits as stored, scales halved (f16)."""
    if K % 32 or K % gs:
        raise SafetensorsError("ShapeMismatch", f"{weight.name}: K={K} vs group {gs}")
    codes = _bytes_of(weight, f"[{M}x{K}] 1-bit codes", M * K // 8, {"U8", "U32"})
    ng = M * (K // gs)
    s = _raw16(scales, ng, "f16 group scales", {"F16"}).view(np.float16)
    b = None
    if strict and biases is not None:
        b = _raw16(biases, ng, "f16 group biases", {"F16"}).view(np.float16)
    try:
        half = fm.q1_affine_to_symmetric(s, b, check=b is not None)
    except ValueError as e:
        raise SafetensorsError("InexactAffine", f"{weight.name}: {e}") from None
    return fm.QWeight(1, M, K, gs, codes.view("<u4").reshape(M, K // 32),
                      half.reshape(M, K // gs), None, fm.DT_F16)


def _bf16_raw(desc: TensorDescriptor, n: int, what: str) -> np.ndarray:
    """copyRawBF16 (model.zig:1169-1220) for the F16 / BF16 sources the 4-bit
    loader accepts (model.zig:974-986)."""
    raw = _raw16(desc, n, what, {"F16", "BF16"})
    if desc.dtype == "BF16":
        return raw
    return fm.to_bf16_truncate(raw.view(np.float16))


def q4_projection(weight: TensorDescriptor, scales: TensorDescriptor,
                  biases: TensorDescriptor, M: int, K: int, gs: int) -> fm.QWeight:
    """loadQ4Projection: nibbles as stored, scales/biases as raw BF16."""
    if K % 8 or K % gs:
        raise SafetensorsError("ShapeMismatch", f"{weight.name}: K={K} vs group {gs}")
    codes = _bytes_of(weight, f"[{M}x{K}] 4-bit codes", M * K // 2, {"U8", "U32"})
    ng = M * (K // gs)
    s = _bf16_raw(scales, ng, "group scales").reshape(M, K // gs)
    b = _bf16_raw(biases, ng, "group biases").reshape(M, K // gs)
    return fm.QWeight(4, M, K, gs, codes.view("<u4").reshape(M, K // 8), s, b, fm.DT_BF16)


def norm_scale(desc: TensorDescriptor, n: int) -> np.ndarray:
    """loadNormScale (model.zig:1030-1056) + copyOrConvertF32 (:1130-1167)."""
    if desc.dtype == "F32":
        return _bytes_of(desc, f"f32 norm [{n}]", 4 * n, {"F32"}).view("<f4")
    raw = _raw16(desc, n, f"norm [{n}]", {"F16", "BF16"})
    if desc.dtype == "F16":
        return raw.view(np.float16).astype(np.float32)
    return (raw.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _projection(files, prefix: str, M: int, K: int, cfg_gs: int, quant: str, strict: bool):
    w = find_tensor(files, prefix + ".weight")
    s = find_tensor(files, prefix + ".scales")
    if quant == QUANT_Q4:
        return q4_projection(w, s, find_tensor(files, prefix + ".biases"), M, K, cfg_gs)
    b = None
    if strict:
        for f in files:
            b = f.get_tensor(prefix + ".biases")
            if b is not None:
                break
    return q1_projection(w, s, b, M, K, cfg_gs, strict)


def read_weights(files, cfg: DecoderConfig, quant: str = QUANT_Q1,
                 tie_word_embeddings: bool = True, strict: bool = True) -> DecoderWeights:
    """Build DecoderWeights from opened shards (loadWeights, model.zig:196-242).

    Arrays are zero-copy views into the mapped shards: keep ``files`` open
    until the weights are uploaded, or use :func:`load_checkpoint`, which
    copies.  The embedding table is a quantised matrix like every projection;
    with tied embeddings the LM head is that same matrix.
    """
    if quant not in (QUANT_Q1, QUANT_Q4):
        raise ValueError(f"quant must be {QUANT_Q1!r} or {QUANT_Q4!r}")
    V, H, gs = cfg.vocab_size, cfg.hidden_size, cfg.group_size
    dw = DecoderWeights(cfg)
    dw.embed_q1 = _projection(files, "model.embed_tokens", V, H, gs, quant, strict)
    dw.final_norm = norm_scale(find_tensor(files, "model.norm.weight"), H)
    dw.lm_head = dw.embed_q1 if tie_word_embeddings else \
        _projection(files, "lm_head", V, H, gs, quant, strict)
    for l in range(cfg.num_layers):
        layer = {}
        for name in PROJS:
            M, K = proj_shape(cfg, name)
            layer[name] = _projection(files, layer_tensor_name(l, LAYER_PROJ_NAMES[name], ""),
                                      M, K, gs, quant, strict)
        for key, comp in LAYER_NORM_NAMES.items():
            n = cfg.head_dim if key in ("q_norm", "k_norm") else H
            layer[key] = norm_scale(find_tensor(files, layer_tensor_name(l, comp, ".weight")), n)
        dw.layers.append(layer)
    return dw


def _copy_q(w: fm.QWeight) -> fm.QWeight:
    return fm.QWeight(w.bits, w.M, w.K, w.group_size, np.array(w.codes), np.array(w.scales),
                      None if w.biases is None else np.array(w.biases), w.scale_dtype)


def load_checkpoint(paths, cfg: DecoderConfig, quant: str = QUANT_Q1,
                    tie_word_embeddings: bool = True, strict: bool = True) -> DecoderWeights:
    """Open ``paths`` (shard files, or one model directory), read every
    tensor the configuration needs and return owned copies."""
    if isinstance(paths, (str, os.PathLike)):
        paths = find_shards(paths) if os.path.isdir(paths) else [paths]
    with ExitStack() as stack:
        files = [stack.enter_context(SafetensorsFile.open(p)) for p in paths]
        dw = read_weights(files, cfg, quant, tie_word_embeddings, strict)
        out = DecoderWeights(cfg)
        out.embed_q1 = _copy_q(dw.embed_q1)
        out.lm_head = out.embed_q1 if dw.lm_head is dw.embed_q1 else _copy_q(dw.lm_head)
        out.final_norm = np.array(dw.final_norm)
        out.layers = [{k: (_copy_q(v) if isinstance(v, fm.QWeight) else np.array(v))
                       for k, v in layer.items()} for layer in dw.layers]
        del dw
    return out


def config_from_hf(config: dict | str | os.PathLike, max_context_length: int = 32768,
                   max_prefill_length: int = 512) -> tuple[DecoderConfig, str, bool]:
    """(DecoderConfig, quant, tie_word_embeddings) from a Hugging Face /
    MLX ``config.json`` (a dict, the file, or its model directory).  The
    reference fixes these values at compile time instead
    (nnmetal/src/transformer.zig:284-360); this reads the same fields."""
    if not isinstance(config, dict):
        p = os.fspath(config)
        if os.path.isdir(p):
            p = os.path.join(p, "config.json")
        with open(p, encoding="utf-8") as f:
            config = json.load(f)
    q = config.get("quantization") or config.get("quantization_config") or {}
    bits = int(q.get("bits", 1))
    if bits not in (1, 4):
        raise ValueError(f"unsupported quantisation: {bits} bits")
    heads = int(config["num_attention_heads"])
    hidden = int(config["hidden_size"])
    cfg = DecoderConfig(
        vocab_size=int(config["vocab_size"]), hidden_size=hidden,
        intermediate_size=int(config["intermediate_size"]),
        num_layers=int(config["num_hidden_layers"]), num_query_heads=heads,
        num_kv_heads=int(config.get("num_key_value_heads", heads)),
        head_dim=int(config.get("head_dim", hidden // heads)),
        max_context_length=max_context_length, max_prefill_length=max_prefill_length,
        group_size=int(q.get("group_size", 128 if bits == 1 else 64)),
        rope_theta=float(config.get("rope_theta", 1e6)),
        rms_eps=float(config.get("rms_norm_eps", 1e-6)),
        embed_kind=0 if bits == 1 else 2, lm_head_kind=0 if bits == 1 else 2,
        quant_format=0 if bits == 1 else 1)
    return cfg, (QUANT_Q1 if bits == 1 else QUANT_Q4), bool(config.get("tie_word_embeddings", True))

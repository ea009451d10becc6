"""Safetensors reader and MLX checkpoint loader (CPU).

The first six tests restate nnmetal/src/safetensors_test.zig case by case
(same headers, same expected descriptors and errors).  The loader tests
write synthetic MLX-format shards and pin the load transforms against the
affine definition ``w = scale * q + bias`` rather than against the
transform's own formula: the 1-bit symmetric form must reproduce it exactly
(model.zig:911-960, :1058-1070), the 4-bit form must equal it with scale
and bias truncated to BF16 (model.zig:962-1026, :1169-1220).
"""
import json
import os
import struct

import numpy as np
import pytest

from nnzap_amd import checkpoint as ck
from nnzap_amd import configs as cf
from nnzap_amd import formats as fm
from nnzap_amd import safetensors as st
from nnzap_amd import synth as S
from oracle import oracle as O

from ckpt_util import write_mlx_checkpoint


def build(json_str: str, data_size: int) -> bytes:
    """buildTestFile (safetensors_test.zig:8-32): u64 LE length, header,
    zero-filled data region."""
    h = json_str.encode()
    return struct.pack("<Q", len(h)) + h + bytes(data_size)


# -- safetensors_test.zig ------------------------------------------------------

def test_parse_header_from_bytes():
    sf = st.SafetensorsFile.from_bytes(build(
        '{"tensor_a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]}}', 24))
    assert sf.count == 1
    d = sf.tensors[0]
    assert d.name == "tensor_a" and d.dtype == "F32"
    assert d.rank == 2 and d.shape == (2, 3)
    assert len(d.data) == 24
    assert d.element_count() == 6 and d.size_bytes() == 24


def test_get_tensor_returns_correct_descriptor():
    sf = st.SafetensorsFile.from_bytes(build(
        '{"weight": {"dtype": "F16", "shape": [4],\n"data_offsets": [0, 8]},\n'
        '"bias": {"dtype": "F32", "shape": [2],\n"data_offsets": [8, 16]}}', 16))
    assert sf.count == 2
    bias = sf.get_tensor("bias")
    assert bias.name == "bias" and bias.dtype == "F32" and bias.rank == 1
    assert bias.shape == (2,) and len(bias.data) == 8
    weight = sf.get_tensor("weight")
    assert weight.name == "weight" and weight.dtype == "F16"
    assert sf.get_tensor("nonexistent") is None


def test_data_offsets_are_validated():
    with pytest.raises(st.SafetensorsError) as e:
        st.SafetensorsFile.from_bytes(build(
            '{"bad": {"dtype": "F32", "shape": [2], "data_offsets": [0, 999]}}', 24))
    assert e.value.kind == "DataOffsetOutOfBounds"


def test_metadata_key_is_skipped():
    sf = st.SafetensorsFile.from_bytes(build(
        '{"real_tensor": {"dtype": "U8", "shape": [4],\n"data_offsets": [0, 4]},\n'
        '"__metadata__": {"format": "test",\n"version": "1.0"}}', 4))
    assert sf.count == 1
    assert sf.tensors[0].name == "real_tensor" and sf.tensors[0].dtype == "U8"
    assert sf.get_tensor("__metadata__") is None
    assert sf.metadata == {"format": "test", "version": "1.0"}


def test_dtype_from_string_round_trips():
    for s in ("U8", "F16", "F32", "BF16"):
        assert st.dtype_from_string(s) == s
    with pytest.raises(st.SafetensorsError) as e:
        st.dtype_from_string("I32")
    assert e.value.kind == "UnsupportedDtype"


def test_dtype_size_bytes():
    assert [st.dtype_size(s) for s in ("U8", "F16", "BF16", "F32", "U32")] == [1, 2, 2, 4, 4]


# -- the rest of the parser's error paths (safetensors.zig:226-572) ------------

@pytest.mark.parametrize("header,size,kind", [
    ('{"a": {"dtype": "F32", "shape": [2], "data_offsets": [8, 4]}}', 8, "InvalidDataOffsets"),
    ('{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0]}}', 8, "InvalidDataOffsets"),
    ('{"a": {"dtype": "F32", "shape": [2], "data_offsets": [-1, 4]}}', 8, "InvalidDataOffsets"),
    ('{"a": {"dtype": "F32", "shape": [2]}}', 8, "MissingDataOffsets"),
    ('{"a": {"shape": [2], "data_offsets": [0, 8]}}', 8, "MissingDtype"),
    ('{"a": {"dtype": 3, "shape": [2], "data_offsets": [0, 8]}}', 8, "InvalidDtype"),
    ('{"a": {"dtype": "I64", "shape": [1], "data_offsets": [0, 8]}}', 8, "UnsupportedDtype"),
    ('{"a": {"dtype": "F32", "data_offsets": [0, 8]}}', 8, "MissingShape"),
    ('{"a": {"dtype": "F32", "shape": [1,1,1,1,2], "data_offsets": [0, 8]}}', 8,
     "TooManyDimensions"),
    ('{"a": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}', 8, "InvalidShape"),
    ('{"a": {"dtype": "F32", "shape": [2.5], "data_offsets": [0, 8]}}', 8, "InvalidShape"),
    ('{"a": {"dtype": "F32", "shape": 2, "data_offsets": [0, 8]}}', 8, "InvalidShape"),
    ('{"a": [1, 2]}', 8, "InvalidTensorEntry"),
    ('[1, 2]', 8, "InvalidJson"),
    ('{"a": ', 8, "InvalidJson"),
])
def test_header_errors(header, size, kind):
    with pytest.raises(st.SafetensorsError) as e:
        st.SafetensorsFile.from_bytes(build(header, size))
    assert e.value.kind == kind


def test_header_length_beyond_file():
    b = bytearray(build('{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1))
    b[0:8] = struct.pack("<Q", len(b))
    with pytest.raises(st.SafetensorsError) as e:
        st.SafetensorsFile.from_bytes(bytes(b))
    assert e.value.kind == "InvalidHeader"
    b[0:8] = struct.pack("<Q", st.MAX_HEADER_BYTES + 1)
    with pytest.raises(st.SafetensorsError) as e:
        st.SafetensorsFile.from_bytes(bytes(b))
    assert e.value.kind == "InvalidHeader"


def test_too_many_tensors():
    ok = {f"t{i}": {"dtype": "U8", "shape": [1], "data_offsets": [i, i + 1]}
          for i in range(st.MAX_TENSORS)}
    assert st.SafetensorsFile.from_bytes(build(json.dumps(ok), st.MAX_TENSORS)).count == \
        st.MAX_TENSORS
    ok["extra"] = {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}
    with pytest.raises(st.SafetensorsError) as e:
        st.SafetensorsFile.from_bytes(build(json.dumps(ok), st.MAX_TENSORS))
    assert e.value.kind == "TooManyTensors"


def test_save_then_mmap_round_trip(tmp_path):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.arange(6, dtype=np.float16)
    c = np.array([1, 2, 3], dtype=np.uint8)
    d = ("BF16", np.array([0x3F80, 0xC000], dtype=np.uint16))
    e = np.array([7, 0xFFFFFFFF], dtype=np.uint32)
    p = tmp_path / "x.safetensors"
    st.save(p, {"a": a, "b": b, "c": c, "d": d, "e": e}, metadata={"k": "v"})
    raw = p.read_bytes()
    (hlen,) = struct.unpack_from("<Q", raw)
    assert (8 + hlen) % 8 == 0
    with st.SafetensorsFile.open(p) as sf:
        assert sf.names() == ["a", "b", "c", "d", "e"] and sf.metadata == {"k": "v"}
        np.testing.assert_array_equal(sf.get_tensor("a").array(), a)
        np.testing.assert_array_equal(sf.get_tensor("b").array(), b)
        np.testing.assert_array_equal(sf.get_tensor("c").array(), c)
        assert sf.get_tensor("d").dtype == "BF16"
        np.testing.assert_array_equal(sf.get_tensor("d").array(), d[1])
        np.testing.assert_array_equal(sf.get_tensor("e").array(), e)


# -- MLX checkpoint loader -----------------------------------------------------

CFG = cf.DecoderConfig(vocab_size=500, hidden_size=256, intermediate_size=512, num_layers=2,
                       num_query_heads=4, num_kv_heads=2, head_dim=64, max_context_length=256,
                       max_prefill_length=64, group_size=128, rope_theta=10000.0,
                       embed_kind=0, lm_head_kind=0)


def _bf16_trunc_f64(x_f16):
    f = np.asarray(x_f16, dtype=np.float16).astype(np.float32)
    return (f.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)


def test_find_shards_sorted(tmp_path):
    with pytest.raises(st.SafetensorsError) as e:
        ck.find_shards(tmp_path)
    assert e.value.kind == "NoSafetensorFiles"
    for n in ("b.safetensors", "a.safetensors", "c.txt"):
        (tmp_path / n).write_bytes(b"")
    assert [os.path.basename(p) for p in ck.find_shards(tmp_path)] == \
        ["a.safetensors", "b.safetensors"]


@pytest.fixture(scope="module")
def q1_ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("q1")
    src = write_mlx_checkpoint(d, CFG, bits=1, tie=True)
    return d, src


def test_q1_checkpoint_matches_affine_definition(q1_ckpt):
    d, src = q1_ckpt
    w = ck.load_checkpoint(d, CFG)
    assert w.lm_head is w.embed_q1
    mats = [("model.embed_tokens", w.embed_q1)]
    for l, layer in enumerate(w.layers):
        for name in cf.PROJS:
            mats.append((ck.layer_tensor_name(l, ck.LAYER_PROJ_NAMES[name], ""), layer[name]))
    assert len(mats) == 1 + 7 * CFG.num_layers
    for prefix, q in mats:
        codes, scale, bias = src[prefix]
        assert q.bits == 1 and q.scale_dtype == fm.DT_F16
        np.testing.assert_array_equal(q.codes, codes, err_msg=prefix)
        # symmetric +-s' reproduces scale*bit + bias exactly
        aff = O.dequant_q1_affine(codes, scale, bias, q.M, q.K, q.group_size)
        np.testing.assert_array_equal(O.dequant_q1(q), aff, err_msg=prefix)


def test_norms_widened_exactly(q1_ckpt):
    d, src = q1_ckpt
    w = ck.load_checkpoint(d, CFG)
    for l, layer in enumerate(w.layers):
        for key, comp in ck.LAYER_NORM_NAMES.items():
            v = src[ck.layer_tensor_name(l, comp, ".weight")]
            want = (S.bf16_bits_to_f32(v[1]) if isinstance(v, tuple)
                    else np.asarray(v).astype(np.float32))
            assert layer[key].dtype == np.float32
            np.testing.assert_array_equal(layer[key], want)
    np.testing.assert_array_equal(w.final_norm, src["model.norm.weight"].astype(np.float32))


def test_embedding_rows_match_oracle_lookup(q1_ckpt):
    d, src = q1_ckpt
    w = ck.load_checkpoint(d, CFG)
    codes, scale, bias = src["model.embed_tokens"]
    ids = [0, 17, 499]
    aff = O.dequant_q1_affine(codes, scale, bias, CFG.vocab_size, CFG.hidden_size,
                              CFG.group_size)[ids]
    got = O.embed_q1(ids, w.embed_q1.codes.view(np.uint8).reshape(-1),
                     w.embed_q1.scales.view(np.float16).reshape(-1), CFG.hidden_size,
                     CFG.group_size)
    np.testing.assert_array_equal(got, aff)


def test_q1_inexact_bias_rejected_unless_lenient(tmp_path):
    small = cf.DecoderConfig(**{**CFG.__dict__, "num_layers": 1})
    write_mlx_checkpoint(tmp_path, small, bits=1, bias_rule="off")
    with pytest.raises(st.SafetensorsError) as e:
        ck.load_checkpoint(tmp_path, small)
    assert e.value.kind == "InexactAffine"
    w = ck.load_checkpoint(tmp_path, small, strict=False)   # the reference's behaviour
    assert w.embed_q1.bits == 1


@pytest.mark.parametrize("scale_dtype", ["F16", "BF16"])
def test_q4_checkpoint_bf16_truncation(tmp_path, scale_dtype):
    cfg = cf.DecoderConfig(**{**CFG.__dict__, "num_layers": 1, "group_size": 64})
    src = write_mlx_checkpoint(tmp_path, cfg, bits=4, tie=False, scale_dtype=scale_dtype)
    w = ck.load_checkpoint(tmp_path, cfg, quant=ck.QUANT_Q4, tie_word_embeddings=False)
    assert w.lm_head is not w.embed_q1
    for prefix, q in [("model.embed_tokens", w.embed_q1), ("lm_head", w.lm_head),
                      ("model.layers.0.mlp.down_proj", w.layers[0]["down"]),
                      ("model.layers.0.self_attn.v_proj", w.layers[0]["v"])]:
        codes, scale, bias = src[prefix]
        assert q.bits == 4 and q.scale_dtype == fm.DT_BF16
        np.testing.assert_array_equal(q.codes, codes, err_msg=prefix)
        n = fm.unpack_q4(codes, q.K).astype(np.float64)
        s = np.repeat(_bf16_trunc_f64(scale), q.group_size, axis=1)
        b = np.repeat(_bf16_trunc_f64(bias), q.group_size, axis=1)
        if scale_dtype == "BF16":   # stored bf16 bits are taken unchanged
            s = np.repeat(S.bf16_bits_to_f32(S.f32_to_bf16_bits(scale.astype(np.float32)))
                          .astype(np.float64), q.group_size, axis=1)
            b = np.repeat(S.bf16_bits_to_f32(S.f32_to_bf16_bits(bias.astype(np.float32)))
                          .astype(np.float64), q.group_size, axis=1)
        want = (s * n + b).astype(np.float32).astype(np.float64)
        np.testing.assert_array_equal(O.dequant_q4(q), want, err_msg=prefix)


def test_loader_errors(tmp_path, q1_ckpt):
    d, _ = q1_ckpt
    # a layer the checkpoint does not have
    more = cf.DecoderConfig(**{**CFG.__dict__, "num_layers": 3})
    with pytest.raises(st.SafetensorsError) as e:
        ck.load_checkpoint(d, more)
    assert e.value.kind == "TensorNotFound" and "model.layers.2." in str(e.value)
    # a shape that disagrees with the configuration
    wide = cf.DecoderConfig(**{**CFG.__dict__, "intermediate_size": 640})
    with pytest.raises(st.SafetensorsError) as e:
        ck.load_checkpoint(d, wide)
    assert e.value.kind == "ShapeMismatch"
    # 1-bit scales must be F16 (model.zig:919)
    p = tmp_path / "bad.safetensors"
    st.save(p, {"model.embed_tokens.weight": np.zeros((4, 4), np.uint32),
                "model.embed_tokens.scales": ("BF16", np.zeros((4, 1), np.uint16))})
    with st.SafetensorsFile.open(p) as f:
        with pytest.raises(st.SafetensorsError) as e:
            ck._projection([f], "model.embed_tokens", 4, 128, 128, ck.QUANT_Q1, False)
    assert e.value.kind == "UnsupportedDtype"


def test_config_from_hf(tmp_path):
    cfg_json = {"vocab_size": 151669, "hidden_size": 2048, "intermediate_size": 6144,
                "num_hidden_layers": 28, "num_attention_heads": 16, "num_key_value_heads": 8,
                "head_dim": 128, "rope_theta": 1000000.0, "rms_norm_eps": 1e-6,
                "tie_word_embeddings": True, "quantization": {"group_size": 128, "bits": 1}}
    (tmp_path / "config.json").write_text(json.dumps(cfg_json))
    cfg, quant, tie = ck.config_from_hf(tmp_path)
    # the reference's compile-time Bonsai1_7B (transformer.zig:284-296)
    assert (cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_layers) == \
        (151669, 2048, 6144, 28)
    assert (cfg.num_query_heads, cfg.num_kv_heads, cfg.head_dim, cfg.group_size) == \
        (16, 8, 128, 128)
    assert cfg.rope_theta == 1e6 and quant == ck.QUANT_Q1 and tie
    assert cfg.embed_kind == 0 and cfg.lm_head_kind == 0
    cfg_json["quantization"] = {"group_size": 64, "bits": 4}
    cfg_json["vocab_size"] = 151936
    cfg4, quant4, _ = ck.config_from_hf(cfg_json)
    assert quant4 == ck.QUANT_Q4 and cfg4.group_size == 64
    assert (cfg4.embed_kind, cfg4.lm_head_kind, cfg4.quant_format) == (2, 2, 1)

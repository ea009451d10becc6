"""ctypes binding of include/nnz.h (the C ABI of libnnzap_amd.so).

The library is loaded from the package directory only; if it is missing the
import of anything that needs it raises -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libnnzap_amd.so"
HEADER = HERE.parent / "include" / "nnz.h"

OK, EINVAL, EUNSUPPORTED, EHIP, ENOMEM, ETIMEOUT, ESTATE = 0, -1, -2, -3, -4, -5, -6
F32, F16, BF16 = 0, 1, 2
GEMM_STORE_F16, GEMM_STORE_F32, GEMM_RESADD, GEMM_SILU_PAIR = 0, 1, 2, 3
GQA_NOALLOC_MAX_BYTES = 8 << 20   # NNZ_GQA_NOALLOC_MAX_BYTES
EMBED_Q1, EMBED_BF16, EMBED_Q4 = 0, 1, 2
LMHEAD_Q1, LMHEAD_TIED_BF16, LMHEAD_Q4 = 0, 1, 2
OPT_Q1_MATRIX_CORES = 1
QUANT_FORMAT_Q1, QUANT_FORMAT_Q4 = 0, 1

u32, f32, vp, i32, sz = C.c_uint32, C.c_float, C.c_void_p, C.c_int32, C.c_size_t


class QMVDims(C.Structure):
    _fields_ = [("M", u32), ("K", u32), ("group_size", u32)]


class RMSNormDims(C.Structure):
    _fields_ = [("hidden_size", u32), ("num_tokens", u32), ("eps", f32)]


class RoPEDims(C.Structure):
    _fields_ = [("num_heads", u32), ("head_dim", u32), ("position", u32), ("rope_theta", f32)]


class KVUpdateDims(C.Structure):
    _fields_ = [("num_kv_heads", u32), ("head_dim", u32), ("position", u32),
                ("max_context_length", u32)]


class FusedRoPEKVDims(C.Structure):
    _fields_ = [("num_kv_heads", u32), ("head_dim", u32), ("position", u32),
                ("max_context_length", u32), ("rope_theta", f32)]


class FusedNormRoPEDims(C.Structure):
    _fields_ = [("num_heads", u32), ("head_dim", u32), ("position", u32), ("eps", f32),
                ("rope_theta", f32)]


class FusedKNormRoPEKVDims(C.Structure):
    _fields_ = [("num_kv_heads", u32), ("head_dim", u32), ("position", u32),
                ("max_context_length", u32), ("eps", f32), ("rope_theta", f32)]


class GQADims(C.Structure):
    _fields_ = [("num_query_heads", u32), ("num_kv_heads", u32), ("head_dim", u32),
                ("seq_len", u32), ("max_context_length", u32), ("heads_per_kv_group", u32)]


class GQAFusedDims(C.Structure):
    _fields_ = [("num_query_heads", u32), ("num_kv_heads", u32), ("head_dim", u32),
                ("seq_len", u32), ("max_context_length", u32), ("heads_per_kv_group", u32),
                ("position", u32), ("eps", f32), ("rope_theta", f32)]


class EmbedDims(C.Structure):
    _fields_ = [("vocab_size", u32), ("hidden_size", u32), ("num_tokens", u32),
                ("group_size", u32)]


class QWeightDesc(C.Structure):
    _fields_ = [("codes", vp), ("scales", vp), ("biases", vp), ("packed_count", u32),
                ("group_size", u32), ("bits", u32), ("scale_dtype", u32)]


class QmvStack(C.Structure):
    """nnz_qmv_stack: `count` matrices at fixed byte strides (stacked launch)."""
    _fields_ = [("count", u32), ("blocks_per_matrix", u32), ("codes_stride", C.c_uint64),
                ("scales_stride", C.c_uint64), ("input_stride", C.c_uint64),
                ("output_stride", C.c_uint64)]


class SamplingParams(C.Structure):
    """nnz_sampling_params (SamplingParams, transformer.zig:3652-3657)."""
    _fields_ = [("temperature", f32), ("top_k", u32), ("top_p", f32), ("reserved", u32),
                ("seed", C.c_uint64)]


class ModelConfig(C.Structure):
    _fields_ = [("vocab_size", u32), ("hidden_size", u32), ("intermediate_size", u32),
                ("num_layers", u32), ("num_query_heads", u32), ("num_kv_heads", u32),
                ("head_dim", u32), ("max_context_length", u32), ("max_prefill_length", u32),
                ("group_size", u32), ("rope_theta", f32), ("rms_eps", f32),
                ("embed_kind", u32), ("lm_head_kind", u32), ("quant_format", u32)]


P = C.POINTER
QW = P(QWeightDesc)

# name -> (restype, argtypes)
PROTOS = {
    "nnz_version": (C.c_char_p, []),
    "nnz_ctx_create": (C.c_int, [C.c_int, vp, P(vp)]),
    "nnz_ctx_destroy": (C.c_int, [vp]),
    "nnz_ctx_stream": (vp, [vp]),
    "nnz_last_error": (C.c_char_p, [vp]),
    "nnz_alloc": (C.c_int, [vp, sz, P(vp)]),
    "nnz_free": (C.c_int, [vp, vp]),
    "nnz_upload": (C.c_int, [vp, vp, vp, sz]),
    "nnz_download": (C.c_int, [vp, vp, vp, sz]),
    "nnz_stream_sync": (C.c_int, [vp, u32]),
    "nnz_graph_begin": (C.c_int, [vp]),
    "nnz_graph_end": (C.c_int, [vp, P(vp)]),
    "nnz_graph_replay": (C.c_int, [vp, vp]),
    "nnz_graph_destroy": (C.c_int, [vp]),
    "nnz_ctx_set_option": (C.c_int, [vp, C.c_int, C.c_int]),
    "nnz_timer_mark": (C.c_int, [vp, C.c_int]),
    "nnz_timer_elapsed_ms": (C.c_int, [vp, C.c_int, C.c_int, P(f32)]),
    # Q1
    "nnz_dispatch_qmv": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_f16in": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_f16io": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_f16io_resadd": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_fused_pair": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_fused_pair_f16in": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_fused_pair_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_fused_pair_silu_f16io": (C.c_int, [vp, QW, QW, vp, vp, QMVDims]),
    "nnz_dispatch_qmv_fused_pair_silu": (C.c_int, [vp, QW, QW, vp, vp, QMVDims]),
    "nnz_dispatch_fused_norm_pair_silu_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_fused_norm_qmv_f16io": (C.c_int, [vp, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_fused_norm_pair_qmv_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, vp, QMVDims]),
    "nnz_dispatch_fused_norm_qkv_f16io": (C.c_int, [vp, QW, QW, QW, vp, vp, vp, vp, vp, QMVDims,
                                                    u32]),
    "nnz_dispatch_fused_norm_qmv_f16in": (C.c_int, [vp, QW, vp, vp, vp, QMVDims]),
    # Q4
    "nnz_dispatch_q4mv": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_q4mv_f16io": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_q4mv_f16in": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_q4mv_f16io_resadd": (C.c_int, [vp, QW, vp, vp, QMVDims]),
    "nnz_dispatch_q4mv_fused_pair_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_q4mv_fused_pair_silu_f16io": (C.c_int, [vp, QW, QW, vp, vp, QMVDims]),
    "nnz_dispatch_q4_fused_norm_qmv_f16io": (C.c_int, [vp, QW, vp, vp, vp, QMVDims]),
    "nnz_dispatch_q4_fused_norm_pair_qmv_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, vp, QMVDims]),
    "nnz_dispatch_q4_fused_norm_pair_silu_f16io": (C.c_int, [vp, QW, QW, vp, vp, vp, QMVDims]),
    # stacked
    "nnz_dispatch_qmv_stacked": (C.c_int, [vp, QW, vp, vp, QMVDims, P(QmvStack)]),
    "nnz_dispatch_q4mv_stacked": (C.c_int, [vp, QW, vp, vp, QMVDims, P(QmvStack)]),
    "nnz_dispatch_qmv_fused_pair_silu_stacked": (C.c_int, [vp, QW, QW, vp, vp, QMVDims,
                                                           P(QmvStack)]),
    # dequant / gemm
    "nnz_dispatch_dequant": (C.c_int, [vp, QW, vp, QMVDims]),
    "nnz_dispatch_dequant_gemm": (C.c_int, [vp, QW, QW, vp, u32, vp, C.c_int, QMVDims]),
    # transformer
    "nnz_dispatch_rms_norm": (C.c_int, [vp, vp, vp, vp, C.c_int, C.c_int, RMSNormDims]),
    "nnz_dispatch_silu": (C.c_int, [vp, vp, vp, u32]),
    "nnz_dispatch_silu_elementwise_mul": (C.c_int, [vp, vp, vp, vp, C.c_int, u32]),
    "nnz_dispatch_rope": (C.c_int, [vp, vp, C.c_int, RoPEDims]),
    "nnz_dispatch_kv_cache_update": (C.c_int, [vp, vp, vp, C.c_int, vp, vp, C.c_int, KVUpdateDims]),
    "nnz_dispatch_fused_rope_kv_cache": (C.c_int, [vp, vp, vp, vp, vp, FusedRoPEKVDims]),
    "nnz_dispatch_fused_norm_rope": (C.c_int, [vp, vp, vp, FusedNormRoPEDims]),
    "nnz_dispatch_fused_k_norm_rope_kv_cache": (C.c_int, [vp, vp, vp, vp, vp, vp,
                                                          FusedKNormRoPEKVDims]),
    "nnz_gqa_scratch_bytes": (sz, [GQADims]),
    "nnz_dispatch_gqa_attention": (C.c_int, [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, vp,
                                             C.c_int, vp, sz, i32, f32, GQADims]),
    "nnz_dispatch_gqa_attention_noalloc": (C.c_int, [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int,
                                                     vp, C.c_int, i32, f32, GQADims]),
    "nnz_dispatch_gqa_attention_fused": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz,
                                                   GQAFusedDims]),
    "nnz_dispatch_gqa_attention_fused_1pass": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                                         sz, vp, GQAFusedDims]),
    "nnz_gqa_partial_chunks": (u32, [u32]),
    "nnz_dispatch_gqa_attention_partials": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                                      vp, GQAFusedDims]),
    "nnz_dispatch_qmv_merge_f16io_resadd": (C.c_int, [vp, QW, vp, vp, vp, u32, u32, vp, QMVDims]),
    "nnz_dispatch_embedding_lookup": (C.c_int, [vp, vp, vp, vp, vp, EmbedDims]),
    "nnz_dispatch_embedding_lookup_q4": (C.c_int, [vp, vp, vp, vp, vp, vp, EmbedDims]),
    "nnz_dispatch_embedding_lookup_bf16": (C.c_int, [vp, vp, vp, vp, EmbedDims]),
    "nnz_dispatch_residual_add": (C.c_int, [vp, vp, vp, u32]),
    "nnz_dispatch_argmax": (C.c_int, [vp, vp, u32, vp, vp]),
    "nnz_sample_workspace_bytes": (sz, [u32]),
    "nnz_rng_seed": (C.c_int, [vp, C.c_uint64, vp]),
    "nnz_dispatch_sample": (C.c_int, [vp, vp, u32, vp, vp, vp, sz, vp, vp]),
    "nnz_dispatch_lm_head_bf16": (C.c_int, [vp, vp, vp, vp, u32, u32]),
    # model
    "nnz_model_create": (C.c_int, [vp, P(ModelConfig), P(vp)]),
    "nnz_model_destroy": (C.c_int, [vp]),
    "nnz_model_tensor": (C.c_int, [vp, C.c_int, u32, P(vp), P(sz)]),
    "nnz_model_forward_decode": (C.c_int, [vp, u32, u32]),
    "nnz_model_prefill": (C.c_int, [vp, vp, u32, u32]),
    "nnz_model_generate": (C.c_int, [vp, vp, u32, u32, vp, vp, vp, C.c_int, vp]),
    "nnz_model_decode_begin": (C.c_int, [vp, vp, u32, u32]),
    "nnz_model_decode_steps": (C.c_int, [vp, u32]),
    "nnz_model_decode_read": (C.c_int, [vp, u32, vp, vp]),
    "nnz_model_decode_end": (C.c_int, [vp]),
    "nnz_model_set_sampling": (C.c_int, [vp, vp]),
    "nnz_model_set_eos": (C.c_int, [vp, vp, u32]),
    "nnz_model_decode_status": (C.c_int, [vp, vp, vp]),
    "nnz_synth_normal_bf16": (C.c_int, [vp, vp, C.c_uint64, C.c_uint64, C.c_double]),
}


def header_functions(path: Path = HEADER) -> list[str]:
    """Every function name declared in include/*.h (used by the ABI test)."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nnz_[a-z0-9_]+)\s*\(", text)))


class NnzError(RuntimeError):
    def __init__(self, name: str, code: int, msg: str):
        super().__init__(f"{name} failed with {code}: {msg}")
        self.code = code


_LIB = None


def lib() -> C.CDLL:
    """Load libnnzap_amd.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m nnzap_amd.build` "
                              "(there is no CPU fallback for the HIP path)")
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in PROTOS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def check(ctx, name: str, rc: int) -> None:
    if rc != OK:
        msg = lib().nnz_last_error(ctx).decode() if ctx else ""
        raise NnzError(name, rc, msg)

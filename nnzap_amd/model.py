"""Host wrapper of the C-ABI decoder model (Model(Config) + generate).

Mirrors nnmetal/src/model.zig (Model: init + loadWeights) and
nnmetal/src/transformer.zig:3942 (generate) for the synthetic BASELINE
config-5 model.  All compute runs in libnnzap_amd.so.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from . import _lib as L
from . import synth as S
from .configs import PROJS, DecoderConfig, DecoderWeights
from . import ops
from .ops import Device

_CODES = {"q": 10, "k": 12, "v": 14, "o": 16, "gate": 18, "up": 20, "down": 22}
T_EMBED_CODES, T_EMBED_SCALES, T_LM_CODES, T_LM_SCALES, T_FINAL_NORM = 0, 1, 2, 3, 4
T_ATTN_NORM, T_FFN_NORM, T_Q_NORM, T_K_NORM = 24, 25, 26, 27
T_K_CACHE, T_V_CACHE, T_LOGITS, T_RESIDUAL = 30, 31, 40, 41
T_EMBED_BIASES, T_LM_BIASES = 5, 6
_BIASES = {"q": 50, "k": 51, "v": 52, "o": 53, "gate": 54, "up": 55, "down": 56}


class DecoderModel:
    """One decoder instance resident in HBM on ``dev``."""

    def __init__(self, dev: Device, cfg: DecoderConfig):
        self.dev, self.cfg = dev, cfg
        c = L.ModelConfig(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_layers,
                          cfg.num_query_heads, cfg.num_kv_heads, cfg.head_dim,
                          cfg.max_context_length, cfg.max_prefill_length, cfg.group_size,
                          cfg.rope_theta, cfg.rms_eps, cfg.embed_kind, cfg.lm_head_kind,
                          cfg.quant_format)
        h = C.c_void_p()
        dev.call("nnz_model_create", C.byref(c), C.byref(h))
        self.h = h
        ops.track(self)

    def close(self):
        if self.h:
            L.lib().nnz_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            if sys.is_finalizing():  # HIP runtime may be gone; see ops.Device
                return
            self.close()
        except Exception:   # module globals may already be gone at teardown
            pass

    def _mcall(self, name, *args):
        rc = getattr(L.lib(), name)(self.h, *args)
        L.check(self.dev.ctx, name, rc)

    def tensor(self, tid: int, layer: int = 0):
        p, n = C.c_void_p(), C.c_size_t()
        self._mcall("nnz_model_tensor", tid, layer, C.byref(p), C.byref(n))
        return p.value, n.value

    def upload(self, tid: int, layer: int, arr: np.ndarray) -> None:
        ptr, nbytes = self.tensor(tid, layer)
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != nbytes:
            raise ValueError(f"tensor {tid}/{layer}: {arr.nbytes} bytes given, {nbytes} expected")
        self.dev.call("nnz_upload", C.c_void_p(ptr), arr.ctypes.data_as(C.c_void_p), nbytes)

    def download(self, tid: int, layer: int = 0, dtype=np.float32) -> np.ndarray:
        ptr, nbytes = self.tensor(tid, layer)
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        self.dev.call("nnz_download", out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), nbytes)
        return out

    def load(self, w: DecoderWeights, embed_on_device: bool = False) -> None:
        """Upload weights (model.zig:196-242 loadWeights).  With
        ``embed_on_device`` the bf16 embedding table is generated on the GPU
        from the same seeded stream instead of being uploaded."""
        cfg = self.cfg
        bits = 4 if cfg.quant_format == L.QUANT_FORMAT_Q4 else 1
        for l, layer in enumerate(w.layers):
            for name in PROJS:
                if layer[name].bits != bits:
                    raise ValueError(f"layer {l} {name}: this decoder holds {bits}-bit projections, "
                                     f"got {layer[name].bits}-bit")
        if len(w.layers) != cfg.num_layers:
            raise ValueError(f"{len(w.layers)} layers given, config has {cfg.num_layers}")
        if cfg.embed_kind == L.EMBED_BF16:
            if embed_on_device:
                ptr, nbytes = self.tensor(T_EMBED_CODES)
                self.dev.call("nnz_synth_normal_bf16", C.c_void_p(ptr), nbytes // 2,
                              S.SEED_MODEL_BASE + 0, 0.02)
            else:
                self.upload(T_EMBED_CODES, 0, w.embed_bf16)
        else:
            if w.embed_q1 is None or w.embed_q1.bits != bits:
                raise ValueError(f"config asks for a {bits}-bit embedding table")
            self._upload_q(T_EMBED_CODES, T_EMBED_SCALES, T_EMBED_BIASES, 0, w.embed_q1)
        if cfg.lm_head_kind in (L.LMHEAD_Q1, L.LMHEAD_Q4):
            if w.lm_head is None or w.lm_head.bits != bits:
                raise ValueError(f"config asks for a {bits}-bit LM head")
            self._upload_q(T_LM_CODES, T_LM_SCALES, T_LM_BIASES, 0, w.lm_head)
        self.upload(T_FINAL_NORM, 0, w.final_norm)
        for l, layer in enumerate(w.layers):
            for name in PROJS:
                cid = _CODES[name]
                self._upload_q(cid, cid + 1, _BIASES[name], l, layer[name])
            self.upload(T_ATTN_NORM, l, layer["attn_norm"])
            self.upload(T_FFN_NORM, l, layer["ffn_norm"])
            self.upload(T_Q_NORM, l, layer["q_norm"])
            self.upload(T_K_NORM, l, layer["k_norm"])
        self.dev.sync()

    def _upload_q(self, t_codes: int, t_scales: int, t_biases: int, layer: int, q) -> None:
        """Codes and scales, plus the biases of a 4-bit (q4_mlx) matrix."""
        self.upload(t_codes, layer, q.codes)
        self.upload(t_scales, layer, q.scales)
        if q.bits == 4:
            self.upload(t_biases, layer, q.biases)

    def load_weights(self, paths, quant: str = "q1", tie_word_embeddings: bool = True,
                     strict: bool = True) -> None:
        """loadWeights(file_paths) (model.zig:196-242): read an MLX-format
        checkpoint (shard files or a model directory) straight from the
        mapped shards into device memory."""
        from contextlib import ExitStack
        import os
        from . import checkpoint as ck
        from .safetensors import SafetensorsFile
        cfg = self.cfg
        q4 = cfg.quant_format == L.QUANT_FORMAT_Q4
        if q4 != (quant == ck.QUANT_Q4):
            raise ValueError(f"quant {quant!r} does not match the model's quant_format")
        want = (L.EMBED_Q4, L.LMHEAD_Q4) if q4 else (L.EMBED_Q1, L.LMHEAD_Q1)
        if (cfg.embed_kind, cfg.lm_head_kind) != want:
            raise ValueError("checkpoint models need a quantised embedding and LM head "
                             "(EMBED_Q1/LMHEAD_Q1, or EMBED_Q4/LMHEAD_Q4 for q4_mlx)")
        if isinstance(paths, (str, os.PathLike)):
            paths = ck.find_shards(paths) if os.path.isdir(paths) else [paths]
        with ExitStack() as stack:
            files = [stack.enter_context(SafetensorsFile.open(p)) for p in paths]
            w = ck.read_weights(files, cfg, quant, tie_word_embeddings, strict)
            self.load(w)
            del w

    def forward_decode(self, token: int, position: int) -> np.ndarray:
        self._mcall("nnz_model_forward_decode", token, position)
        self.dev.sync()
        return self.download(T_LOGITS)

    def prefill(self, tokens: np.ndarray, start: int = 0) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self._mcall("nnz_model_prefill", t.ctypes.data_as(C.c_void_p), len(t), start)
        self.dev.sync()
        return self.download(T_LOGITS)

    # -- streaming decode: begin (prefill + capture), enqueue steps, read -----
    def decode_begin(self, prompt: np.ndarray, max_new: int) -> None:
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        self._mcall("nnz_model_decode_begin", p.ctypes.data_as(C.c_void_p), len(p), max_new)

    def decode_steps(self, n: int) -> None:
        self._mcall("nnz_model_decode_steps", n)

    def decode_read(self, n: int):
        toks = np.zeros(n, dtype=np.uint32)
        margins = np.zeros(n, dtype=np.float32)
        self._mcall("nnz_model_decode_read", n, toks.ctypes.data_as(C.c_void_p),
                    margins.ctypes.data_as(C.c_void_p))
        return toks, margins

    def decode_end(self) -> None:
        self._mcall("nnz_model_decode_end")

    def set_sampling(self, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                     seed: int = 42) -> None:
        """GenerateOpts.params (SamplingParams, transformer.zig:3652-3657);
        temperature 0 is greedy."""
        p = L.SamplingParams(temperature, top_k, top_p, 0, seed)
        self._mcall("nnz_model_set_sampling", C.byref(p))

    def set_eos(self, ids) -> None:
        """GenerateOpts.eos_ids: a picked stop token ends generation unemitted."""
        a = np.ascontiguousarray(list(ids), dtype=np.uint32)
        self._mcall("nnz_model_set_eos", a.ctypes.data_as(C.c_void_p) if len(a) else None, len(a))

    def decode_status(self):
        """(tokens emitted, stopped by a stop token) of the current stream."""
        n, stopped = C.c_uint32(), C.c_int()
        self._mcall("nnz_model_decode_status", C.byref(n), C.byref(stopped))
        return n.value, bool(stopped.value)

    def generate(self, prompt: np.ndarray, n_new: int, use_graph: bool = True,
                 step_ms: bool = False):
        """generate (transformer.zig:3942): up to n_new tokens, fewer when a
        stop token ends the stream.  Returns (tokens, per-token values,
        per-step ms or None); the values are top-2 logit margins (greedy) or
        the sampled tokens' probabilities."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.zeros(n_new, dtype=np.uint32)
        margins = np.zeros(n_new, dtype=np.float32)
        ms = np.zeros(n_new, dtype=np.float32) if step_ms else None
        count = C.c_uint32()
        self._mcall("nnz_model_generate", p.ctypes.data_as(C.c_void_p), len(p), n_new,
                    toks.ctypes.data_as(C.c_void_p), margins.ctypes.data_as(C.c_void_p),
                    ms.ctypes.data_as(C.c_void_p) if ms is not None else None, int(use_graph),
                    C.byref(count))
        n = count.value
        return toks[:n], margins[:n], (ms[:n] if ms is not None else None)

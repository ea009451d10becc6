"""Python mirror of nnmetal's kernel-dispatch API on top of libnnzap_amd.so.

Each ``dispatch_*`` function mirrors one reference helper in
nnmetal/src/transformer.zig (cited per function) and calls the matching C-ABI
entry point of include/nnz.h.  Buffers are torch tensors on the GPU (torch is
only the allocator/stream plumbing); quantised matrices are
:class:`DeviceQWeight` objects.  Errors raise :class:`NnzError` -- the
reference asserts instead.
"""
from __future__ import annotations

import atexit
import ctypes as C
import sys
import weakref

import numpy as np

from . import _lib as L
from .formats import QWeight, DT_BF16, DT_F16
from ._lib import NnzError, QMVDims, lib  # noqa: F401  (re-exported)


def _torch():
    import torch
    return torch


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_DT = {"float32": L.F32, "float16": L.F16, "bfloat16": L.BF16}


def dtype_code(t) -> int:
    return _DT[str(t.dtype).replace("torch.", "")]


# Objects that own library handles (contexts, models), in creation order.
# Teardown contract: the caller closes them (close()); whatever is still
# open when the interpreter exits is closed here, newest first (a model
# before the context it runs on), from an atexit hook -- atexit runs before
# interpreter finalization, while the HIP runtime is fully alive.  Nothing
# is released from __del__ during finalization: the runtime's own C++
# state may already be destroyed then.
_LIVE: list = []


def track(obj) -> None:
    _LIVE.append(weakref.ref(obj))


@atexit.register
def _close_live() -> None:
    while _LIVE:
        o = _LIVE.pop()()
        if o is not None:
            try:
                o.close()
            except Exception:
                pass


class Device:
    """Replaces metal.Device (nnmetal/src/metal.zig:839-1372): a context bound
    to torch's current stream on ``cuda:index``."""

    def __init__(self, index: int = 0, own_stream: bool = False):
        """``own_stream``: the context creates its own non-blocking HIP stream
        (needed for graph capture; then exchange data through nnz_upload /
        nnz_download, not through torch ops on another stream)."""
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError("nnzap_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
        torch.cuda.set_device(index)
        self.index = index
        self.torch_device = torch.device("cuda", index)
        self.stream = None if own_stream else torch.cuda.current_stream(index)
        if self.stream is not None and self.stream.cuda_stream == 0:
            # torch's legacy default stream has handle 0, which nnz_ctx_create
            # reads as "create your own stream": the library's launches would
            # then not be ordered with torch's ops (nor with its caching
            # allocator's reuse of freed tensors).  Make a dedicated stream
            # (default priority) current for torch and share it instead.
            self.stream = torch.cuda.Stream(index)
            torch.cuda.set_stream(self.stream)
        ctx = C.c_void_p()
        handle = None if own_stream else C.c_void_p(self.stream.cuda_stream)
        rc = lib().nnz_ctx_create(index, handle, C.byref(ctx))
        if rc != 0:
            raise NnzError("nnz_ctx_create", rc, "")
        self.ctx = ctx
        track(self)

    def close(self) -> None:
        if self.ctx:
            lib().nnz_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        # During interpreter finalization the HIP runtime's C++ state may
        # already be destroyed; the atexit hook above has closed every live
        # object before that point.
        try:
            if sys.is_finalizing():
                return
            self.close()
        except Exception:   # module globals may already be gone at teardown
            pass

    def call(self, name: str, *args) -> None:
        rc = getattr(lib(), name)(self.ctx, *args)
        L.check(self.ctx, name, rc)

    def sync(self, timeout_ms: int = 60000) -> None:
        self.call("nnz_stream_sync", timeout_ms)

    def mark(self, slot: int) -> None:
        self.call("nnz_timer_mark", slot)

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        self.call("nnz_timer_elapsed_ms", a, b, C.byref(ms))
        return float(ms.value)


class DeviceQWeight:
    """A quantised matrix resident in device memory (PackedBuffer/Q4Buffer)."""

    def __init__(self, dev: Device, w: QWeight):
        torch = _torch()
        self.host = w
        self.M, self.K, self.group_size, self.bits = w.M, w.K, w.group_size, w.bits
        td = dev.torch_device
        self.codes = torch.from_numpy(np.ascontiguousarray(w.codes).view(np.int32)).to(td)
        self.scales = torch.from_numpy(np.ascontiguousarray(w.scales).view(np.int16)).to(td)
        self.biases = (torch.from_numpy(np.ascontiguousarray(w.biases).view(np.int16)).to(td)
                       if w.biases is not None else None)
        self.desc = L.QWeightDesc(self.codes.data_ptr(), self.scales.data_ptr(),
                                  _ptr(self.biases), w.M * w.K, w.group_size, w.bits,
                                  w.scale_dtype)

    @property
    def ref(self):
        return C.byref(self.desc)

    def dims(self) -> QMVDims:
        return QMVDims(self.M, self.K, self.group_size)


def _v(t):
    return C.c_void_p(_ptr(t))


class StackedQWeights:
    """`count` independently drawn quantised matrices of one shape [M x K],
    generated on the device (seeded torch generator): codes uniform random
    bits (Q1) or nibbles (Q4), 16-bit scales ~U(scale_range) and, for Q4,
    biases ~U(bias_range).  Matrix i lives at a fixed stride in three device
    arrays -- the layout nnz_dispatch_*_stacked reads.  Rows of every array
    are padded to 16 bytes per matrix so the strides keep the codes aligned."""

    def __init__(self, dev: Device, M: int, K: int, group_size: int, bits: int, count: int,
                 seed: int, scale_range=(0.01, 0.05), bias_range=(-0.1, 0.1),
                 scale_dtype: int = DT_F16, pad_bytes: int = 0):
        torch = _torch()
        td = dev.torch_device
        g = torch.Generator(device=td)
        g.manual_seed(seed)
        self.M, self.K, self.group_size, self.bits, self.count = M, K, group_size, bits, count
        self.scale_dtype = scale_dtype
        words = M * K * bits // 32
        ng = M * K // group_size
        # pad_bytes (a multiple of 16): extra bytes between consecutive
        # matrices' codes and scales, so that their starts need not share
        # the same low address bits
        assert pad_bytes % 16 == 0
        wpad = (words + 3) // 4 * 4 + pad_bytes // 4
        gpad = (ng + 7) // 8 * 8 + pad_bytes // 2
        self.codes = torch.randint(-2 ** 31, 2 ** 31 - 1, (count, wpad), dtype=torch.int32,
                                   generator=g, device=td)
        sdt = torch.float16 if scale_dtype == DT_F16 else torch.bfloat16

        def uni(lo, hi):
            return (lo + (hi - lo) * torch.rand(count, gpad, generator=g, device=td)) \
                .to(sdt).view(torch.int16)
        self.scales = uni(*scale_range)
        self.biases = uni(*bias_range) if bits == 4 else None
        self.desc = L.QWeightDesc(self.codes.data_ptr(), self.scales.data_ptr(),
                                  _ptr(self.biases), M * K, group_size, bits, scale_dtype)
        self.codes_stride = wpad * 4
        self.scales_stride = gpad * 2

    @property
    def ref(self):
        return C.byref(self.desc)

    @property
    def nbytes_each(self) -> int:
        """Algorithmic bytes of one matrix (codes, scales and biases)."""
        n = self.M * self.K * self.bits // 8 + self.M * self.K // self.group_size * 2
        return n + (self.M * self.K // self.group_size * 2 if self.bits == 4 else 0)

    def dims(self) -> QMVDims:
        return QMVDims(self.M, self.K, self.group_size)

    def stack(self, input_stride: int, output_stride: int, blocks_per_matrix: int = 0):
        return L.QmvStack(self.count, blocks_per_matrix, self.codes_stride, self.scales_stride,
                          input_stride, output_stride)

    def host(self, i: int) -> QWeight:
        """Host copy of matrix i (for checks against the oracle)."""
        words = self.M * self.K * self.bits // 32
        ng = self.M * self.K // self.group_size
        codes = self.codes[i, :words].cpu().numpy().view(np.uint32).reshape(self.M, -1)
        sc = self.scales[i, :ng].cpu().numpy().view(np.uint16).reshape(self.M, -1)
        bi = (self.biases[i, :ng].cpu().numpy().view(np.uint16).reshape(self.M, -1)
              if self.biases is not None else None)
        return QWeight(self.bits, self.M, self.K, self.group_size, codes, sc, bi,
                       self.scale_dtype)


def _stack_io(x, y):
    """Byte strides between the matrices' inputs x[count, K] and outputs y[count, M]."""
    return x.stride(0) * x.element_size(), y.stride(0) * y.element_size()


def dispatch_qmv_stacked(dev, sw: StackedQWeights, x, y, blocks_per_matrix: int = 0):
    """Config-2 arithmetic (Q1, f32 in/out) over sw.count matrices in one
    launch: y[i] = W_i . x[i]."""
    xs, ys = _stack_io(x, y)
    st = sw.stack(xs, ys, blocks_per_matrix)
    dev.call("nnz_dispatch_qmv_stacked", sw.ref, _v(x), _v(y), sw.dims(), C.byref(st))


def dispatch_q4mv_stacked(dev, sw: StackedQWeights, x, y, blocks_per_matrix: int = 0):
    """Config-1 arithmetic (Q4, f32 in/out) over sw.count matrices in one launch."""
    xs, ys = _stack_io(x, y)
    st = sw.stack(xs, ys, blocks_per_matrix)
    dev.call("nnz_dispatch_q4mv_stacked", sw.ref, _v(x), _v(y), sw.dims(), C.byref(st))


def dispatch_qmv_fused_pair_silu_stacked(dev, wa: StackedQWeights, wb: StackedQWeights, x, y,
                                         blocks_per_matrix: int = 0):
    """Config-3 arithmetic (silu(Wg x) * (Wu x), f32 in/out) over wa.count
    gate/up pairs in one launch; the two stacks share their strides."""
    assert (wa.codes_stride, wa.scales_stride, wa.count) == \
        (wb.codes_stride, wb.scales_stride, wb.count), "pair stacks differ in layout"
    xs, ys = _stack_io(x, y)
    st = wa.stack(xs, ys, blocks_per_matrix)
    dev.call("nnz_dispatch_qmv_fused_pair_silu_stacked", wa.ref, wb.ref, _v(x), _v(y),
             wa.dims(), C.byref(st))


# ----------------------------------------------------------------- QMV, Q1
def dispatch_qmv(dev, w, x, y, dims=None):
    """transformer.zig:1565 dispatchQMV (f32 in, f32 out)."""
    dev.call("nnz_dispatch_qmv", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_qmv_f16in(dev, w, x, y, dims=None):
    """transformer.zig:1653 dispatchQMVf16in."""
    dev.call("nnz_dispatch_qmv_f16in", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_qmv_f16io(dev, w, x, y, dims=None):
    """transformer.zig:1728 dispatchQMVf16io."""
    dev.call("nnz_dispatch_qmv_f16io", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_qmv_f16io_resadd(dev, w, x, residual, dims=None):
    """transformer.zig:1806 dispatchQMVf16ioResadd."""
    dev.call("nnz_dispatch_qmv_f16io_resadd", w.ref, _v(x), _v(residual), dims or w.dims())


def dispatch_qmv_fused_pair(dev, wa, wb, x, ya, yb, dims=None):
    """transformer.zig:1120 dispatchQMVFusedPair."""
    dev.call("nnz_dispatch_qmv_fused_pair", wa.ref, wb.ref, _v(x), _v(ya), _v(yb), dims or wa.dims())


def dispatch_qmv_fused_pair_f16in(dev, wa, wb, x, ya, yb, dims=None):
    """transformer.zig:1181 dispatchQMVFusedPairf16in."""
    dev.call("nnz_dispatch_qmv_fused_pair_f16in", wa.ref, wb.ref, _v(x), _v(ya), _v(yb),
             dims or wa.dims())


def dispatch_qmv_fused_pair_f16io(dev, wa, wb, x, ya, yb, dims=None):
    """transformer.zig:1238 dispatchQMVFusedPairf16io."""
    dev.call("nnz_dispatch_qmv_fused_pair_f16io", wa.ref, wb.ref, _v(x), _v(ya), _v(yb),
             dims or wa.dims())


def dispatch_qmv_fused_pair_silu_f16io(dev, wa, wb, x, y, dims=None):
    """transformer.zig:1309 dispatchQMVFusedPairSiLUf16io."""
    dev.call("nnz_dispatch_qmv_fused_pair_silu_f16io", wa.ref, wb.ref, _v(x), _v(y),
             dims or wa.dims())


def dispatch_qmv_fused_pair_silu(dev, wa, wb, x, y, dims=None):
    """BASELINE config 3 (f32 I/O) form of transformer.zig:1309."""
    dev.call("nnz_dispatch_qmv_fused_pair_silu", wa.ref, wb.ref, _v(x), _v(y), dims or wa.dims())


def dispatch_fused_norm_pair_silu_f16io(dev, wa, wb, residual, y, norm_scale, dims=None):
    """transformer.zig:1373 dispatchFusedNormPairSiLUf16io."""
    dev.call("nnz_dispatch_fused_norm_pair_silu_f16io", wa.ref, wb.ref, _v(residual), _v(y),
             _v(norm_scale), dims or wa.dims())


def dispatch_fused_norm_qmv_f16io(dev, w, residual, y, norm_scale, dims=None):
    """transformer.zig:1438 dispatchFusedNormQMVf16io."""
    dev.call("nnz_dispatch_fused_norm_qmv_f16io", w.ref, _v(residual), _v(y), _v(norm_scale),
             dims or w.dims())


def dispatch_fused_norm_pair_qmv_f16io(dev, wa, wb, residual, ya, yb, norm_scale, dims=None):
    """transformer.zig:1501 dispatchFusedNormPairQMVf16io."""
    dev.call("nnz_dispatch_fused_norm_pair_qmv_f16io", wa.ref, wb.ref, _v(residual), _v(ya),
             _v(yb), _v(norm_scale), dims or wa.dims())


def dispatch_fused_norm_qkv_f16io(dev, wq, wk, wv, residual, q, k, v, norm_scale):
    """transformer.zig:1438 + :1501 as one launch (shared normalised input)."""
    dev.call("nnz_dispatch_fused_norm_qkv_f16io", wq.ref, wk.ref, wv.ref, _v(residual), _v(q), _v(k),
             _v(v), _v(norm_scale), wq.dims(), wk.M)


def dispatch_fused_norm_qmv_f16in(dev, w, residual, y, norm_scale, dims=None):
    """transformer.zig:669 (rms_norm_f16out) + :1653 dispatchQMVf16in as one launch."""
    dev.call("nnz_dispatch_fused_norm_qmv_f16in", w.ref, _v(residual), _v(y), _v(norm_scale),
             dims or w.dims())


# ----------------------------------------------------------------- QMV, Q4
def dispatch_q4mv(dev, w, x, y, dims=None):
    """f32 x -> f32 y, plain fp32 result."""
    dev.call("nnz_dispatch_q4mv", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_q4mv_f16io(dev, w, x, y, dims=None):
    """transformer.zig:1903 dispatchQ4MVf16io."""
    dev.call("nnz_dispatch_q4mv_f16io", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_q4mv_f16in(dev, w, x, y, dims=None):
    """transformer.zig:1944 dispatchQ4MVf16in."""
    dev.call("nnz_dispatch_q4mv_f16in", w.ref, _v(x), _v(y), dims or w.dims())


def dispatch_q4mv_f16io_resadd(dev, w, x, residual, dims=None):
    """transformer.zig:1987 dispatchQ4MVf16ioResadd."""
    dev.call("nnz_dispatch_q4mv_f16io_resadd", w.ref, _v(x), _v(residual), dims or w.dims())


def dispatch_q4mv_fused_pair_f16io(dev, wa, wb, x, ya, yb, dims=None):
    """transformer.zig:2069 dispatchQ4MVFusedPairf16io."""
    dev.call("nnz_dispatch_q4mv_fused_pair_f16io", wa.ref, wb.ref, _v(x), _v(ya), _v(yb),
             dims or wa.dims())


def dispatch_q4mv_fused_pair_silu_f16io(dev, wa, wb, x, y, dims=None):
    """transformer.zig:2118 dispatchQ4MVFusedPairSiLUf16io."""
    dev.call("nnz_dispatch_q4mv_fused_pair_silu_f16io", wa.ref, wb.ref, _v(x), _v(y),
             dims or wa.dims())


def dispatch_q4_fused_norm_qmv_f16io(dev, w, residual, y, norm_scale, dims=None):
    """transformer.zig:2166 dispatchQ4FusedNormQMVf16io."""
    dev.call("nnz_dispatch_q4_fused_norm_qmv_f16io", w.ref, _v(residual), _v(y), _v(norm_scale),
             dims or w.dims())


def dispatch_q4_fused_norm_pair_qmv_f16io(dev, wa, wb, residual, ya, yb, norm_scale, dims=None):
    """transformer.zig:2237 dispatchQ4FusedNormPairQMVf16io."""
    dev.call("nnz_dispatch_q4_fused_norm_pair_qmv_f16io", wa.ref, wb.ref, _v(residual), _v(ya),
             _v(yb), _v(norm_scale), dims or wa.dims())


def dispatch_q4_fused_norm_pair_silu_f16io(dev, wa, wb, residual, y, norm_scale, dims=None):
    """transformer.zig:2318 dispatchQ4FusedNormPairSiLUf16io."""
    dev.call("nnz_dispatch_q4_fused_norm_pair_silu_f16io", wa.ref, wb.ref, _v(residual), _v(y),
             _v(norm_scale), dims or wa.dims())


# ---------------------------------------------------------- dequant / GEMM
def dispatch_dequant(dev, w, out):
    dev.call("nnz_dispatch_dequant", w.ref, _v(out), w.dims())


def dispatch_dequant_gemm(dev, wa, a_f16, out, mode, wb=None):
    P = a_f16.shape[0]
    dev.call("nnz_dispatch_dequant_gemm", wa.ref, wb.ref if wb is not None else None, _v(a_f16),
             P, _v(out), mode, wa.dims())


# ------------------------------------------------------------ transformer
def dispatch_rms_norm(dev, x, scale, out, hidden, num_tokens, eps=1e-6, bf16_trunc=False):
    """transformer.zig:669 dispatchRMSNorm (variant chosen by ``out``'s dtype)."""
    dev.call("nnz_dispatch_rms_norm", _v(x), _v(scale), _v(out), dtype_code(out), int(bf16_trunc),
             L.RMSNormDims(hidden, num_tokens, eps))


def dispatch_silu(dev, x, out):
    """transformer.zig:700 dispatchSiLU."""
    dev.call("nnz_dispatch_silu", _v(x), _v(out), x.numel())


def dispatch_silu_elementwise_mul(dev, gate, up, out):
    """transformer.zig:719 dispatchSiLUElementwiseMul."""
    dev.call("nnz_dispatch_silu_elementwise_mul", _v(gate), _v(up), _v(out), dtype_code(out),
             out.numel())


def dispatch_rope(dev, data, num_heads, head_dim, position, theta):
    """transformer.zig:740 dispatchRoPE (in place)."""
    dev.call("nnz_dispatch_rope", _v(data), dtype_code(data),
             L.RoPEDims(num_heads, head_dim, position, theta))


def dispatch_kv_cache_update(dev, k, v, k_cache, v_cache, num_kv_heads, head_dim, position,
                             max_ctx):
    """transformer.zig:760 dispatchKVCacheUpdate."""
    dev.call("nnz_dispatch_kv_cache_update", _v(k), _v(v), dtype_code(k), _v(k_cache),
             _v(v_cache), dtype_code(k_cache),
             L.KVUpdateDims(num_kv_heads, head_dim, position, max_ctx))


def dispatch_fused_rope_kv_cache(dev, k, v, k_cache, v_cache, dims: L.FusedRoPEKVDims):
    """transformer.zig:792 dispatchFusedRoPEKVCache."""
    dev.call("nnz_dispatch_fused_rope_kv_cache", _v(k), _v(v), _v(k_cache), _v(v_cache), dims)


def dispatch_fused_norm_rope(dev, data, scale, dims: L.FusedNormRoPEDims):
    """transformer.zig:829 dispatchFusedNormRoPE."""
    dev.call("nnz_dispatch_fused_norm_rope", _v(data), _v(scale), dims)


def dispatch_fused_k_norm_rope_kv_cache(dev, k, v, k_cache, v_cache, k_scale,
                                        dims: L.FusedKNormRoPEKVDims):
    """transformer.zig:866 dispatchFusedKNormRoPEKVCache."""
    dev.call("nnz_dispatch_fused_k_norm_rope_kv_cache", _v(k), _v(v), _v(k_cache), _v(v_cache),
             _v(k_scale), dims)


def gqa_scratch_bytes(dims: L.GQADims) -> int:
    return int(lib().nnz_gqa_scratch_bytes(dims))


def dispatch_gqa_attention(dev, q, k_cache, v_cache, out, scratch, dims: L.GQADims,
                           v_transposed=True, rope_position=-1, rope_theta=0.0):
    """transformer.zig:1030 dispatchGQAAttention / :915 dispatchGQAAttentionTG."""
    dev.call("nnz_dispatch_gqa_attention", _v(q), dtype_code(q), _v(k_cache), _v(v_cache),
             dtype_code(k_cache), int(v_transposed), _v(out), dtype_code(out), _v(scratch),
             scratch.numel() * scratch.element_size(), int(rope_position), float(rope_theta), dims)


def dispatch_gqa_attention_fused(dev, q, k_cache, v_cache, out, k_raw, v_raw, q_norm, k_norm,
                                 scratch, dims: L.GQAFusedDims):
    """transformer.zig:962 dispatchGQAAttentionFusedTG."""
    dev.call("nnz_dispatch_gqa_attention_fused", _v(q), _v(k_cache), _v(v_cache), _v(out),
             _v(k_raw), _v(v_raw), _v(q_norm), _v(k_norm), _v(scratch),
             scratch.numel() * scratch.element_size(), dims)


def dispatch_gqa_attention_fused_1pass(dev, q, k_cache, v_cache, out, k_raw, v_raw, q_norm,
                                       k_norm, scratch, dims: L.GQAFusedDims, d_seq_len=None):
    """transformer.zig:962 dispatchGQAAttentionFusedTG as one launch (graph
    replay form; ``scratch`` must start zeroed, see include/nnz.h)."""
    dev.call("nnz_dispatch_gqa_attention_fused_1pass", _v(q), _v(k_cache), _v(v_cache), _v(out),
             _v(k_raw), _v(v_raw), _v(q_norm), _v(k_norm), _v(scratch),
             scratch.numel() * scratch.element_size(), _v(d_seq_len), dims)


def gqa_partial_chunks(seq_len: int) -> int:
    return int(L.lib().nnz_gqa_partial_chunks(seq_len))


def dispatch_gqa_attention_partials(dev, q, k_cache, v_cache, k_raw, v_raw, q_norm, k_norm,
                                    part_o, part_ml, dims: L.GQAFusedDims, d_seq_len=None,
                                    rope_inv_freq=None):
    """The decode step's attention half: transformer.zig:3244-3370 up to the
    per-chunk partials (part_o [n][Hq*D] in the merge's unit-major column
    order, part_ml [n][Hq][2], n = gqa_partial_chunks(seq_len))."""
    dev.call("nnz_dispatch_gqa_attention_partials", _v(q), _v(k_cache), _v(v_cache), _v(k_raw),
             _v(v_raw), _v(q_norm), _v(k_norm), _v(rope_inv_freq), _v(part_o), _v(part_ml),
             _v(d_seq_len), dims)


def dispatch_qmv_merge_f16io_resadd(dev, w, part_o, part_ml, seq_len, head_dim, residual,
                                    d_seq_len=None, dims=None):
    """residual += W . merge(partials), the merge rounded to f16 (the O
    projection of transformer.zig:1686 on the attention output)."""
    dev.call("nnz_dispatch_qmv_merge_f16io_resadd", w.ref, _v(part_o), _v(part_ml), _v(d_seq_len),
             seq_len, head_dim, _v(residual), dims or w.dims())


def dispatch_embedding_lookup(dev, ids, bits, scales, out, dims: L.EmbedDims):
    """transformer.zig:1072 dispatchEmbeddingLookup."""
    dev.call("nnz_dispatch_embedding_lookup", _v(ids), _v(bits), _v(scales), _v(out), dims)


def dispatch_embedding_lookup_q4(dev, ids, nibs, scales, biases, out, dims: L.EmbedDims):
    """transformer.zig:2625-2691 (Q4 branch of encodeEmbeddingLookup)."""
    dev.call("nnz_dispatch_embedding_lookup_q4", _v(ids), _v(nibs), _v(scales), _v(biases),
             _v(out), dims)


def dispatch_embedding_lookup_bf16(dev, ids, table, out, dims: L.EmbedDims):
    dev.call("nnz_dispatch_embedding_lookup_bf16", _v(ids), _v(table), _v(out), dims)


def dispatch_residual_add(dev, residual, addition):
    """transformer.zig:1097 dispatchResidualAdd."""
    dev.call("nnz_dispatch_residual_add", _v(residual), _v(addition), residual.numel())


def dispatch_argmax(dev, logits, out_index, out_value=None):
    """transformer.zig:3694 argmax, on device."""
    dev.call("nnz_dispatch_argmax", _v(logits), logits.numel(), _v(out_index), _v(out_value))


def sample_workspace_bytes(count: int) -> int:
    return int(L.lib().nnz_sample_workspace_bytes(count))


def rng_seed(dev, seed: int, state):
    """std.Random.DefaultPrng.init(seed) into a device uint64[4] (int64 tensor)."""
    dev.call("nnz_rng_seed", C.c_uint64(seed & (2**64 - 1)), _v(state))


def dispatch_sample(dev, logits, out_index, rng, workspace, temperature: float,
                    top_k: int = 0, top_p: float = 1.0, out_prob=None):
    """transformer.zig:3860 sampleToken, on device (one draw from ``rng``)."""
    p = L.SamplingParams(temperature, top_k, top_p, 0, 0)
    dev.call("nnz_dispatch_sample", _v(logits), logits.numel(), C.byref(p), _v(rng),
             _v(workspace), workspace.numel() * workspace.element_size() if workspace is not None
             else 0, _v(out_index), _v(out_prob))


def dispatch_lm_head_bf16(dev, table, x, logits):
    """LM head of transformer.zig:2730-2785 with the tied bf16 embedding
    table (:297): logits = table . x, table bf16 [V, H], x f16 [H]."""
    V, H = table.shape
    dev.call("nnz_dispatch_lm_head_bf16", _v(table), _v(x), _v(logits), V, H)


__all__ = [n for n in dir() if n.startswith("dispatch_")] + ["Device", "DeviceQWeight",
                                                             "NnzError", "gqa_scratch_bytes",
                                                             "rng_seed", "sample_workspace_bytes"]

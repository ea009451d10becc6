"""GPU check of the allocation-free decode attention entry point
(nnz_dispatch_gqa_attention_noalloc), called through the C ABI.

Its output must equal nnz_dispatch_gqa_attention's (the workspace variant:
same kernels, same chunk plan) bit for bit, on two calls in a row where the
second is smaller than the first (the fixed partials buffer keeps the first
call's contents), and match the CPU oracle to the 1e-3 bar.  A shape whose
partials exceed the fixed buffer is refused with NNZ_EUNSUPPORTED before
anything is launched."""
import numpy as np
import pytest
import torch

from nnzap_amd import _lib as L
from nnzap_amd import configs as cf
from nnzap_amd import ops
from nnzap_amd import synth as S
from oracle import oracle as O

from gpu_util import assert_close, from_bits16, host

pytestmark = pytest.mark.gpu


def _noalloc(dev, q, k, v, out, dims, rope_position, rope_theta):
    rc = L.lib().nnz_dispatch_gqa_attention_noalloc(
        dev.ctx, q.data_ptr(), ops.dtype_code(q), k.data_ptr(), v.data_ptr(), ops.dtype_code(k),
        0, out.data_ptr(), ops.dtype_code(out), rope_position, rope_theta, dims)
    return rc


def _case(dev, L_, hkv=8):
    print(f"noalloc attention L={L_} hkv={hkv}", flush=True)
    q, k, v = cf.config4(L_, hkv=hkv)
    qd, kd, vd = from_bits16(q, "bf16"), from_bits16(k, "bf16"), from_bits16(v, "bf16")
    dims = L.GQADims(16, hkv, 128, L_, L_, 16 // hkv)
    ref_out = torch.empty(16, 128, dtype=torch.float32, device="cuda")
    scratch = torch.empty((ops.gqa_scratch_bytes(dims) + 3) // 4, dtype=torch.float32, device="cuda")
    ops.dispatch_gqa_attention(dev, qd, kd, vd, ref_out, scratch, dims, v_transposed=False,
                               rope_position=L_, rope_theta=1e6)
    out = torch.full((16, 128), float("nan"), dtype=torch.float32, device="cuda")
    rc = _noalloc(dev, qd, kd, vd, out, dims, L_, 1e6)
    L.check(dev.ctx, "nnz_dispatch_gqa_attention_noalloc", rc)
    dev.sync()
    got, want = host(out), host(ref_out)
    assert np.array_equal(got, want), f"L={L_}: differs from the workspace entry point"
    qf = O.rope(S.bf16_bits_to_f32(q).astype(np.float64), L_, 1e6)
    ref = O.attention_decode(qf, S.bf16_bits_to_f32(k), S.bf16_bits_to_f32(v), L_, False)
    assert_close(got, ref, what=f"noalloc L={L_}")


def test_noalloc_attention_matches_workspace_variant(dev):
    _case(dev, 32768)   # the config-4 shape at its longest (the streaming plan)
    _case(dev, 4096)    # then a smaller call over the previous contents


def _largest_accepted(hq, hkv, d):
    """The longest seq_len whose partials fit the fixed buffer (the need
    grows by one chunk row every 64 tokens)."""
    seq = 64
    while ops.gqa_scratch_bytes(L.GQADims(hq, hkv, d, seq + 64, seq + 64, hq // hkv)) \
            <= L.GQA_NOALLOC_MAX_BYTES:
        seq += 64
    return seq


def test_noalloc_attention_fills_the_buffer(dev):
    """16 query heads over 2 KV heads (groups of 8) take the 64-token chunk
    plan: at the longest accepted length its partials end within one chunk
    row of the buffer's end.  That call matches the workspace entry point and
    the oracle; a smaller call follows over its contents; one more token is
    refused."""
    hq, hkv, d = 16, 2, 128
    seq = _largest_accepted(hq, hkv, d)
    need = ops.gqa_scratch_bytes(L.GQADims(hq, hkv, d, seq, seq, hq // hkv))
    assert L.GQA_NOALLOC_MAX_BYTES - need < hq * (d + 2) * 4
    _case(dev, seq, hkv=hkv)
    _case(dev, 1000, hkv=hkv)
    over = seq + 1
    dims = L.GQADims(hq, hkv, d, over, over, hq // hkv)
    assert ops.gqa_scratch_bytes(dims) > L.GQA_NOALLOC_MAX_BYTES
    qz = torch.zeros(hq, d, dtype=torch.float32, device="cuda")
    kz = torch.zeros(hkv, over, d, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(hq, d, dtype=torch.float32, device="cuda")
    assert _noalloc(dev, qz, kz, kz, out, dims, -1, 0.0) == L.EUNSUPPORTED


def test_noalloc_attention_rejects_oversize(dev):
    hq, hkv, d, seq = 16, 8, 128, 70000
    dims = L.GQADims(hq, hkv, d, seq, seq, 2)
    assert ops.gqa_scratch_bytes(dims) > L.GQA_NOALLOC_MAX_BYTES
    q = torch.zeros(hq, d, dtype=torch.float32, device="cuda")
    # full-size caches, so that even a launch would stay in bounds
    k = torch.zeros(hkv, seq, d, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros(hkv, seq, d, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(hq, d, dtype=torch.float32, device="cuda")
    assert _noalloc(dev, q, k, v, out, dims, -1, 0.0) == L.EUNSUPPORTED
    assert b"fixed buffer" in L.lib().nnz_last_error(dev.ctx)

"""GPU parity of the QMV family (Q1 and Q4) against the CPU oracle.

Bar (north star): dequantised weights bit-exact; fp32-accumulated outputs
within max relative error 1e-3 (relative to |ref| + 1e-2 rms(ref)); f16
outputs add at most one f16 rounding (< 1e-3); Q4 "BF16-faithful" outputs
within one bf16 ulp of the truncated oracle value (see gpu_util).
"""
import numpy as np
import pytest
import torch

from nnzap_amd import configs as cf
from nnzap_amd import formats as fm
from nnzap_amd import ops
from nnzap_amd import synth as S
from oracle import oracle as O

from gpu_util import assert_bf16_faithful, assert_close, host, tdev

pytestmark = pytest.mark.gpu


def _dw(dev, w):
    return ops.DeviceQWeight(dev, w)


def _f16(x):
    return O.f16(x)


# ------------------------------------------------------------ dequant -----
@pytest.mark.parametrize("bits", [1, 4])
def test_dequant_bit_exact(dev, bits):
    w = cf.q1_matrix(64, 512, 128, 201, 202) if bits == 1 else cf.q4_matrix(64, 512, 64, 203, 204, 205)
    dw = _dw(dev, w)
    out = torch.empty(w.M * w.K, dtype=torch.float32, device="cuda")
    ops.dispatch_dequant(dev, dw, out)
    dev.sync()
    ref = O.dequant(w).astype(np.float32).reshape(-1)
    assert np.array_equal(out.cpu().numpy(), ref)


# ------------------------------------------------------------ Q1 family ---
def test_config2_q1_qmv_f32(dev):
    """W[2048 x 6144] gs128, f32 x/y."""
    w, x = cf.config2()
    dw = _dw(dev, w)
    y = torch.empty(w.M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv(dev, dw, tdev(x), y)
    dev.sync()
    assert_close(host(y), O.qmv(w, x), what="config2")


@pytest.mark.parametrize("M,K", [(64, 5504), (48, 128), (33, 256), (130, 2048), (20, 4096),
                                 (3, 2048), (1, 4096)])
def test_q1_qmv_shapes(dev, M, K):
    w = cf.q1_matrix(M, K, 128, 300 + K, 301 + K)
    x = S.normal(302, K).astype(np.float32)
    dw = _dw(dev, w)
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv(dev, dw, tdev(x), y)
    dev.sync()
    assert_close(host(y), O.qmv(w, x), what=f"q1 {M}x{K}")


def test_q1_reference_fixture_k5504(dev):
    """transformer_test.zig:1606-1695 fixture (createTestPackedBuffer, seed 0x5A,
    sin input), tolerance tightened from the reference's 2e-3 absolute."""
    from test_oracle import reference_test_packed
    w = reference_test_packed(64, 5504, 0x5A)
    x = (np.float32(0.1) * np.sin(np.arange(5504, dtype=np.float32) * np.float32(0.037))
         + np.float32(0.05)).astype(np.float32)
    y = torch.empty(64, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv(dev, _dw(dev, w), tdev(x), y)
    dev.sync()
    ref = O.qmv(w, x)
    assert_close(host(y), ref, what="fixture")
    assert np.max(np.abs(host(y) - ref)) < 2e-3


@pytest.mark.parametrize("K", [2048, 6144])
def test_q1_f16_variants(dev, K):
    M = 1024
    w = cf.q1_matrix(M, K, 128, 310, 311)
    wb = cf.q1_matrix(M, K, 128, 312, 313)
    x16 = S.normal(314, K).astype(np.float16)
    x = x16.astype(np.float64)
    a, b = _dw(dev, w), _dw(dev, wb)
    xd = tdev(x16)
    ra, rb = O.qmv(w, x), O.qmv(wb, x)
    # f16in -> f32
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_f16in(dev, a, xd, y)
    dev.sync()
    assert_close(host(y), ra, what="f16in")
    # f16io
    y16 = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_qmv_f16io(dev, a, xd, y16)
    dev.sync()
    assert_close(host(y16), _f16(ra), what="f16io")
    # resadd
    res0 = S.normal(315, M).astype(np.float32)
    res = tdev(res0)
    ops.dispatch_qmv_f16io_resadd(dev, a, xd, res)
    dev.sync()
    assert_close(host(res), res0.astype(np.float64) + ra, what="resadd")
    # fused pair f16io / f16in
    ya = torch.empty(M, dtype=torch.float16, device="cuda")
    yb = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_qmv_fused_pair_f16io(dev, a, b, xd, ya, yb)
    dev.sync()
    assert_close(host(ya), _f16(ra), what="pair a")
    assert_close(host(yb), _f16(rb), what="pair b")
    fa = torch.empty(M, dtype=torch.float32, device="cuda")
    fb = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_fused_pair_f16in(dev, a, b, xd, fa, fb)
    dev.sync()
    assert_close(host(fa), ra, what="pair f16in a")
    assert_close(host(fb), rb, what="pair f16in b")
    # fused pair + silu (f16)
    ops.dispatch_qmv_fused_pair_silu_f16io(dev, a, b, xd, y16)
    dev.sync()
    assert_close(host(y16), _f16(O.silu(ra) * rb), what="pair silu f16io")


def test_q1_fused_pair_f32(dev):
    w = cf.q1_matrix(256, 2048, 128, 320, 321)
    wb = cf.q1_matrix(256, 2048, 128, 322, 323)
    x = S.normal(324, 2048).astype(np.float32)
    ya = torch.empty(256, dtype=torch.float32, device="cuda")
    yb = torch.empty(256, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_fused_pair(dev, _dw(dev, w), _dw(dev, wb), tdev(x), ya, yb)
    dev.sync()
    assert_close(host(ya), O.qmv(w, x), what="a")
    assert_close(host(yb), O.qmv(wb, x), what="b")


def test_config3_fused_gate_up_silu(dev):
    """silu(Wg x) * (Wu x), f32 x/out, [6144 x 2048] each."""
    wg, wu, x = cf.config3()
    out = torch.empty(wg.M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_fused_pair_silu(dev, _dw(dev, wg), _dw(dev, wu), tdev(x), out)
    dev.sync()
    assert_close(host(out), O.qmv_pair_silu(wg, wu, x), what="config3")


@pytest.mark.parametrize("K", [2048, 1024])
def test_q1_fused_norm_variants(dev, K):
    M = 512
    wa, wb = cf.q1_matrix(M, K, 128, 330, 331), cf.q1_matrix(M, K, 128, 332, 333)
    res = S.normal(334, K).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(335, K)).astype(np.float32)
    xn = O.norm_to_half(res, nw)
    a, b = _dw(dev, wa), _dw(dev, wb)
    rd, nd = tdev(res), tdev(nw)
    y = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_fused_norm_qmv_f16io(dev, a, rd, y, nd)
    dev.sync()
    assert_close(host(y), _f16(O.qmv(wa, xn)), what="norm qmv")
    ya = torch.empty(M, dtype=torch.float16, device="cuda")
    yb = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_fused_norm_pair_qmv_f16io(dev, a, b, rd, ya, yb, nd)
    dev.sync()
    assert_close(host(ya), _f16(O.qmv(wa, xn)), what="norm pair a")
    assert_close(host(yb), _f16(O.qmv(wb, xn)), what="norm pair b")
    ops.dispatch_fused_norm_pair_silu_f16io(dev, a, b, rd, y, nd)
    dev.sync()
    assert_close(host(y), _f16(O.qmv_pair_silu(wa, wb, xn)), what="norm pair silu")


@pytest.mark.parametrize("qrows,kvrows,K", [(2048, 1024, 2048), (256, 128, 256)])
def test_fused_norm_qkv_and_norm_lm_head(dev, qrows, kvrows, K):
    """One-launch norm + Q/K/V (equals the reference's norm-Q plus norm-KV-pair
    dispatches) and norm + f32-output QMV (rms_norm_f16out + qmv_f16in)."""
    wq = cf.q1_matrix(qrows, K, 128, 380, 381)
    wk = cf.q1_matrix(kvrows, K, 128, 382, 383)
    wv = cf.q1_matrix(kvrows, K, 128, 384, 385)
    res = S.normal(386, K).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(387, K)).astype(np.float32)
    xn = O.norm_to_half(res, nw)
    q = torch.empty(qrows, dtype=torch.float16, device="cuda")
    k = torch.empty(kvrows, dtype=torch.float16, device="cuda")
    v = torch.empty(kvrows, dtype=torch.float16, device="cuda")
    rd, nd = tdev(res), tdev(nw)
    ops.dispatch_fused_norm_qkv_f16io(dev, _dw(dev, wq), _dw(dev, wk), _dw(dev, wv), rd, q, k, v, nd)
    y = torch.empty(qrows, dtype=torch.float32, device="cuda")
    ops.dispatch_fused_norm_qmv_f16in(dev, _dw(dev, wq), rd, y, nd)
    dev.sync()
    assert_close(host(q), _f16(O.qmv(wq, xn)), what="qkv q")
    assert_close(host(k), _f16(O.qmv(wk, xn)), what="qkv k")
    assert_close(host(v), _f16(O.qmv(wv, xn)), what="qkv v")
    assert_close(host(y), O.qmv(wq, xn), what="norm lm head")


def test_norm_lm_head_vocabulary_rows_ragged(dev):
    """A vocabulary-sized norm + QMV (the LM head's form: nibble tables, 8
    rows per wave step) with a row count that is not a multiple of the rows
    per step: the last step is clamped back onto rows [M - 8, M) and must
    store only the rows no other step wrote."""
    M, K = 65536 + 13, 2048
    w = cf.q1_matrix(M, K, 128, 390, 391)
    res = S.normal(392, K).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(393, K)).astype(np.float32)
    y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
    ops.dispatch_fused_norm_qmv_f16in(dev, _dw(dev, w), tdev(res), y, tdev(nw))
    dev.sync()
    assert_close(host(y), O.qmv(w, O.norm_to_half(res, nw)), what="vocabulary rows")


@pytest.mark.parametrize("M", [6145, 5, 1])
def test_q4_qmv_ragged_rows(dev, M):
    """4-bit QMV on an f32 input (two rows per wave step) with row counts
    that leave a partial last step, or fewer rows than a step."""
    w = cf.q4_matrix(M, 2048, 64, 344, 345, 346)
    x = S.normal(347, 2048).astype(np.float32)
    y = torch.full((M,), float("nan"), dtype=torch.float32, device="cuda")
    ops.dispatch_q4mv(dev, _dw(dev, w), tdev(x), y)
    dev.sync()
    assert_close(host(y), O.qmv(w, x), what=f"q4 M={M}")


# ------------------------------------------------------------ Q4 family ---
def test_config1_q4_qmv_f32(dev):
    """W[6144 x 2048] gs64, f16 scale/bias, f32 x/y."""
    w, x = cf.config1()
    y = torch.empty(w.M, dtype=torch.float32, device="cuda")
    ops.dispatch_q4mv(dev, _dw(dev, w), tdev(x), y)
    dev.sync()
    assert_close(host(y), O.qmv(w, x), what="config1")


@pytest.mark.parametrize("gs,sdt", [(64, fm.DT_BF16), (128, fm.DT_F16), (32, fm.DT_BF16)])
def test_q4_f32_group_sizes(dev, gs, sdt):
    w = cf.q4_matrix(300, 1024, gs, 340, 341, 342, scale_dtype=sdt)
    x = S.normal(343, 1024).astype(np.float32)
    y = torch.empty(300, dtype=torch.float32, device="cuda")
    ops.dispatch_q4mv(dev, _dw(dev, w), tdev(x), y)
    dev.sync()
    assert_close(host(y), O.qmv(w, x), what=f"q4 gs{gs}")


@pytest.mark.parametrize("K", [2048, 6144])
def test_q4_faithful_variants(dev, K):
    """The reference's BF16-faithful Q4 kernels (bf16 scales, truncated outputs)."""
    M = 512
    wa = cf.q4_matrix(M, K, 64, 350, 351, 352, scale_dtype=fm.DT_BF16)
    wb = cf.q4_matrix(M, K, 64, 353, 354, 355, scale_dtype=fm.DT_BF16)
    x16 = (0.5 * S.normal(356, K)).astype(np.float16)
    x = x16.astype(np.float64)
    a, b = _dw(dev, wa), _dw(dev, wb)
    xd = tdev(x16)
    ra, rb = O.qmv(wa, x), O.qmv(wb, x)
    y16 = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_q4mv_f16io(dev, a, xd, y16)
    dev.sync()
    assert_bf16_faithful(host(y16), ra, "q4 f16io")
    y32 = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.dispatch_q4mv_f16in(dev, a, xd, y32)
    dev.sync()
    assert_bf16_faithful(host(y32), ra, "q4 f16in")
    res0 = S.normal(357, M).astype(np.float32)
    res = tdev(res0)
    ops.dispatch_q4mv_f16io_resadd(dev, a, xd, res)
    dev.sync()
    assert_close(host(res), res0 + O.bf16_trunc(ra), rtol=1e-2, what="q4 resadd")
    ya = torch.empty(M, dtype=torch.float16, device="cuda")
    yb = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_q4mv_fused_pair_f16io(dev, a, b, xd, ya, yb)
    dev.sync()
    assert_bf16_faithful(host(ya), ra, "q4 pair a")
    assert_bf16_faithful(host(yb), rb, "q4 pair b")
    ops.dispatch_q4mv_fused_pair_silu_f16io(dev, a, b, xd, y16)
    dev.sync()
    assert_bf16_faithful(host(y16), O.silu(ra) * rb, "q4 pair silu")


def test_q4_fused_norm_variants(dev):
    M, K = 512, 2048
    wa = cf.q4_matrix(M, K, 64, 360, 361, 362, scale_dtype=fm.DT_BF16)
    wb = cf.q4_matrix(M, K, 64, 363, 364, 365, scale_dtype=fm.DT_BF16)
    res = S.normal(366, K).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(367, K)).astype(np.float32)
    xn = O.norm_to_half(res, nw, q4_faithful=True)
    a, b = _dw(dev, wa), _dw(dev, wb)
    rd, nd = tdev(res), tdev(nw)
    y = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_q4_fused_norm_qmv_f16io(dev, a, rd, y, nd)
    dev.sync()
    assert_bf16_faithful(host(y), O.qmv(wa, xn), "q4 norm")
    ya = torch.empty(M, dtype=torch.float16, device="cuda")
    yb = torch.empty(M, dtype=torch.float16, device="cuda")
    ops.dispatch_q4_fused_norm_pair_qmv_f16io(dev, a, b, rd, ya, yb, nd)
    dev.sync()
    assert_bf16_faithful(host(ya), O.qmv(wa, xn), "q4 norm pair a")
    assert_bf16_faithful(host(yb), O.qmv(wb, xn), "q4 norm pair b")
    ops.dispatch_q4_fused_norm_pair_silu_f16io(dev, a, b, rd, y, nd)
    dev.sync()
    assert_bf16_faithful(host(y), O.qmv_pair_silu(wa, wb, xn), "q4 norm silu")


# ------------------------------------------------- committed golden vectors --
def test_configs_against_committed_vectors(dev):
    """Configs 1-3 (first 64 outputs) and the K=5504 fixture against the
    vectors committed in tests/golden/small_vectors.json."""
    import json
    import os
    from test_oracle import reference_test_packed
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "small_vectors.json")))
    w1, x1 = cf.config1()
    y = torch.empty(w1.M, dtype=torch.float32, device="cuda")
    ops.dispatch_q4mv(dev, _dw(dev, w1), tdev(x1), y)
    w2, x2 = cf.config2()
    y2 = torch.empty(w2.M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv(dev, _dw(dev, w2), tdev(x2), y2)
    wg, wu, x3 = cf.config3()
    y3 = torch.empty(wg.M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_fused_pair_silu(dev, _dw(dev, wg), _dw(dev, wu), tdev(x3), y3)
    wf = reference_test_packed(64, 5504, 0x5A)
    xf = (np.float32(0.1) * np.sin(np.arange(5504, dtype=np.float32) * np.float32(0.037))
          + np.float32(0.05)).astype(np.float32)
    yf = torch.empty(64, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv(dev, _dw(dev, wf), tdev(xf), yf)
    dev.sync()
    assert_close(host(y)[:64], g["config1"]["y64"], what="config1 golden")
    assert_close(host(y2)[:64], g["config2"]["y64"], what="config2 golden")
    assert_close(host(y3)[:64], g["config3"]["y64"], what="config3 golden")
    assert_close(host(yf), g["q1_fixture_k5504"]["y"], what="K=5504 golden")


# ----------------------------------------------------------- error paths ---
def test_qmv_rejects_bad_dims(dev):
    w = cf.q1_matrix(64, 256, 128, 370, 371)
    dw = _dw(dev, w)
    x = torch.zeros(256, dtype=torch.float32, device="cuda")
    y = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(ops.NnzError) as e:
        ops.dispatch_qmv(dev, dw, x, y, ops.QMVDims(64, 250, 128))
    assert e.value.code == -1
    with pytest.raises(ops.NnzError):
        ops.dispatch_q4mv(dev, dw, x, y)  # Q1 weight into a Q4 entry point


def test_c_abi_config2_from_c(dev):
    """BASELINE config 2 through the C ABI from a C translation unit
    (tests/c/abi_check.c: nnz_ctx_create, nnz_alloc, nnz_upload,
    nnz_dispatch_qmv, nnz_stream_sync, nnz_download), against the oracle and
    the committed golden vector."""
    import ctypes as C
    import json
    import os
    from pathlib import Path
    print("config2 QMV from C", flush=True)
    so = Path(__file__).resolve().parent / "c" / "libnnz_abi_check.so"
    if not so.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("nnz_c_tests_build", so.parent / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    lib = C.CDLL(str(so))
    w, x = cf.config2()
    y = np.zeros(w.M, dtype=np.float32)
    codes = np.ascontiguousarray(w.codes, dtype=np.uint32)
    scales = np.ascontiguousarray(w.scales, dtype=np.uint16)
    xc = np.ascontiguousarray(x, dtype=np.float32)
    err = C.create_string_buffer(256)
    rc = lib.nnz_abi_qmv_config(codes.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p),
                                xc.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p),
                                C.c_uint32(w.M), C.c_uint32(w.K), C.c_uint32(w.group_size), err)
    assert rc == 0, err.value.decode()
    assert_close(y, O.qmv(w, x), what="config2 from C")
    gold = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "small_vectors.json")))
    assert_close(y[:64], np.array(gold["config2"]["y64"]), what="config2 golden")


@pytest.mark.parametrize("V,H", [(5003, 2048), (1000, 4096), (777, 2560)])
def test_lm_head_bf16(dev, V, H):
    """Tied bf16 LM head (nnz_dispatch_lm_head_bf16): logits = table . x with
    f32 accumulation; the pipelined kernel (hidden 2048 / 4096, ragged row
    count) and the lane-group kernel (hidden 2560)."""
    table = S.f64_to_bf16_bits(0.02 * S.normal(600 + H, V * H)).reshape(V, H)
    x = S.normal(601, H).astype(np.float16)
    tb = torch.from_numpy(table.view(np.int16)).cuda().view(torch.bfloat16)
    y = torch.full((V,), float("nan"), dtype=torch.float32, device="cuda")
    ops.dispatch_lm_head_bf16(dev, tb, tdev(x), y)
    dev.sync()
    ref = S.bf16_bits_to_f32(table).astype(np.float64) @ x.astype(np.float64)
    assert_close(host(y), ref, what=f"lm_head_bf16 V={V} H={H}")

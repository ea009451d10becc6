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

from gpu_util import assert_bf16_faithful, assert_close, assert_close_f16, host, tdev

pytestmark = pytest.mark.gpu


@pytest.fixture
def q1_cores(dev):
    """Sets NNZ_OPT_Q1_MATRIX_CORES for one test, back to the default after."""
    from nnzap_amd import _lib as L

    def set_(v):
        dev.call("nnz_ctx_set_option", L.OPT_Q1_MATRIX_CORES, v)
    yield set_
    set_(0)


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


# ------------------------------------------------- stacked (one launch) ---
@pytest.mark.parametrize("kind", ["config1_q4", "config2_q1", "config3_pair_silu"])
@pytest.mark.parametrize("bpm", [0, 1, 3])
@pytest.mark.parametrize("cores", [1, 2])
def test_stacked_matches_single(dev, kind, bpm, cores, q1_cores):
    """nnz_dispatch_*_stacked: 5 independently drawn matrices of a config
    shape in one launch (blocks per matrix: library choice, 1, 3); every
    matrix's output equals the single-matrix launch bit for bit (a row is
    reduced by one wave in a fixed order, whatever the grid) and the oracle
    within the 1e-3 bar.  Both 1-bit kernels (matrix cores on / off: the
    K = 2048 pair has both)."""
    q1_cores(cores)
    n = 5
    if kind == "config1_q4":
        M, K, gs, bits = 6144, 2048, 64, 4
        sw = [ops.StackedQWeights(dev, M, K, gs, 4, n, 11, (0.005, 0.02), (-0.1, 0.1))]
    elif kind == "config2_q1":
        M, K, gs, bits = 2048, 6144, 128, 1
        sw = [ops.StackedQWeights(dev, M, K, gs, 1, n, 12, (0.01, 0.05))]
    else:
        M, K, gs, bits = 6144, 2048, 128, 1
        sw = [ops.StackedQWeights(dev, M, K, gs, 1, n, 13 + i, (0.01, 0.05)) for i in range(2)]
    x = torch.randn(n, K, device="cuda", generator=torch.Generator("cuda").manual_seed(14))
    y = torch.full((n, M), float("nan"), device="cuda")
    if kind == "config1_q4":
        ops.dispatch_q4mv_stacked(dev, sw[0], x, y, bpm)
    elif kind == "config2_q1":
        ops.dispatch_qmv_stacked(dev, sw[0], x, y, bpm)
    else:
        ops.dispatch_qmv_fused_pair_silu_stacked(dev, sw[0], sw[1], x, y, bpm)
    dev.sync()
    for i in (0, 2, n - 1):
        ws = [s.host(i) for s in sw]
        dws = [_dw(dev, w) for w in ws]
        y1 = torch.empty(M, device="cuda")
        if kind == "config1_q4":
            ops.dispatch_q4mv(dev, dws[0], x[i].contiguous(), y1)
        elif kind == "config2_q1":
            ops.dispatch_qmv(dev, dws[0], x[i].contiguous(), y1)
        else:
            ops.dispatch_qmv_fused_pair_silu(dev, dws[0], dws[1], x[i].contiguous(), y1)
        dev.sync()
        assert torch.equal(y[i], y1), f"{kind} matrix {i}: stacked != single launch"
        xi = x[i].cpu().numpy()
        ref = O.qmv(ws[0], xi) if kind != "config3_pair_silu" else O.qmv_pair_silu(ws[0], ws[1], xi)
        assert_close(host(y[i]), ref, what=f"{kind} matrix {i}")


def test_stacked_refuses_bad_strides(dev):
    """A stride that breaks the 16-byte code alignment, a zero count and a
    missing stack descriptor are refused with an error code, never launched."""
    import ctypes as C
    from nnzap_amd import _lib as L
    sw = ops.StackedQWeights(dev, 64, 2048, 128, 1, 2, 15)
    x = torch.zeros(2, 2048, device="cuda")
    y = torch.zeros(2, 64, device="cuda")
    bad = L.QmvStack(2, 0, sw.codes_stride + 4, sw.scales_stride, 2048 * 4, 64 * 4)
    rc = L.lib().nnz_dispatch_qmv_stacked(dev.ctx, sw.ref, C.c_void_p(x.data_ptr()),
                                          C.c_void_p(y.data_ptr()), sw.dims(), C.byref(bad))
    assert rc == L.EINVAL
    zero = L.QmvStack(0, 0, sw.codes_stride, sw.scales_stride, 2048 * 4, 64 * 4)
    rc = L.lib().nnz_dispatch_qmv_stacked(dev.ctx, sw.ref, C.c_void_p(x.data_ptr()),
                                          C.c_void_p(y.data_ptr()), sw.dims(), C.byref(zero))
    assert rc == L.EINVAL
    rc = L.lib().nnz_dispatch_qmv_stacked(dev.ctx, sw.ref, C.c_void_p(x.data_ptr()),
                                          C.c_void_p(y.data_ptr()), sw.dims(), None)
    assert rc == L.EINVAL


# ------------------------------------------- 1-bit on the matrix cores ---
def _cores_pair(dev, q1_cores, run):
    """run() under matrix cores forced on, then off: (mfma, valu) outputs."""
    q1_cores(1)
    a = run()
    q1_cores(2)
    b = run()
    return a, b


def _near_valu(a, b, what):
    """The two 1-bit kernels sum in different orders: agree to float32
    rounding, max |a - b| <= 1e-5 max |b| (the SiLU products are
    heavy-tailed, so max |b|, not rms, is the scale)."""
    a, b = host(a), host(b)
    d = np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-30)
    assert d <= 1e-5, f"{what}: matrix cores vs VALU kernel differ by {d:.2e} of max |y|"


@pytest.mark.parametrize("M", [1, 16, 33, 2048, 20011])
def test_q1_matrix_cores_qmv(dev, q1_cores, M):
    """dispatchQMV (f32 in/out) and dispatchQMVf16in at K = 2048, gs 128 on
    the block-scaled MFMA kernel (x split into five e4m3 terms, bits as fp4
    +-1): the oracle within 1e-3, the VALU kernel within float32 rounding;
    ragged row counts (1, 33, 20011 rows: partial 16-row tiles)."""
    w = cf.q1_matrix(M, 2048, 128, 700 + M % 97, 701)
    x = S.normal(702, 2048).astype(np.float32)
    dw = _dw(dev, w)
    xd = tdev(x)
    x16 = tdev(x, torch.float16)

    def run32():
        y = torch.full((M,), float("nan"), device="cuda")
        ops.dispatch_qmv(dev, dw, xd, y)
        dev.sync()
        return y

    def run16():
        y = torch.full((M,), float("nan"), device="cuda")
        ops.dispatch_qmv_f16in(dev, dw, x16, y)
        dev.sync()
        return y
    a, b = _cores_pair(dev, q1_cores, run32)
    assert_close(host(a), O.qmv(w, x), what=f"f32 M={M}")
    _near_valu(a, b, f"f32 M={M}")
    a, b = _cores_pair(dev, q1_cores, run16)
    assert_close(host(a), O.qmv(w, x16.cpu().numpy().astype(np.float64)), what=f"f16in M={M}")
    _near_valu(a, b, f"f16in M={M}")


@pytest.mark.parametrize("M", [6144, 151936])
def test_q1_matrix_cores_norm_lm_head(dev, q1_cores, M):
    """Final RMSNorm + LM head (f16-rounded normalised input, f32 logits) on
    the matrix cores, at the decoder's vocabulary size and a layer's."""
    w = cf.q1_matrix(M, 2048, 128, 710, 711)
    res = S.normal(712, 2048).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(713, 2048)).astype(np.float32)
    dw, rd, nd = _dw(dev, w), tdev(res), tdev(nw)

    def run():
        y = torch.full((M,), float("nan"), device="cuda")
        ops.dispatch_fused_norm_qmv_f16in(dev, dw, rd, y, nd)
        dev.sync()
        return y
    a, b = _cores_pair(dev, q1_cores, run)
    assert_close(host(a), O.qmv(w, O.norm_to_half(res, nw)), what=f"norm lm head M={M}")
    _near_valu(a, b, f"norm lm head M={M}")


@pytest.mark.parametrize("M", [6144, 100])
def test_q1_matrix_cores_pair_and_resadd(dev, q1_cores, M):
    """Config 3 (fused gate/up + SiLU, f32 I/O), the decoder's fused norm +
    gate/up + SiLU (f16 out) and the f16io residual add on the matrix cores."""
    wg, wu = cf.q1_matrix(M, 2048, 128, 720, 721), cf.q1_matrix(M, 2048, 128, 722, 723)
    x = S.normal(724, 2048).astype(np.float32)
    res = S.normal(725, 2048).astype(np.float32)
    nw = (1.0 + 0.1 * S.normal(726, 2048)).astype(np.float32)
    dg, du, xd, rd, nd = _dw(dev, wg), _dw(dev, wu), tdev(x), tdev(res), tdev(nw)

    def pair():
        y = torch.full((M,), float("nan"), device="cuda")
        ops.dispatch_qmv_fused_pair_silu(dev, dg, du, xd, y)
        dev.sync()
        return y

    def norm_pair():
        y = torch.full((M,), float("nan"), dtype=torch.float16, device="cuda")
        ops.dispatch_fused_norm_pair_silu_f16io(dev, dg, du, rd, y, nd)
        dev.sync()
        return y
    a, b = _cores_pair(dev, q1_cores, pair)
    assert_close(host(a), O.qmv_pair_silu(wg, wu, x), what="pair silu")
    _near_valu(a, b, "pair silu")
    a, b = _cores_pair(dev, q1_cores, norm_pair)
    xn = O.norm_to_half(res, nw)
    ref = O.qmv_pair_silu(wg, wu, xn)
    assert_close_f16(host(a), ref, what="norm pair silu (matrix cores)")
    assert_close_f16(host(b), ref, what="norm pair silu (VALU)")
    wo = cf.q1_matrix(M, 2048, 128, 727, 728)
    do = _dw(dev, wo)
    x16 = tdev((0.05 * x).astype(np.float16))
    base = S.normal(729, M).astype(np.float32)

    def resadd():
        r = tdev(base)
        ops.dispatch_qmv_f16io_resadd(dev, do, x16, r)
        dev.sync()
        return r
    a, b = _cores_pair(dev, q1_cores, resadd)
    ref = base.astype(np.float64) + O.qmv(wo, x16.cpu().numpy().astype(np.float64))
    assert_close(host(a), ref, what="f16io resadd")
    _near_valu(a, b, "f16io resadd")

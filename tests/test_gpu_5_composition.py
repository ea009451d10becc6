"""The reference's composed-path fixtures on the GPU, through the C ABI:

* "single-block forward matches CPU reference" (transformer_test.zig:1697-1997)
  as the reference's forwardBlock does it -- one dispatch per op family
  (fused norm + Q/K/V, fused attention with q/k norm, RoPE and KV append,
  O projection +=, fused norm + gate/up + SiLU*mul, down projection +=);
* "forwardDecode full path matches CPU reference" (:2086-2489) through the
  decoder model (nnz_model_forward_decode);
* the random-weight fixture of tests/test_oracle_composition.py through the
  model, five consecutive positions.

Bars: the TinyBlock outputs within 1e-3 per element (relative, floor 1e-2
rms) of the oracle, the random-weight logits within 1e-3 normwise, (whose composition tests/test_oracle_composition.py pins to a scalar
restatement of the reference's CPU functions), and within the reference
test's own tolerance of its float32 CPU path.
"""
import numpy as np
import pytest
import torch

import ref_cpu as R
from nnzap_amd import _lib as L
from nnzap_amd import ops
from nnzap_amd.model import DecoderModel
from nnzap_amd.ops import Device
from oracle.decoder import OracleDecoder

from gpu_util import assert_close, assert_close_normwise, host, tdev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mdev():
    d = Device(0, own_stream=True)
    yield d
    d.close()


def test_single_block_fixture_through_dispatches(dev):
    cfg, w, res, k, v, pos = R.single_block_case()
    print("single-block fixture (TinyBlock, position 3)", flush=True)
    wd = R.decoder_weights(cfg, [w])
    L0 = wd.layers[0]
    H, HD, I = cfg["hidden_size"], cfg["head_dim"], cfg["intermediate_size"]
    NQH, NKVH, MAXC = cfg["num_query_heads"], cfg["num_kv_heads"], cfg["max_context_length"]
    QD, KVD = NQH * HD, NKVH * HD
    dq = {n: ops.DeviceQWeight(dev, L0[n]) for n in ("q", "k", "v", "o", "gate", "up", "down")}
    norms = {n: tdev(L0[n]) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")}
    residual = tdev(np.array(res, dtype=np.float32))
    kc = R.kv_as_array(k, cfg).astype(np.float16)                       # [h][t][d]
    vc = R.kv_as_array(v, cfg).astype(np.float16).transpose(0, 2, 1)     # [h][d][t]
    kc_d, vc_d = tdev(kc), tdev(np.ascontiguousarray(vc))
    q = torch.empty(QD, dtype=torch.float16, device="cuda")
    kr = torch.empty(KVD, dtype=torch.float16, device="cuda")
    vr = torch.empty(KVD, dtype=torch.float16, device="cuda")
    att = torch.empty(QD, dtype=torch.float16, device="cuda")
    hid = torch.empty(I, dtype=torch.float16, device="cuda")
    ops.dispatch_fused_norm_qkv_f16io(dev, dq["q"], dq["k"], dq["v"], residual, q, kr, vr,
                                      norms["attn_norm"])
    fd = L.GQAFusedDims(NQH, NKVH, HD, pos + 1, MAXC, NQH // NKVH, pos, 1e-6, cfg["rope_theta"])
    gd = L.GQADims(NQH, NKVH, HD, pos + 1, MAXC, NQH // NKVH)
    scratch = torch.empty((ops.gqa_scratch_bytes(gd) + 3) // 4, dtype=torch.float32, device="cuda")
    ops.dispatch_gqa_attention_fused(dev, q, kc_d, vc_d, att, kr, vr, norms["q_norm"],
                                     norms["k_norm"], scratch, fd)
    ops.dispatch_qmv_f16io_resadd(dev, dq["o"], att, residual)
    ops.dispatch_fused_norm_pair_silu_f16io(dev, dq["gate"], dq["up"], residual, hid,
                                            norms["ffn_norm"])
    ops.dispatch_qmv_f16io_resadd(dev, dq["down"], hid, residual)
    dev.sync()
    got = host(residual)

    od = OracleDecoder(wd)
    od.kc[0] = R.kv_as_array(k, cfg)
    od.vc[0] = R.kv_as_array(v, cfg)
    want = od.layer(0, np.array([float(x) for x in res])[None, :], pos)[0]
    assert_close(got, want, what="single block residual")
    # the appended K row (float16, normed + roped) and V row
    kk, vv = host(kc_d), host(vc_d).transpose(0, 2, 1)
    assert np.max(np.abs(kk[:, pos] - od.kc[0, :, pos])) <= 2.0 ** -10 * np.max(np.abs(od.kc[0]))
    assert np.max(np.abs(vv[:, pos] - od.vc[0, :, pos])) <= 2.0 ** -10 * np.max(np.abs(od.vc[0]))
    assert np.array_equal(kk[:, :pos], od.kc[0, :, :pos])           # history untouched
    # the reference test's bar against its float32 CPU path (:1990-1995)
    want32 = np.array([float(x) for x in R.Ref().forward_block(cfg, res, w, list(k), list(v),
                                                                 pos, pos + 1)])
    assert np.max(np.abs(got - want32)) <= 8.0


def test_forward_decode_fixture_through_model(mdev):
    cfg, emb, layers, fnorm, tok, pos = R.forward_decode_case()
    print("forwardDecode fixture (TinyBlock, token 1, position 0)", flush=True)
    wd = R.decoder_weights(cfg, layers, emb, fnorm)
    m = DecoderModel(mdev, R.decoder_config(cfg))
    try:
        m.load(wd)
        got = m.forward_decode(tok, pos)
    finally:
        m.close()
    want = OracleDecoder(wd).forward([tok], pos)[0]
    assert_close(got, want, what="forwardDecode logits")
    n = cfg["num_kv_heads"] * cfg["max_context_length"] * cfg["head_dim"]
    want32 = np.array([float(x) for x in R.Ref().forward_decode(
        cfg, emb, layers, fnorm, tok, pos, [[np.float16(0)] * n], [[np.float16(0)] * n])])
    assert np.max(np.abs(got - want32)) <= 5e-2                     # the test's bar (:2480-2486)
    assert np.max(got) - np.min(got) > 1e-3
    assert int(np.argmax(got)) == int(np.argmax(want))


def test_random_fixture_steps_through_model(mdev):
    cfg, emb, layers, fnorm, w = R.soft_case()
    tokens = [3, 500, 77, 77, 260]
    print("random-weight fixture, 5 positions", flush=True)
    m = DecoderModel(mdev, R.decoder_config(cfg))
    od = OracleDecoder(w)
    try:
        m.load(w)
        for p, t in enumerate(tokens):
            got = m.forward_decode(t, p)
            # decoder bar (normwise): two layers of random weights with norm
            # scales near 1 let float16 rounding flips propagate -- the same
            # algorithm with float32 products lands up to 2.6e-2 per element
            # (near-zero logits) and 2.8e-4 normwise from the float64 oracle
            assert_close_normwise(got, od.forward([t], p)[0], what=f"position {p}")
    finally:
        m.close()

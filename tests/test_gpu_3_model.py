"""GPU parity of the whole decoder (forwardDecode / prefill / greedy generate).

Tiny model: logits of prefill and of single decode steps against the CPU
oracle (relative error <= 1e-3) and greedy tokens identical to the oracle.
Full Bonsai-1.7B shape: 512-token prompt through the
dequant-GEMM prefill, 256 greedy decode steps, tokens compared with the
committed golden fixture made by the oracle (tests/golden/make_golden.py).
"""
import json
import os

import numpy as np
import pytest

from nnzap_amd import configs as cf
from nnzap_amd.model import DecoderModel
from nnzap_amd.ops import Device
from oracle.decoder import OracleDecoder

from gpu_util import assert_close, assert_close_normwise

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def mdev():
    d = Device(0, own_stream=True)
    yield d
    d.close()


@pytest.fixture(scope="module")
def tiny():
    cfg = cf.TINY
    return cfg, cf.decoder_weights(cfg, norm_mode="unit")


def test_tiny_prefill_and_decode_logits(mdev, tiny):
    cfg, w = tiny
    m = DecoderModel(mdev, cfg)
    try:
        m.load(w)
        ids = cf.prompt_ids(cfg, 40)
        ref = OracleDecoder(w)
        ref_logits = ref.forward(list(ids), 0)
        got = m.prefill(ids, 0)
        assert_close_normwise(got, ref_logits[-1], what="prefill logits")
        assert int(np.argmax(got)) == int(np.argmax(ref_logits[-1]))
        # decode three more tokens one at a time (forwardDecode)
        for i, t in enumerate([5, 77, 300]):
            pos = len(ids) + i
            r = ref.forward([t], pos)[0]
            g = m.forward_decode(t, pos)
            assert_close_normwise(g, r, what=f"decode pos {pos}")
    finally:
        m.close()


def test_tiny_prefill_chunks_match_single_prefill(mdev, tiny):
    """Two prefill calls (start 0, start 30) equal one call over the same tokens."""
    cfg, w = tiny
    ids = cf.prompt_ids(cfg, 60)
    a = DecoderModel(mdev, cfg)
    b = DecoderModel(mdev, cfg)
    try:
        a.load(w)
        la = a.prefill(ids, 0)
        b.load(w)
        b.prefill(ids[:30], 0)
        lb = b.prefill(ids[30:], 30)
        assert_close_normwise(lb, la, rtol=1e-4, what="chunked prefill")
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_generate_matches_oracle(mdev, tiny, use_graph):
    cfg, w = tiny
    m = DecoderModel(mdev, cfg)
    try:
        m.load(w)
        prompt = cf.prompt_ids(cfg, 32)
        toks, margins, _ = m.generate(prompt, 48, use_graph=use_graph)
        ref_toks, ref_margins = OracleDecoder(w).generate(prompt, 48)
        assert np.array_equal(toks, ref_toks), (toks, ref_toks)
        # margins are logit differences: two logit errors of <= 1e-3 max|logit|
        assert np.max(np.abs(margins - ref_margins)) < 2e-3
    finally:
        m.close()


def test_tiny_tied_bf16_lm_head(mdev):
    cfg = cf.DecoderConfig(**{**cf.TINY.__dict__, "lm_head_kind": 1})
    w = cf.decoder_weights(cfg, norm_mode="unit")
    m = DecoderModel(mdev, cfg)
    try:
        m.load(w)
        ids = cf.prompt_ids(cfg, 16)
        assert_close_normwise(m.prefill(ids, 0), OracleDecoder(w).forward(list(ids), 0)[-1],
                              what="tied lm")
    finally:
        m.close()


def test_device_embedding_generator_matches_host(mdev):
    """nnz_synth_normal_bf16 reproduces synth.normal -> bf16 bit for bit."""
    import ctypes as C
    import torch
    from nnzap_amd import synth as S
    n = 1 << 20
    t = torch.empty(n, dtype=torch.int16, device="cuda")
    mdev.call("nnz_synth_normal_bf16", C.c_void_p(t.data_ptr()), n, 100, 0.02)
    mdev.sync()
    host = t.cpu().numpy().view(np.uint16)
    ref = S.f64_to_bf16_bits(0.02 * S.normal(100, n))
    assert np.array_equal(host, ref)


def test_config5_golden_tokens(mdev):
    """BASELINE config 5 at full size: 512 prompt ids, 256 greedy steps; tokens
    must equal the oracle's golden list (committed fixture)."""
    path = os.path.join(GOLDEN, "config5_tokens.json")
    if not os.path.exists(path):
        pytest.skip("golden fixture not generated yet")
    gold = json.load(open(path))
    cfg = cf.BONSAI_1_7B
    print("config5: building weights", flush=True)
    w = cf.decoder_weights(cfg, norm_mode=gold["norm_mode"], host_embed=False)
    m = DecoderModel(mdev, cfg)
    try:
        m.load(w, embed_on_device=True)
        prompt = cf.prompt_ids(cfg, gold["n_prompt"])
        print("config5: generating", flush=True)
        toks, margins, _ = m.generate(prompt, gold["n_new"], use_graph=True)
    finally:
        m.close()
    ref = np.array(gold["tokens"], dtype=np.uint32)
    first_bad = int(np.argmax(toks != ref)) if np.any(toks != ref) else -1
    assert first_bad == -1, (f"first mismatch at step {first_bad}: got {toks[first_bad]}, "
                            f"want {ref[first_bad]} (oracle margin {gold['margins'][first_bad]:.3e})")

"""GPU parity of device-side sampling (sampleToken on device) and of the
decode loop's stop tokens.

* The device random stream equals the oracle's restatement of Zig's
  DefaultPrng word for word after every draw.
* Tokens drawn on the device equal the oracle's for the same logits and the
  same stream wherever the oracle's draw (and top-p cut) lies farther from a
  decision boundary than float32 summation rounding (1e-5 + 2.5e-7 sqrt(V));
  nearer than that, the order of the sum decides and the device's token must
  be the inverse-CDF pick of r within that tolerance.
* Device draws follow the filtered softmax (chi-square).
* The model's generate with sampling equals the oracle's generate up to the
  first step whose decision margin is below 1e-4 (the model's logits differ
  from the oracle's by float32 rounding), and stop tokens end it unemitted.
"""
import numpy as np
import pytest
import torch

from nnzap_amd import _lib as L
from nnzap_amd import configs as cf
from nnzap_amd import ops
from nnzap_amd.model import DecoderModel
from nnzap_amd.ops import Device, NnzError
from oracle import sampling as SM
from oracle.decoder import OracleDecoder

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sdev():
    d = Device(0, own_stream=True)
    yield d
    d.close()


def _buffers(n, draws):
    ws = torch.empty(ops.sample_workspace_bytes(n), dtype=torch.uint8, device="cuda")
    rng = torch.zeros(4, dtype=torch.int64, device="cuda")
    out = torch.full((draws,), -1, dtype=torch.int32, device="cuda")
    prob = torch.zeros(draws, dtype=torch.float32, device="cuda")
    return ws, rng, out, prob


def _state(rng):
    return [int(v) for v in rng.cpu().numpy().view(np.uint64)]


def test_rng_stream_matches_oracle(sdev):
    ws, rng, out, prob = _buffers(1000, 64)
    logits = torch.randn(1000, device="cuda")
    ops.rng_seed(sdev, 12345, rng)
    p = SM.ZigPrng(12345)
    assert _state(rng) == p.s
    for i in range(64):
        ops.dispatch_sample(sdev, logits, out[i:i + 1], rng, ws, 1.0)
        p.float32()
    sdev.sync()
    assert _state(rng) == p.s


def _logits(n, seed, kind):
    g = np.random.default_rng(seed)
    x = g.normal(0.0, 2.5, n).astype(np.float32)
    if kind == "ties":            # coarse grid: many equal logits, ties at every cut
        x = (np.round(x * 2) / 2).astype(np.float32)
    if kind == "peaked":
        x[g.integers(0, n, 3)] += 12.0
    return x


CASES = [
    # (vocab, temperature, top_k, top_p, kind, draws)
    (1000, 1.0, 0, 1.0, "normal", 200),
    (1000, 0.7, 40, 1.0, "normal", 200),
    (1000, 0.8, 50, 0.9, "normal", 200),
    (1000, 1.2, 0, 0.95, "normal", 200),
    (1000, 1.0, 1, 1.0, "normal", 50),
    (1000, 1.0, 0, 1e-6, "normal", 50),     # smallest nucleus: the first candidate
    (1000, 1.0, 20, 0.7, "ties", 200),
    (1000, 1.0, 0, 0.6, "ties", 200),
    (777, 0.9, 2000, 0.5, "peaked", 100),
    (3000, 1.0, 1500, 1.0, "normal", 100),
    (151936, 0.8, 40, 0.95, "normal", 24),
    (151936, 1.0, 0, 0.9, "normal", 12),
    (151936, 0.6, 0, 1.0, "peaked", 12),
    (151936, 0.9, 0, 0.9, "peaked", 12),      # nucleus within the 64 largest
    (151936, 1.0, 100, 0.9, "normal", 12),    # lists cut below k, survivors > 64
    (151936, 1.0, 10000, 1.0, "normal", 6),   # cut lists miss part of the top-k set
    (4096, 1.0, 64, 0.8, "normal", 100),      # 64 survivors: one wave
    (4096, 1.0, 65, 1.0, "normal", 100),      # 65: the block-wide path
]


@pytest.mark.parametrize("V,T,k,p,kind,draws", CASES)
def test_sample_matches_oracle(sdev, V, T, k, p, kind, draws):
    x = _logits(V, V + draws, kind)
    ws, rng, out, prob = _buffers(V, draws)
    logits = torch.from_numpy(x).cuda()
    seed = 1000 + V + draws
    ops.rng_seed(sdev, seed, rng)
    print(f"sample V={V} T={T} k={k} p={p} {kind}", flush=True)
    for i in range(draws):
        ops.dispatch_sample(sdev, logits, out[i:i + 1], rng, ws, T, k, p, out_prob=prob[i:i + 1])
    sdev.sync()
    got = out.cpu().numpy()
    gp = prob.cpu().numpy()
    prng = SM.ZigPrng(seed)
    tol = SM.summation_tolerance(V)
    exact = 0
    for i in range(draws):
        d = SM.sample_token(x, T, k, p, prng)
        if d.margin >= tol:
            exact += 1
            assert got[i] == d.token, (i, got[i], d.token, d.margin)
            assert abs(gp[i] - d.prob) <= 1e-4 * max(d.prob, 1e-3) + 1e-6, (i, gp[i], d.prob)
        else:   # near a boundary: the pick must still be the inverse CDF of r
            assert d.within(int(got[i]), tol + 2 * d.q_cut), (i, got[i], d.token, d.margin)
    if V <= 3000:
        assert exact >= draws * 0.8
    assert _state(rng) == prng.s


def test_sample_distribution(sdev):
    V, T, k, p, n = 40, 0.9, 12, 0.85, 6000
    x = _logits(V, 3, "normal")
    want = SM.filtered_distribution(x, T, k, p)
    ws, rng, out, prob = _buffers(V, n)
    logits = torch.from_numpy(x).cuda()
    ops.rng_seed(sdev, 99, rng)
    for i in range(n):
        ops.dispatch_sample(sdev, logits, out[i:i + 1], rng, ws, T, k, p)
    sdev.sync()
    counts = np.bincount(out.cpu().numpy(), minlength=V).astype(np.float64)
    assert np.all(counts[want == 0] == 0)
    m = want > 0
    chi2 = np.sum((counts[m] - n * want[m]) ** 2 / (n * want[m]))
    dof = m.sum() - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof) + 10, (chi2, dof)


def test_temperature_zero_is_argmax(sdev):
    x = _logits(5000, 8, "normal")
    ws, rng, out, prob = _buffers(5000, 1)
    ops.dispatch_sample(sdev, torch.from_numpy(x).cuda(), out, rng, ws, 0.0)
    sdev.sync()
    assert int(out.cpu()[0]) == int(np.argmax(x))


# -- the decode loop ---------------------------------------------------------------

@pytest.fixture(scope="module")
def tiny():
    cfg = cf.TINY
    return cfg, cf.decoder_weights(cfg, norm_mode="unit")


@pytest.mark.parametrize("params", [(1.2, 5, 1.0, 5), (0.8, 40, 0.9, 7)])
def test_generate_sampled_matches_oracle(sdev, tiny, params):
    cfg, w = tiny
    prompt = cf.prompt_ids(cfg, 32)
    ref_toks, ref_probs, margins = OracleDecoder(w).generate_sampled(prompt, 24, *params)
    m = DecoderModel(sdev, cfg)
    try:
        m.load(w)
        m.set_sampling(*params)
        toks, probs, _ = m.generate(prompt, 24, use_graph=True)
        toks2, _, _ = m.generate(prompt, 24, use_graph=False)
    finally:
        m.close()
    assert np.array_equal(toks, toks2)          # graph replay == eager steps
    # steps before the first near-boundary decision must agree exactly
    bad = np.nonzero(margins < 1e-4)[0]
    n_cmp = int(bad[0]) if len(bad) else len(ref_toks)
    assert n_cmp >= 8
    assert np.array_equal(toks[:n_cmp], ref_toks[:n_cmp]), (toks, ref_toks, margins)
    np.testing.assert_allclose(probs[:n_cmp], ref_probs[:n_cmp], rtol=2e-3)


@pytest.mark.parametrize("use_graph", [True, False])
def test_generate_stops_at_eos(sdev, tiny, use_graph):
    cfg, w = tiny
    prompt = cf.prompt_ids(cfg, 32)
    ref, _ = OracleDecoder(w).generate(prompt, 16)
    # a stop token first produced at step j > 0
    j = next(i for i in range(1, 16) if ref[i] not in ref[:i])
    eos = int(ref[j])
    ref_eos, _ = OracleDecoder(w).generate(prompt, 16, eos=(eos, 7777))
    assert len(ref_eos) == j
    m = DecoderModel(sdev, cfg)
    try:
        m.load(w)
        m.set_eos([7777, eos])
        toks, margins, _ = m.generate(prompt, 16, use_graph=use_graph)
        assert np.array_equal(toks, ref[:j]) and len(margins) == j
        assert m.decode_status() == (j, True)
        m.set_eos([int(ref[0])])                  # stop token picked first: nothing emitted
        toks, _, _ = m.generate(prompt, 16, use_graph=use_graph)
        assert len(toks) == 0
        m.set_eos([])
        toks, _, _ = m.generate(prompt, 16, use_graph=use_graph)
        assert np.array_equal(toks, ref)
    finally:
        m.close()


@pytest.mark.parametrize("top_p", [float("nan"), 0.0, -0.5])
def test_bad_top_p_is_rejected(sdev, tiny, top_p):
    """applyTopP asserts 0 < p <= 1 (transformer.zig:3781-3790): NaN and
    p <= 0 are refused by both the model and the sampling dispatch (p >= 1
    stays "off", :3878)."""
    cfg, w = tiny
    m = DecoderModel(sdev, cfg)
    try:
        with pytest.raises(NnzError) as e:
            m.set_sampling(0.8, 0, top_p, 1)
        assert e.value.code == L.EINVAL
        m.set_sampling(0.8, 0, 1.5, 1)      # >= 1: top-p off, accepted
    finally:
        m.close()
    x = _logits(1000, 3, "normal")
    ws, rng, out, prob = _buffers(1000, 1)
    with pytest.raises(NnzError) as e:
        ops.dispatch_sample(sdev, torch.from_numpy(x).cuda(), out, rng, ws, 1.0, 0, top_p)
    assert e.value.code == L.EINVAL

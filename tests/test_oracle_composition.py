"""Pins the oracle's whole decode step (OracleDecoder) -- its op order and
rounding points -- to the reference's two composed-path tests, restated as
scalar loops in tests/ref_cpu.py independently of oracle/:

* "single-block forward matches CPU reference" (transformer_test.zig:1697-1997):
  TinyBlock, KV pre-filled for 3 positions, one token at position 3;
* "forwardDecode full path matches CPU reference" (:2086-2489): embedding ->
  block -> final norm -> tied LM head for token 1 at position 0.

Three comparisons per fixture:
1. oracle with the decode kernels' float16 rounding points vs the scalar
   restatement evaluated in float64 with the same rounding points (hooks):
   equal to float32 resolution -- pins op order and rounding points;
2. oracle without the activation roundings vs the restatement in the
   reference's own float32 arithmetic: equal to float32 summation error --
   pins the composition to the reference's CPU semantics;
3. oracle (rounded) vs the float32 restatement within the reference's own
   tolerances (8.0 absolute on the residual, 5e-2 on the logits).

The reference's pre-filled keys make every softmax one-hot, so its fixtures
cannot see a positive rescaling of q or k (a missing q_norm or k_norm).  A
third fixture (random weights, two layers, five consecutive positions) closes
that gap, and planted mistakes (gate/up swapped, a missing q_norm or k_norm,
k/v swapped, the two block norms exchanged, the wrong KV head, a dropped rounding point) are shown to
fail comparison 1.  Two closed forms pin what the fixtures leave open: with
zero O and down scales every block is the identity, and at position 0 the
attention output is v.
"""
import numpy as np
import pytest

import ref_cpu as R
from nnzap_amd import configs as cf
from nnzap_amd import formats as fm
from oracle import oracle as O
from oracle.decoder import OracleDecoder

TIGHT = 2e-7   # normwise, float32 resolution
# The reference's CPU path sums in float32, one term at a time: over K = 128
# to 512 terms of random sign the rounding error relative to the result is
# up to ~K * 2^-24 * sum|terms| / |sum| -- a few 1e-5 after two blocks.
F32_SUM = 5e-5


def normwise(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def _ref64(r16=True):
    return R.Ref(ft=float, r16=R.round16 if r16 else None, rope="build")


def _oracle_block(w_dec, k, v, cfg, res, pos, round16=True):
    od = OracleDecoder(w_dec, round16=round16)
    od.kc[0] = R.kv_as_array(k, cfg)
    od.vc[0] = R.kv_as_array(v, cfg)
    out = od.layer(0, np.array([float(x) for x in res])[None, :], pos)[0]
    return out, od


@pytest.fixture(scope="module")
def block():
    cfg, w, res, k, v, pos = R.single_block_case()
    return cfg, w, res, k, v, pos, R.decoder_weights(cfg, [w])


@pytest.fixture(scope="module")
def decode():
    cfg, emb, layers, fnorm, tok, pos = R.forward_decode_case()
    return cfg, emb, layers, fnorm, tok, pos, R.decoder_weights(cfg, layers, emb, fnorm)


def _block_ref(ref, cfg, w, res, k, v, pos):
    kc, vc = list(k), list(v)
    out = ref.forward_block(cfg, res, w, kc, vc, pos, pos + 1)
    return np.array([float(x) for x in out]), kc, vc


def test_single_block_rounding_points_pinned(block):
    cfg, w, res, k, v, pos, wd = block
    want, kc, vc = _block_ref(_ref64(), cfg, w, res, k, v, pos)
    got, od = _oracle_block(wd, k, v, cfg, res, pos)
    assert normwise(got, want) <= TIGHT
    # the appended K/V rows (float16) are identical
    assert np.array_equal(od.kc[0], R.kv_as_array(kc, cfg))
    assert np.array_equal(od.vc[0], R.kv_as_array(vc, cfg))


def test_single_block_matches_reference_f32(block):
    cfg, w, res, k, v, pos, wd = block
    want32, _, _ = _block_ref(R.Ref(), cfg, w, res, k, v, pos)
    got, _ = _oracle_block(wd, k, v, cfg, res, pos, round16=False)
    assert normwise(got, want32) <= F32_SUM
    # the rounded oracle (what the GPU is checked against) meets the
    # reference test's own bar against its float32 CPU path (:1990-1995)
    got_r, _ = _oracle_block(wd, k, v, cfg, res, pos)
    assert np.max(np.abs(got_r - want32)) <= 8.0


def _oracle_logits(wd, tok, pos, round16=True):
    return OracleDecoder(wd, round16=round16).forward([tok], pos)[0]


def _decode_ref(ref, cfg, emb, layers, fnorm, tok, pos):
    n = cfg["num_kv_heads"] * cfg["max_context_length"] * cfg["head_dim"]
    kcs = [[np.float16(0)] * n for _ in layers]
    vcs = [[np.float16(0)] * n for _ in layers]
    return np.array([float(x) for x in ref.forward_decode(cfg, emb, layers, fnorm, tok, pos,
                                                           kcs, vcs)])


def test_forward_decode_rounding_points_pinned(decode):
    cfg, emb, layers, fnorm, tok, pos, wd = decode
    want = _decode_ref(_ref64(), cfg, emb, layers, fnorm, tok, pos)
    assert normwise(_oracle_logits(wd, tok, pos), want) <= TIGHT


def test_forward_decode_matches_reference_f32(decode):
    cfg, emb, layers, fnorm, tok, pos, wd = decode
    want32 = _decode_ref(R.Ref(), cfg, emb, layers, fnorm, tok, pos)
    assert normwise(_oracle_logits(wd, tok, pos, round16=False), want32) <= F32_SUM
    got = _oracle_logits(wd, tok, pos)
    assert np.max(np.abs(got - want32)) <= 5e-2          # the test's bar (:2480-2486)
    assert np.max(got) - np.min(got) > 1e-3              # non-degenerate (:2380-2392)


# -- planted mistakes: each one must break comparison 1 ----------------------

def _mutated(wd, fn):
    import copy
    w2 = copy.deepcopy(wd)
    fn(w2.layers[0])
    return w2


@pytest.fixture(scope="module")
def soft():
    return R.soft_case()


def _soft_steps(ref, cfg, emb, layers, fnorm, tokens):
    """Consecutive decode steps of the restatement (positions 0..n-1)."""
    n = cfg["num_kv_heads"] * cfg["max_context_length"] * cfg["head_dim"]
    kcs = [[np.float16(0)] * n for _ in layers]
    vcs = [[np.float16(0)] * n for _ in layers]
    return [np.array([float(x) for x in ref.forward_decode(cfg, emb, layers, fnorm, t, p, kcs,
                                                            vcs)])
            for p, t in enumerate(tokens)]


SOFT_TOKENS = [3, 500, 77, 77, 260]


def _oracle_steps(w, tokens, round16=True):
    od = OracleDecoder(w, round16=round16)
    return [od.forward([t], p)[0] for p, t in enumerate(tokens)]


@pytest.fixture(scope="module")
def soft_want(soft):
    cfg, emb, layers, fnorm, w = soft
    return _soft_steps(_ref64(), cfg, emb, layers, fnorm, SOFT_TOKENS)


def test_soft_fixture_steps_pinned(soft, soft_want):
    """Random weights, two layers, five consecutive positions (attention over
    1..5 keys, GQA group 2): every step's logits equal the restatement's."""
    cfg, emb, layers, fnorm, w = soft
    want = soft_want
    got = _oracle_steps(w, SOFT_TOKENS)
    for p, (g, r) in enumerate(zip(got, want)):
        assert normwise(g, r) <= TIGHT, f"position {p}"
    want32 = _soft_steps(R.Ref(), cfg, emb, layers, fnorm, SOFT_TOKENS)
    for p, (g, r) in enumerate(zip(_oracle_steps(w, SOFT_TOKENS, round16=False), want32)):
        assert normwise(g, r) <= F32_SUM, f"position {p} (float32 reference)"


@pytest.mark.parametrize("mistake", ["swap_gate_up", "no_q_norm", "no_k_norm", "swap_k_v",
                                     "swap_norms"])
def test_planted_weight_mistakes_are_caught(soft, soft_want, mistake):
    cfg, emb, layers, fnorm, w = soft
    want = soft_want[2]

    def mutate(layer):
        if mistake == "swap_gate_up":
            layer["gate"], layer["up"] = layer["up"], layer["gate"]
        elif mistake == "no_q_norm":
            layer["q_norm"] = np.ones_like(layer["q_norm"])
        elif mistake == "no_k_norm":
            layer["k_norm"] = np.ones_like(layer["k_norm"])
        elif mistake == "swap_k_v":
            layer["k"], layer["v"] = layer["v"], layer["k"]
        else:   # attention-input and MLP-input norms exchanged
            layer["attn_norm"], layer["ffn_norm"] = layer["ffn_norm"], layer["attn_norm"]
    got = _oracle_steps(_mutated(w, mutate), SOFT_TOKENS[:3])[-1]
    assert normwise(got, want) > 1e3 * TIGHT


def test_planted_rounding_mistake_is_caught(block, decode):
    """Dropping the activation roundings changes the result far beyond the
    tight bar: the fixtures see the rounding points."""
    cfg, w, res, k, v, pos, wd = block
    want, _, _ = _block_ref(_ref64(), cfg, w, res, k, v, pos)
    got, _ = _oracle_block(wd, k, v, cfg, res, pos, round16=False)
    assert normwise(got, want) > 1e2 * TIGHT
    cfg, emb, layers, fnorm, tok, pos, wd = decode
    want = _decode_ref(_ref64(), cfg, emb, layers, fnorm, tok, pos)
    assert normwise(_oracle_logits(wd, tok, pos, round16=False), want) > 1e2 * TIGHT


def test_planted_gqa_head_mistake_is_caught(soft):
    """Query head h must read KV head h // group: a restatement that pairs
    the query heads with the other KV head differs from the oracle."""
    cfg, emb, layers, fnorm, w = soft

    class WrongHead(R.Ref):
        def gqa(self, q, k_cache, v_cache, nqh, hd, seq_len, max_ctx, group):
            out = []
            for h in range(nqh):
                out += self.attention_head(q[h * hd:(h + 1) * hd], k_cache, v_cache,
                                           (nqh - 1 - h) // group, hd, seq_len, max_ctx)
            return out
    bad = _soft_steps(WrongHead(ft=float, r16=R.round16, rope="build"), cfg, emb, layers, fnorm,
                      SOFT_TOKENS[:3])[-1]
    got = _oracle_steps(w, SOFT_TOKENS[:3])[-1]
    assert normwise(got, bad) > 1e3 * TIGHT


# -- closed forms ----------------------------------------------------------------

def _zero_scales(q):
    return fm.QWeight(q.bits, q.M, q.K, q.group_size, q.codes, np.zeros_like(q.scales), q.biases,
                      q.scale_dtype)


def test_zero_o_and_down_make_every_block_the_identity():
    """With the O and down projections zero, the residual passes every block
    unchanged: logits = LM head(f16(rmsnorm(embedding) * final_norm))."""
    cfg = cf.TINY
    w = cf.decoder_weights(cfg, norm_mode="unit")
    for layer in w.layers:
        layer["o"] = _zero_scales(layer["o"])
        layer["down"] = _zero_scales(layer["down"])
    ids = cf.prompt_ids(cfg, 5)
    got = OracleDecoder(w).forward(list(ids), 0)
    e = np.stack([np.float64(np.float32(x)) for x in
                  (w.embed_bf16[ids].astype(np.uint32) << 16).view(np.float32)])
    xn = e / np.sqrt(np.mean(e * e, axis=1, keepdims=True) + cfg.rms_eps) * w.final_norm
    xn = xn.astype(np.float16).astype(np.float64)
    lm = np.where(fm.unpack_q1(w.lm_head.codes, w.lm_head.K).astype(bool), 1.0, -1.0) * \
        np.repeat(w.lm_head.scales.view(np.float16).astype(np.float64), cfg.group_size, axis=1)
    want = (xn @ lm.T).astype(np.float32).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-9)


def test_position_zero_attention_output_is_v():
    """At position 0 the softmax has one key: each query head's output is the
    value row of its KV head (h // group), whatever q and k are.  With the
    gate scales zero (silu(0) = 0) the MLP adds nothing, so one block maps
    r to f32(r + W_o f16(v)) with v = f16(W_v f16(rmsnorm(r) * attn_norm))."""
    cfg = cf.DecoderConfig(**{**cf.TINY.__dict__, "num_layers": 1})
    w = cf.decoder_weights(cfg, norm_mode="unit")
    w.layers[0]["gate"] = _zero_scales(w.layers[0]["gate"])
    tok = 17
    od = OracleDecoder(w)
    res0 = od.embed_rows([tok])
    got = od.layer(0, res0.astype(np.float32).astype(np.float64), 0)[0]
    L0 = w.layers[0]
    r = res0[0]
    xn = (r / np.sqrt(np.mean(r * r) + cfg.rms_eps) * L0["attn_norm"]).astype(np.float16)
    Wv = O.dequant(L0["v"])
    v = (Wv @ xn.astype(np.float64)).astype(np.float16).astype(np.float64)
    D, g = cfg.head_dim, cfg.num_query_heads // cfg.num_kv_heads
    att = np.concatenate([v[(h // g) * D:(h // g + 1) * D] for h in range(cfg.num_query_heads)])
    want = (r + O.dequant(L0["o"]) @ att).astype(np.float32).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_torch_cpu_prefill_matches_oracle():
    """The CPU baseline's batched prefill (oracle/torch_cpu.py) equals the
    oracle's prompt pass (without the float16 activation roundings), in one
    call and in two chunks, and leaves the cache a following decode step
    continues from."""
    import torch
    from oracle.torch_cpu import TorchDecoder
    cfg = cf.TINY
    w = cf.decoder_weights(cfg, norm_mode="unit")
    od = OracleDecoder(w, round16=False)
    ids = list(cf.prompt_ids(cfg, 20))
    want = od.forward(ids, 0)[-1]
    xs = torch.from_numpy(od.embed_rows(ids).astype(np.float32))
    td = TorchDecoder(w, cfg.max_context_length)
    assert normwise(td.prefill(xs, 0).numpy(), want) <= 4 * F32_SUM
    x = torch.from_numpy(od.embed_rows([7])[0].astype(np.float32))
    assert normwise(td.step(x, 20).numpy(), od.forward([7], 20)[0]) <= 4 * F32_SUM
    tc = TorchDecoder(w, cfg.max_context_length)
    tc.prefill(xs[:12], 0)
    assert normwise(tc.prefill(xs[12:], 12).numpy(), want) <= 4 * F32_SUM


def test_torch_cpu_baseline_matches_oracle():
    """The timed CPU baseline (oracle/torch_cpu.py, float32 torch) computes the
    oracle's decode step (without the float16 activation roundings), both
    with pre-dequantised weights and dequantising on every call."""
    import torch
    from oracle.torch_cpu import TorchDecoder
    cfg = cf.TINY
    w = cf.decoder_weights(cfg, norm_mode="unit")
    od = OracleDecoder(w, round16=False)
    tds = [TorchDecoder(w, cfg.max_context_length, predequantise=p) for p in (True, False)]
    for pos, tok in enumerate([5, 300, 300, 17]):
        want = od.forward([tok], pos)[0]
        x = torch.from_numpy(od.embed_rows([tok])[0].astype(np.float32))
        for td in tds:
            got = td.step(x, pos).numpy()
            # float32 sums, plus the float16 KV cache: a float32 k or v can
            # round to the neighbouring float16 of the float64 one
            assert normwise(got, want) <= 4 * F32_SUM, f"position {pos}"

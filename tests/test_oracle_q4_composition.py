"""Pins the oracle's q4_mlx decode step (OracleDecoder with a 4-bit config):
its op order and every BF16 truncation point, against the independent
restatement in tests/ref_cpu_q4.py (written from the reference's Q4 Metal
kernels, q4mv_bf16_specialized.metal and transformer.metal:505-677).

* The restatement, token by token with its own KV caches, and the oracle's
  batched prefill agree on every token's logits to float32 resolution, and
  on the float16 caches bit for bit.
* Each BF16 truncation point dropped in turn from the restatement (the
  embedding row, the fused-norm inputs, the Q/K/V stores, the O and down
  residual additions, the SiLU*mul store, the final norm, the logits) makes
  it disagree with the oracle by orders of magnitude more than that: every
  point is observable, and the oracle has each of them where the reference
  kernels put it.
"""
import numpy as np
import pytest

import ref_cpu as R
import ref_cpu_q4 as R4
from nnzap_amd import configs as cf
from oracle.decoder import OracleDecoder

TIGHT = 2e-7      # normwise, float32 resolution (as for the 1-bit composition)
PLANTED = 1e-5    # a dropped truncation moves values by up to 2^-8 of themselves

# A small q4_mlx model: two layers, two query heads over one KV head, group
# size 64 (the Bonsai*_Q4 presets' group size), tied Q4 embedding / LM head.
CFG = cf.DecoderConfig(vocab_size=256, hidden_size=128, intermediate_size=256, num_layers=2,
                       num_query_heads=2, num_kv_heads=1, head_dim=64, max_context_length=8,
                       max_prefill_length=4, group_size=64, rope_theta=10000.0,
                       embed_kind=2, lm_head_kind=2, quant_format=1)
TOKENS = [17, 200, 3]


def normwise(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.fixture(scope="module")
def model():
    w = cf.decoder_weights(CFG, norm_mode="unit")
    od = OracleDecoder(w)
    logits = od.forward(TOKENS, 0)
    return w, od, logits


def _restated(w, drop=(), upto=len(TOKENS)):
    ref = R4.RefQ4(w, drop)
    kcs, vcs = ref.new_caches()
    out = [ref.decode(t, p, kcs, vcs) for p, t in enumerate(TOKENS[:upto])]
    return np.array(out), kcs, vcs


def test_q4_step_rounding_points_pinned(model):
    w, od, logits = model
    got, kcs, vcs = _restated(w)
    for p in range(len(TOKENS)):
        assert normwise(got[p], logits[p]) <= TIGHT, f"token {p}"
    cfg = {"num_kv_heads": CFG.num_kv_heads, "max_context_length": CFG.max_context_length,
           "head_dim": CFG.head_dim}
    for l in range(CFG.num_layers):
        assert np.array_equal(od.kc[l], R.kv_as_array(kcs[l], cfg))
        assert np.array_equal(od.vc[l], R.kv_as_array(vcs[l], cfg))


def test_q4_truncations_change_values(model):
    """The BF16 truncations are not no-ops on this model: the oracle's Q4
    logits differ from the same composition with every truncation dropped."""
    w, _, logits = model
    got, _, _ = _restated(w, drop=R4.POINTS, upto=1)
    assert normwise(got[0], logits[0]) > PLANTED


@pytest.mark.parametrize("point", R4.POINTS)
def test_q4_dropped_truncation_fails(model, point):
    w, _, logits = model
    # the logits point only touches the last step; the others propagate
    got, _, _ = _restated(w, drop=(point,), upto=2)
    err = normwise(got[1], logits[1])
    assert err > PLANTED, f"dropping the {point} truncation went unnoticed ({err:.2e})"


def test_bf16_round_is_truncation():
    """bf16_round keeps the high 16 bits of the float32 value: toward zero,
    for both signs, exact on BF16 values (q4mv_bf16_specialized.metal:52-57)."""
    x = np.float32(1.0) + np.float32(2.0 ** -8) * np.float32(0.99)   # just below 1 + 2^-8
    assert R4.bf16_round(float(x)) == 1.0
    assert R4.bf16_round(-float(x)) == -1.0
    assert R4.bf16_round(1.0 + 2.0 ** -7) == 1.0 + 2.0 ** -7
    assert R4.raw16(0x3F80, True) == 1.0 and R4.raw16(0xC000, True) == -2.0

"""Sampling oracle (CPU): the random stream and sampleToken.

Pins for oracle/sampling.py:
* SplitMix64 and xoshiro256++ reproduce published known answers (the
  SplitMix64 reference outputs for seed 0; the xoshiro256++ reference
  outputs from the state {1, 2, 3, 4});
* Random.float(f32) by its distribution (range, mean, quartiles, the small
  values the exponent construction reaches);
* the filters by the reference's own tests (transformer_test.zig:2561-2671);
* the sampler by its output distribution against the filtered softmax
  evaluated from the definition in float64 (chi-square).
"""
import numpy as np
import pytest

from oracle import sampling as SM


def test_splitmix64_known_answers():
    st, a = SM.splitmix64(0)
    st, b = SM.splitmix64(st)
    assert (a, b) == (0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4)


def test_xoshiro256pp_known_answers():
    p = SM.ZigPrng(state=[1, 2, 3, 4])
    assert [p.next() for _ in range(10)] == [
        41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205,
        9973669472204895162, 14011001112246962877, 12406186145184390807,
        15849039046786891736, 10450023813501588000]


def test_seeding_uses_four_splitmix_outputs():
    st, outs = 42, []
    for _ in range(4):
        st, o = SM.splitmix64(st)
        outs.append(o)
    assert SM.ZigPrng(42).s == outs


def test_float32_distribution():
    p = SM.ZigPrng(7)
    u = np.array([p.float32() for _ in range(200_000)], dtype=np.float64)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.004
    for q in (0.1, 0.25, 0.5, 0.75, 0.9):
        assert abs(np.mean(u < q) - q) < 0.004
    # the exponent comes from leading zeros: P(u < 2^-8) = 2^-8
    assert abs(np.mean(u < 2.0 ** -8) - 2.0 ** -8) < 0.0006


def test_float32_exponent_construction():
    """A draw with the top bit set lands in [0.5, 1); one with 40 leading
    zeros in [2^-41, 2^-40)."""
    class Fixed(SM.ZigPrng):
        def __init__(self, vals):
            self.vals = list(vals)

        def next(self):
            return self.vals.pop(0)
    assert 0.5 <= Fixed([(1 << 63) | 5]).float32() < 1.0
    v = Fixed([(1 << 23) | 3]).float32()    # clz = 40
    assert 2.0 ** -41 <= v < 2.0 ** -40


# -- the reference's sampling tests (transformer_test.zig:2561-2671) ------------

def test_greedy_returns_argmax():
    logits = np.array([0.1, 5.0, 2.0, 3.0], dtype=np.float32)
    tok = SM.sample_token(logits, 0.0, 0, 1.0, SM.ZigPrng(999)).token
    assert tok == int(np.argmax(logits)) == 1


def test_apply_temperature_scales():
    out = SM.apply_temperature(np.array([4.0, 8.0, -2.0, 6.0]), 2.0)
    np.testing.assert_allclose(out, [2.0, 4.0, -1.0, 3.0], atol=1e-6)


def test_apply_top_k_keeps_largest():
    out = SM.apply_top_k(np.array([1.0, 5.0, 3.0, 2.0, 4.0], dtype=np.float32), 2)
    assert out[1] == 5.0 and out[4] == 4.0
    assert np.all(np.isneginf(out[[0, 2, 3]]))


def test_apply_top_p_keeps_dominant():
    out, _, _ = SM.apply_top_p(np.array([0.0, 0.0, 10.0, 0.0], dtype=np.float32), 0.8)
    assert out[2] > -100.0
    assert np.all(np.isneginf(out[[0, 1, 3]]))


def test_top_k_keeps_ties_at_threshold():
    x = np.array([3.0, 1.0, 2.0, 2.0, 2.0, 0.5], dtype=np.float32)
    out = SM.apply_top_k(x, 2)          # threshold 2.0: three tokens tie
    assert np.isfinite(out).sum() == 4


@pytest.mark.parametrize("T,k,p", [(1.0, 0, 1.0), (0.7, 6, 1.0), (1.3, 0, 0.8), (0.9, 10, 0.9)])
def test_sampler_matches_filtered_distribution(T, k, p):
    rng = np.random.default_rng(5)
    logits = rng.normal(0, 1.5, 24).astype(np.float32)
    want = SM.filtered_distribution(logits, T, k, p)
    prng = SM.ZigPrng(123)
    n = 12000
    counts = np.zeros(len(logits))
    for _ in range(n):
        counts[SM.sample_token(logits, T, k, p, prng).token] += 1
    assert np.all(counts[want == 0] == 0)
    m = want > 0
    chi2 = np.sum((counts[m] - n * want[m]) ** 2 / (n * want[m]))
    dof = m.sum() - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof) + 10, (chi2, dof)

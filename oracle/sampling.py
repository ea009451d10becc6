"""CPU oracle of token sampling -- TEST INFRASTRUCTURE ONLY.

Restates nnmetal's sampleToken (nnmetal/src/transformer.zig:3860-3894) with
its filters -- applyTemperature (:3709-3719), applyTopK (:3743-3766),
applyTopP (:3768-3816), softmaxInPlace (:3721-3741) -- and the inverse-CDF
draw sampleFromDistribution (:3896-3908), in float32 with the reference's
sequential summation order.

The random stream is generate's ``std.Random.DefaultPrng.init(seed)``
(:3969-3972).  That generator lives in the Zig standard library (Zig 0.15.2,
``nnmetal/build.zig.zon:5``), which is not part of the reference tree; its
published algorithms are restated here:

* ``Xoshiro256`` = xoshiro256++ (Blackman and Vigna, 2018), 4 x u64 state;
* ``Xoshiro256.init`` fills the state with four SplitMix64 outputs
  (Steele, Lea and Flood, 2014) started from the seed;
* ``Random.int(u64)`` is one ``next()``; ``Random.float(f32)`` takes 23
  random mantissa bits and an exponent of ``126 - clz`` of the same 64-bit
  draw (further draws only when clz >= 41).

Pinning: SplitMix64 and xoshiro256++ against published known answers, the
float conversion by its distribution, the filters by the reference's own
tests (transformer_test.zig:2561-2671) and the sampler by its output
distribution (tests/test_sampling.py).  The exact draw sequence of Zig's
generator cannot be run here (no Zig toolchain): parity with Zig itself is
unpinned beyond the restated published algorithm.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1


def splitmix64(state: int):
    """One SplitMix64 step: (new state, output)."""
    state = (state + 0x9E3779B97F4A7C15) & M64
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return state, z ^ (z >> 31)


def _rotl(x: int, k: int) -> int:
    return ((x << k) | (x >> (64 - k))) & M64


class ZigPrng:
    """std.Random.DefaultPrng (Xoshiro256) with Random.float(f32)."""

    def __init__(self, seed: int | None = None, state=None):
        if state is not None:
            self.s = [int(v) & M64 for v in state]
            return
        st, self.s = seed & M64, []
        for _ in range(4):
            st, out = splitmix64(st)
            self.s.append(out)

    def next(self) -> int:
        s = self.s
        r = (_rotl((s[0] + s[3]) & M64, 23) + s[0]) & M64
        t = (s[1] << 17) & M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = _rotl(s[3], 45)
        return r

    def float32(self) -> np.float32:
        rnd = self.next()
        lz = 64 - rnd.bit_length()
        if lz >= 41:
            lz = 41 + (64 - self.next().bit_length())
            if lz == 41 + 64:
                lz += 32 - ((self.next() & 0xFFFFFFFF) | 0x7FF).bit_length()
        bits = ((126 - lz) << 23) | (rnd & 0x7FFFFF)
        return np.array([bits], dtype=np.uint32).view(np.float32)[0]


def _softmax_f32(x: np.ndarray) -> np.ndarray:
    """softmaxInPlace: max, exp(x - max), sequential f32 sum, * (1/sum)."""
    m = np.max(x)
    e = np.exp((x - m).astype(np.float32)).astype(np.float32)
    s = np.cumsum(e, dtype=np.float32)[-1]
    inv = np.float32(1.0) / s
    return (e * inv).astype(np.float32)


def apply_temperature(x: np.ndarray, temperature: float) -> np.ndarray:
    inv_t = np.float32(1.0) / np.float32(temperature)
    return (np.asarray(x, dtype=np.float32) * inv_t).astype(np.float32)


def apply_top_k(x: np.ndarray, k: int) -> np.ndarray:
    """applyTopK: the k-th largest value is the threshold, smaller -> -inf."""
    x = x.copy()
    if k >= len(x):
        return x
    thr = np.sort(x)[::-1][k - 1]
    x[x < thr] = -np.inf
    return x


def apply_top_p(x: np.ndarray, p: float):
    """applyTopP: walk tokens by probability (descending; ties by index),
    accumulate in f32, drop everything after the cumulative reaches p.
    Returns (filtered x, |cumulative at the cut - p| in float64, probability
    of the token at the cut)."""
    x = x.copy()
    q = _softmax_f32(x)
    order = np.argsort(-q.astype(np.float64), kind="stable")
    cum = np.cumsum(q[order], dtype=np.float32)
    hit = np.nonzero(cum >= np.float32(p))[0]
    margin, q_cut = np.inf, 0.0
    if len(hit):
        j = int(hit[0])
        x[order[j + 1:]] = -np.inf
        c64 = np.cumsum(q[order].astype(np.float64))
        margin = min(abs(c64[j] - p), abs(c64[j - 1] - p) if j > 0 else np.inf)
        q_cut = float(max(q[order[j]], q[order[j + 1]] if j + 1 < len(q) else 0.0))
    return x, margin, q_cut


class Draw:
    """One sampleToken result: ``token``, its probability ``prob``, the draw
    ``r``, the float64 cumulative distribution ``cdf`` it was drawn from, the
    float64 distance ``margin`` of r and of the top-p cut from the decision
    boundaries, and ``q_cut``, the probability at the top-p cut."""

    def __init__(self, token, prob, r, cdf, margin, q_cut):
        self.token, self.prob, self.r, self.cdf = token, prob, r, cdf
        self.margin, self.q_cut = margin, q_cut

    def __iter__(self):            # (token, prob, margin)
        return iter((self.token, self.prob, self.margin))

    def within(self, token: int, tol: float) -> bool:
        """Whether ``token`` is the inverse-CDF pick of r under this
        distribution when the boundaries may move by ``tol``."""
        if token == len(self.cdf) - 1 and self.r >= self.cdf[-1] - tol:
            return True
        if not 0 <= token < len(self.cdf):
            return False
        lo = self.cdf[token - 1] if token > 0 else 0.0
        return self.cdf[token] > lo and lo - tol <= self.r <= self.cdf[token] + tol


def summation_tolerance(n: int) -> float:
    """Typical rounding of a float32 sum of n probabilities, in any order:
    decisions closer than this to a boundary depend on the order."""
    return 1e-5 + 2.5e-7 * float(np.sqrt(n))


def sample_token(logits, temperature: float, top_k: int, top_p: float, prng: ZigPrng) -> Draw:
    """sampleToken (transformer.zig:3860-3894) with the reference's float32
    arithmetic and sequential sums."""
    x = np.asarray(logits, dtype=np.float32)
    if temperature == 0.0:
        i = int(np.argmax(x))
        cdf = np.zeros(len(x))
        cdf[i:] = 1.0
        return Draw(i, 1.0, 0.5, cdf, np.inf, 0.0)
    x = apply_temperature(x, temperature)
    if top_k > 0:
        x = apply_top_k(x, top_k)
    margin, q_cut = np.inf, 0.0
    if top_p < 1.0:
        x, margin, q_cut = apply_top_p(x, top_p)
    probs = _softmax_f32(x)
    r = prng.float32()
    cum = np.cumsum(probs, dtype=np.float32)
    hit = np.nonzero(cum > r)[0]
    c64 = np.cumsum(probs.astype(np.float64))
    if not len(hit):
        return Draw(len(x) - 1, 0.0, float(r), c64, min(margin, abs(c64[-1] - float(r))), q_cut)
    i = int(hit[0])
    lo = c64[i - 1] if i > 0 else 0.0
    margin = min(margin, abs(c64[i] - float(r)), abs(float(r) - lo) if probs[i] > 0 else np.inf)
    return Draw(i, float(probs[i]), float(r), c64, margin, q_cut)


def filtered_distribution(logits, temperature: float, top_k: int, top_p: float) -> np.ndarray:
    """The distribution sampleToken draws from, by definition and in float64:
    softmax(logits / T) restricted to the k largest (ties at the k-th value
    kept) and then to the smallest most-probable set holding mass >= p."""
    x = np.asarray(logits, dtype=np.float64) / temperature
    keep = np.ones(len(x), dtype=bool)
    if 0 < top_k < len(x):
        keep &= x >= np.sort(x)[::-1][top_k - 1]
    e = np.where(keep, np.exp(x - x[keep].max()), 0.0)
    q = e / e.sum()
    if top_p < 1.0:
        order = np.argsort(-q, kind="stable")
        cum = np.cumsum(q[order])
        j = int(np.searchsorted(cum, top_p, side="left"))
        drop = order[j + 1:]
        q[drop] = 0.0
        q /= q.sum()
    return q

"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each check is chosen so that a plausible mistake in the oracle (wrong bit or
nibble order, dropped bias term, sign flip, transposed operand, wrong RoPE
pairing, wrong KV layout) fails it.  Anchors: the reference's known-answer
tests and fixtures (cited), closed forms, and brute-force loops written
independently of the oracle's vectorised code.
"""
import math

import numpy as np
import pytest

from nnzap_amd import formats as fm
from nnzap_amd import synth as S
from nnzap_amd import configs as cf
from oracle import oracle as O


# ---------------------------------------------------------------- fixtures --
def reference_test_packed(M, K, seed, gs=128):
    """createTestPackedBuffer (transformer_test.zig:886-923): byte i =
    seed +% (i % 37); scale i = f16(0.1 + (seed % 10) * 0.01 + i * 0.005)."""
    nbytes = M * K // 8
    raw = ((seed + (np.arange(nbytes) % 37)) & 0xFF).astype(np.uint8)
    G = M * K // gs
    sc = (np.float32(0.1) + np.float32(seed % 10) * np.float32(0.01)
          + np.arange(G, dtype=np.float32) * np.float32(0.005)).astype(np.float16)
    return fm.QWeight(1, M, K, gs, raw.view("<u4").reshape(M, K // 32).copy(),
                      sc.view(np.uint16).reshape(M, K // gs), None, fm.DT_F16)


def brute_q1_row(w: fm.QWeight, x, r):
    """cpuQMV (transformer_test.zig:303-330) as a scalar loop over bytes."""
    by = np.ascontiguousarray(w.codes).view(np.uint8).reshape(-1)
    sc = np.ascontiguousarray(w.scales).view(np.float16).reshape(-1)
    acc = 0.0
    for c in range(w.K):
        flat = r * w.K + c
        bit = (int(by[flat // 8]) >> (flat % 8)) & 1
        s = float(sc[flat // w.group_size])
        acc += (s if bit else -s) * float(x[c])
    return acc


def brute_q4_row(w: fm.QWeight, x, r):
    wd = np.ascontiguousarray(w.codes).reshape(-1)
    sc = O.raw16_to_f64(w.scales.reshape(-1), w.scale_dtype)
    bi = O.raw16_to_f64(w.biases.reshape(-1), w.scale_dtype)
    acc = 0.0
    for c in range(w.K):
        flat = r * w.K + c
        n = (int(wd[flat // 8]) >> (4 * (flat % 8))) & 0xF
        g = flat // w.group_size
        acc += (sc[g] * n + bi[g]) * float(x[c])
    return acc


# ------------------------------------------------------------ known answers --
def test_embedding_known_answer_0xAA():
    """transformer_test.zig:1450-1541: bits 0xAA, scale 0.5, tokens [1, 3]
    -> alternating -0.5, +0.5 (bit 0 of 0xAA is clear)."""
    by = np.full(8, 0xAA, dtype=np.uint8)
    out = O.embed_q1([1, 3], by, np.array([0.5], dtype=np.float16), hidden=16, gs=128)
    expect = np.tile([-0.5, 0.5], 8)
    assert np.array_equal(out[0], expect) and np.array_equal(out[1], expect)


def test_scale_halving_known_answers():
    """model_test.zig:251-295: 1->0.5, 2->1, 0.5->0.25, -1->-0.5, 0.125->0.0625."""
    src = np.array([1.0, 2.0, 0.5, -1.0, 0.125], dtype=np.float16)
    got = fm.q1_affine_to_symmetric(src, None, check=False).view(np.float16).astype(np.float64)
    assert np.array_equal(got, [0.5, 1.0, 0.25, -0.5, 0.0625])


def test_affine_bias_equals_symmetric_config2():
    """BASELINE config 2 gives bias = -scale/2; then scale*bit + bias equals
    the symmetric +-scale/2 exactly, so dropping the bias is lossless."""
    w, x, scale, bias = cf.config2(return_affine=True)
    sub = slice(0, 16)
    aff = O.dequant_q1_affine(w.codes[sub], scale[sub], bias[sub], 16, w.K, w.group_size)
    w16 = fm.QWeight(1, 16, w.K, w.group_size, w.codes[sub], w.scales[sub], None, fm.DT_F16)
    assert np.array_equal(aff, O.dequant_q1(w16))


def test_affine_check_rejects_other_bias():
    with pytest.raises(ValueError):
        fm.q1_affine_to_symmetric(np.array([1.0], np.float16), np.array([-0.25], np.float16))


def test_argmax_first_maximum_wins():
    """transformer_test.zig:2495-2526: ties resolve to the first maximum."""
    assert O.argmax_first([1.0, 3.0, 2.0, 3.0]) == 1
    assert O.argmax_first([-1.0, -1.0]) == 0


def test_bf16_trunc_and_f16_round():
    # 1 + 2^-8 + 2^-20: truncation keeps 1 + 2^-8 ... no, bf16 has 7 mantissa
    # bits, so anything below 2^-7 is dropped by truncation.
    assert O.bf16_trunc(1.0 + 2 ** -7 + 2 ** -9) == 1.0 + 2 ** -7
    assert O.bf16_trunc(-(1.0 + 2 ** -8)) == -1.0            # toward zero
    assert O.f16(1.0 + 2 ** -11) == 1.0                      # tie to even
    assert O.f16(1.0 + 3 * 2 ** -11) == 1.0 + 2 ** -9


# ----------------------------------------------------------------- formats --
def test_q1_pack_bit_order():
    bits = np.zeros((1, 32), np.uint8)
    bits[0, 0] = 1
    bits[0, 9] = 1
    assert fm.pack_q1(bits)[0, 0] == (1 | (1 << 9))
    rnd = (S.words(99, 64).view(np.uint8) & 1).reshape(4, 64)
    assert np.array_equal(fm.unpack_q1(fm.pack_q1(rnd), 64), rnd)


def test_q4_pack_nibble_order():
    nib = np.arange(8, dtype=np.uint8)[None, :]
    assert fm.pack_q4(nib)[0, 0] == 0x76543210
    rnd = (S.words(98, 16).view(np.uint8) & 0xF).reshape(4, 16)
    assert np.array_equal(fm.unpack_q4(fm.pack_q4(rnd), 16), rnd)


# --------------------------------------------------------------------- QMV --
def test_qmv_reference_fixture_k5504():
    """transformer_test.zig:1606-1695: M=64, K=5504, seed 0x5A, x = 0.1 sin(0.037 i)
    + 0.05 (f32).  Oracle vs the scalar byte loop on sampled rows."""
    w = reference_test_packed(64, 5504, 0x5A)
    x = (np.float32(0.1) * np.sin(np.arange(5504, dtype=np.float32) * np.float32(0.037))
         + np.float32(0.05)).astype(np.float32)
    y = O.qmv(w, x)
    for r in (0, 1, 31, 63):
        assert abs(y[r] - brute_q1_row(w, x, r)) <= 1e-9 * (1 + abs(y[r]))


def test_q4_matches_scalar_loop():
    w = cf.q4_matrix(8, 256, 64, 21, 22, 23)
    x = S.normal(24, 256)
    y = O.qmv(w, x)
    for r in range(8):
        assert abs(y[r] - brute_q4_row(w, x, r)) <= 1e-9 * (1 + abs(y[r]))


def test_q4_bf16_scales_zero_extend():
    w = cf.q4_matrix(4, 64, 64, 31, 32, 33, scale_dtype=fm.DT_BF16)
    x = S.normal(34, 64)
    y = O.qmv(w, x)
    for r in range(4):
        assert abs(y[r] - brute_q4_row(w, x, r)) <= 1e-9 * (1 + abs(y[r]))


def test_qmv_invariants_q1():
    w = cf.q1_matrix(16, 512, 128, 41, 42)
    x1, x2 = S.normal(43, 512), S.normal(44, 512)
    # linearity
    assert np.allclose(O.qmv(w, 2 * x1 - 3 * x2), 2 * O.qmv(w, x1) - 3 * O.qmv(w, x2), rtol=1e-12,
                       atol=1e-12)
    # all bits flipped -> -y
    wf = fm.QWeight(1, w.M, w.K, w.group_size, ~w.codes, w.scales, None, fm.DT_F16)
    assert np.allclose(O.qmv(wf, x1), -O.qmv(w, x1), rtol=0, atol=1e-12)
    # all ones -> sum_g s_g * sum_{c in g} x_c
    w1 = fm.QWeight(1, w.M, w.K, w.group_size, np.full_like(w.codes, 0xFFFFFFFF), w.scales, None,
                    fm.DT_F16)
    s = w.scales.view(np.float16).astype(np.float64)
    gx = x1.reshape(-1, 128).sum(axis=1)
    assert np.allclose(O.qmv(w1, x1), s @ gx, rtol=1e-12)
    # x = e_j selects column j
    j = 77
    e = np.zeros(512)
    e[j] = 1.0
    assert np.array_equal(O.qmv(w, e), O.dequant_q1(w)[:, j])


def test_qmv_invariants_q4():
    w = cf.q4_matrix(8, 256, 64, 51, 52, 53)
    x = S.normal(54, 256)
    c = 11
    wc = fm.QWeight(4, w.M, w.K, w.group_size, np.full_like(w.codes, c * 0x11111111), w.scales,
                    w.biases, w.scale_dtype)
    s = O.raw16_to_f64(w.scales, w.scale_dtype)
    b = O.raw16_to_f64(w.biases, w.scale_dtype)
    gx = x.reshape(-1, 64).sum(axis=1)
    expect = ((s * c + b) * gx[None, :]).sum(axis=1)
    assert np.allclose(O.qmv(wc, x), expect, rtol=1e-9)


def test_fused_silu_equals_unfused():
    wg = cf.q1_matrix(32, 256, 128, 61, 62)
    wu = cf.q1_matrix(32, 256, 128, 63, 64)
    x = S.normal(65, 256)
    g, u = O.qmv(wg, x), O.qmv(wu, x)
    assert np.allclose(O.qmv_pair_silu(wg, wu, x), g / (1 + np.exp(-g)) * u, rtol=1e-14)


# ------------------------------------------------------------ norm / rope --
def test_rmsnorm_matches_scalar_formula():
    x = S.normal(71, 64)
    w = S.normal(72, 64)
    ms = sum(float(v) ** 2 for v in x) / 64
    expect = [float(x[i]) / math.sqrt(ms + 1e-6) * float(w[i]) for i in range(64)]
    assert np.allclose(O.rmsnorm(x, w), expect, rtol=1e-12)


def test_rope_reference_case():
    """transformer_test.zig:1185-1240: 2 heads x 8, position 3, theta 1e4,
    x_i = (i+1)*0.1; the reference's CPU form uses 1/pow(theta, 2p/d)."""
    x = (np.arange(16) + 1) * 0.1
    got = O.rope(x.reshape(2, 8), 3, 10000.0).reshape(-1)
    exp = x.copy()
    for h in range(2):
        for p in range(4):
            ang = 3 * (1.0 / 10000.0 ** (2 * p / 8))
            a, b = x[h * 8 + 2 * p], x[h * 8 + 2 * p + 1]
            exp[h * 8 + 2 * p] = a * math.cos(ang) - b * math.sin(ang)
            exp[h * 8 + 2 * p + 1] = a * math.sin(ang) + b * math.cos(ang)
    assert np.allclose(got, exp, atol=1e-6)


def test_rope_invariants():
    x = S.normal(73, 4 * 128).reshape(4, 128)
    assert np.array_equal(O.rope(x, 0, 1e6), x)                 # position 0 = identity
    y = O.rope(x, 12345, 1e6)
    n0 = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
    n1 = y[:, 0::2] ** 2 + y[:, 1::2] ** 2
    assert np.allclose(n0, n1, rtol=1e-12)                      # pair norms preserved
    # consecutive pairs, not NeoX halves: pair 0 is (x0, x1)
    e = np.zeros(128)
    e[0] = 1.0
    r = O.rope(e[None, :], 1, 1e6)[0]
    assert r[1] != 0.0 and r[64] == 0.0


# ---------------------------------------------------------------- attention --
def test_attention_single_token_returns_v():
    q = S.normal(81, 4 * 64).reshape(4, 64)
    K = S.normal(82, 2 * 8 * 64).reshape(2, 8, 64)
    V = S.normal(83, 2 * 8 * 64).reshape(2, 8, 64)
    out = O.attention_decode(q, K, V, 1, v_transposed=False)
    assert np.allclose(out[0], V[0, 0]) and np.allclose(out[3], V[1, 0])
    # transposed-V layout gives the same result
    out_t = O.attention_decode(q, K, V.transpose(0, 2, 1).copy(), 1, v_transposed=True)
    assert np.array_equal(out, out_t)


def test_attention_identical_keys_give_mean_v():
    q = S.normal(84, 2 * 64).reshape(2, 64)
    K = np.tile(S.normal(85, 64), (1, 5, 1)).reshape(1, 5, 64)
    V = S.normal(86, 5 * 64).reshape(1, 5, 64)
    out = O.attention_decode(q, K, V, 5, v_transposed=False)
    assert np.allclose(out[0], V[0].mean(axis=0), rtol=1e-12)


def test_attention_brute_force_with_reference_kv_fixture():
    """populateTestKVCache (transformer_test.zig:850-881): k = (h*L*D + t*D + d + 1)*0.05,
    v = ...*0.025 as f16; scalar-loop softmax attention."""
    Hkv, L, D, Hq = 2, 4, 8, 4
    k = np.zeros((Hkv, L, D))
    v = np.zeros((Hkv, L, D))
    for h in range(Hkv):
        for t in range(L):
            for d in range(D):
                seed = h * L * D + t * D + d + 1
                k[h, t, d] = O.f16(seed * 0.05)
                v[h, t, d] = O.f16(seed * 0.025)
    q = S.normal(87, Hq * D).reshape(Hq, D) * 0.1
    out = O.attention_decode(q, k, v, L, v_transposed=False)
    for h in range(Hq):
        kv = h // 2
        sc = [sum(q[h, d] * k[kv, t, d] for d in range(D)) / math.sqrt(D) for t in range(L)]
        m = max(sc)
        e = [math.exp(s - m) for s in sc]
        tot = sum(e)
        for d in range(D):
            assert abs(out[h, d] - sum(e[t] / tot * v[kv, t, d] for t in range(L))) < 1e-12


def test_embed_q4_truncates():
    w = cf.q4_matrix(4, 64, 64, 91, 92, 93, scale_dtype=fm.DT_BF16)
    out = O.embed_q4([2], w.codes, w.scales, w.biases, 64, 64, fm.DT_BF16)
    deq = O.dequant_q4(w)[2]
    assert np.array_equal(out[0], O.bf16_trunc(deq))


# -------------------------------------------------------------- decoder ----
@pytest.mark.parametrize("cfg", [cf.TINY, cf.TINY_Q4], ids=["q1", "q4"])
def test_decoder_batched_prefill_equals_token_by_token(cfg):
    """The oracle's batched prefill must equal the reference's token-by-token
    prefill (transformer.zig:4032-4068) on a tiny model (1-bit, and q4_mlx
    with its bf16 rounding points)."""
    from oracle.decoder import OracleDecoder
    w = cf.decoder_weights(cfg, norm_mode="unit")
    ids = cf.prompt_ids(cfg, 6)
    a = OracleDecoder(w)
    la = a.forward(list(ids), 0)
    b = OracleDecoder(w)
    lb = np.stack([b.forward([int(t)], i)[0] for i, t in enumerate(ids)])
    assert np.allclose(la, lb, rtol=0, atol=1e-9)
    assert np.array_equal(a.kc, b.kc)

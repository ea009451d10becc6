"""GPU parity of attention, norms, RoPE, KV append, embeddings, argmax and the
prefill dequant-GEMM against the CPU oracle."""
import numpy as np
import pytest
import torch

from nnzap_amd import _lib as L
from nnzap_amd import configs as cf
from nnzap_amd import ops
from nnzap_amd import synth as S
from oracle import oracle as O

from gpu_util import (assert_bf16_faithful, assert_close, assert_close_normwise, from_bits16, host,
                      tdev)

pytestmark = pytest.mark.gpu


def _scratch(dims):
    n = ops.gqa_scratch_bytes(dims)
    return torch.empty((n + 3) // 4, dtype=torch.float32, device="cuda")


# --------------------------------------------------------------- attention --
@pytest.mark.parametrize("L_", [512, 4096, 32768])
def test_config4_gqa_decode(dev, L_):
    """q bf16 [16,128] roped at position L, KV bf16 [8,L,128],
    scale 1/sqrt(128), fp32 accumulate; V given as [8, L, 128]."""
    print(f"config4 L={L_}", flush=True)
    q, k, v = cf.config4(L_)
    qd, kd, vd = from_bits16(q, "bf16"), from_bits16(k, "bf16"), from_bits16(v, "bf16")
    out = torch.empty(16, 128, dtype=torch.float32, device="cuda")
    dims = L.GQADims(16, 8, 128, L_, L_, 2)
    ops.dispatch_gqa_attention(dev, qd, kd, vd, out, _scratch(dims), dims, v_transposed=False,
                               rope_position=L_, rope_theta=1e6)
    dev.sync()
    qf = O.rope(S.bf16_bits_to_f32(q).astype(np.float64), L_, 1e6)
    ref = O.attention_decode(qf, S.bf16_bits_to_f32(k), S.bf16_bits_to_f32(v), L_, False)
    assert_close(host(out), ref, what=f"config4 L={L_}")


@pytest.mark.parametrize("L_,max_ctx,hq,hkv,d", [(1, 8, 4, 2, 64), (77, 128, 16, 8, 128),
                                                 (700, 1024, 8, 8, 128), (3000, 4096, 16, 2, 64),
                                                 (2000, 2048, 16, 4, 128), (104, 104, 16, 8, 128),
                                                 (99, 104, 8, 8, 128), (20000, 20000, 2, 1, 128),
                                                 (9000, 9216, 4, 2, 128)])
def test_gqa_transposed_v_f16(dev, L_, max_ctx, hq, hkv, d):
    """Reference layout: f16 caches, V transposed [h][d][max_ctx], f16 q/out."""
    rng_q = (0.3 * S.normal(400, hq * d)).astype(np.float16).reshape(hq, d)
    kf = np.zeros((hkv, max_ctx, d), np.float16)
    vf = np.zeros((hkv, d, max_ctx), np.float16)
    kf[:, :L_] = S.normal(401, hkv * L_ * d).astype(np.float16).reshape(hkv, L_, d)
    vf[:, :, :L_] = S.normal(402, hkv * L_ * d).astype(np.float16).reshape(hkv, d, L_)
    out = torch.empty(hq, d, dtype=torch.float16, device="cuda")
    dims = L.GQADims(hq, hkv, d, L_, max_ctx, hq // hkv)
    ops.dispatch_gqa_attention(dev, tdev(rng_q), tdev(kf), tdev(vf), out, _scratch(dims), dims)
    dev.sync()
    ref = O.attention_decode(rng_q.astype(np.float64), kf.astype(np.float64), vf.astype(np.float64),
                             L_, True)
    assert_close(host(out), O.f16(ref), what=f"gqa L={L_}")


@pytest.mark.parametrize("vt", [False, True])
def test_gqa_long_ragged_bf16(dev, vt):
    """16397 tokens (16384 + 13): the launcher walks chunks of two 64-token
    sub-chunks with an online softmax, the last chunk holding one ragged
    sub-chunk; bf16 caches in both V layouts, f32 q roped at 16397, f32 out."""
    L_, max_ctx, hq, hkv, d = 16397, 16400, 16, 8, 128
    print(f"gqa long ragged vt={vt}", flush=True)
    q = S.normal(410, hq * d).astype(np.float32).reshape(hq, d)
    kb = S.f32_to_bf16_bits(S.normal(411, hkv * max_ctx * d).astype(np.float32)).reshape(hkv, max_ctx, d)
    vb = S.f32_to_bf16_bits(S.normal(412, hkv * max_ctx * d).astype(np.float32))
    vb = vb.reshape(hkv, d, max_ctx) if vt else vb.reshape(hkv, max_ctx, d)
    out = torch.empty(hq, d, dtype=torch.float32, device="cuda")
    dims = L.GQADims(hq, hkv, d, L_, max_ctx, hq // hkv)
    ops.dispatch_gqa_attention(dev, tdev(q), from_bits16(kb, "bf16"), from_bits16(vb, "bf16"), out,
                               _scratch(dims), dims, v_transposed=vt, rope_position=L_,
                               rope_theta=1e6)
    dev.sync()
    qf = O.rope(q.astype(np.float64), L_, 1e6)
    ref = O.attention_decode(qf, S.bf16_bits_to_f32(kb), S.bf16_bits_to_f32(vb), L_, vt)
    assert_close(host(out), ref, what=f"gqa long vt={vt}")


@pytest.mark.parametrize("pos", [0, 5, 600, 1500])
def test_gqa_fused_norm_rope_kv(dev, pos):
    """transformer.metal:1467-1695 semantics: q/k per-head RMSNorm + RoPE, K/V
    append at `pos`, attention over pos+1 tokens; cache contents checked too."""
    hq, hkv, d, max_ctx, theta = 16, 8, 128, 2048, 1e6
    q = S.normal(410, hq * d).astype(np.float16).reshape(hq, d)
    kr = S.normal(411, hkv * d).astype(np.float16).reshape(hkv, d)
    vr = S.normal(412, hkv * d).astype(np.float16).reshape(hkv, d)
    qn = (1 + 0.1 * S.normal(413, d)).astype(np.float32)
    kn = (1 + 0.1 * S.normal(414, d)).astype(np.float32)
    kc = np.zeros((hkv, max_ctx, d), np.float16)
    vc = np.zeros((hkv, d, max_ctx), np.float16)
    if pos:
        kc[:, :pos] = (0.5 * S.normal(415, hkv * pos * d)).astype(np.float16).reshape(hkv, pos, d)
        vc[:, :, :pos] = S.normal(416, hkv * pos * d).astype(np.float16).reshape(hkv, d, pos)
    kcd, vcd = tdev(kc), tdev(vc)
    out = torch.empty(hq, d, dtype=torch.float16, device="cuda")
    fd = L.GQAFusedDims(hq, hkv, d, pos + 1, max_ctx, hq // hkv, pos, 1e-6, theta)
    dims = L.GQADims(hq, hkv, d, pos + 1, max_ctx, hq // hkv)
    ops.dispatch_gqa_attention_fused(dev, tdev(q), kcd, vcd, out, tdev(kr), tdev(vr), tdev(qn),
                                     tdev(kn), _scratch(dims), fd)
    dev.sync()
    kc_ref, vc_ref = kc.astype(np.float64), vc.astype(np.float64)
    ref = O.gqa_fused_step(q.astype(np.float64), kr.astype(np.float64), vr.astype(np.float64),
                           kc_ref, vc_ref, qn, kn, pos, theta, v_transposed=True)
    kg = host(kcd)
    assert_close(kg[:, pos], kc_ref[:, pos], what="k cache row")
    assert np.array_equal(host(vcd)[:, :, pos], vc_ref[:, :, pos])
    assert np.array_equal(kg[:, :pos], kc_ref[:, :pos])  # earlier rows untouched
    assert_close(host(out), O.f16(ref), what=f"fused pos={pos}")


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (4, 2, 64), (8, 8, 128)])
def test_gqa_fused_1pass_successive_positions(dev, hq, hkv, d):
    """Fused attention (one kernel, plus a merge kernel past one chunk) at
    consecutive positions sharing one scratch, with the sequence length read
    from device memory as in graph replay."""
    max_ctx, theta = 2048, 1e6
    qn = (1 + 0.1 * S.normal(417, d)).astype(np.float32)
    kn = (1 + 0.1 * S.normal(418, d)).astype(np.float32)
    kc = np.zeros((hkv, max_ctx, d), np.float16)
    vc = np.zeros((hkv, d, max_ctx), np.float16)
    start = 1400
    kc[:, :start] = (0.5 * S.normal(419, hkv * start * d)).astype(np.float16).reshape(hkv, start, d)
    vc[:, :, :start] = S.normal(420, hkv * start * d).astype(np.float16).reshape(hkv, d, start)
    kcd, vcd = tdev(kc), tdev(vc)
    kc_ref, vc_ref = kc.astype(np.float64), vc.astype(np.float64)
    max_seq = start + 8
    dims = L.GQAFusedDims(hq, hkv, d, max_seq, max_ctx, hq // hkv, 0, 1e-6, theta)
    gd = L.GQADims(hq, hkv, d, max_seq, max_ctx, hq // hkv)
    scr = torch.zeros(ops.gqa_scratch_bytes(gd) // 4 + 64, dtype=torch.float32, device="cuda")
    dseq = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty(hq, d, dtype=torch.float16, device="cuda")
    for i, pos in enumerate(range(start, start + 8)):
        q = S.normal(430 + i, hq * d).astype(np.float16).reshape(hq, d)
        kr = S.normal(440 + i, hkv * d).astype(np.float16).reshape(hkv, d)
        vr = S.normal(450 + i, hkv * d).astype(np.float16).reshape(hkv, d)
        dseq.fill_(pos + 1)
        ops.dispatch_gqa_attention_fused_1pass(dev, tdev(q), kcd, vcd, out, tdev(kr), tdev(vr),
                                               tdev(qn), tdev(kn), scr, dims, d_seq_len=dseq)
        dev.sync()
        ref = O.gqa_fused_step(q.astype(np.float64), kr.astype(np.float64), vr.astype(np.float64),
                               kc_ref, vc_ref, qn, kn, pos, theta, v_transposed=True)
        assert_close(host(out), O.f16(ref), what=f"1pass pos={pos}")
    assert_close(host(kcd)[:, start:start + 8], kc_ref[:, start:start + 8], what="k rows")
    assert np.array_equal(host(vcd)[:, :, start:start + 8], vc_ref[:, :, start:start + 8])


@pytest.mark.parametrize("pos", [30, 700, 1023])
@pytest.mark.parametrize("freq_table", [False, True])
@pytest.mark.parametrize("hq,hkv", [(16, 8), (24, 12)])
def test_attention_partials_merged_o_projection(dev, pos, freq_table, hq, hkv):
    """The decode step's two halves: attention to per-chunk partials, then the
    1-bit O projection (residual +=) merging them in its prologue.  Checked
    against the one-call fused attention + plain O projection on the GPU
    (same f16 attention output, different QMV order: 1e-4), and against the
    oracle (normwise, after the f16 rounding of the attention output).
    24 heads: K = 3072, rows of one and a half wave-widths (the second unit
    block is half past the row end)."""
    d, max_ctx, theta = 128, 1024, 1e6
    H = 2048
    qn = (1 + 0.1 * S.normal(461, d)).astype(np.float32)
    kn = (1 + 0.1 * S.normal(462, d)).astype(np.float32)
    kc = np.zeros((hkv, max_ctx, d), np.float16)
    vc = np.zeros((hkv, d, max_ctx), np.float16)
    kc[:, :pos] = (0.5 * S.normal(463, hkv * pos * d)).astype(np.float16).reshape(hkv, pos, d)
    vc[:, :, :pos] = S.normal(464, hkv * pos * d).astype(np.float16).reshape(hkv, d, pos)
    q = S.normal(465, hq * d).astype(np.float16).reshape(hq, d)
    kr = S.normal(466, hkv * d).astype(np.float16).reshape(hkv, d)
    vr = S.normal(467, hkv * d).astype(np.float16).reshape(hkv, d)
    wo = cf.q1_matrix(H, hq * d, 128, 468, 469)
    res0 = S.normal(470, H).astype(np.float32)
    dwo = ops.DeviceQWeight(dev, wo)
    seq = pos + 1
    dims = L.GQAFusedDims(hq, hkv, d, seq, max_ctx, hq // hkv, pos, 1e-6, theta)
    dseq = torch.full((1,), seq, dtype=torch.int32, device="cuda")
    n = ops.gqa_partial_chunks(seq)
    assert 1 <= n <= 16
    part_o = torch.empty(hq * n * d, dtype=torch.float32, device="cuda")
    part_ml = torch.empty(hq * n * 2, dtype=torch.float32, device="cuda")
    freqs = tdev(O.rope_inv_freq(d, theta)) if freq_table else None
    # path 1: partials + merged O projection
    kc1, vc1, res1 = tdev(kc), tdev(vc), tdev(res0)
    ops.dispatch_gqa_attention_partials(dev, tdev(q), kc1, vc1, tdev(kr), tdev(vr), tdev(qn),
                                        tdev(kn), part_o, part_ml, dims, d_seq_len=dseq,
                                        rope_inv_freq=freqs)
    ops.dispatch_qmv_merge_f16io_resadd(dev, dwo, part_o, part_ml, seq, d, res1, d_seq_len=dseq)
    # path 2: fused attention output + plain O projection
    kc2, vc2, res2 = tdev(kc), tdev(vc), tdev(res0)
    gd = L.GQADims(hq, hkv, d, seq, max_ctx, hq // hkv)
    scr = torch.zeros(ops.gqa_scratch_bytes(gd) // 4 + 64, dtype=torch.float32, device="cuda")
    att = torch.empty(hq * d, dtype=torch.float16, device="cuda")
    ops.dispatch_gqa_attention_fused_1pass(dev, tdev(q), kc2, vc2, att, tdev(kr), tdev(vr),
                                           tdev(qn), tdev(kn), scr, dims, d_seq_len=dseq)
    ops.dispatch_qmv_f16io_resadd(dev, dwo, att, res2)
    dev.sync()
    assert np.array_equal(host(kc1), host(kc2)) and np.array_equal(host(vc1), host(vc2))
    # The two O projections sum the same f32 products in different orders,
    # and the merge divides by the softmax sum as a reciprocal product, so an
    # f16 input where num * (1 / den) and num / den straddle a rounding edge
    # moves by one ulp.  Per row |res1 - res2| stays within 64 float32 ulps of
    # the sum of |terms| plus one ulp of the residual: two summation orders
    # emulated in float32 reach 0.04 of that, one flipped input ~0.06.
    r1, r2 = host(res1), host(res2)
    terms = np.abs(O.dequant(wo)) @ np.abs(host(att))
    bound = 64 * 2.0 ** -24 * terms + 2.0 ** -23 * np.abs(r2)
    worst = float(np.max(np.abs(r1 - r2) / bound))
    assert worst <= 1.0, f"merged vs unmerged pos={pos}: {worst:.2f} x the rounding bound"
    ref_att = O.f16(O.gqa_fused_step(q.astype(np.float64), kr.astype(np.float64),
                                     vr.astype(np.float64), kc.astype(np.float64),
                                     vc.astype(np.float64), qn, kn, pos, theta, v_transposed=True))
    ref = res0.astype(np.float64) + O.qmv(wo, ref_att.reshape(-1))
    assert_close_normwise(host(res1), ref, rtol=1e-3, what=f"oracle pos={pos}")


# ------------------------------------------------------------------ norms ---
@pytest.mark.parametrize("variant", ["f32", "f16", "bf16_f16"])
@pytest.mark.parametrize("H,T", [(2048, 3), (2560, 5), (4096, 9), (200, 2), (512, 513)])
def test_rms_norm_variants(dev, variant, H, T):
    """Wave-per-row path (hidden a multiple of 256 up to 4096, any row count)
    and the block-per-row path (hidden 200)."""
    x = S.normal(420, H * T).astype(np.float32)
    w = (1 + 0.1 * S.normal(421, H)).astype(np.float32)
    odt = torch.float32 if variant == "f32" else torch.float16
    out = torch.empty(T * H, dtype=odt, device="cuda")
    ops.dispatch_rms_norm(dev, tdev(x), tdev(w), out, H, T, bf16_trunc=(variant == "bf16_f16"))
    dev.sync()
    ref = O.rmsnorm(x.reshape(T, H), w).reshape(-1)
    if variant == "f16":
        ref = O.f16(ref)
    elif variant == "bf16_f16":
        ref = O.f16(O.bf16_trunc(ref))
        assert_close(host(out), ref, rtol=1e-2, what=variant)  # 1 bf16 ulp band
        return
    assert_close(host(out), ref, what=variant)


def test_rope_and_kv_update(dev):
    """rope (transformer_test.zig:1185-1240 case) and kv_cache_update (:1242-1336)."""
    vals = ((np.arange(16) + 1) * 0.1).astype(np.float32)
    t = tdev(vals)
    ops.dispatch_rope(dev, t, 2, 8, 3, 10000.0)
    dev.sync()
    assert_close(host(t), O.rope(vals.reshape(2, 8), 3, 10000.0).reshape(-1), rtol=1e-5, what="rope")
    # large position, f16 in place
    x = S.normal(430, 16 * 128).astype(np.float16)
    t16 = tdev(x)
    ops.dispatch_rope(dev, t16, 16, 128, 30000, 1e6)
    dev.sync()
    assert_close(host(t16), O.f16(O.rope(x.astype(np.float64).reshape(16, 128), 30000, 1e6).reshape(-1)),
                 what="rope f16")
    # kv update: K[h][pos][d], V[h][d][pos]
    hkv, d, max_ctx, pos = 2, 4, 8, 2
    k = (np.arange(hkv * d) * 0.5).astype(np.float32)
    v = (np.arange(hkv * d) * -0.25).astype(np.float32)
    kc = torch.zeros(hkv * max_ctx * d, dtype=torch.float16, device="cuda")
    vc = torch.zeros(hkv * max_ctx * d, dtype=torch.float16, device="cuda")
    ops.dispatch_kv_cache_update(dev, tdev(k), tdev(v), kc, vc, hkv, d, pos, max_ctx)
    dev.sync()
    K = host(kc).reshape(hkv, max_ctx, d)
    V = host(vc).reshape(hkv, d, max_ctx)
    assert np.array_equal(K[:, pos], k.reshape(hkv, d))
    assert np.array_equal(V[:, :, pos], v.reshape(hkv, d))
    K[:, pos] = 0
    V[:, :, pos] = 0
    assert not K.any() and not V.any()


def test_fused_rope_kernels(dev):
    hkv, hq, d, max_ctx, pos, theta = 8, 16, 128, 64, 17, 1e6
    k = S.normal(440, hkv * d).astype(np.float16)
    v = S.normal(441, hkv * d).astype(np.float16)
    ks = (1 + 0.1 * S.normal(442, d)).astype(np.float32)
    kc = torch.zeros(hkv, max_ctx, d, dtype=torch.float16, device="cuda")
    vc = torch.zeros(hkv, d, max_ctx, dtype=torch.float16, device="cuda")
    ops.dispatch_fused_rope_kv_cache(dev, tdev(k), tdev(v), kc, vc,
                                     L.FusedRoPEKVDims(hkv, d, pos, max_ctx, theta))
    dev.sync()
    kr = O.f16(O.rope(k.astype(np.float64).reshape(hkv, d), pos, theta))
    assert_close(host(kc)[:, pos], kr, what="fused rope kv")
    assert np.array_equal(host(vc)[:, :, pos], v.reshape(hkv, d).astype(np.float64))
    ops.dispatch_fused_k_norm_rope_kv_cache(dev, tdev(k), tdev(v), kc, vc, tdev(ks),
                                            L.FusedKNormRoPEKVDims(hkv, d, pos + 1, max_ctx, 1e-6, theta))
    dev.sync()
    kr2 = O.f16(O.head_norm_rope(k.astype(np.float64).reshape(hkv, d), ks, pos + 1, theta))
    assert_close(host(kc)[:, pos + 1], kr2, what="fused k norm rope kv")
    q = S.normal(443, hq * d).astype(np.float16)
    qd = tdev(q)
    ops.dispatch_fused_norm_rope(dev, qd, tdev(ks), L.FusedNormRoPEDims(hq, d, pos, 1e-6, theta))
    dev.sync()
    assert_close(host(qd).reshape(hq, d),
                 O.f16(O.head_norm_rope(q.astype(np.float64).reshape(hq, d), ks, pos, theta)),
                 what="fused norm rope")


# ------------------------------------------------------- embedding / misc ---
def test_embedding_known_answer(dev):
    """transformer_test.zig:1450-1541 (bits 0xAA, scale 0.5, tokens [1, 3])."""
    ids = tdev(np.array([1, 3], np.int32))
    bits = tdev(np.full(8, 0xAA, np.uint8))
    sc = tdev(np.array([0.5], np.float16))
    out = torch.empty(32, dtype=torch.float32, device="cuda")
    ops.dispatch_embedding_lookup(dev, ids, bits, sc, out, L.EmbedDims(4, 16, 2, 128))
    dev.sync()
    assert np.array_equal(host(out), np.tile([-0.5, 0.5], 16))


def test_embedding_q1_q4_bf16_random(dev):
    V, H = 64, 256
    w1 = cf.q1_matrix(V, H, 128, 450, 451)
    ids = np.array([0, 63, 17, 17, 5], np.int32)
    out = torch.empty(len(ids) * H, dtype=torch.float32, device="cuda")
    ops.dispatch_embedding_lookup(dev, tdev(ids), tdev(w1.codes.view(np.uint8)),
                                  tdev(w1.scales.view(np.float16)), out,
                                  L.EmbedDims(V, H, len(ids), 128))
    dev.sync()
    ref = O.embed_q1(ids, w1.codes.view(np.uint8).reshape(-1), w1.scales.view(np.float16).reshape(-1), H, 128)
    assert np.array_equal(host(out), ref.reshape(-1))
    w4 = cf.q4_matrix(V, H, 64, 452, 453, 454, scale_dtype=1 + 1)
    ops.dispatch_embedding_lookup_q4(dev, tdev(ids), tdev(w4.codes), tdev(w4.scales.view(np.int16)),
                                     tdev(w4.biases.view(np.int16)), out, L.EmbedDims(V, H, len(ids), 64))
    dev.sync()
    ref4 = O.embed_q4(ids, w4.codes, w4.scales, w4.biases, H, 64, 2)
    assert np.array_equal(host(out), ref4.reshape(-1))
    tab = S.f64_to_bf16_bits(S.normal(455, V * H)).reshape(V, H)
    ops.dispatch_embedding_lookup_bf16(dev, tdev(ids), tdev(tab.view(np.int16)), out,
                                       L.EmbedDims(V, H, len(ids), 0))
    dev.sync()
    assert np.array_equal(host(out), S.bf16_bits_to_f32(tab[ids]).reshape(-1).astype(np.float64))


def test_residual_silu_argmax(dev):
    r = tdev(np.arange(1, 9, dtype=np.float32))
    a = tdev((np.arange(1, 9) * 0.1).astype(np.float32))
    ops.dispatch_residual_add(dev, r, a)
    x = S.normal(460, 1000).astype(np.float32)
    s = torch.empty(1000, dtype=torch.float32, device="cuda")
    ops.dispatch_silu(dev, tdev(x), s)
    g, u = S.normal(461, 1000).astype(np.float16), S.normal(462, 1000).astype(np.float16)
    sm = torch.empty(1000, dtype=torch.float16, device="cuda")
    ops.dispatch_silu_elementwise_mul(dev, tdev(g), tdev(u), sm)
    logits = S.normal(463, 151936).astype(np.float32)
    logits[[100, 90000]] = 9.0  # tie: the first maximum wins
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    val = torch.zeros(2, dtype=torch.float32, device="cuda")
    ops.dispatch_argmax(dev, tdev(logits), idx, val)
    dev.sync()
    assert np.allclose(host(r), np.arange(1, 9) * 1.1, rtol=1e-6)
    assert_close(host(s), O.silu(x), rtol=1e-5, what="silu")
    assert_close(host(sm), O.f16(O.silu(g.astype(np.float64)) * u), what="silu mul f16")
    assert int(idx.item()) == 100
    assert host(val)[0] == 9.0 and host(val)[1] == 9.0


# ------------------------------------------------------------ prefill GEMM --
@pytest.mark.parametrize("P", [1, 37, 512])
def test_dequant_gemm_modes(dev, P):
    M, K = 1024, 2048
    wa, wb = cf.q1_matrix(M, K, 128, 470, 471), cf.q1_matrix(M, K, 128, 472, 473)
    a16 = (0.5 * S.normal(474, P * K)).astype(np.float16).reshape(P, K)
    A = a16.astype(np.float64)
    da, db = ops.DeviceQWeight(dev, wa), ops.DeviceQWeight(dev, wb)
    ad = tdev(a16)
    ra, rb = A @ O.dequant(wa).T, A @ O.dequant(wb).T
    out16 = torch.empty(P, M, dtype=torch.float16, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out16, L.GEMM_STORE_F16)
    out32 = torch.empty(P, M, dtype=torch.float32, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out32, L.GEMM_STORE_F32)
    res0 = S.normal(475, P * M).astype(np.float32).reshape(P, M)
    res = tdev(res0)
    ops.dispatch_dequant_gemm(dev, da, ad, res, L.GEMM_RESADD)
    ops.dispatch_dequant_gemm(dev, da, ad, out16, L.GEMM_SILU_PAIR, wb=db)
    dev.sync()
    assert_close(host(out32), ra, what="gemm f32")
    assert_close(host(res), res0 + ra, what="gemm resadd")
    assert_close(host(out16), O.f16(O.silu(ra) * rb), what="gemm silu pair")


@pytest.mark.parametrize("P,M,K,gs", [(100, 192, 2112, 64), (512, 128, 6144, 128),
                                       (64, 64, 192, 64), (1024, 64, 320, 64),
                                       (512, 4096, 576, 64)])
def test_dequant_gemm_shapes(dev, P, M, K, gs):
    """K not a multiple of the stage (last stage partial), group size 64,
    token tiles that do and do not divide by 8, grids of up to one block per
    CU (eight k-phases) and beyond (four), and the silu pair."""
    wa, wb = cf.q1_matrix(M, K, gs, 490, 491), cf.q1_matrix(M, K, gs, 492, 493)
    a16 = (0.5 * S.normal(494, P * K)).astype(np.float16).reshape(P, K)
    A = a16.astype(np.float64)
    da, db = ops.DeviceQWeight(dev, wa), ops.DeviceQWeight(dev, wb)
    ra, rb = A @ O.dequant(wa).T, A @ O.dequant(wb).T
    ad = tdev(a16)   # held until the sync: the kernels run on the library's stream
    out32 = torch.empty(P, M, dtype=torch.float32, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out32, L.GEMM_STORE_F32)
    out16 = torch.empty(P, M, dtype=torch.float16, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out16, L.GEMM_SILU_PAIR, wb=db)
    dev.sync()
    assert_close(host(out32), ra, what="gemm f32")
    assert_close(host(out16), O.f16(O.silu(ra) * rb), what="gemm silu pair")


@pytest.mark.parametrize("P,M,K,gs,sdt", [(37, 256, 2048, 64, 2), (512, 512, 2048, 64, 2),
                                           (100, 128, 6144, 128, 1), (64, 64, 192, 64, 2),
                                           (512, 2560, 2048, 64, 2)])
def test_dequant_gemm_q4_modes(dev, P, M, K, gs, sdt):
    """4-bit (q4_mlx) weights: s * (A . n) + b * sum(A) per group on the MFMA,
    every mode BF16-faithful like the Q4 decode kernels (one bf16 ulp bar).
    The last case has 320 blocks (more than one per CU), so the single-matrix
    modes run the two-k-phase kernel real 4-bit prefill takes at hidden 2560."""
    from nnzap_amd import formats as fm
    sd = fm.DT_BF16 if sdt == 2 else fm.DT_F16
    wa = cf.q4_matrix(M, K, gs, 520, 521, 522, scale_dtype=sd)
    wb = cf.q4_matrix(M, K, gs, 523, 524, 525, scale_dtype=sd)
    a16 = (0.5 * S.normal(526, P * K)).astype(np.float16).reshape(P, K)
    A = a16.astype(np.float64)
    da, db = ops.DeviceQWeight(dev, wa), ops.DeviceQWeight(dev, wb)
    ra, rb = A @ O.dequant(wa).T, A @ O.dequant(wb).T
    ad = tdev(a16)   # held until the sync: the kernels run on the library's stream
    out16 = torch.empty(P, M, dtype=torch.float16, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out16, L.GEMM_STORE_F16)
    out32 = torch.empty(P, M, dtype=torch.float32, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, out32, L.GEMM_STORE_F32)
    res0 = S.normal(527, P * M).astype(np.float32).reshape(P, M)
    res = tdev(res0)
    ops.dispatch_dequant_gemm(dev, da, ad, res, L.GEMM_RESADD)
    pair = torch.empty(P, M, dtype=torch.float16, device="cuda")
    ops.dispatch_dequant_gemm(dev, da, ad, pair, L.GEMM_SILU_PAIR, wb=db)
    dev.sync()
    # fp32 summation error of a K-term sum (random-walk bound, 4 sigma)
    se = 4 * 2.0 ** -24 * np.sqrt(K) * (np.abs(A) @ np.abs(O.dequant(wa)).T)
    assert_bf16_faithful(host(out32), ra, "q4 gemm f32", sum_err=se)
    assert_bf16_faithful(host(out16), ra, "q4 gemm f16", sum_err=se)
    # residual += bf16(sum): one bf16 ulp of the added term (the GPU's fp32 sum
    # and the fp64 oracle may straddle a truncation boundary) plus the f32 add
    ref = res0 + O.bf16_trunc(ra)
    err = np.abs(host(res).astype(np.float64) - ref)
    assert (err <= 2.0 ** -7 * np.abs(ra) + 2.0 ** -23 * np.abs(ref) + se + 2.0 ** -30).all(), \
        f"q4 gemm resadd: {int((err > 2.0 ** -7 * np.abs(ra)).sum())} elements beyond one bf16 ulp"
    # silu(a) * b: the fp32 summation errors of a and b propagate through
    # d(silu(a) b) = silu'(a) b da + silu(a) db, |silu'| <= 1.1
    se_b = 4 * 2.0 ** -24 * np.sqrt(K) * (np.abs(A) @ np.abs(O.dequant(wb)).T)
    se_pair = 1.1 * np.abs(rb) * se + np.abs(O.silu(ra)) * se_b
    assert_bf16_faithful(host(pair), O.silu(ra) * rb, "q4 gemm silu pair", sum_err=se_pair)


def test_gemm_row_equals_decode_qmv(dev):
    """Per-token equivalence: GEMM row p equals the decode QMV of token p."""
    M, K, P = 512, 2048, 8
    w = cf.q1_matrix(M, K, 128, 480, 481)
    a16 = S.normal(482, P * K).astype(np.float16).reshape(P, K)
    dw = ops.DeviceQWeight(dev, w)
    out = torch.empty(P, M, dtype=torch.float32, device="cuda")
    ops.dispatch_dequant_gemm(dev, dw, tdev(a16), out, L.GEMM_STORE_F32)
    y = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.dispatch_qmv_f16in(dev, dw, tdev(a16[5]), y)
    dev.sync()
    assert_close(host(out)[5], host(y), rtol=1e-4, what="gemm row vs qmv")

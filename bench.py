"""Benchmark of the MI355X decode hot path (one GPU).

Headline (BASELINE.json metric): greedy decode tok/s of the Bonsai-1.7B-shaped
config-5 model at batch 1 -- 28 layers, 1-bit gs128 linears, bf16 embeddings,
512-token prompt prefilled through the dequant-GEMM, then decode steps, each a
replay of one captured hipGraph with on-device argmax.  A "step" is one decode
token.  W warm-up steps run in a separate pass; the K timed steps are the first
K steps after a fresh 512-token prefill (positions 512..512+K-1), bracketed by
stream synchronisation.

Also reported (same JSON line):
  roofline      the dominant decode kernel: algorithmic bytes / average launch
                duration, the "stacked" figure: N launches back to back in one
                hipGraph, HIP events on the library's stream around the replay,
                every working set (weights, KV caches) rotated through >= 64
                distinct copies and >= 640 MB so every launch streams from HBM;
                per-dispatch device durations from rocprofv3 are in profiles/;
  qmv           configs 1-4 (4-bit QMV, 1-bit QMV, fused gate/up+SiLU, GQA
                decode attention at L = 512/4096/32768) in the same way;
  decode        also prefill tok/s and p50/p99 per-token latency of a host
                loop that waits for each token (the reference bench's outputs);
  decode_tied_lm_head  the same decoder with the tied bf16 embedding table
                as LM head (622 MB per token), and that GEMV's HBM fraction;
  cpu_baseline  the full 28-layer decode step in PyTorch float32 on this
                host's cores (pre-dequantised weights: 5 warm-ups, median of
                30; dequantising every step: a shorter sample);
  cpu_configs   configs 1-4 in PyTorch float32 on this host (median of 7
                after 2 warm-ups; --cpu-full: median of 30 after 5).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--lm-head q1|tied] [--quick]
                [--cpu-full]
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16/bf16 MFMA
BASELINE_TOKS = 182.8  # reference decode tok/s, Bonsai-1.7B Q1 bs1 (README.md:71-77)
ROTATE_BYTES = 640 << 20
MIN_COPIES = 64


def random_copies(shape, dtype, per_copy_bytes, seed):
    """Independently drawn N(0,1) device tensors (cast to dtype), at least
    MIN_COPIES of them and at least ROTATE_BYTES in all."""
    import torch
    n = max(MIN_COPIES, int(ROTATE_BYTES // per_copy_bytes) + 1)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    out = [torch.randn(shape, device="cuda", generator=g).to(dtype) for _ in range(n)]
    torch.cuda.synchronize()
    return out


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- decode ----
def bench_decode(args, dev, lm_head=None, latency=True):
    """Headline decode tok/s (see the module docstring), plus the
    reference bench's other outputs (bonsai_bench.zig:255-320): prefill tok/s
    (512 prompt tokens / prefill wall time, median of 3 after a warm-up) and
    the p50 / p99 per-token latency of a host loop that waits for every token
    before asking for the next (8 warm-up + 64 measured tokens; p50 =
    sorted[n/2], p99 = sorted[n*99/100])."""
    from nnzap_amd import configs as cf
    from nnzap_amd.model import DecoderModel

    lm_head = lm_head or args.lm_head
    cfg = cf.DecoderConfig(**{**cf.BONSAI_1_7B.__dict__,
                              "lm_head_kind": 1 if lm_head == "tied" else 0})
    t = time.time()
    # the tied model's table is generated on the device: build the host
    # weights without it
    w = cf.decoder_weights(cf.DecoderConfig(**{**cfg.__dict__, "lm_head_kind": 0}),
                           norm_mode="small", host_embed=False)
    if lm_head == "tied":
        w.lm_head = None
    m = DecoderModel(dev, cfg)
    m.load(w, embed_on_device=True)
    log(f"model ({lm_head} LM head) ready in {time.time() - t:.1f}s")
    prompt = cf.prompt_ids(cfg, args.prompt)
    # warm-up pass (separate prefill)
    m.decode_begin(prompt, max(args.warmup, 1))
    m.decode_steps(max(args.warmup, 1))
    m.decode_read(1)
    m.decode_end()
    # measured pass: prefill (timed separately), then exactly K decode steps
    dev.sync()
    tp0 = time.perf_counter()
    m.decode_begin(prompt, args.steps)
    dev.sync()
    tp1 = time.perf_counter()
    m.decode_steps(args.steps)
    dev.sync()
    t1 = time.perf_counter()
    toks, margins = m.decode_read(args.steps)
    m.decode_end()
    dt = t1 - tp1
    out = {
        "tok_s": args.steps / dt,
        "ms_per_step": 1000.0 * dt / args.steps,
        "prefill_ms_incl_capture": 1000.0 * (tp1 - tp0),
        "min_margin": float(np.min(margins)),
        "tokens_head": toks[:8].tolist(),
    }
    if latency:
        pf = []
        for i in range(4):
            dev.sync()
            a = time.perf_counter()
            m.prefill(prompt, 0)
            pf.append(time.perf_counter() - a)
        t_pf = float(np.median(pf[1:]))
        out["prefill_ms"] = round(1000.0 * t_pf, 3)
        out["prefill_tok_s"] = round(len(prompt) / t_pf, 1)
        n_warm, n_lat = 8, 64
        m.decode_begin(prompt, n_warm + n_lat)
        lat = []
        for i in range(n_warm + n_lat):
            a = time.perf_counter()
            m.decode_steps(1)
            m.decode_read(i + 2)          # waits for this token, copies it to the host
            if i >= n_warm:
                lat.append(time.perf_counter() - a)
        m.decode_end()
        srt = sorted(lat)
        out["latency_us"] = {"p50": round(1e6 * srt[len(srt) // 2], 1),
                             "p99": round(1e6 * srt[len(srt) * 99 // 100], 1),
                             "tokens": n_lat, "warmup": n_warm,
                             "mode": "one graph replay + bounded sync + token read per token"}
    gold = os.path.join(ROOT, "tests", "golden", "config5_tokens.json")
    if os.path.exists(gold) and lm_head == "q1" and args.prompt == 512:
        g = json.load(open(gold))
        n = min(len(g["tokens"]), args.steps)
        out["tokens_match_golden"] = bool(np.array_equal(toks[:n], np.array(g["tokens"][:n])))
        out["golden_compared"] = n
    gold = os.path.join(ROOT, "tests", "golden", "config5_unit_tokens.json")
    if os.path.exists(gold) and lm_head == "q1" and args.prompt == 512:
        out.update(golden_unit_prefix(m, cfg, prompt, json.load(open(gold))))
    m.close()
    return out


def golden_unit_prefix(m, cfg, prompt, g):
    """Free-running greedy stream of the loaded decoder with its norm weights
    switched to the fixture's (1 + N(0, 0.02)), against the oracle's 256
    golden tokens: the length of the matching prefix, and the first step
    where the oracle's top-2 margin is a near-tie (below twice the logit bar
    of the parity test), from which on the streams may part.  Runs after the
    timed region; the loaded model is left in the fixture's norm mode."""
    from nnzap_amd import configs as cf
    from nnzap_amd import model as MD
    from nnzap_amd import synth as S

    mode = g["norm_mode"]
    m.upload(MD.T_FINAL_NORM, 0, cf.norm_weights(S.SEED_MODEL_BASE + 3, cfg.hidden_size, mode))
    tids = {"attn_norm": MD.T_ATTN_NORM, "ffn_norm": MD.T_FFN_NORM,
            "q_norm": MD.T_Q_NORM, "k_norm": MD.T_K_NORM}
    for l in range(cfg.num_layers):
        for name, arr in cf.layer_norm_weights(cfg, l, mode).items():
            m.upload(tids[name], l, arr)
    n = int(g["n_new"])
    m.decode_begin(prompt, n)
    m.decode_steps(n)
    toks, _ = m.decode_read(n)
    m.decode_end()
    ref = np.array(g["tokens"][:n], dtype=np.int64)
    toks = np.asarray(toks[:n], dtype=np.int64)
    bad = np.nonzero(toks != ref)[0]
    near = 2 * max(1e-3, 4 * g.get("fp32_noise", 0.0)) * g["logits"][0]["max_abs"]
    ties = [i for i, mg in enumerate(g["margins"][:n]) if mg < near]
    return {"tokens_match_golden_unit": int(bad[0]) if len(bad) else n,
            "golden_unit_compared": n,
            "golden_unit_first_near_tie": ties[0] if ties else None}


def bench_decode_q4(args, dev):
    """Decode tok/s of a Bonsai-1.7B_Q4-shaped decoder (q4_mlx: 4-bit gs64
    linears, Q4 embedding tied into the LM head, transformer.zig:336-350).
    Codes, scales and biases are filled on the device from a seeded normal
    stream (throughput only; the Q4 numerics are covered by the parity
    tests); a 32-token prompt is prefilled through the 4-bit GEMM, then
    ``steps`` decode steps are timed like the headline figure."""
    from nnzap_amd import configs as cf
    from nnzap_amd import model as MD
    import ctypes as C

    cfg = cf.DecoderConfig(**{**cf.BONSAI_1_7B.__dict__, "group_size": 64, "embed_kind": 2,
                              "lm_head_kind": 2, "quant_format": 1})
    m = MD.DecoderModel(dev, cfg)
    seed = [7000]

    def fill(tid, layer=0, scale=1.0):
        ptr, nbytes = m.tensor(tid, layer)
        dev.call("nnz_synth_normal_bf16", C.c_void_p(ptr), nbytes // 2, seed[0], scale)
        seed[0] += 1

    for base in ((MD.T_EMBED_CODES, MD.T_EMBED_SCALES, MD.T_EMBED_BIASES),
                 (MD.T_LM_CODES, MD.T_LM_SCALES, MD.T_LM_BIASES)):
        fill(base[0]), fill(base[1], 0, 0.01), fill(base[2], 0, 0.01)
    for l in range(cfg.num_layers):
        for name in cf.PROJS:
            fill(MD._CODES[name], l), fill(MD._CODES[name] + 1, l, 0.01), fill(MD._BIASES[name], l, 0.01)
        for tid, n in ((MD.T_ATTN_NORM, cfg.hidden_size), (MD.T_FFN_NORM, cfg.hidden_size),
                       (MD.T_Q_NORM, cfg.head_dim), (MD.T_K_NORM, cfg.head_dim)):
            m.upload(tid, l, cf.norm_weights(tid + 64 * l, n, "unit"))
    m.upload(MD.T_FINAL_NORM, 0, cf.norm_weights(3, cfg.hidden_size, "unit"))
    prompt = cf.prompt_ids(cfg, 32)
    m.decode_begin(prompt, max(args.warmup, 1))
    m.decode_steps(max(args.warmup, 1))
    m.decode_read(1)
    m.decode_end()
    dev.sync()
    tp0 = time.perf_counter()
    m.decode_begin(prompt, args.steps)
    dev.sync()
    tp1 = time.perf_counter()
    m.decode_steps(args.steps)
    dev.sync()
    t1 = time.perf_counter()
    m.decode_read(args.steps)
    m.decode_end()
    m.close()
    dt = t1 - tp1
    return {"tok_s": round(args.steps / dt, 2), "ms_per_step": round(1000.0 * dt / args.steps, 4),
            "prefill_32_ms_incl_capture": round(1000.0 * (tp1 - tp0), 2),
            "workload": "Bonsai-1.7B_Q4 shape: 28 layers, q4_mlx gs64 linears, Q4 tied "
                        "embedding/LM head (vocab 151936), device-filled random weights"}


# --------------------------------------------------------------- kernels ----
class Rot:
    """Distinct device copies of one quantised matrix (same values, distinct
    addresses): at least MIN_COPIES and at least ``total_bytes`` in all, so
    that cycling through them streams every launch from HBM (the 256 MB
    Infinity Cache holds any single working set)."""

    def __init__(self, dev, w, total_bytes):
        import torch
        from nnzap_amd import ops
        base = ops.DeviceQWeight(dev, w)
        self.n = max(MIN_COPIES, int(total_bytes // max(1, w.nbytes)) + 1)
        self.ws = [base]
        for _ in range(self.n - 1):
            c = object.__new__(ops.DeviceQWeight)
            c.__dict__.update(base.__dict__)
            c.codes, c.scales = base.codes.clone(), base.scales.clone()
            c.biases = base.biases.clone() if base.biases is not None else None
            from nnzap_amd import _lib as L
            c.desc = L.QWeightDesc(c.codes.data_ptr(), c.scales.data_ptr(),
                                   c.biases.data_ptr() if c.biases is not None else None,
                                   w.M * w.K, w.group_size, w.bits, w.scale_dtype)
            self.ws.append(c)
        torch.cuda.synchronize()

    def __getitem__(self, i):
        return self.ws[i % self.n]


def time_launches(dev, fn, n_iter, reps=3):
    """Average duration of one launch as the decoder runs it: ``n_iter``
    launches captured into one hipGraph on the library stream and replayed,
    HIP events around each replay, best of ``reps`` replays."""
    import ctypes as C
    from nnzap_amd import _lib as L

    fn(0)
    dev.sync()
    g = C.c_void_p()
    dev.call("nnz_graph_begin")
    try:
        for i in range(n_iter):
            fn(i + 1)
    finally:
        dev.call("nnz_graph_end", C.byref(g))
    try:
        dev.call("nnz_graph_replay", g)
        dev.sync()
        best = None
        for _ in range(reps):
            dev.mark(0)
            dev.call("nnz_graph_replay", g)
            dev.mark(1)
            ms = dev.elapsed_ms(0, 1) / n_iter
            best = ms if best is None else min(best, ms)
    finally:
        L.lib().nnz_graph_destroy(g)
    return best * 1000.0  # us


def _kernel_cases():
    """Named kernel timings: name -> fn(dev, n_iter) -> (us, algorithmic
    bytes per launch, launches per decode token or None).  The decode cases
    are the launches the captured decode step makes, at config-5 shapes."""
    import torch
    from nnzap_amd import _lib as L
    from nnzap_amd import configs as cf
    from nnzap_amd import formats as fm
    from nnzap_amd import ops

    f32, f16 = torch.float32, torch.float16
    H, I, QD, KVD, V = 2048, 6144, 2048, 1024, 151936

    def act():
        rng = np.random.default_rng(0)
        res_d = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).cuda()
        return res_d, torch.ones(H, dtype=f32, device="cuda")

    def config1(dev, n):
        w1, x1 = cf.config1()
        r = Rot(dev, w1, ROTATE_BYTES)
        xd, y = torch.from_numpy(x1).cuda(), torch.empty(6144, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_q4mv(dev, r[i], xd, y), n)
        return us, w1.nbytes + 2048 * 4 + 6144 * 4, None

    def config2(dev, n):
        w2, x2 = cf.config2()
        r = Rot(dev, w2, ROTATE_BYTES)
        xd, y = torch.from_numpy(x2).cuda(), torch.empty(2048, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv(dev, r[i], xd, y), n)
        return us, w2.nbytes + 6144 * 4 + 2048 * 4, None

    def config3(dev, n):
        wg, wu, x3 = cf.config3()
        rg, ru = Rot(dev, wg, ROTATE_BYTES // 2), Rot(dev, wu, ROTATE_BYTES // 2)
        xd, y = torch.from_numpy(x3).cuda(), torch.empty(6144, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv_fused_pair_silu(dev, rg[i], ru[i], xd, y), n)
        return us, wg.nbytes + wu.nbytes + 2048 * 4 + 6144 * 4, None

    def dec_qkv(dev, n):
        res_d, nw = act()
        wq = cf.q1_matrix(QD, H, 128, 500, 501)
        wk, wv = cf.q1_matrix(KVD, H, 128, 502, 503), cf.q1_matrix(KVD, H, 128, 504, 505)
        rq = Rot(dev, wq, ROTATE_BYTES // 2)
        rk, rv = Rot(dev, wk, ROTATE_BYTES // 4), Rot(dev, wv, ROTATE_BYTES // 4)
        q = torch.empty(QD, dtype=f16, device="cuda")
        k, v = torch.empty(KVD, dtype=f16, device="cuda"), torch.empty(KVD, dtype=f16, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_fused_norm_qkv_f16io(
            dev, rq[i], rk[i], rv[i], res_d, q, k, v, nw), n)
        return us, wq.nbytes + wk.nbytes + wv.nbytes + H * 8 + (QD + 2 * KVD) * 2, 28

    def dec_attention(dev, n):
        # one decode layer's attention: q/k norm + RoPE, KV append, attention
        # over 640 tokens (the mean context of the timed steps), merge
        seq, max_ctx = 640, 1024
        kcs = random_copies((8, max_ctx, 128), f16, 8 * max_ctx * 128 * 4, 23)
        vcs = random_copies((8, 128, max_ctx), f16, 8 * max_ctx * 128 * 4, 24)
        qr = torch.randn(16 * 128, device="cuda").to(f16)
        kr = torch.randn(8 * 128, device="cuda").to(f16)
        vr = torch.randn(8 * 128, device="cuda").to(f16)
        qn = torch.ones(128, dtype=f32, device="cuda")
        att = torch.empty(16, 128, dtype=f16, device="cuda")
        fd = L.GQAFusedDims(16, 8, 128, seq, max_ctx, 2, seq - 1, 1e-6, 1e6)
        scr = torch.zeros(ops.gqa_scratch_bytes(L.GQADims(16, 8, 128, seq, max_ctx, 2)) // 4 + 64,
                          dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_gqa_attention_fused_1pass(
            dev, qr, kcs[i % len(kcs)], vcs[i % len(vcs)], att, kr, vr, qn, qn, scr, fd), n)
        return us, 2 * 8 * seq * 128 * 2 + 16 * 128 * 4 + 8 * 128 * 8, None

    def dec_attention_partials(dev, n):
        # the decoder's attention launch: q/k norm + RoPE (frequency table),
        # KV append, split-sequence attention to per-chunk partials, at the
        # mean context of the timed steps (640 tokens)
        seq, max_ctx = 640, 1024
        kcs = random_copies((8, max_ctx, 128), f16, 8 * max_ctx * 128 * 4, 21)
        vcs = random_copies((8, 128, max_ctx), f16, 8 * max_ctx * 128 * 4, 22)
        qr = torch.randn(16 * 128, device="cuda").to(f16)
        kr = torch.randn(8 * 128, device="cuda").to(f16)
        vr = torch.randn(8 * 128, device="cuda").to(f16)
        qn = torch.ones(128, dtype=f32, device="cuda")
        freqs = torch.from_numpy((1e6 ** (-np.arange(0, 128, 2) / 128.0)).astype(np.float32)).cuda()
        nch = ops.gqa_partial_chunks(seq)
        po = torch.empty(16 * nch * 128, dtype=f32, device="cuda")
        pm = torch.empty(16 * nch * 2, dtype=f32, device="cuda")
        fd = L.GQAFusedDims(16, 8, 128, seq, max_ctx, 2, seq - 1, 1e-6, 1e6)
        us = time_launches(dev, lambda i: ops.dispatch_gqa_attention_partials(
            dev, qr, kcs[i % len(kcs)], vcs[i % len(vcs)], kr, vr, qn, qn, po, pm, fd,
            rope_inv_freq=freqs), n)
        # K and V of 640 tokens x 8 heads, q/k/v in, new K/V row out, partials out
        nbytes = 2 * 8 * seq * 128 * 2 + (16 + 16) * 128 * 2 + 8 * 128 * 4 + 16 * nch * 130 * 4
        return us, nbytes, 28

    def dec_o_merge(dev, n):
        # the decoder's O projection: merge of the attention partials in the
        # prologue, residual +=
        seq = 640
        nch = ops.gqa_partial_chunks(seq)
        wo = cf.q1_matrix(H, QD, 128, 506, 507)
        r = Rot(dev, wo, ROTATE_BYTES)
        po = torch.randn(16 * nch * 128, dtype=f32, device="cuda")
        pm = torch.stack([torch.randn(16 * nch, device="cuda"),
                          1 + torch.rand(16 * nch, device="cuda")], 1).reshape(-1).contiguous()
        resid = torch.zeros(H, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv_merge_f16io_resadd(
            dev, r[i], po, pm, seq, 128, resid), n)
        return us, wo.nbytes + 16 * nch * 130 * 4 + H * 8, 28

    def dec_o(dev, n):
        wo = cf.q1_matrix(H, QD, 128, 506, 507)
        r = Rot(dev, wo, ROTATE_BYTES)
        x16 = torch.randn(QD, dtype=f16, device="cuda") * 0.05
        resid = torch.zeros(H, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv_f16io_resadd(dev, r[i], x16, resid), n)
        return us, wo.nbytes + QD * 2 + H * 8, None

    def dec_gate_up(dev, n):
        res_d, nw = act()
        wg5, wu5 = cf.q1_matrix(I, H, 128, 508, 509), cf.q1_matrix(I, H, 128, 510, 511)
        rg, ru = Rot(dev, wg5, ROTATE_BYTES // 2), Rot(dev, wu5, ROTATE_BYTES // 2)
        h = torch.empty(I, dtype=f16, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_fused_norm_pair_silu_f16io(
            dev, rg[i], ru[i], res_d, h, nw), n)
        return us, wg5.nbytes + wu5.nbytes + H * 8 + I * 2, 28

    def dec_down(dev, n):
        wd = cf.q1_matrix(H, I, 128, 512, 513)
        r = Rot(dev, wd, ROTATE_BYTES)
        x16 = torch.randn(I, dtype=f16, device="cuda") * 0.05
        resid = torch.zeros(H, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv_f16io_resadd(dev, r[i], x16, resid), n)
        return us, wd.nbytes + I * 2 + H * 8, 28

    def dec_lm_head(dev, n):
        res_d, nw = act()
        wl = cf.q1_matrix(V, H, 128, 514, 515)
        r = Rot(dev, wl, ROTATE_BYTES)
        logits = torch.empty(V, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_fused_norm_qmv_f16in(
            dev, r[i], res_d, logits, nw), max(16, n // 8))
        return us, wl.nbytes + H * 8 + V * 4, 1

    def dec_lm_head_f16in(dev, n):
        # the unfused alternative: f16 normalised input, f32 logits
        wl = cf.q1_matrix(V, H, 128, 514, 515)
        r = Rot(dev, wl, ROTATE_BYTES)
        x16 = torch.randn(H, dtype=f16, device="cuda") * 0.05
        logits = torch.empty(V, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_qmv_f16in(dev, r[i], x16, logits),
                           max(16, n // 8))
        return us, wl.nbytes + H * 2 + V * 4, None

    def dec_lm_head_tied(dev, n):
        # the tied bf16 LM head (622 MB per token): two tables alternate, each
        # larger than the 256 MB Infinity Cache, so every launch streams HBM
        g = torch.Generator(device="cuda")
        g.manual_seed(516)
        tabs = [(torch.randn(V, H, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
                for _ in range(2)]
        x16 = torch.randn(H, dtype=f16, device="cuda") * 0.05
        logits = torch.empty(V, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_lm_head_bf16(dev, tabs[i % 2], x16, logits),
                           max(8, n // 16))
        del tabs
        return us, V * H * 2 + H * 2 + V * 4, None

    def floor_small(dev, n):
        # launch floor: one tiny kernel (residual += addition over 2048 f32)
        a = torch.zeros(H, dtype=f32, device="cuda")
        b = torch.ones(H, dtype=f32, device="cuda")
        us = time_launches(dev, lambda i: ops.dispatch_residual_add(dev, a, b), n)
        return us, 3 * H * 4, None

    def config4(L_):
        def run(dev, n):
            per = 8 * L_ * 128 * 2
            kbs = random_copies((8, L_, 128), torch.bfloat16, 2 * per, 40 + L_)
            vbs = random_copies((8, L_, 128), torch.bfloat16, 2 * per, 41 + L_)
            qb = torch.randn(16, 128, device="cuda").to(torch.bfloat16)
            ob = torch.empty(16, 128, dtype=f32, device="cuda")
            d4 = L.GQADims(16, 8, 128, L_, L_, 2)
            s4 = torch.empty(ops.gqa_scratch_bytes(d4) // 4 + 64, dtype=f32, device="cuda")
            us = time_launches(dev, lambda i: ops.dispatch_gqa_attention(
                dev, qb, kbs[i % len(kbs)], vbs[i % len(vbs)], ob, s4, d4, v_transposed=False,
                rope_position=L_, rope_theta=1e6), max(16, n // 4))
            del kbs, vbs
            return us, 4096 * L_ + 12288, None
        return run

    def prefill_gemm(M_, K_, mode, pair=False, q4=False):
        # one prefill dequant-GEMM of the decoder at a 512-token prompt:
        # C[512 x M] = A[512 x K] . W^T (1-bit W, or q4_mlx gs64 with bf16
        # scales/biases; f16 A), reported as MFMA throughput; weights rotated
        # like the QMV cases
        def mat(seed):
            if q4:
                return cf.q4_matrix(M_, K_, 64, seed, seed + 10, seed + 20, scale_dtype=fm.DT_BF16)
            return cf.q1_matrix(M_, K_, 128, seed, seed + 10)

        def run(dev, n):
            P = 512
            wa = mat(600)
            ra = Rot(dev, wa, ROTATE_BYTES // (2 if pair else 1))
            rb = Rot(dev, mat(602), ROTATE_BYTES // 2) if pair else None
            a16 = (torch.randn(P, K_, device="cuda") * 0.5).to(f16)
            o = torch.empty(P, M_, dtype=f16 if mode in (L.GEMM_STORE_F16, L.GEMM_SILU_PAIR) else f32,
                            device="cuda")
            us = time_launches(dev, lambda i: ops.dispatch_dequant_gemm(
                dev, ra[i], a16, o, mode, wb=rb[i] if pair else None), max(16, n // 8))
            flops = 2 * P * M_ * K_ * (2 if pair else 1)
            nbytes = wa.nbytes * (2 if pair else 1) + P * K_ * 2 + P * M_ * o.element_size()
            return us, nbytes, None, flops
        return run

    def sample(T, k, p, peaked=False):
        # device sampling over the 151,936 logits the LM head just wrote
        # (sampleToken on device: temperature, top-k, top-p, one draw);
        # logits N(0, 2.5^2), "peaked": 8 tokens raised by 12
        def run(dev, n):
            g = np.random.default_rng(3)
            x = g.normal(0.0, 2.5, V).astype(np.float32)
            if peaked:
                x[g.integers(0, V, 8)] += 12.0
            logits = torch.from_numpy(x).cuda()
            ws = torch.empty(ops.sample_workspace_bytes(V), dtype=torch.uint8, device="cuda")
            rng = torch.zeros(4, dtype=torch.int64, device="cuda")
            out = torch.zeros(1, dtype=torch.int32, device="cuda")
            ops.rng_seed(dev, 42, rng)
            us = time_launches(dev, lambda i: ops.dispatch_sample(dev, logits, out, rng, ws, T, k, p),
                               max(16, n // 8))
            return us, V * 4, None
        return run

    def stacked(kind, pad=0, bpm=0):
        # One launch over `count` independently drawn matrices of a config
        # shape (>= 256 of them and >= 450 MB in all, so the launch streams
        # from HBM): the kernel's streaming rate without the per-launch
        # floor.  HIP events on the library stream around single launches,
        # best of 5 after a warm-up.
        def run(dev, n):
            # The working set comes from fresh device memory: served from
            # segments the allocator cached for the cases before it, the
            # 1.8 GB config-1 stack streamed 20-25 % slower (399.6 against
            # 326.0 us after an empty_cache, 318.8 us run alone).
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            shp = {"config1": (6144, 2048, 64, 4), "config2": (2048, 6144, 128, 1),
                   "config3": (6144, 2048, 128, 1), "q1_6144x2048": (6144, 2048, 128, 1)}[kind]
            M_, K_, gs, bits = shp
            nmat = 2 if kind == "config3" else 1
            each = (M_ * K_ * bits // 8 + M_ * K_ // gs * 2 * (2 if bits == 4 else 1)) * nmat
            # a multiple of 256 matrices (>= 64, >= 640 MB where that is fewer):
            # the matrix-core kernel runs one block per CU and matrix
            count = max(256, -(-max(MIN_COPIES * each, ROTATE_BYTES) // each))
            count = -(-count // 256) * 256
            rng = (0.005, 0.02) if bits == 4 else (0.01, 0.05)
            sws = [ops.StackedQWeights(dev, M_, K_, gs, bits, count, 900 + i, rng, pad_bytes=pad)
                   for i in range(nmat)]
            x = torch.randn(count, K_, device="cuda")
            y = torch.empty(count, M_, device="cuda")
            if kind == "config1":
                fn = lambda: ops.dispatch_q4mv_stacked(dev, sws[0], x, y, bpm)  # noqa: E731
            elif kind in ("config2", "q1_6144x2048"):
                fn = lambda: ops.dispatch_qmv_stacked(dev, sws[0], x, y, bpm)  # noqa: E731
            else:
                fn = lambda: ops.dispatch_qmv_fused_pair_silu_stacked(dev, sws[0], sws[1], x, y, bpm)  # noqa: E731
            fn()
            dev.sync()
            best = None
            for _ in range(5):
                dev.mark(0)
                fn()
                dev.mark(1)
                ms = dev.elapsed_ms(0, 1)
                best = ms if best is None else min(best, ms)
            nbytes = count * (each + K_ * 4 + M_ * 4)
            del sws
            return best * 1000.0, nbytes, None, None, {"matrices": count,
                                                       "us_per_matrix": round(best * 1000.0 / count, 3)}
        return run

    def cores(case, value):
        # the same case with NNZ_OPT_Q1_MATRIX_CORES forced (1: the
        # block-scaled MFMA 1-bit kernel wherever it applies, 2: never)
        def run(dev, n):
            dev.call("nnz_ctx_set_option", L.OPT_Q1_MATRIX_CORES, value)
            try:
                r = case(dev, n)   # an A/B variant: not a launch of the decode step
                return (r[0], r[1], None) + tuple(r[3:])
            finally:
                dev.call("nnz_ctx_set_option", L.OPT_Q1_MATRIX_CORES, 0)
        return run

    def q1_big(dev, n):
        # one 1-bit matrix of 256 x 6144 rows, K = 2048 (~500 MB): a single
        # ordinary launch, every CU sweeping neighbouring tiles of one region
        M_ = 6144 * 256
        sw = ops.StackedQWeights(dev, M_, 2048, 128, 1, 1, 950)
        x = torch.randn(2048, device="cuda")
        y = torch.empty(M_, device="cuda")
        fn = lambda: ops.dispatch_qmv(dev, sw, x, y)  # noqa: E731
        fn()
        dev.sync()
        best = None
        for _ in range(5):
            dev.mark(0)
            fn()
            dev.mark(1)
            ms = dev.elapsed_ms(0, 1)
            best = ms if best is None else min(best, ms)
        del sw
        return best * 1000.0, M_ * (256 + 32) + 2048 * 4 + M_ * 4, None

    def copy_calib(dev, n):
        # a plain device copy of known size: the scale for FETCH/WRITE_SIZE
        a = torch.ones(64 << 20, dtype=f32, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(8):
            b.copy_(a)
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1000.0 / 8, 2 * a.numel() * 4, None

    return {
        "config1_q4mv": config1, "config2_qmv": config2, "config3_gate_up_silu": config3,
        "dec_qkv_norm": dec_qkv, "dec_attention_partials": dec_attention_partials,
        "dec_o_merge_resadd": dec_o_merge, "dec_gate_up_norm_silu": dec_gate_up,
        "attention_fused_seq640": dec_attention, "o_resadd": dec_o,
        "dec_down_resadd": dec_down, "dec_lm_head_norm": dec_lm_head,
        "dec_lm_head_f16in": dec_lm_head_f16in, "dec_lm_head_tied": dec_lm_head_tied,
        "floor_residual_add": floor_small,
        "config4_attention_L512": config4(512), "config4_attention_L4096": config4(4096),
        "config4_attention_L32768": config4(32768), "copy_256MiB": copy_calib,
        "stacked_config1_q4mv": stacked("config1"), "stacked_config2_qmv": stacked("config2"),
        "stacked_config3_gate_up_silu": stacked("config3"),
        "stacked_config3_gate_up_silu_valu": cores(stacked("config3"), 2),
        "stacked_q1_6144x2048": stacked("q1_6144x2048"),
        "q1_big_mfma": cores(q1_big, 1),
        "q1_big_valu": cores(q1_big, 2),
        "stacked_q1_6144x2048_bpm4": stacked("q1_6144x2048", 0, 4),
        "stacked_config3_bpm4": stacked("config3", 0, 4),
        "stacked_q1_6144x2048_valu": cores(stacked("q1_6144x2048"), 2),
        "dec_lm_head_norm_valu": cores(dec_lm_head, 2),
        "dec_lm_head_norm_mfma": cores(dec_lm_head, 1),
        "config3_gate_up_silu_mfma": cores(config3, 1),
        "dec_gate_up_norm_silu_mfma": cores(dec_gate_up, 1),
        "prefill_gemm_q": prefill_gemm(QD, H, L.GEMM_STORE_F16),
        "prefill_gemm_kv": prefill_gemm(KVD, H, L.GEMM_STORE_F16),
        "prefill_gemm_o_resadd": prefill_gemm(H, QD, L.GEMM_RESADD),
        "prefill_gemm_gate_up_silu": prefill_gemm(I, H, L.GEMM_SILU_PAIR, pair=True),
        "prefill_gemm_down_resadd": prefill_gemm(H, I, L.GEMM_RESADD),
        "prefill_gemm_q4_gate_up_silu": prefill_gemm(I, H, L.GEMM_SILU_PAIR, pair=True, q4=True),
        "prefill_gemm_q4_down_resadd": prefill_gemm(H, I, L.GEMM_RESADD, q4=True),
        "sample_topk40_topp095": sample(0.8, 40, 0.95),
        "sample_topp090": sample(1.0, 0, 0.9),
        "sample_topp090_peaked": sample(1.0, 0, 0.9, peaked=True),
        "sample_temperature_only": sample(0.7, 0, 1.0),
    }


def bench_kernels(dev, quick=False, only=None):
    import torch

    n_iter = 64 if quick else 256
    cases = _kernel_cases()
    names = list(cases) if not only else only.split(",")
    res = {}
    for name in names:
        r = cases[name](dev, n_iter)
        us, nbytes, per_token = r[:3]
        torch.cuda.synchronize()
        gbs = nbytes / (us * 1e-6) / 1e9
        if len(r) > 3 and r[3] is not None:   # MFMA-bound: FLOP/s against the dense f16 peak
            tf = r[3] / (us * 1e-6) / 1e12
            res[name] = {"us": round(us, 3), "flops": int(r[3]), "TFLOPs": round(tf, 1),
                         "frac": round(tf / PEAK_F16_TFLOPS, 4)}
            log(f"{name:28s} {us:8.2f} us  {tf:8.1f} TFLOP/s  ({r[3]} FLOP)")
            continue
        res[name] = {"us": round(us, 3), "bytes": int(nbytes), "GBs": round(gbs, 1),
                     "frac": round(gbs / PEAK_HBM_GBS, 4)}
        if per_token is not None:
            res[name]["per_token"] = per_token
        if len(r) > 4:
            res[name].update(r[4])
        log(f"{name:28s} {us:8.2f} us  {gbs:8.1f} GB/s  ({nbytes} B)")
    return res


def sources_digest():
    """sha256 (first 16 hex digits) of the HIP sources the library is built
    from and of its build flags (nnzap_amd/csrc/*.hip, *.h, include/nnz.h and
    nnzap_amd/build.py, sorted by name): the profiles under profiles/ record
    the digest of the sources they measured."""
    import hashlib
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(ROOT, "nnzap_amd", "csrc", "*.hip")) +
                   glob.glob(os.path.join(ROOT, "nnzap_amd", "csrc", "*.h")) +
                   [os.path.join(ROOT, "include", "nnz.h"),
                    os.path.join(ROOT, "nnzap_amd", "build.py")], key=os.path.basename)
    for f in files:
        h.update(os.path.basename(f).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()[:16]


def load_trace_us():
    """Mean per-dispatch device duration (us) and kernel name(s) of every
    kernel case from the committed rocprofv3 kernel-trace summary
    (profiles/kernel_case_traces.md, first table: the case's kernels summed),
    and the sources digest that summary records ("Sources: <digest>")."""
    path = os.path.join(ROOT, "profiles", "kernel_case_traces.md")
    out, digest = {}, None
    if not os.path.exists(path):
        return out, digest
    for line in open(path):
        if line.startswith("Sources:"):
            digest = line.split()[1].strip("`")
        f = [x.strip() for x in line.strip().strip("|").split("|")]
        if len(f) >= 10 and f[0] and f[0] not in out:
            try:
                out[f[0]] = (float(f[3]), f[1].strip("`"))
            except ValueError:
                pass
    return out, digest


def load_traffic():
    """HBM bytes per launch of the decode kernel cases, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/pmc_traffic.md):
    fetch_KiB * fetch_scale + write_KiB * write_scale, the scales calibrated
    on a copy of known size."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.md")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        f = line.split()
        if len(f) == 6 and f[0] == "TRAFFIC":
            out[f[1]] = int(round((float(f[2]) * float(f[4]) + float(f[3]) * float(f[5])) * 1024))
    return out


# ------------------------------------------------------------ CPU baseline --
def cpu_threads() -> int:
    """Threads the CPU legs use: OMP_NUM_THREADS (the GPU box sets it to its
    CPU share, 16 per GPU) or every core os.cpu_count() reports."""
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def _median_time(fn, warmup=5, runs=30):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(pos=512, warmup=5, runs=30, dq_warmup=1, dq_runs=3):
    """The config-5 decoder's decode step in PyTorch float32 on this host's
    cores (oracle/torch_cpu.py): all 28 layers + the 1-bit LM head, KV cache
    holding `pos` tokens.  Pre-dequantised float32 weights: `warmup` steps
    then the median of `runs` (the headline value).  Dequantised from the
    packed codes on every step: `dq_warmup` then the median of `dq_runs`
    (several seconds per step, so a shorter sample)."""
    import torch
    from nnzap_amd import configs as cf
    from oracle.torch_cpu import TorchDecoder

    threads = cpu_threads()
    torch.set_num_threads(threads)
    cfg = cf.BONSAI_1_7B
    w = cf.decoder_weights(cfg, norm_mode="small", host_embed=False)
    t0 = time.perf_counter()
    td = TorchDecoder(w, pos + 8, predequantise=True)
    t_deq = time.perf_counter() - t0
    td.fill_cache(pos)
    x = torch.randn(cfg.hidden_size, generator=torch.Generator().manual_seed(1)) * 0.02
    t_pre = _median_time(lambda: td.step(x, pos), warmup, runs)
    # the 512-token prompt as one batch (the reference prefills token by
    # token; one warm-up, the median of 3)
    xs = torch.randn(512, cfg.hidden_size, generator=torch.Generator().manual_seed(2)) * 0.02
    t_pf = _median_time(lambda: td.prefill(xs, 0), 1, 3)
    del td
    tq = TorchDecoder(w, pos + 8, predequantise=False)
    tq.fill_cache(pos)
    t_dq = _median_time(lambda: tq.step(x, pos), dq_warmup, dq_runs)
    del tq
    log(f"cpu decode (torch f32, {threads} threads): {1 / t_pre:.2f} tok/s pre-dequantised, "
        f"{1 / t_dq:.3f} tok/s dequantising every step (one-time dequant {t_deq:.1f}s); "
        f"prefill of 512 tokens {1000 * t_pf:.0f} ms")
    return {"value": round(1.0 / t_pre, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "impl": "PyTorch CPU float32 (oracle/torch_cpu.py)", "cpu_model": cpu_model(),
            "cpu_count": os.cpu_count(),
            "ms_per_token_predequantised": round(1000 * t_pre, 2),
            "ms_per_token_dequant_each_call": round(1000 * t_dq, 1),
            "tok_s_dequant_each_call": round(1.0 / t_dq, 4),
            "prefill_512_ms": round(1000 * t_pf, 1),
            "prefill_tok_s": round(512 / t_pf, 1),
            "sample": (f"one decode step of the full config-5 decoder (28 layers + 1-bit LM head, "
                       f"KV cache of {pos} tokens) in torch float32 on {threads} threads; "
                       f"value: weights pre-dequantised, {warmup} warm-up steps then the median "
                       f"of {runs}; dequantising every step: {dq_warmup} warm-up then the median "
                       f"of {dq_runs}; prefill: the 512-token prompt as one batch "
                       f"(pre-dequantised), 1 warm-up then the median of 3")}


def cpu_configs(full=False):
    """Configs 1-4 in PyTorch float32 on this host (oracle/torch_cpu.py), 5
    warm-up calls then the median of 30 (without --cpu-full: 2 and 7).  Two
    variants per config: dequantise (or widen the bf16 caches) on every
    call, and the same product on pre-dequantised float32 operands."""
    import torch
    from nnzap_amd import configs as cf
    from nnzap_amd import formats as fm
    from oracle import torch_cpu as T

    torch.set_num_threads(cpu_threads())
    wu, nr = (5, 30) if full else (2, 7)
    out = {}
    w1, x1 = cf.config1()
    x1t = torch.from_numpy(x1)
    deq1 = lambda: T.dequant_q4(w1.codes, w1.scales, w1.biases, w1.M, w1.K, w1.group_size,  # noqa: E731
                                w1.scale_dtype == fm.DT_BF16)
    d1 = deq1()
    out["config1_q4mv"] = (lambda: deq1() @ x1t, lambda: d1 @ x1t, w1.nbytes + 8192 + 24576)
    w2, x2 = cf.config2()
    x2t = torch.from_numpy(x2)
    deq2 = lambda: T.dequant_q1(w2.codes, w2.scales, w2.M, w2.K, w2.group_size)  # noqa: E731
    d2 = deq2()
    out["config2_qmv"] = (lambda: deq2() @ x2t, lambda: d2 @ x2t, w2.nbytes + 24576 + 8192)
    wg, wup, x3 = cf.config3()
    x3t = torch.from_numpy(x3)
    dq = lambda q: T.dequant_q1(q.codes, q.scales, q.M, q.K, q.group_size)  # noqa: E731
    dg, du = dq(wg), dq(wup)
    silu = torch.nn.functional.silu
    out["config3_gate_up_silu"] = (lambda: silu(dq(wg) @ x3t) * (dq(wup) @ x3t),
                                   lambda: silu(dg @ x3t) * (du @ x3t),
                                   wg.nbytes + wup.nbytes + 8192 + 24576)
    p = torch.arange(64, dtype=torch.float64)
    inv = torch.exp2(-(2.0 * p / 128) * np.log2(1e6)).float()

    def attn(q, k, v, L_):
        qr = T.rope(q, L_, inv).view(8, 2, 128)
        s = torch.matmul(qr, k.transpose(1, 2)) / np.sqrt(128)
        return torch.matmul(torch.softmax(s, dim=-1), v).reshape(16, 128)

    def bf16(bits, shape):
        return (torch.from_numpy(bits.view(np.int16)).to(torch.int32) << 16).view(torch.float32) \
            .reshape(shape)
    for L_ in (512, 4096, 32768):
        q, k, v = cf.config4(L_)
        qf, kf, vf = bf16(q, (16, 128)), bf16(k, (8, L_, 128)), bf16(v, (8, L_, 128))
        out[f"config4_attention_L{L_}"] = (
            lambda q=q, k=k, v=v, L_=L_: attn(bf16(q, (16, 128)), bf16(k, (8, L_, 128)),
                                              bf16(v, (8, L_, 128)), L_),
            lambda qf=qf, kf=kf, vf=vf, L_=L_: attn(qf, kf, vf, L_),
            4096 * L_ + 12288)
    res = {}
    with torch.no_grad():
        for name, (f_dq, f_pre, nbytes) in out.items():
            t_dq = _median_time(f_dq, wu, nr)
            t_pre = _median_time(f_pre, wu, nr)
            res[name] = {"us_dequant_each_call": round(t_dq * 1e6, 1),
                         "us_predequantised": round(t_pre * 1e6, 1),
                         "GBs_dequant_each_call": round(nbytes / t_dq / 1e9, 3)}
            log(f"cpu {name:26s} {t_dq * 1e6:12.1f} us (dequant each call) "
                f"{t_pre * 1e6:12.1f} us (pre-dequantised)")
    return {"kind": "port", "impl": "PyTorch CPU float32 (oracle/torch_cpu.py)", "warmup": wu,
            "runs": nr, "stat": "median", "threads": cpu_threads(), "cpu_model": cpu_model(),
            "cpu_count": os.cpu_count(), "configs": res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--lm-head", choices=("q1", "tied"), default="q1")
    ap.add_argument("--quick", action="store_true", help="fewer kernel timing iterations")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-full", action="store_true",
                    help="per-config CPU timings with 5 warm-ups and the median of 30")
    ap.add_argument("--skip-kernels", action="store_true")
    ap.add_argument("--skip-q4", action="store_true", help="leave out the 4-bit decode figure")
    ap.add_argument("--skip-tied", action="store_true",
                    help="leave out the tied bf16 LM head decode figure")
    ap.add_argument("--skip-decode", action="store_true",
                    help="kernel timings only (profiling runs); no JSON line")
    ap.add_argument("--only", default=None,
                    help="comma-separated kernel cases to time (e.g. for --pmc runs)")
    ap.add_argument("--details", default=None, help="write the full result dict here")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the decode path has no multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)

    import torch
    from nnzap_amd.ops import Device

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = Device(0, own_stream=True)
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.skip_decode:
        bench_kernels(dev, quick=args.quick, only=args.only)
        return
    dec = bench_decode(args, dev)
    dec_tied = None if args.skip_tied or args.lm_head == "tied" else \
        bench_decode(args, dev, lm_head="tied", latency=False)
    if dec_tied:
        log(f"tied bf16 LM head decode: {dec_tied['tok_s']:.1f} tok/s")
    dec_q4 = None if args.skip_q4 else bench_decode_q4(args, dev)
    if dec_q4:
        log(f"q4 decode: {dec_q4['tok_s']} tok/s")
    log(f"decode: {dec['tok_s']:.1f} tok/s ({dec['ms_per_step']:.3f} ms/step)")
    kern = {} if args.skip_kernels else bench_kernels(dev, quick=args.quick, only=args.only)

    roofline = None
    dec_k = {k: v for k, v in kern.items() if "per_token" in v}
    if dec_k:
        dom = max(dec_k, key=lambda k: dec_k[k]["us"] * dec_k[k]["per_token"])
        d = dec_k[dom]
        traffic = load_traffic().get(dom)
        roofline = {"kernel": dom, "bound": "hbm", "achieved": d["GBs"], "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(d["GBs"] / PEAK_HBM_GBS, 4), "traffic": traffic,
                    "avg_launch_us": d["us"], "algorithmic_bytes": d["bytes"],
                    "timing": "live: launches back to back in one hipGraph, HIP events on the "
                              "library stream / launches",
                    "traffic_source": "profiles/pmc_traffic.md" if traffic else None}
        traces, digest = load_trace_us()
        tr = traces.get(dom)
        if tr:   # the committed rocprofv3 per-dispatch mean of the same case
            us_tr, kname = tr
            roofline.update({"trace_us": us_tr,
                             "achieved_trace": round(d["bytes"] / (us_tr * 1e-6) / 1e9, 1),
                             "frac_trace": round(d["bytes"] / (us_tr * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                             "trace_kernel": kname,
                             "trace_source": "profiles/kernel_case_traces.md (committed "
                                             "rocprofv3 summary, not re-measured by this run)",
                             "trace_matches_sources": digest == sources_digest()})
    cpu = None if args.skip_cpu else cpu_baseline()
    cpu_cfg = None if args.skip_cpu else cpu_configs(full=args.cpu_full)

    line = {
        "metric": "decode tok/s (Bonsai-1.7B, bs1) + QMV achieved HBM GB/s vs peak",
        "value": round(dec["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(dec["tok_s"] / BASELINE_TOKS, 2),
        "dtype": "q1-weights/f16-act/f32-acc",
        "data": "synthetic: seeded random-init weights, uniform random prompt ids",
        "config": {"workload": "config5 Bonsai-1.7B-shaped decoder: 28 layers, hidden 2048, "
                               "MLP 6144, 16Q/8KV x 128, vocab 151936, 1-bit gs128 linears, "
                               "bf16 embeddings/norms, 512-token GEMM prefill, greedy decode",
                   "lm_head": args.lm_head, "prompt": args.prompt, "batch": 1,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "tokens_match_golden_unit": dec.get("tokens_match_golden_unit"),
        "cpu_baseline": cpu,
        "cpu_configs": cpu_cfg,
        "decode": dec,
        "decode_q4": dec_q4,
        "decode_tied_lm_head": dec_tied and {
            "tok_s": round(dec_tied["tok_s"], 2), "ms_per_step": round(dec_tied["ms_per_step"], 4),
            "lm_head_kernel": kern.get("dec_lm_head_tied"),
            "workload": "config 5 with the tied bf16 embedding table as LM head (622 MB/token)"},
        "qmv": {k: v for k, v in kern.items() if k.startswith("config")},
        "qmv_stacked": {k: v for k, v in kern.items() if k.startswith("stacked_")},
        "copy_ceiling": kern.get("copy_256MiB"),
        "prefill_gemm": {k: v for k, v in kern.items() if k.startswith("prefill_gemm")},
        "decode_kernels": dec_k,
    }
    if args.details:
        with open(args.details, "w") as f:
            json.dump(line, f, indent=1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()

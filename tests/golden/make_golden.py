"""Writes the committed golden fixtures under tests/golden/ with the CPU oracle.

The reference ships no numeric expected outputs for this path (its tests
recompute CPU references at run time and its e2e goldens need real Bonsai
checkpoints), so these fixtures are produced by the oracle from seeded
synthetic inputs -- the seeds make the inputs reproducible on any host.

  python tests/golden/make_golden.py small     # kernel-level vectors (seconds)
  python tests/golden/make_golden.py config5        # 28-layer greedy tokens + logits (minutes, ~20 GB RAM)
  python tests/golden/make_golden.py config5_unit [--all-steps]
                                                    # the same with norm weights 1 + N(0, 0.02);
                                                    # --all-steps: logits of every decode step
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from nnzap_amd import configs as cf  # noqa: E402
from nnzap_amd import synth as S  # noqa: E402
from oracle import oracle as O  # noqa: E402
from oracle.decoder import OracleDecoder  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def small():
    out = {}
    # reference fixture: transformer_test.zig:1606-1695 (K=5504, seed 0x5A)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from test_oracle import reference_test_packed
    w = reference_test_packed(64, 5504, 0x5A)
    x = (np.float32(0.1) * np.sin(np.arange(5504, dtype=np.float32) * np.float32(0.037))
         + np.float32(0.05)).astype(np.float32)
    out["q1_fixture_k5504"] = {"y": O.qmv(w, x).tolist()}
    # configs 1-3: input hashes + first 64 outputs
    w1, x1 = cf.config1()
    out["config1"] = {"sha256": sha(w1.codes, w1.scales, w1.biases, x1), "y64": O.qmv(w1, x1)[:64].tolist()}
    w2, x2 = cf.config2()
    out["config2"] = {"sha256": sha(w2.codes, w2.scales, x2), "y64": O.qmv(w2, x2)[:64].tolist()}
    wg, wu, x3 = cf.config3()
    out["config3"] = {"sha256": sha(wg.codes, wg.scales, wu.codes, wu.scales, x3),
                      "y64": O.qmv_pair_silu(wg, wu, x3)[:64].tolist()}
    # config 4 at L=512
    q, k, v = cf.config4(512)
    qf = O.rope(S.bf16_bits_to_f32(q).astype(np.float64), 512, 1e6)
    y4 = O.attention_decode(qf, S.bf16_bits_to_f32(k), S.bf16_bits_to_f32(v), 512, False)
    out["config4_L512"] = {"sha256": sha(q, k, v), "out": y4.tolist()}
    # tiny decoder: prefill logits (first 64) + 48 greedy tokens
    cfg = cf.TINY
    wt = cf.decoder_weights(cfg, norm_mode="unit")
    prompt = cf.prompt_ids(cfg, 32)
    od = OracleDecoder(wt)
    logits = od.forward(list(prompt), 0)[-1]
    toks, margins = OracleDecoder(wt).generate(prompt, 48)
    out["tiny_decoder"] = {"prompt": prompt.tolist(), "prefill_logits64": logits[:64].tolist(),
                           "tokens": toks.tolist(), "margins": margins.tolist()}
    with open(os.path.join(HERE, "small_vectors.json"), "w") as f:
        json.dump(out, f)
    print("wrote small_vectors.json")


LOGIT_STEPS = 16     # decode steps whose logits are recorded at LOGIT_STRIDE
LOGIT_STRIDE = 512   # every 512th logit is recorded besides the top 8
LATE_STRIDE = 1024   # steps past LOGIT_STEPS (all of them with --all-steps)


def logit_summary(logits, stride=LOGIT_STRIDE):
    """What the GPU test compares at full size: the top 8 (index, value), a
    strided sample of the whole vector, max |logit|, and a sha256 of the
    float32 values (identifies the vector; not compared on the GPU)."""
    lg = np.asarray(logits, dtype=np.float64)
    top = np.argsort(-lg, kind="stable")[:8]
    return {"top8_idx": top.tolist(), "top8_val": lg[top].tolist(),
            "sample": lg[::stride].tolist(), "stride": stride,
            "max_abs": float(np.max(np.abs(lg))),
            "sha256": sha(lg.astype(np.float32))}


def fp32_noise(w, prompt, summary) -> float:
    """Normwise spread (max |err| / max |logit| over the recorded entries)
    between the float64 oracle's last-prompt-token logits and the same
    algorithm with every weight product in float32 -- the rounding noise any
    float32 implementation carries end to end at this size (float16
    activation roundings flip and propagate through the 28 layers)."""
    od = OracleDecoder(w, max_ctx=len(prompt) + 8, matmul_dtype=np.float32)
    lg = od.forward(list(prompt), 0)[-1]
    idx = np.concatenate([np.array(summary["top8_idx"]), np.arange(0, len(lg), LOGIT_STRIDE)])
    want = np.concatenate([np.array(summary["top8_val"]), np.array(summary["sample"])])
    return float(np.max(np.abs(lg[idx] - want)) / summary["max_abs"])


def add_noise(name: str):
    path = os.path.join(HERE, name)
    g = json.load(open(path))
    cfg = cf.BONSAI_1_7B
    w = cf.decoder_weights(cfg, norm_mode=g["norm_mode"], host_embed=False)
    g["fp32_noise"] = fp32_noise(w, cf.prompt_ids(cfg, g["n_prompt"]), g["logits"][0])
    with open(path, "w") as f:
        json.dump(g, f)
    print(f"{name}: fp32 noise {g['fp32_noise']:.3e}")


def config5(n_prompt=512, n_new=256, norm_mode="small", out_name="config5_tokens.json",
            all_steps=False):
    """Greedy tokens of the full-size decoder and the logit summaries of the
    last prompt token and of the first LOGIT_STEPS decode steps (every step
    with all_steps: the later ones sampled every LATE_STRIDE logits), so the
    GPU test can teacher-force the golden tokens through the whole stream."""
    t0 = time.time()
    cfg = cf.BONSAI_1_7B
    w = cf.decoder_weights(cfg, norm_mode=norm_mode, host_embed=False)  # rows on demand
    print(f"weights {time.time() - t0:.0f}s", flush=True)
    od = OracleDecoder(w, max_ctx=n_prompt + n_new + 8)
    print(f"dequant {time.time() - t0:.0f}s", flush=True)
    prompt = cf.prompt_ids(cfg, n_prompt)
    logits = od.forward(list(prompt), 0)[-1]
    print(f"prefill {time.time() - t0:.0f}s", flush=True)
    summaries = [logit_summary(logits)]      # last prefill token, then decode steps
    pos = n_prompt
    toks, margins = [], []
    for i in range(n_new):
        t = O.argmax_first(logits)
        srt = np.sort(logits)
        toks.append(int(t))
        margins.append(float(srt[-1] - srt[-2]))
        logits = od.forward([t], pos)[0]
        if i < LOGIT_STEPS:
            summaries.append(logit_summary(logits))
        elif all_steps and i < n_new - 1:
            summaries.append(logit_summary(logits, LATE_STRIDE))
        pos += 1
        if i % 16 == 0:
            print(f"step {i} token {t} margin {margins[-1]:.3e} ({time.time() - t0:.0f}s)", flush=True)
    del od
    noise = fp32_noise(w, prompt, summaries[0])
    res = {"n_prompt": n_prompt, "n_new": n_new, "norm_mode": norm_mode, "lm_head": "q1",
           "fp32_noise": noise,
           "prompt_sha256": sha(prompt), "tokens": toks, "margins": margins,
           "min_margin": min(margins), "distinct_tokens": len(set(toks)),
           "logit_stride": LOGIT_STRIDE,
           "logits": summaries}
    with open(os.path.join(HERE, out_name), "w") as f:
        json.dump(res, f)
    print(f"wrote {out_name} in {time.time() - t0:.0f}s; min margin {min(margins):.3e}; "
          f"{len(set(toks))} distinct tokens")


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "small"
    if what == "small":
        small()
    elif what == "config5":
        config5()
    elif what == "noise":
        # record the float32 noise in existing config-5 fixtures
        add_noise("config5_tokens.json")
        add_noise("config5_unit_tokens.json")
    elif what == "config5_unit":
        # norm weights 1 + N(0, 0.02): the fallback of the norm-weight
        # decision, whose token stream is not periodic
        config5(norm_mode="unit", out_name="config5_unit_tokens.json",
                all_steps="--all-steps" in sys.argv)
    else:
        raise SystemExit(f"unknown fixture set {what}")

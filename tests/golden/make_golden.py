"""Writes the committed golden fixtures under tests/golden/ with the CPU oracle.

The reference ships no numeric expected outputs for this path (its tests
recompute CPU references at run time and its e2e goldens need real Bonsai
checkpoints), so these fixtures are produced by the oracle from seeded
synthetic inputs -- the seeds make the inputs reproducible on any host.

  python tests/golden/make_golden.py small     # kernel-level vectors (seconds)
  python tests/golden/make_golden.py config5   # 28-layer greedy tokens (minutes, ~20 GB RAM)
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


def config5(n_prompt=512, n_new=256, norm_mode="small"):
    t0 = time.time()
    cfg = cf.BONSAI_1_7B
    w = cf.decoder_weights(cfg, norm_mode=norm_mode, host_embed=False)  # rows on demand
    print(f"weights {time.time() - t0:.0f}s", flush=True)
    od = OracleDecoder(w, max_ctx=n_prompt + n_new + 8)
    print(f"dequant {time.time() - t0:.0f}s", flush=True)
    prompt = cf.prompt_ids(cfg, n_prompt)
    logits = od.forward(list(prompt), 0)[-1]
    print(f"prefill {time.time() - t0:.0f}s", flush=True)
    pos = n_prompt
    toks, margins = [], []
    for i in range(n_new):
        t = O.argmax_first(logits)
        srt = np.sort(logits)
        toks.append(int(t))
        margins.append(float(srt[-1] - srt[-2]))
        logits = od.forward([t], pos)[0]
        pos += 1
        if i % 16 == 0:
            print(f"step {i} token {t} margin {margins[-1]:.3e} ({time.time() - t0:.0f}s)", flush=True)
    res = {"n_prompt": n_prompt, "n_new": n_new, "norm_mode": norm_mode, "lm_head": "q1",
           "prompt_sha256": sha(prompt), "tokens": toks, "margins": margins,
           "min_margin": min(margins)}
    with open(os.path.join(HERE, "config5_tokens.json"), "w") as f:
        json.dump(res, f)
    print(f"wrote config5_tokens.json in {time.time() - t0:.0f}s; min margin {min(margins):.3e}")


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "small"
    if what == "small":
        small()
    elif what == "config5":
        config5()
    else:
        raise SystemExit(f"unknown fixture set {what}")

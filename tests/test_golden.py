"""The committed golden fixtures are reproduced bit-for-bit by the seeded input
generator and the oracle on this host (CPU only)."""
import json
import os

import numpy as np
import pytest

from nnzap_amd import configs as cf
from nnzap_amd import synth as S
from oracle import oracle as O

HERE = os.path.join(os.path.dirname(__file__), "golden")
G = json.load(open(os.path.join(HERE, "small_vectors.json")))


def _sha(*arrays):
    import hashlib
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_config_inputs_hash_and_outputs():
    w1, x1 = cf.config1()
    assert _sha(w1.codes, w1.scales, w1.biases, x1) == G["config1"]["sha256"]
    assert np.allclose(O.qmv(w1, x1)[:64], G["config1"]["y64"], rtol=1e-12, atol=1e-12)
    w2, x2 = cf.config2()
    assert _sha(w2.codes, w2.scales, x2) == G["config2"]["sha256"]
    assert np.allclose(O.qmv(w2, x2)[:64], G["config2"]["y64"], rtol=1e-12, atol=1e-12)
    wg, wu, x3 = cf.config3()
    assert _sha(wg.codes, wg.scales, wu.codes, wu.scales, x3) == G["config3"]["sha256"]


def test_config4_hash():
    q, k, v = cf.config4(512)
    assert _sha(q, k, v) == G["config4_L512"]["sha256"]


def test_tiny_decoder_tokens_reproduce():
    from oracle.decoder import OracleDecoder
    cfg = cf.TINY
    w = cf.decoder_weights(cfg, norm_mode="unit")
    prompt = cf.prompt_ids(cfg, 32)
    assert prompt.tolist() == G["tiny_decoder"]["prompt"]
    toks, _ = OracleDecoder(w).generate(prompt, 48)
    assert toks.tolist() == G["tiny_decoder"]["tokens"]


def test_config5_fixture_prompt():
    path = os.path.join(HERE, "config5_tokens.json")
    if not os.path.exists(path):
        pytest.skip("config5 fixture not generated")
    g = json.load(open(path))
    assert _sha(cf.prompt_ids(cf.BONSAI_1_7B, g["n_prompt"])) == g["prompt_sha256"]
    assert len(g["tokens"]) == g["n_new"] and all(0 <= t < 151936 for t in g["tokens"])

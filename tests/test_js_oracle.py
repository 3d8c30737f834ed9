"""The single-threaded JavaScript restatement of the decode pass
(oracle/js/decode.js, the CPU "JS path" baseline) against the C oracle on
the same generated weights and K/V: a 2-block SmolLM2-shaped model, three
chats, two greedy passes. JavaScript sums in f64 and the oracle in f32, so
the logits agree to rounding (1e-3 absolute) and the greedy ids agree
wherever the oracle's top-1/top-2 margin exceeds that."""
import os

import numpy as np
import pytest

from chattorrent_amd import configs
from oracle import jsdecode as J
from oracle import lib as L
from oracle import model as Mo

pytestmark = pytest.mark.skipif(J.node_binary() is None, reason="node is not installed")

SEED = 1234


def test_js_pass_matches_the_c_oracle(tmp_path):
    d = configs.with_layers(configs.SMOLLM2, 2)
    ctxs = [17, 130, 70]
    first = [int(i) for i in L.gen_ids(SEED, 0x5EED, len(ctxs), d["vocab"])]
    J.write_inputs(str(tmp_path), d, SEED, ctxs, first, steps=2, logits_out="logits0.f32")
    got = J.run(str(tmp_path), 2, timeout=300)
    om = Mo.Model(d, n_slots=len(ctxs), max_pages=4)
    om.gen_weights(SEED)
    for s, T in enumerate(ctxs):
        om.fill_random_kv(s, T, SEED, s + 1)
    logits0 = np.fromfile(os.path.join(str(tmp_path), "logits0.f32"), np.float32).reshape(len(ctxs), d["vocab"])
    ids = first
    for step in range(2):
        jobs = [dict(slot=s, past=T + step, n=1, ids=[ids[s]], sampled=1, topk=2) for s, T in enumerate(ctxs)]
        want = np.concatenate([w["logits"] for w in om.pass_(jobs)])
        if step == 0:
            assert np.abs(logits0 - want).max() <= 1e-3, np.abs(logits0 - want).max()
        for s in range(len(ctxs)):
            order = np.argsort(-want[s], kind="stable")
            if want[s, order[0]] - want[s, order[1]] > 1e-3:
                assert got["ids"][step][s] == order[0], (step, s)
            assert abs(got["top"][step][s] - want[s, got["ids"][step][s]]) <= 1e-3
        ids = got["ids"][step]
    assert got["steps"] == 2 and got["ms_per_step"] > 0

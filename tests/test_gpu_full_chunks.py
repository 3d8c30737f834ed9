"""configs[4] at its own depth: the Llama-3.1-8B-shaped model (32 blocks,
untied head, llama3 RoPE scaling) with a 512-row prompt chunk packed beside
decode rows, against the oracle on identical seeded inputs, over three passes
(web/model/stage.js:1314-1481 #pass with prefill chunks, as route.js feeds
them):

1. 24 decode rows (chats with random int8 KV, contexts log-uniform in
   [32, 4096]) and the first 512-token chunk of a new chat's prompt (not
   sampled);
2. the decode rows' next tokens and the prompt's last 100 tokens, its last
   row sampled;
3. all 25 chats decoding, the new one from its first sample.
Both sides always continue with the oracle's greedy ids, so a near tie
cannot split the trajectories.

Bars: every sampled row's logits within 1e-2 of the oracle's; greedy ids
equal wherever the oracle's top-1/top-2 margin exceeds twice the row's logit
difference (closer rows are reported); the new chat's K/V rows of both chunks
in blocks 0 and 31 within one code and scales within 1e-5 relative, from
inputs both sides share bit for bit (block 0's is the rounded embedding;
block 31 is re-run on the GPU from the oracle's own rows into it); and the device's page tables equal the oracle's ensurePages replay
(web/model/model.js:185-211) after every pass."""
import json

import numpy as np
import pytest

from chattorrent_amd import configs
from test_gpu_full import _progress, _report, _top2

pytestmark = pytest.mark.gpu

SEED = 1234 + 5
DECODE = 24
PROMPT = 612
CHUNK = 512
TOL = 1e-2


def _check_kv(c, om, d, slot, t0, t1, layer):
    """The device's K/V rows t0..t1-1 of `slot` in `layer` against the
    oracle's: (equal codes, codes, largest code difference, largest relative
    scale difference)."""
    D, nKV = d["head_dim"], d["n_kv_heads"]
    same = total = dmax = 0
    rmax = 0.0
    for which in (0, 1):
        for h in range(nKV):
            g = c.read_kv(layer, which, slot, h, t0, t1)
            w = om.kv_rows(layer, which, slot, t0, t1, h)
            gc = g[:, :D // 4].view(np.int8).astype(np.int32)
            wc = w[:, :D // 4].view(np.int8).astype(np.int32)
            gs, ws = g[:, D // 4:].view(np.float32), w[:, D // 4:].view(np.float32)
            dmax = max(dmax, int(np.abs(gc - wc).max()))
            rmax = max(rmax, float((np.abs(gs - ws) / np.maximum(np.abs(ws), 1e-30)).max()))
            same += int((gc == wc).sum())
            total += gc.size
    return same, total, dmax, rmax


def test_config4_8b_full_depth_chunk_beside_decode(gpu):
    from chattorrent_amd.ccdecode import Context
    from oracle import lib as L
    from oracle import model as Mo
    d = configs.LLAMA8B
    V = d["vocab"]
    rng = np.random.default_rng(SEED)
    ctxs = [int(t) for t in np.exp(rng.uniform(np.log(32), np.log(4096), DECODE))]
    new = DECODE                                      # the new chat's frame
    n_max = 4096 + 64
    max_pages = n_max // 64
    c = Context(d, n_max=n_max, t_max=DECODE + CHUNK, slots=DECODE + 1, sessions=DECODE + 1, max_jobs=DECODE + 1)
    om = Mo.Model(d, n_slots=DECODE + 1, max_pages=max_pages)
    try:
        c.fill_random(SEED)
        om.gen_weights(SEED)
        _progress("configs[4] 8B oracle weights generated")
        for s, T in enumerate(ctxs):
            c.fill_random_kv(s, T, SEED, s + 1)
            om.fill_random_kv(s, T, SEED, s + 1)
        prompt = L.gen_ids(SEED, 0x8B, PROMPT, V)
        toks = [int(x) for x in rng.integers(0, V, DECODE)]
        new_tok = None
        rec = {"passes": [], "contexts": ctxs}
        last_in = []
        for p in range(3):
            jobs = [dict(slot=s, past=T + p, n=1, ids=[toks[s]], sampled=1, topk=2) for s, T in enumerate(ctxs)]
            if p == 0:
                jobs.append(dict(slot=new, past=0, n=CHUNK, ids=[int(x) for x in prompt[:CHUNK]], sampled=0, topk=2))
            elif p == 1:
                jobs.append(dict(slot=new, past=CHUNK, n=PROMPT - CHUNK, ids=[int(x) for x in prompt[CHUNK:]],
                                 sampled=1, topk=2))
            else:
                jobs.append(dict(slot=new, past=PROMPT, n=1, ids=[new_tok], sampled=1, topk=2))
            _, ids = c.step(jobs, topk=2)
            sampled = [j for j in jobs if j["sampled"]]
            got = c.read_logits(len(sampled))
            cap = {}
            out = om.pass_(jobs, capture=lambda layer, x: cap.__setitem__(layer, x[-jobs[-1]["n"]:].copy())
                           if layer == d["n_layer"] - 2 else None)
            want = [w for w, j in zip(out, jobs) if j["sampled"]]
            if p < 2:
                last_in.append((jobs[-1], L.to_f16(cap[d["n_layer"] - 2])))   # the new chat's rows into block 31
            _progress(f"configs[4] pass {p} checked against the oracle")
            max_err, near, nxt = 0.0, [], []
            for r, (j, w) in enumerate(zip(sampled, want)):
                err = float(np.abs(got[r] - w["logits"][0]).max())
                max_err = max(max_err, err)
                assert err <= TOL, (p, j["slot"], err)
                want_id, margin = _top2(w["logits"][0])
                if margin > 2 * err:
                    assert int(ids[r, 0]) == want_id, (p, j["slot"], int(ids[r, 0]), want_id, margin, err)
                else:
                    near.append({"slot": j["slot"], "margin": margin, "err": err,
                                 "same_id": int(ids[r, 0]) == want_id})
                nxt.append(want_id)                  # both sides continue with the oracle's id
            for s in range(DECODE):
                assert list(c.pages(s)) == om.frames[s]["owned"], (p, s)
            assert list(c.pages(new)) == om.frames[new]["owned"], p
            toks = nxt[:DECODE]
            if p >= 1:
                new_tok = nxt[DECODE]
            rec["passes"].append({"rows": sum(j["n"] for j in jobs), "sampled": len(sampled), "max_logit_err": max_err,
                                  "rows_inside_noise": near})
        # block 0's input is the rounded embedding on both sides, bit for bit;
        # the last block's rows are checked after re-running it on the GPU
        # from the oracle's own input rows (its f16 residual after block 30)
        # for both chunks, as a downstream peer would enter it
        for j, rows in last_in:
            c.step([dict(slot=new, past=j["past"], n=j["n"], hidden=rows)], at=d["n_layer"], to=d["n_layer"] + 1)
        for layer in (0, d["n_layer"] - 1):
            codes_max, rtol, frac = 1, 1e-5, 0.99
            same, total, dmax, rmax = _check_kv(c, om, d, new, 0, PROMPT, layer)
            rec[f"kv_block{layer}"] = {"codes_equal_frac": same / total, "max_code_diff": dmax,
                                       "max_scale_rel_diff": rmax}
            assert dmax <= codes_max and rmax <= rtol and same / total > frac, (layer, rec[f"kv_block{layer}"])
        _report("configs[4] 8B 32 layers: 512-row chunk beside decode rows", rec)
        print(json.dumps(rec))
    finally:
        c.close()

"""configs[3] at its own depth: speculative verify on the 27B-class model
(64 blocks), 16 chats x 8 rows (1 real + 7 drafts), contexts U[4096, 32768],
against the layer-streamed oracle (oracle.model.StreamedModel) on identical
seeded inputs.

The drafts are built so that acceptance is exercised: each chat's drafts are
its own greedy continuation (decoded on the GPU one row at a time first),
broken after a[s] = s % 8 accepted drafts by an id that differs from the
greedy one. #finish's rule (web/model/stage.js:1522-1541) then accepts a[s]
drafts on the GPU, because row i of a verify carries the bits of the one-row
pass at the same position (test_verify_rows_equal_one_row_jobs); the oracle's
own acceptance must agree wherever its top-1/top-2 margins are clear of the
logit difference (the reference's greedy check of this kind is
web/dev/verify.js:241-262).

Bars, as at configs[2] (tests/test_gpu_full.py):
* per block: each of the 64 blocks run on the GPU from the oracle's own input
  rows gives the oracle's output within 2 f16 steps at the scale of the
  block's sublayer outputs; the distribution at each value's own scale is
  reported;
* end to end: the 128 rows' logits within max(1e-2, 2 x floor), the floor
  being the logit change the oracle itself shows when one f16 step is added
  to one element of a chat's entry row (measured here on four chats, whose
  rows are independent of the other chats', so the floor can only be
  smaller than over all sixteen);
* greedy ids equal wherever the oracle's margin exceeds twice the row's
  logit difference; the accepted-draft count per chat equal wherever every
  row it depends on is so;
* the K/V rows the verify appended at all 8 positions, in blocks 0, 31 and
  63: codes within one code of the oracle's (the same f32 inputs up to the
  matmul's rounding) and scales within 1e-5 relative."""
import json
import math

import numpy as np
import pytest

from chattorrent_amd import configs
from test_gpu_full import _f16_steps, _progress, _report, _top2

pytestmark = pytest.mark.gpu

SEED = 1234 + 3           # bench.py c4's contexts: default_rng(seed + 3)
CHATS, ROWS = 16, 8
TOL = 1e-2
KV_LAYERS = (0, 31, 63)


def _accepted(samples, drafts):
    """#finish's verify rule (web/model/stage.js:1522-1541): row i's sample
    is accepted while it equals draft i+1; the first mismatch stops."""
    a = 0
    while a < len(drafts) - 1 and int(samples[a]) == int(drafts[a + 1]):
        a += 1
    return a


def test_config3_27b_full_depth_verify(gpu):
    from chattorrent_amd.ccdecode import Context
    from oracle import lib as L
    from oracle import model as Mo
    d = configs.M27B
    V, D, nKV = d["vocab"], d["head_dim"], d["n_kv_heads"]
    rng = np.random.default_rng(SEED)
    pasts = [int(t) for t in rng.integers(4096, 32769, CHATS)]
    n_max = 64 * math.ceil((max(pasts) + ROWS + 8) / 64)
    c = Context(d, n_max=n_max, t_max=CHATS * ROWS, slots=CHATS, sessions=CHATS, max_jobs=CHATS)
    try:
        c.fill_random(SEED)
        for s, T in enumerate(pasts):
            c.fill_random_kv(s, T, SEED, s + 1)
        # each chat's greedy continuation, one row a pass
        chain = np.zeros((CHATS, ROWS), np.int64)
        chain[:, 0] = rng.integers(0, V, CHATS)
        for k in range(ROWS - 1):
            _, ids = c.step([dict(slot=s, past=T + k, n=1, ids=[int(chain[s, k])], sampled=1)
                             for s, T in enumerate(pasts)], topk=1)
            chain[:, k + 1] = ids[:, 0]
        want_acc = [s % ROWS for s in range(CHATS)]
        drafts = chain.copy()
        for s, a in enumerate(want_acc):
            if a + 1 < ROWS:
                drafts[s, a + 1] = (chain[s, a + 1] + 1 + s) % V
                drafts[s, a + 2:] = rng.integers(0, V, ROWS - a - 2)
        jobs = [dict(slot=s, past=T, n=ROWS, ids=[int(x) for x in drafts[s]], sampled=ROWS, topk=2)
                for s, T in enumerate(pasts)]
        _, ids = c.step(jobs, topk=2)
        logits = c.read_logits(CHATS * ROWS)
        got_ids = ids[:, 0].reshape(CHATS, ROWS)
        got_acc = [_accepted(got_ids[s], drafts[s]) for s in range(CHATS)]
        assert got_acc == want_acc, (got_acc, want_acc)
        _progress("configs[3] GPU verify pass done")

        ctxs = [(T, s + 1) for s, T in enumerate(pasts)]
        sm = Mo.StreamedModel(d, SEED, ctxs, ROWS)
        sm.on_layer = lambda layer: _progress(f"configs[3] oracle block {layer} done")
        after, terms = [], []
        sm.on_sublayers = lambda layer, a, m: terms.append(np.maximum(np.sqrt((a * a).mean(axis=1, keepdims=True)),
                                                                      np.sqrt((m * m).mean(axis=1, keepdims=True))))
        want = sm.pass_(jobs, capture=lambda layer, x: after.append(L.to_f16(x)))

        # the floor, on four chats: one f16 step added to the entry row
        fl = [0, 5, 10, 15]
        sp = Mo.StreamedModel(d, SEED, [ctxs[s] for s in fl], 1)
        sp.on_layer = lambda layer: _progress(f"configs[3] perturbed oracle block {layer} done")
        codes, sc = sp.w["wte"]
        pj = []
        for i, s in enumerate(fl):
            h = L.to_f16(L.round_f16(L.gather_embed_q8(np.array([int(drafts[s, 0])], np.int32), codes, sc, 32)))
            h[0, 0] += 1
            pj.append(dict(slot=i, past=pasts[s], n=1, ids=None, hidden=L.from_f16(h), sampled=1, topk=2))
        moved = sp.pass_(pj)
        floor = max(float(np.abs(moved[i]["logits"][0] - want[s]["logits"][0]).max()) for i, s in enumerate(fl))

        # per block: the GPU from the oracle's rows before each block
        emb = np.concatenate([L.to_f16(L.round_f16(L.gather_embed_q8(np.array(j["ids"], np.int32), codes, sc, 32)))
                              for j in jobs])
        entry = c.step([dict(slot=s, past=T, n=ROWS, ids=jobs[s]["ids"]) for s, T in enumerate(pasts)], at=0, to=1)
        assert np.array_equal(entry, emb)                       # gather + round is exact
        worst_scaled = worst_own = 0.0
        within1, within2 = [], []
        rows_in = emb
        for b in range(d["n_layer"]):
            hj = [dict(slot=s, past=T, n=ROWS, hidden=rows_in[ROWS * s:ROWS * (s + 1)]) for s, T in enumerate(pasts)]
            got = c.step(hj, at=b + 1, to=b + 2)
            scaled, own = _f16_steps(got, after[b], rows_in, terms[b])
            assert scaled.max() <= 2, (b, float(scaled.max()))
            worst_scaled, worst_own = max(worst_scaled, float(scaled.max())), max(worst_own, float(own.max()))
            within1.append(float((own <= 1).mean()))
            within2.append(float((own <= 2).mean()))
            rows_in = after[b]
        _progress("configs[3] per-block checks done")

        # the appended K/V rows: after the per-block passes every block's rows
        # come from the oracle's own input rows
        same = total = 0
        for layer in KV_LAYERS:
            for which in (0, 1):
                for s, T in enumerate(pasts):
                    w = np.stack([sm.kept[layer][(s, t)][which] for t in range(T, T + ROWS)])   # [t, nKV, RW]
                    for h in range(nKV):
                        g = c.read_kv(layer, which, s, h, T, T + ROWS)
                        gc = g[:, :D // 4].view(np.int8).astype(np.int32)
                        wc = np.ascontiguousarray(w[:, h, :D // 4]).view(np.int8).astype(np.int32)
                        assert np.abs(gc - wc).max() <= 1, (layer, which, s, h)
                        gs = g[:, D // 4:].view(np.float32)
                        ws = np.ascontiguousarray(w[:, h, D // 4:]).view(np.float32)
                        assert np.allclose(gs, ws, rtol=1e-5, atol=1e-30), (layer, which, s, h)
                        same += int((gc == wc).sum())
                        total += gc.size
        assert same / total > 0.99, same / total

        # end to end: logits, ids and acceptance
        bound = max(TOL, 2.0 * floor)
        max_err, near, margins = 0.0, [], []
        ok_rows = np.zeros((CHATS, ROWS), bool)
        ids_equal = 0
        for s in range(CHATS):
            for i in range(ROWS):
                g, w = logits[ROWS * s + i], want[s]["logits"][i]
                err = float(np.abs(g - w).max())
                max_err = max(max_err, err)
                assert err <= bound, ((s, i), err, bound)
                want_id, margin = _top2(w)
                margins.append(margin)
                ids_equal += int(got_ids[s, i]) == want_id
                if margin > 2 * err:
                    assert int(got_ids[s, i]) == want_id, ((s, i), int(got_ids[s, i]), want_id, margin, err)
                    ok_rows[s, i] = True
                else:
                    near.append({"chat": s, "row": i, "margin": margin, "err": err,
                                 "same_id": int(got_ids[s, i]) == want_id})
        acc_checked = 0
        oracle_acc = []
        for s in range(CHATS):
            wa = _accepted([_top2(want[s]["logits"][i])[0] for i in range(ROWS)], drafts[s])
            oracle_acc.append(wa)
            decided = min(wa + 1, ROWS - 1)              # rows 0 .. the first mismatch decide it
            if ok_rows[s, :decided].all():
                assert wa == got_acc[s], (s, wa, got_acc[s])
                acc_checked += 1
        m = np.array(margins)
        rec = {"rows": CHATS * ROWS, "contexts": pasts, "max_logit_err": max_err, "floor_one_step_perturbation": floor,
               "logit_bound": bound, "ids_equal": ids_equal, "min_margin": float(m.min()),
               "median_margin": float(np.median(m)), "rows_inside_noise": near,
               "accepted_gpu": got_acc, "accepted_oracle": oracle_acc, "acceptance_checked_chats": acc_checked,
               "per_block_max_steps_at_scale": worst_scaled, "per_block_max_steps_own": worst_own,
               "per_block_min_frac_within_one_own_step": min(within1),
               "per_block_min_frac_within_two_own_steps": min(within2),
               "kv_codes_equal_frac": same / total}
        _report("configs[3] 27B 64 layers x 16 chats x 8 verify rows", rec)
        print(json.dumps(rec))
        assert acc_checked >= CHATS // 2, rec
    finally:
        c.close()

"""Hybrid (Qwen3.5-architecture) models through cc_step against the oracle's
HybridModel on identical weights (tests/hybrid_weights.py): Gated DeltaNet
blocks with each session's recurrent state and conv ring carried across
passes (web/model/model.js:418-527), full-attention blocks with q_norm /
k_norm, partial rotary and the output gate (:368-410), in packed ragged
batches; a session restarted at position 0 starts from a zero state."""
import numpy as np
import pytest

import hybrid_weights as HW
from oracle import hybrid as Hy

pytestmark = pytest.mark.gpu
SEED = 11


def _ids(rng, n, vocab):
    return rng.integers(0, vocab, size=n).astype(np.int32)


def _check(got_vals, got_ids, want, ctx):
    """Whole logits rows within 2e-3 of the rows' largest magnitude; greedy
    ids equal unless the oracle's top-2 margin is below that."""
    logits = np.concatenate([w["logits"] for w in want])
    full = ctx.read_logits(logits.shape[0])
    tol = max(1e-2, 2e-3 * np.abs(logits).max())
    err = np.abs(full - logits).max()
    assert err <= tol, (err, tol)
    for r in range(logits.shape[0]):
        order = np.argsort(-logits[r], kind="stable")
        if logits[r, order[0]] - logits[r, order[1]] > tol:
            assert got_ids[r, 0] == order[0], (r, got_ids[r, 0], order[0])
    return logits


def _pair(d, slots=3, n_max=512, t_max=64):
    from chattorrent_amd.ccdecode import Context
    c = Context(d, n_max=n_max, t_max=t_max, slots=slots)
    om = Hy.HybridModel(d, n_slots=slots, max_pages=-(-n_max // 64))
    om.w = HW.make(d, SEED)
    HW.upload(c, om.w, d)
    return c, om


@pytest.mark.parametrize("cfg", ["spike", "wide", "d256"])
def test_hybrid_passes_match_oracle(gpu, cfg):
    """Prefill of two sessions, decode steps fed back greedily, a 3-row verify
    beside a decode, then a new session in a used slot (state reset)."""
    d = {"spike": HW.SPIKE, "wide": HW.WIDE, "d256": HW.D256}[cfg]
    c, om = _pair(d)
    rng = np.random.default_rng(3)
    V = d["vocab"]
    try:
        jobs = [dict(slot=0, past=0, n=12, ids=_ids(rng, 12, V), sampled=1, topk=4),
                dict(slot=1, past=0, n=5, ids=_ids(rng, 5, V), sampled=1, topk=4)]
        pasts = [12, 5]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        nxt = [int(ids[0, 0]), int(ids[1, 0])]
        for step in range(4):
            jobs = [dict(slot=s, past=pasts[s], n=1, ids=np.array([nxt[s]], np.int32), sampled=1, topk=4)
                    for s in (0, 1)]
            vals, ids = c.step(jobs, topk=4)
            logits = _check(vals, ids, om.pass_(jobs), c)
            nxt = [int(np.argmax(logits[0])), int(np.argmax(logits[1]))]
            pasts = [pasts[0] + 1, pasts[1] + 1]
        # a verify of 3 rows on session 0 beside a decode row on session 1
        jobs = [dict(slot=0, past=pasts[0], n=3, ids=_ids(rng, 3, V), sampled=3, topk=4),
                dict(slot=1, past=pasts[1], n=1, ids=np.array([nxt[1]], np.int32), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        # slot 1 taken by a new session: its pages go back, it starts at 0
        c.release(1)
        om.base.pool.release(om.base.frames[1])
        jobs = [dict(slot=1, past=0, n=7, ids=_ids(rng, 7, V), sampled=1, topk=4),
                dict(slot=0, past=pasts[0] + 3, n=1, ids=np.array([nxt[0]], np.int32), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
    finally:
        c.close()


def test_hybrid_state_carries_across_passes_bitwise(gpu):
    """A prompt in one pass, in two and in three gives the last row's logits
    bit for bit: the recurrent state and the conv ring are stored as f32
    between passes and each token runs the same arithmetic."""
    d = HW.SPIKE
    rng = np.random.default_rng(9)
    prompt = _ids(rng, 12, d["vocab"])
    got = []
    for cuts in ([12], [5, 7], [5, 1, 6], [1, 1, 1, 9]):
        c, _ = _pair(d, slots=1)
        try:
            past = 0
            for n in cuts:
                job = dict(slot=0, past=past, n=n, ids=prompt[past:past + n], sampled=1, topk=2)
                c.step([job], topk=2)
                past += n
            got.append(c.read_logits(1).copy())
        finally:
            c.close()
    for g in got[1:]:
        assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32))


def test_hybrid_batch_mates_do_not_change_bits(gpu):
    """A session's logits do not depend on the other sessions packed with it."""
    d = HW.WIDE
    rng = np.random.default_rng(4)
    p0, p1 = _ids(rng, 9, d["vocab"]), _ids(rng, 20, d["vocab"])
    c, _ = _pair(d)
    try:
        c.step([dict(slot=0, past=0, n=9, ids=p0, sampled=1, topk=2)], topk=2)
        alone = c.read_logits(1).copy()
        c.release(0)
        c.step([dict(slot=1, past=0, n=20, ids=p1, sampled=1, topk=2),
                dict(slot=0, past=0, n=9, ids=p0, sampled=1, topk=2)], topk=2)
        both = c.read_logits(2)
        assert np.array_equal(both[1].view(np.uint32), alone[0].view(np.uint32))
    finally:
        c.close()


def _run(c, jobs, topk=2):
    c.step(jobs, topk=topk)
    return c.read_logits(sum(j.get("sampled", 1) for j in jobs)).copy()


@pytest.mark.parametrize("keep", [0, 2, 4])
def test_hybrid_verify_rollback_matches_oracle(gpu, keep):
    """A 4-row verify (snap) beside another session's decode, then the next
    job rolls the linear blocks back to before the verify and re-runs its
    first `keep` rows (stage.js:1248-1283, model.js:447-470); the following
    decode continues from there. Every pass against the oracle."""
    d = HW.SPIKE
    c, om = _pair(d)
    rng = np.random.default_rng(21)
    V = d["vocab"]
    try:
        jobs = [dict(slot=0, past=0, n=12, ids=_ids(rng, 12, V), sampled=1, topk=4),
                dict(slot=1, past=0, n=6, ids=_ids(rng, 6, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        jobs = [dict(slot=0, past=12, n=4, ids=_ids(rng, 4, V), sampled=4, topk=4, snap=True),
                dict(slot=1, past=6, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        jobs = [dict(slot=0, past=12 + keep, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4, keep=keep),
                dict(slot=1, past=7, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        jobs = [dict(slot=0, past=13 + keep, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
    finally:
        c.close()


def test_hybrid_rollback_equals_plain_feed_bitwise(gpu):
    """A verify of [t, d1, d2, d3] rolled back to keep 2, then token x, gives
    the same logits bit for bit as feeding [t, d1] and then x plainly: the
    recurrent state is replayed with the same arithmetic, and the rejected
    rows' KV is overwritten or masked."""
    d = HW.SPIKE
    rng = np.random.default_rng(22)
    V = d["vocab"]
    prompt, ver, x = _ids(rng, 10, V), _ids(rng, 4, V), _ids(rng, 1, V)
    c, _ = _pair(d, slots=1)
    try:
        _run(c, [dict(slot=0, past=0, n=10, ids=prompt, sampled=1)])
        _run(c, [dict(slot=0, past=10, n=4, ids=ver, sampled=4, snap=True)])
        spec = _run(c, [dict(slot=0, past=12, n=1, ids=x, sampled=1, keep=2)])
    finally:
        c.close()
    c, _ = _pair(d, slots=1)
    try:
        _run(c, [dict(slot=0, past=0, n=10, ids=prompt, sampled=1)])
        _run(c, [dict(slot=0, past=10, n=2, ids=ver[:2], sampled=1)])
        plain = _run(c, [dict(slot=0, past=12, n=1, ids=x, sampled=1)])
    finally:
        c.close()
    assert np.array_equal(spec.view(np.uint32), plain.view(np.uint32))


def test_hybrid_refuses_what_it_cannot_replay(gpu):
    """A rollback with no verify before it, one past the verify's rows, a
    plain job that skips or rewinds rows, and a verify above 8 rows are
    refused (cold / bad job) and change nothing."""
    from chattorrent_amd.ccdecode import CC_COLD, CC_EARG, CCError
    d = HW.SPIKE
    rng = np.random.default_rng(23)
    V = d["vocab"]
    c, _ = _pair(d, slots=1, t_max=64)
    try:
        _run(c, [dict(slot=0, past=0, n=5, ids=_ids(rng, 5, V), sampled=1)])
        for job, code in ((dict(slot=0, past=5, n=1, keep=0), CC_COLD),        # no verify to return to
                          (dict(slot=0, past=7, n=1), CC_COLD),                # skips rows
                          (dict(slot=0, past=3, n=1), CC_COLD),                # rewinds
                          (dict(slot=0, past=5, n=9, snap=True), CC_EARG)):    # verify above 8 rows
            job = dict(job, ids=_ids(rng, job["n"], V), sampled=1)
            with pytest.raises(CCError) as e:
                c.step([job], topk=2)
            assert e.value.status == code, (job, e.value)
        _run(c, [dict(slot=0, past=5, n=3, ids=_ids(rng, 3, V), sampled=3, snap=True)])
        with pytest.raises(CCError) as e:   # keep beyond the verify's 3 rows
            c.step([dict(slot=0, past=9, n=1, ids=_ids(rng, 1, V), sampled=1, keep=4)], topk=2)
        assert e.value.status == CC_COLD
        _run(c, [dict(slot=0, past=8, n=1, ids=_ids(rng, 1, V), sampled=1, keep=3)])
    finally:
        c.close()


def test_hybrid_long_jobs_take_the_row_parallel_conv_bitwise(gpu):
    """A prompt longer than 16 rows runs the conv parallel over rows (ring
    stashed, rows, ring advanced); cut into short jobs it runs the
    one-thread-per-channel conv. Both give the same logits, bit for bit."""
    d = HW.SPIKE
    rng = np.random.default_rng(41)
    prompt = _ids(rng, 40, d["vocab"])
    got = []
    for cuts in ([40], [16, 16, 8], [1, 39], [3, 20, 17]):
        c, _ = _pair(d, slots=1)
        try:
            past = 0
            for n in cuts:
                c.step([dict(slot=0, past=past, n=n, ids=prompt[past:past + n], sampled=1)], topk=2)
                past += n
            got.append(c.read_logits(1).copy())
        finally:
            c.close()
    for g in got[1:]:
        assert np.array_equal(g.view(np.uint32), got[0].view(np.uint32))


def test_hybrid_verify_beside_row_parallel_conv_then_rollback(gpu):
    """A 4-row verify (snap) packed beside another session's 30-row prompt
    chunk, so the pass runs the row-parallel conv (rows > 16), then a
    rollback to keep 2 with the next token beside that session's decode.
    The verifying session's logits equal, bit for bit, the same passes with
    the other session's chunk cut to 3 rows (the one-thread-per-channel
    conv, and the <= 32-row matmul), and every pass matches the oracle."""
    d = HW.SPIKE
    V = d["vocab"]
    rng = np.random.default_rng(43)
    p0, p1 = _ids(rng, 10, V), _ids(rng, 40, V)
    ver, x, y = _ids(rng, 4, V), _ids(rng, 1, V), _ids(rng, 1, V)
    runs = []
    for long_n in (30, 3):
        c, om = _pair(d)
        try:
            passes = [
                [dict(slot=0, past=0, n=10, ids=p0, sampled=1, topk=4),
                 dict(slot=1, past=0, n=5, ids=p1[:5], sampled=1, topk=4)],
                [dict(slot=0, past=10, n=4, ids=ver, sampled=4, topk=4, snap=True),
                 dict(slot=1, past=5, n=long_n, ids=p1[5:5 + long_n], sampled=1, topk=4)],
                [dict(slot=0, past=12, n=1, ids=x, sampled=1, topk=4, keep=2),
                 dict(slot=1, past=5 + long_n, n=1, ids=y, sampled=1, topk=4)],
                [dict(slot=0, past=13, n=1, ids=y, sampled=1, topk=4)],
            ]
            mine = []
            for jobs in passes:
                vals, ids = c.step(jobs, topk=4)
                logits = _check(vals, ids, om.pass_(jobs), c)
                rows = jobs[0]["sampled"]
                mine.append(c.read_logits(logits.shape[0])[:rows].copy())
            runs.append(mine)
        finally:
            c.close()
    for a, b in zip(*runs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_hybrid_long_rollback_job_matches_oracle(gpu):
    """A 40-row prefill beside a short one, a verify on the short session,
    then a 20-row job that rolls it back (keep 1) beside a decode: the long
    path's ring stash, rollback copies and snapshot, against the oracle."""
    d = HW.WIDE
    c, om = _pair(d)
    rng = np.random.default_rng(42)
    V = d["vocab"]
    try:
        jobs = [dict(slot=0, past=0, n=40, ids=_ids(rng, 40, V), sampled=1, topk=4),
                dict(slot=1, past=0, n=3, ids=_ids(rng, 3, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        jobs = [dict(slot=1, past=3, n=4, ids=_ids(rng, 4, V), sampled=4, topk=4, snap=True),
                dict(slot=0, past=40, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
        jobs = [dict(slot=1, past=4, n=20, ids=_ids(rng, 20, V), sampled=1, topk=4, keep=1),
                dict(slot=0, past=41, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        _check(vals, ids, om.pass_(jobs), c)
    finally:
        c.close()


def test_hybrid_split_over_two_peers_bitwise(gpu):
    """Two contexts holding positions [0, 3) and [3, 6) of a 4-block hybrid
    model, rows handed on as f16 bits (stage.js:1340-1346): prefill, a
    verify and a rollback crossing both, each context tracking its own
    recurrent blocks. The head's logits equal the single context's."""
    from chattorrent_amd.ccdecode import Context
    d = HW.SPIKE
    w = HW.make(d, SEED)
    rng = np.random.default_rng(51)
    V = d["vocab"]
    prompt, ver, x = _ids(rng, 9, V), _ids(rng, 4, V), _ids(rng, 1, V)
    plan = [dict(past=0, n=9, ids=prompt), dict(past=9, n=4, ids=ver, snap=True, sampled=4),
            dict(past=11, n=1, ids=x, keep=2)]
    whole = Context(d, n_max=256, t_max=16, slots=1)
    a = Context(d, n_max=256, t_max=16, slots=1, lo=0, hi=3)
    b = Context(d, n_max=256, t_max=16, slots=1, lo=3, hi=6)
    try:
        for c, lo, hi in ((whole, 0, 6), (a, 0, 3), (b, 3, 6)):
            HW.upload(c, w, d, lo, hi)
        for j in plan:
            job = dict(slot=0, sampled=j.get("sampled", 1), **{k: v for k, v in j.items() if k != "sampled"})
            whole.step([job], topk=2)
            want = whole.read_logits(job["sampled"]).copy()
            rows = a.step([dict(job, sampled=0)], at=0, to=3)
            b.step([dict(job, ids=None, hidden=rows)], at=3, to=6, topk=2)
            got = b.read_logits(job["sampled"])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), j
    finally:
        for c in (whole, a, b):
            c.close()


def test_hybrid_qwen38_widths_match_oracle(gpu):
    """Qwen3.8-27B's own widths through four of its blocks (three Gated DeltaNet,
    one full attention) against the oracle: hidden 5120, 24 query / 4 kv heads
    of 256 with a quarter rotary, 16 key / 48 value heads of 128 in the linear
    blocks, ffn 17408 and the untied 248320-row head. Prefill of two sessions,
    a decode step, a 4-row verify (snap) beside a decode, its rollback keeping
    2 rows, then a decode after it (web/model/model.js:411-527,
    web/model/stage.js:1248-1283)."""
    from chattorrent_amd import configs
    d = dict(configs.QWEN38, n_layer=4, layer_types=configs.QWEN38["layer_types"][:4])
    d.pop("mtp_vocab", None)
    c, om = _pair(d, slots=2, n_max=512, t_max=64)
    rng = np.random.default_rng(38)
    V = d["vocab"]
    errs = []

    def check(vals, ids, want):
        logits = _check(vals, ids, want, c)
        errs.append(float(np.abs(c.read_logits(logits.shape[0]) - logits).max()))
        return logits
    try:
        jobs = [dict(slot=0, past=0, n=20, ids=_ids(rng, 20, V), sampled=1, topk=4),
                dict(slot=1, past=0, n=9, ids=_ids(rng, 9, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        logits = check(vals, ids, om.pass_(jobs))
        nxt = [int(np.argmax(logits[0])), int(np.argmax(logits[1]))]
        jobs = [dict(slot=s, past=p, n=1, ids=np.array([nxt[s]], np.int32), sampled=1, topk=4)
                for s, p in ((0, 20), (1, 9))]
        vals, ids = c.step(jobs, topk=4)
        check(vals, ids, om.pass_(jobs))
        jobs = [dict(slot=0, past=21, n=4, ids=_ids(rng, 4, V), sampled=4, topk=4, snap=True),
                dict(slot=1, past=10, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        check(vals, ids, om.pass_(jobs))
        jobs = [dict(slot=0, past=23, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4, keep=2),
                dict(slot=1, past=11, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        check(vals, ids, om.pass_(jobs))
        jobs = [dict(slot=0, past=24, n=1, ids=_ids(rng, 1, V), sampled=1, topk=4)]
        vals, ids = c.step(jobs, topk=4)
        check(vals, ids, om.pass_(jobs))
        print("qwen3.8 widths, max |logit - oracle| per pass:", [round(e, 5) for e in errs])
    finally:
        c.close()

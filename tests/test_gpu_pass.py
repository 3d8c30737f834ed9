"""Pass-level parity: cc_step (Runner.#pass, web/model/stage.js:1314-1481)
against the oracle's restatement of the same pass, on identical seeded
weights and KV (both sides use the shared counter-based generator).

Bars: greedy ids identical (with the top-1/top-2
margin reported for the near-tie case); logits within 1e-2 abs; the f16
residual within 2 f16 ulp; packing, page indices and batch invariance
bit-exact."""
import json
import os
import warnings

import numpy as np
import pytest

from chattorrent_amd import configs

pytestmark = pytest.mark.gpu

SEED = 7


def _setup(gpu, d, contexts, n_max=1024, t_max=64, extra_slots=1):
    from chattorrent_amd.ccdecode import Context
    from oracle import model as Mo
    slots = len(contexts) + extra_slots
    c = Context(d, n_max=n_max, t_max=t_max, slots=slots)
    c.fill_random(SEED)
    om = Mo.Model(d, n_slots=slots, max_pages=-(-n_max // 64))
    om.gen_weights(SEED)
    for s, T in enumerate(contexts):
        if T:
            c.fill_random_kv(s, T, SEED, s + 1)
            om.fill_random_kv(s, T, SEED, s + 1)
    return c, om


def _report(name, rec):
    """A measured distribution, as a warning and, when gpurun_out/ exists,
    in gpurun_out/pass_parity.json."""
    warnings.warn(f"{name}: " + json.dumps(rec), stacklevel=2)
    out = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gpurun_out")
    if os.path.isdir(out):
        path = os.path.join(out, "pass_parity.json")
        try:
            with open(path) as f:
                allr = json.load(f)
        except (OSError, ValueError):
            allr = {}
        allr[name] = rec
        with open(path, "w") as f:
            json.dump(allr, f, indent=1)


def _ids(n, vocab, salt):
    from oracle import lib as L
    return L.gen_ids(SEED, 0x1D5 + salt, n, vocab)


def _f16_ulp_diff(a_bits, b_bits):
    """Distance in f16 steps between two arrays of half bits (same sign run)."""
    def key(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7fff), h & 0x7fff)
    return np.abs(key(a_bits) - key(b_bits))


def _f16_ulp(v):
    """The f16 step at |v| (2^-24 below the normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v.astype(np.float64)), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _ulps_at_scale(got_bits, want_bits, entry_bits):
    """|got - want| in f16 steps at the scale of the values the block handles:
    max(|want|, |entry|). A residual element that cancels to near zero inside
    a block (entry -4e-3 -> out -9e-6) has an error set by the terms that
    cancelled, not by the tiny result, so its step is the entry's."""
    from oracle import lib as L
    g, w, e = L.from_f16(got_bits), L.from_f16(want_bits), L.from_f16(entry_bits)
    scale = np.maximum(np.abs(w), np.abs(e))
    return np.abs(g.astype(np.float64) - w) / _f16_ulp(scale)


def _check_head(d, got_vals, got_ids, want, ctx=None, tol=1e-2):
    """got_*: [rows, M] candidates; want: oracle output rows. With `ctx`, the
    whole logits rows are compared too (cc_read_logits). Greedy ids must be
    equal unless the oracle's top-1/top-2 margin is below 1e-3 (reported)."""
    logits = np.concatenate([w["logits"] for w in want])
    rows = logits.shape[0]
    if ctx is not None:
        full = ctx.read_logits(rows)
        err = np.abs(full - logits).max()
        assert err <= tol, err
    margins = []
    for r in range(rows):
        row = logits[r]
        order = np.argsort(-row, kind="stable")
        margins.append(float(row[order[0]] - row[order[1]]))
        if margins[-1] > 1e-3:
            assert got_ids[r, 0] == order[0], (r, got_ids[r, 0], order[0], margins[-1])
        err = np.abs(got_vals[r] - row[got_ids[r]]).max()
        assert err <= tol, (r, err)
    return margins


@pytest.fixture(scope="module")
def smol(gpu):
    d = configs.with_layers(configs.SMOLLM2, 3)
    c, om = _setup(gpu, d, [17, 130, 511, 200])
    yield d, c, om
    c.close()


def test_decode_step_matches_oracle(smol):
    d, c, om = smol
    jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], s), sampled=1, topk=16)
            for s, T in enumerate([17, 130, 511, 200])]
    vals, ids = c.step(jobs, topk=16)
    want = om.pass_(jobs)
    _check_head(d, vals, ids, want, ctx=c)
    # The new K/V rows of block 0, whose input both sides share bit for bit
    # (the rounded embedding): the same codes except where the f32 K/V differ
    # by an ulp and sit on a rounding boundary (then by one code).
    D, nKV = d["head_dim"], d["n_kv_heads"]
    same = total = 0
    worst_scale = 0.0
    for layer in range(1):
        for which in (0, 1):
            for j in jobs:
                for h in range(nKV):
                    g = c.read_kv(layer, which, j["slot"], h, j["past"], j["past"] + 1)
                    w = om.kv_rows(layer, which, j["slot"], j["past"], j["past"] + 1, h)
                    gc = g[:, :D // 4].view(np.int8).astype(np.int32)
                    wc = w[:, :D // 4].view(np.int8).astype(np.int32)
                    assert np.abs(gc - wc).max() <= 1
                    gs, ws = g[:, D // 4:].view(np.float32), w[:, D // 4:].view(np.float32)
                    assert np.allclose(gs, ws, rtol=1e-5, atol=0)
                    worst_scale = max(worst_scale, float((np.abs(gs - ws) / np.abs(ws)).max()))
                    same += int((gc == wc).sum())
                    total += gc.size
    _report("block-0 new K/V rows, SmolLM2 shape, 4 jobs", {
        "codes": total, "codes_equal": same, "codes_off_by_one": total - same,
        "frac_equal": same / total, "scale_max_rel_diff": worst_scale})
    assert same / total > 0.99


def test_hidden_rows_within_two_f16_ulp_per_block(smol):
    """The f16 residual within 2 f16 ulp per block: each block run alone on
    the GPU (a pass entering at position b+1 with the oracle's f16 rows, as a
    downstream peer would, stage.js:1340-1346) against the oracle's rows after
    that block; the exit rows are f16 (stage.js:1553-1560)."""
    d, c, om = smol
    from oracle import lib as L
    pasts = [17, 130, 511, 200]
    jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 10 + s), sampled=0) for s, T in enumerate(pasts)]
    after = []
    om.pass_(jobs, head=False, capture=lambda layer, x: after.append(L.to_f16(x.copy())))
    entry = c.step(jobs, at=0, to=1)                       # the rounded embedding rows
    per_block = []
    for b in range(d["n_layer"]):
        hj = [dict(j, ids=None, hidden=entry[i:i + 1]) for i, j in enumerate(jobs)]
        got = c.step(hj, at=b + 1, to=b + 2)
        steps = _ulps_at_scale(got, after[b], entry)
        own = _f16_ulp_diff(got, after[b])
        per_block.append((int(steps.max()), float((own == 0).mean()), float((own <= 1).mean()), int(own.max())))
        assert steps.max() <= 2, (b, steps.max())
        assert (own <= 1).mean() > 0.99   # and nearly all within one step of themselves
        entry = after[b]                                   # the next block gets the oracle's rows
    # and the whole pass end to end stays close (one-step flips compound through blocks):
    # nearly every element within 2 f16 steps of itself, and every element within
    # 16 f16 steps at its row's RMS (a wrong channel or row would be off by far more)
    full = c.step(jobs, at=0, to=d["n_layer"] + 1)
    e2e = _f16_ulp_diff(full, after[-1])
    g, w = L.from_f16(full).astype(np.float64), L.from_f16(after[-1]).astype(np.float64)
    rms = np.sqrt((w * w).mean(axis=1, keepdims=True))
    worst = float((np.abs(g - w) / _f16_ulp(np.maximum(np.abs(w), rms))).max())
    _report("hidden rows, SmolLM2 shape, 4 jobs", {
        "blocks": len(per_block),
        "per_block_max_steps_at_scale": max(x[0] for x in per_block),
        "per_block_min_frac_equal": min(x[1] for x in per_block),
        "per_block_min_frac_within_one_own_step": min(x[2] for x in per_block),
        "per_block_max_own_steps": max(x[3] for x in per_block),
        "end_to_end_frac_equal": float((e2e == 0).mean()),
        "end_to_end_frac_within_two_own_steps": float((e2e <= 2).mean()),
        "end_to_end_max_steps_at_row_rms": worst})
    assert (e2e <= 2).mean() > 0.97
    assert worst <= 16, worst


def test_batched_equals_alone_bitwise(smol):
    """web/dev/batch.test.js: a batched pass gives each session the bits it
    gets alone (rows packed in order, every projection row-invariant)."""
    d, c, om = smol
    jobs = [dict(slot=s, past=T, n=n, ids=_ids(n, d["vocab"], 20 + s), sampled=n)
            for s, (T, n) in enumerate([(17, 1), (130, 4), (511, 1), (200, 8)])]
    vals, ids = c.step(jobs, topk=8)
    at = 0
    for j in jobs:
        v1, i1 = c.step([j], topk=8)
        n = j["n"]
        assert np.array_equal(i1, ids[at:at + n])
        assert np.array_equal(v1.view(np.uint32), vals[at:at + n].view(np.uint32))
        at += n


def test_verify_rows_equal_one_row_jobs(smol):
    """docs/model.md 'Matching plain decoding row by row': row i of an 8-row
    verify gives the bits of a one-row job at past + i."""
    d, c, om = smol
    P = 300                                   # slot 4: the spare frame, rows below P never written
    ids8 = _ids(8, d["vocab"], 40)
    vals, ids = c.step([dict(slot=4, past=P, n=8, ids=ids8, sampled=8)], topk=4)
    for i in range(8):
        v1, i1 = c.step([dict(slot=4, past=P + i, n=1, ids=ids8[i:i + 1], sampled=1)], topk=4)
        assert np.array_equal(i1[0], ids[i]) and np.array_equal(v1[0].view(np.uint32), vals[i].view(np.uint32))


def test_deterministic(smol):
    d, c, om = smol
    jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 50 + s), sampled=1)
            for s, T in enumerate([17, 130, 511, 200])]
    a = c.step(jobs, topk=8)
    b = c.step(jobs, topk=8)
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)) and np.array_equal(a[1], b[1])


def test_profile_replay_keeps_results(smol):
    """cc_profile's replay (each class relaunched back-to-back after the step)
    leaves the step's outputs and whole logits rows unchanged and counts one
    launch per block per class (one head launch)."""
    d, c, om = smol
    jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 60 + s), sampled=1)
            for s, T in enumerate([17, 130, 511, 200])]
    a = c.step(jobs, topk=8)
    la = c.read_logits(len(jobs))
    c.profile(True)
    try:
        b = c.step(jobs, topk=8)
        lb = c.read_logits(len(jobs))
        prof = c.profile_read()
    finally:
        c.profile(False)
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32)) and np.array_equal(a[1], b[1])
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    L = d["n_layer"]
    for k in ("qkv", "o", "gate_up", "down", "attn"):
        assert prof[k][1] == L and prof[k][0] > 0, (k, prof[k])
    assert prof["head"][1] == 1 and prof["head"][0] > 0


def test_prefill_and_verify_match_oracle(gpu):
    """Causal rows inside a job: a prefill chunk from position 0 and a verify
    run on top of a random cache, sampled at every row."""
    d = configs.with_layers(configs.SMOLLM2, 2)
    c, om = _setup(gpu, d, [0, 100])
    try:
        jobs = [dict(slot=0, past=0, n=37, ids=_ids(37, d["vocab"], 60), sampled=37),
                dict(slot=1, past=100, n=8, ids=_ids(8, d["vocab"], 61), sampled=8)]
        vals, ids = c.step(jobs, topk=4)
        want = om.pass_(jobs)
        _check_head(d, vals, ids, want, ctx=c)
    finally:
        c.close()


def test_block27b_step_matches_oracle(gpu):
    """One 27B-class block (d 5120, 40/8 heads, D 128, FFN 17408), decode rows
    over ragged contexts, vocab kept full: the head checks the 151936-wide LM
    head too."""
    d = configs.with_layers(configs.M27B, 1)
    ctxs = [256, 1000, 3000]
    c, om = _setup(gpu, d, ctxs, n_max=4096, t_max=16)
    try:
        jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 70 + s), sampled=1, topk=8)
                for s, T in enumerate(ctxs)]
        vals, ids = c.step(jobs, topk=8)
        want = om.pass_(jobs)
        _check_head(d, vals, ids, want, ctx=c)
    finally:
        c.close()


def test_page_allocation_replays_ensure_pages(gpu):
    """web/model/model.js:132-211: lowest index first, pages taken in job order
    and logical order, released last-first — the device table equals the
    oracle pool's replay of the same calls."""
    from chattorrent_amd.ccdecode import Context
    from oracle.model import PagePool
    d = configs.with_layers(configs.SMOLLM2, 1)
    c = Context(d, n_max=512, t_max=32, slots=2, sessions=5, max_jobs=5)
    pool = PagePool(2 * 8)
    frames = [{"pages": np.zeros(8, np.uint32), "owned": [], "max_pages": 8} for _ in range(5)]
    try:
        c.fill_random(SEED)

        def fill(slot, tokens):
            c.fill_random_kv(slot, tokens, SEED, slot + 1)
            assert pool.ensure(frames[slot], tokens)

        def check():
            for s in range(5):
                assert list(c.pages(s)) == frames[s]["owned"], s
            assert c.free_pages() == len(pool.free)

        fill(0, 70)
        fill(1, 129)
        fill(2, 5)
        check()
        c.release(1)
        pool.release(frames[1])
        check()
        jobs = [dict(slot=2, past=5, n=1, ids=[3], sampled=1), dict(slot=3, past=0, n=16, ids=np.arange(16), sampled=1),
                dict(slot=0, past=127, n=2, ids=[1, 2], sampled=1)]
        c.step(jobs, topk=1)
        for j in jobs:
            assert pool.ensure(frames[j["slot"]], j["past"] + j["n"])
        check()
    finally:
        c.close()


def test_error_classes(gpu):
    """#prepare's refusals (web/model/stage.js:1225-1259) and the capacity
    errors (:930-941 busy, :1114-1117 pool too small), per job, before any
    device work."""
    from chattorrent_amd.ccdecode import Context, CCError, CC_EARG, CC_BUSY, CC_EPOOL
    d = configs.with_layers(configs.SMOLLM2, 1)
    c = Context(d, n_max=256, t_max=16, slots=1, sessions=3, max_jobs=3)
    try:
        c.fill_random(SEED)
        with pytest.raises(CCError) as e:
            c.step([dict(slot=0, past=0, n=1, ids=[d["vocab"]], sampled=1)])
        assert e.value.status == CC_EARG and e.value.statuses[0] == CC_EARG
        with pytest.raises(CCError) as e:
            c.step([dict(slot=0, past=250, n=8, ids=np.zeros(8), sampled=1)])
        assert e.value.status == CC_EARG and "exceeds" in str(e.value)
        with pytest.raises(CCError) as e:
            c.step([dict(slot=0, past=0, n=17, ids=np.zeros(17), sampled=1)])
        assert e.value.status == CC_EARG
        with pytest.raises(CCError) as e:
            c.step([dict(slot=1, past=0, n=1, ids=[1], sampled=1), dict(slot=1, past=1, n=1, ids=[1], sampled=1)])
        assert e.value.status == CC_EARG
        c.fill_random_kv(0, 256, SEED, 1)            # the whole pool (1 slot = 4 pages)
        with pytest.raises(CCError) as e:
            c.step([dict(slot=1, past=0, n=1, ids=[1], sampled=1)])
        assert e.value.status == CC_BUSY
        c.release(0)
        out = c.step([dict(slot=1, past=0, n=1, ids=[1], sampled=1)])
        assert out[1].shape == (1, 1)
    finally:
        c.close()
    c = Context(d, n_max=128, t_max=16, slots=1, sessions=1)
    try:
        with pytest.raises(CCError) as e:
            c.fill_random_kv(0, 200, SEED, 1)
        assert e.value.status == CC_EARG
    finally:
        c.close()


def test_decode_steps_equal_step_by_step(smol):
    """cc_decode_steps (K greedy passes back to back on the device, each
    pass's rows packed by k_pack and fed the previous pass's token) gives, pass
    for pass, the ids and candidate bits of K cc_step calls fed the same way."""
    d, c, om = smol
    # past every context the module's other tests wrote, so both runs read the same rows
    slots, pasts = [0, 1, 2, 3], [600, 601, 602, 603]
    first = [int(x) for x in _ids(4, d["vocab"], 90)]
    steps = 6
    vals, ids = c.decode_steps(slots, pasts, first, steps, topk=3)
    toks = first
    for k in range(steps):
        v, i = c.step([dict(slot=s, past=p + k, n=1, ids=[toks[j]], sampled=1) for j, (s, p) in
                       enumerate(zip(slots, pasts))], topk=3)
        assert np.array_equal(i, ids[k]), k
        assert np.array_equal(v.view(np.uint32), vals[k].view(np.uint32)), k
        toks = [int(x) for x in i[:, 0]]


def test_decode_steps_take_pages_as_step_by_step(gpu):
    """cc_decode_steps takes each pass's pages job by job as that pass's
    cc_step would (ensurePages in job order, web/model/model.js:185-202), so
    after a loop whose jobs cross page boundaries at different passes the
    device page tables and the free count equal the oracle pool's replay of
    the passes one by one; the tokens equal a cc_step loop's."""
    from chattorrent_amd.ccdecode import Context
    from oracle.model import PagePool
    d = configs.with_layers(configs.SMOLLM2, 2)
    max_pages, frames_n = 8, 5
    pasts = [60, 127, 5, 190]            # cross a page at passes 4, 1, 59 and 2
    steps = 70
    slots = [3, 0, 4, 1]                 # job order differs from slot order
    c = Context(d, n_max=max_pages * 64, t_max=8, slots=4, sessions=frames_n, max_jobs=4)
    pool = PagePool(4 * max_pages)
    frames = [{"pages": np.zeros(max_pages, np.uint32), "owned": [], "max_pages": max_pages}
              for _ in range(frames_n)]
    try:
        c.fill_random(SEED)
        for s, T in zip(slots, pasts):
            c.fill_random_kv(s, T, SEED, s + 1)
            assert pool.ensure(frames[s], T)
        first = [int(x) for x in _ids(4, d["vocab"], 95)]
        _, ids = c.decode_steps(slots, pasts, first, steps, topk=1)
        for k in range(steps):
            for s, T in zip(slots, pasts):
                assert pool.ensure(frames[s], T + k + 1)
        for s in range(frames_n):
            assert list(c.pages(s)) == frames[s]["owned"], s
        assert c.free_pages() == len(pool.free)
        # the same passes one cc_step at a time give the same tokens
        for s in slots:
            c.release(s)
        for s, T in zip(slots, pasts):
            c.fill_random_kv(s, T, SEED, s + 1)
        toks = first
        for k in range(steps):
            _, i = c.step([dict(slot=s, past=T + k, n=1, ids=[toks[j]], sampled=1)
                           for j, (s, T) in enumerate(zip(slots, pasts))], topk=1)
            assert np.array_equal(i[:, 0], ids[k][:, 0]), k
            toks = [int(x) for x in i[:, 0]]
    finally:
        c.close()

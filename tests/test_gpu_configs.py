"""Pass-level parity at the benchmark's own configurations (the shapes and
job mixes BASELINE names), against the oracle on identical seeded inputs:

* one 27B-class block, 12 chats, contexts U[256, 16384], one
  decode row each entering as f16 ~N(0, 1) rows;
* speculative verify, 16 chats x 8 rows (1 real + 7 drafts),
  contexts U[4096, 32768], K/V appended at all 8 positions, acceptance by
  per-row argmax (web/model/stage.js:1483-1561 #finish);
* the 8B shape (untied head, llama3 RoPE scaling) with 512-row
  prefill chunks packed beside decode rows, over two passes;
* configs[4]'s churn, scaled to a small model: arrivals, chunked prompts,
  decode and retirement over many passes, with the device page tables
  checked against the oracle's replay of ensurePages / freePages
  (web/model/model.js:185-211) after every pass.

Bars as in the other pass tests: greedy ids identical (unless the oracle's
top-1/top-2 margin is under 1e-3), logits within 1e-2 abs, the f16 residual
within 2 f16 ulp of its scale, K/V codes within one code (equal for > 99%),
page indices bit-exact."""
import numpy as np
import pytest

from chattorrent_amd import configs
from test_gpu_pass import SEED, _check_head, _ulps_at_scale, _ids
from test_gpu_full import _progress

pytestmark = pytest.mark.gpu


def _make(d, n_max, t_max, slots, sessions=None, contexts=()):
    from chattorrent_amd.ccdecode import Context
    from oracle import model as Mo
    sessions = sessions or slots
    c = Context(d, n_max=n_max, t_max=t_max, slots=slots, sessions=sessions)
    c.fill_random(SEED)
    max_pages = -(-n_max // 64)
    om = Mo.Model(d, n_slots=sessions, max_pages=max_pages, n_pages=slots * max_pages)
    om.gen_weights(SEED)
    for s, T in enumerate(contexts):
        if T:
            c.fill_random_kv(s, T, SEED, s + 1)
            om.fill_random_kv(s, T, SEED, s + 1)
    return c, om


def _check_kv_rows(c, om, d, jobs, layers=(0,)):
    """The K/V rows a pass appended (positions past .. past+n-1 of every job)
    against the oracle's: the f32 K/V inputs come from matmuls on both sides,
    so a code may differ by one where an input sits on a rounding boundary.
    Block 0's input rows are shared bit for bit; a later block's input is the
    f16 residual, which may differ by an f16 step (2^-11 relative), so its
    scales are held to 2e-3 relative there."""
    D, nKV = d["head_dim"], d["n_kv_heads"]
    same = total = 0
    for layer in layers:
        rtol = 1e-5 if layer == 0 else 2e-3
        for which in (0, 1):
            for j in jobs:
                t0, t1 = j["past"], j["past"] + j["n"]
                for h in range(nKV):
                    g = c.read_kv(layer, which, j["slot"], h, t0, t1)
                    w = om.kv_rows(layer, which, j["slot"], t0, t1, h)
                    gc = g[:, :D // 4].view(np.int8).astype(np.int32)
                    wc = w[:, :D // 4].view(np.int8).astype(np.int32)
                    assert np.abs(gc - wc).max() <= 1, (layer, which, j["slot"], h)
                    gs, ws = g[:, D // 4:].view(np.float32), w[:, D // 4:].view(np.float32)
                    assert np.allclose(gs, ws, rtol=rtol, atol=1e-30), (layer, which, j["slot"], h)
                    same += int((gc == wc).sum())
                    total += gc.size
    assert same / total > (0.99 if max(layers) == 0 else 0.97), same / total


def _accepted(ids, drafts):
    """#finish's verify rule (web/model/stage.js:1483-1561): row i's sample
    is accepted while it equals draft i+1; the first mismatch stops."""
    a = 0
    while a < len(drafts) - 1 and ids[a] == drafts[a + 1]:
        a += 1
    return a


def test_config1_block27b_twelve_chats(gpu):
    """one 27B-class block, 12 chats, contexts U[256, 16384],
    entry rows f16 ~N(0, 1), random int8 KV."""
    from oracle import lib as L
    d = configs.BLOCK27B
    rng = np.random.default_rng(SEED)
    ctxs = [int(t) for t in rng.integers(256, 16385, 12)]
    c, om = _make(d, n_max=16384 + 64, t_max=16, slots=13, contexts=ctxs)
    try:
        entry = L.to_f16(rng.standard_normal((12, d["hidden"])).astype(np.float32))
        jobs = [dict(slot=s, past=T, n=1, hidden=entry[s:s + 1]) for s, T in enumerate(ctxs)]
        got = c.step(jobs, at=1, to=2)
        want = om.pass_([dict(j, hidden=L.from_f16(j["hidden"])) for j in jobs], head=False)
        want = L.to_f16(np.concatenate([w["hidden"] for w in want]))
        steps = _ulps_at_scale(got, want, entry)
        assert steps.max() <= 2, steps.max()
        _check_kv_rows(c, om, d, jobs)
    finally:
        c.close()


def test_config3_verify_sixteen_by_eight(gpu):
    """16 chats x 8 verify rows (1 real + 7 drafts, random ids),
    contexts U[4096, 32768], one 27B-class block with the full head; every row
    sampled, K/V appended at all 8 positions, acceptance per chat."""
    d = configs.BLOCK27B
    rng = np.random.default_rng(SEED + 3)
    ctxs = [int(t) for t in rng.integers(4096, 32769, 16)]
    c, om = _make(d, n_max=32768 + 64, t_max=128, slots=17, contexts=ctxs)
    try:
        jobs = [dict(slot=s, past=T, n=8, ids=_ids(8, d["vocab"], 300 + s), sampled=8, topk=1)
                for s, T in enumerate(ctxs)]
        vals, ids = c.step(jobs, topk=1)
        want = om.pass_(jobs)
        margins = _check_head(d, vals, ids, want, ctx=c)
        _check_kv_rows(c, om, d, jobs)
        for k, (j, w) in enumerate(zip(jobs, want)):
            got_ids = ids[8 * k:8 * k + 8, 0]
            if min(margins[8 * k:8 * k + 8]) > 1e-3:
                assert _accepted(got_ids, j["ids"]) == _accepted(w["ids"][:, 0], j["ids"])
    finally:
        c.close()


def test_config4_llama8b_chunks_beside_decode(gpu):
    """configs[4]'s pass shape: the 8B model (untied head, llama3 RoPE
    scaling; two blocks) with a 512-row prefill chunk packed after seven
    decode rows, then the prompt's second chunk beside the decode rows'
    next step (their greedy tokens fed back)."""
    d = configs.with_layers(configs.LLAMA8B, 2)
    rng = np.random.default_rng(SEED + 4)
    ctxs = [int(t) for t in np.exp(rng.uniform(np.log(32), np.log(4096), 7))]
    c, om = _make(d, n_max=4096 + 64, t_max=576, slots=8, contexts=ctxs)
    try:
        prompt = _ids(1024, d["vocab"], 400)
        dec = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 410 + s), sampled=1, topk=4)
               for s, T in enumerate(ctxs)]
        chunk = dict(slot=7, past=0, n=512, ids=prompt[:512], sampled=0, topk=4)
        jobs = dec + [chunk]
        vals, ids = c.step(jobs, topk=4)
        want = om.pass_(jobs)
        _check_head(d, vals, ids, want[:7], ctx=c)
        _check_kv_rows(c, om, d, jobs, layers=(0, 1))
        nxt = [dict(j, past=j["past"] + 1, ids=[int(ids[s, 0])]) for s, j in enumerate(dec)]
        chunk2 = dict(slot=7, past=512, n=512, ids=prompt[512:], sampled=1, topk=4)
        jobs = nxt + [chunk2]
        vals, ids = c.step(jobs, topk=4)
        want = om.pass_(jobs)
        _check_head(d, vals, ids, want, ctx=c)
        _check_kv_rows(c, om, d, jobs, layers=(0, 1))
    finally:
        c.close()


def test_churn_pages_and_tokens_over_passes(gpu):
    """configs[4]'s churn at a small shape: 6 frames over a pool of 4 slots'
    pages, arrivals with prompts log-uniform in [32, 300] fed as 64-token
    chunks beside the decode rows, retirement after 8-40 generated tokens,
    40 passes. After every pass the device page tables equal the oracle's
    replay and the sampled tokens equal the oracle's."""
    d = configs.with_layers(configs.SMOLLM2, 2)
    n_max, frames, slots = 512, 6, 4
    c, om = _make(d, n_max=n_max, t_max=128, slots=slots, sessions=frames)
    rng = np.random.default_rng(SEED + 5)
    chats = {}            # frame -> {"prompt", "fed", "gen", "stop", "last"}
    arrived = retired = 0
    try:
        for step in range(40):
            # arrivals (at most one a pass) and retirements
            free_frames = [f for f in range(frames) if f not in chats]
            if free_frames and rng.random() < 0.6:
                f = free_frames[0]
                n = int(np.exp(rng.uniform(np.log(32), np.log(300))))
                stop = int(rng.integers(8, 41))
                # admitted only while every chat's whole life fits the pool
                if sum(-(-(len(ch["prompt"]) + ch["stop"]) // 64) for ch in chats.values()) \
                        + -(-(n + stop) // 64) <= om.pool.n_pages:
                    chats[f] = dict(prompt=_ids(n, d["vocab"], 500 + 10 * step), fed=0, gen=0, stop=stop,
                                    last=None)
                    arrived += 1
            jobs, chunked = [], False
            for f in sorted(chats):
                ch = chats[f]
                if ch["fed"] < len(ch["prompt"]):
                    if chunked:
                        continue
                    chunked = True
                    n = min(64, len(ch["prompt"]) - ch["fed"])
                    last = ch["fed"] + n == len(ch["prompt"])
                    jobs.append(dict(slot=f, past=ch["fed"], n=n, ids=ch["prompt"][ch["fed"]:ch["fed"] + n],
                                     sampled=1 if last else 0, topk=2))
                else:
                    jobs.append(dict(slot=f, past=ch["fed"], n=1, ids=[ch["last"]], sampled=1, topk=2))
            if not jobs:
                continue
            vals, ids = c.step(jobs, topk=2)
            want = om.pass_(jobs)
            sampled_want = [w for j, w in zip(jobs, want) if j["sampled"]]
            if sampled_want:
                _check_head(d, vals, ids, sampled_want, ctx=c)
            at = 0
            for j in jobs:
                ch = chats[j["slot"]]
                ch["fed"] += j["n"]
                if j["sampled"]:
                    ch["last"] = int(ids[at, 0])
                    ch["gen"] += 1
                    at += 1
            for f in range(frames):
                assert list(c.pages(f)) == om.frames[f]["owned"], (step, f)
            assert c.free_pages() == len(om.pool.free), step
            for f in [f for f, ch in chats.items() if ch["gen"] >= ch["stop"]]:
                c.release(f)
                om.pool.release(om.frames[f])
                del chats[f]
                retired += 1
                assert list(c.pages(f)) == [] and c.free_pages() == len(om.pool.free)
        assert arrived >= 6 and retired >= 3, (arrived, retired)
    finally:
        c.close()


def test_config4_churn_at_scale_pages_every_pass(gpu):
    """configs[4]'s churn at its own scale: the 8B shape (32 layers, untied
    head, llama3 RoPE scaling), 64 chat frames over one shared pool, Poisson(2)
    arrivals a pass, prompts log-uniform in [32, 4096] fed as 512-token chunks
    beside the decode rows, retirement after U[64, 512] tokens, 2000 passes
    (configs[4]'s length)
    (chattorrent_amd.configs.Churn, the bench's c5 workload). After every pass
    each frame's device page table equals the oracle's replay of ensurePages /
    freePages (web/model/model.js:185-211) over the same jobs, page for page,
    and the free count agrees; every sampled id is a vocabulary id."""
    from chattorrent_amd.ccdecode import Context
    from oracle import model as Mo
    d = dict(configs.LLAMA8B)
    slots, chunk, t_max = 64, 512, 64 + 2 * 512
    n_max = 4096 + 512 + 64
    max_pages = -(-n_max // 64)
    c = Context(d, n_max=n_max, t_max=t_max, slots=slots, sessions=slots, max_jobs=slots)
    pool = Mo.PagePool(slots * max_pages)
    frames = [{"pages": np.zeros(max_pages, np.uint32), "owned": [], "max_pages": max_pages} for _ in range(slots)]
    churn = configs.Churn(d["vocab"], slots, chunk, t_max, SEED + 5)
    passes = rows = most = 0
    try:
        c.fill_random(SEED)
        for step in range(2000):
            if step % 250 == 0:
                _progress(f"churn at scale: pass {step}")
            jobs = churn.jobs()
            if not jobs:
                continue
            for j in jobs:
                assert pool.ensure(frames[j["slot"]], j["past"] + j["n"]), step
            _, ids = c.step(jobs, topk=1)
            assert ids.shape[0] == sum(j["sampled"] for j in jobs)
            assert (ids[:, 0] < d["vocab"]).all(), step
            passes += 1
            rows += sum(j["n"] for j in jobs)
            most = max(most, len(jobs))
            for f in churn.advance(jobs, ids[:, 0]):
                c.release(f)
                pool.release(frames[f])
            for f in range(slots):
                assert list(c.pages(f)) == frames[f]["owned"], (step, f)
            assert c.free_pages() == len(pool.free), step
        st = churn.stats
        assert passes >= 1900 and st["arrived"] >= 200 and st["retired"] >= 100 and st["prefill"] > 0, st
        print(f"churn at scale: {passes} passes, {rows} rows, up to {most} jobs a pass, {st}")
    finally:
        c.close()

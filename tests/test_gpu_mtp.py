"""The MTP draft head (web/model/model.js:529-576, web/model/stage.js:296-320
and :1404-1421) on a hybrid model against the oracle's MtpHead on identical
weights: the MTP layer's KV filled from each MTP job's rows, the session's
kept trunk row, and chains of drafts after a sampled token (argmax over the
draft rows, fed back on the device)."""
import numpy as np
import pytest

import hybrid_weights as HW
from oracle import hybrid as Hy
from test_gpu_hybrid import _check, _ids

pytestmark = pytest.mark.gpu
SEED = 17
V_D = 128


def _setup():
    from chattorrent_amd.ccdecode import Context
    d = dict(HW.SPIKE, mtp_vocab=V_D)
    c = Context(d, n_max=512, t_max=64, slots=2)
    om = Hy.HybridModel(d, n_slots=2, max_pages=8)
    om.w = HW.make(d, SEED)
    HW.upload(c, om.w, d)
    wm = HW.make_mtp(d, SEED, V_D)
    HW.upload_mtp(c, wm, d)
    return d, c, om, Hy.MtpHead(om, wm, V_D)


def _same_drafts(got, want):
    """Draft ids equal step by step while the oracle's top-2 margin is clear
    (after a near tie the chains may part)."""
    assert len(got) == len(want)
    for i, (g, (t, logits)) in enumerate(zip(got, want)):
        top = np.sort(logits)[::-1]
        if top[0] - top[1] <= 2e-3 * max(1.0, abs(top[0])):
            return i
        assert int(g) == t, (i, int(g), t)
    return len(got)


def _pass(c, om, mh, jobs):
    vals, ids = c.step(jobs, topk=4)
    out = om.pass_(jobs)
    for j, o in zip(jobs, out):
        if j.get("mtp"):
            mh.fill(j, o["hidden"])
    return vals, ids, out


def test_mtp_fill_and_drafts_match_oracle(gpu):
    d, c, om, mh = _setup()
    rng = np.random.default_rng(31)
    try:
        job = dict(slot=0, past=0, n=12, ids=_ids(rng, 12, V_D), sampled=1, topk=4, mtp=True)
        vals, ids, out = _pass(c, om, mh, [job])
        _check(vals, ids, out, c)
        t = int(np.argmax(out[0]["logits"][0])) % V_D
        got = c.mtp_draft(0, 11, t, 12, 5)
        assert _same_drafts(got, mh.draft(0, out[0]["hidden"][11], t, 12, 5)) >= 3
        # a verify of the token and four drafts refills the MTP rows the chain wrote
        ver = np.array([t] + [int(g) for g in got[:4]], np.int32)
        job = dict(slot=0, past=12, n=5, ids=ver, sampled=5, topk=4, mtp=True)
        vals, ids, out = _pass(c, om, mh, [job])
        _check(vals, ids, out, c)
        # two drafts accepted: the next token comes from row 2, drafts follow it
        t2 = int(np.argmax(out[0]["logits"][2])) % V_D
        got = c.mtp_draft(0, 2, t2, 15, 4)
        assert _same_drafts(got, mh.draft(0, out[0]["hidden"][2], t2, 15, 4)) >= 3
    finally:
        c.close()


def test_mtp_prefill_chunk_keeps_its_last_row(gpu):
    """A prefill chunk (samples nothing) keeps its last trunk row; the next
    chunk's row 0 pairs with it, beside a second session's job."""
    d, c, om, mh = _setup()
    rng = np.random.default_rng(32)
    try:
        jobs = [dict(slot=0, past=0, n=9, ids=_ids(rng, 9, V_D), sampled=0, topk=4, mtp=True),
                dict(slot=1, past=0, n=4, ids=_ids(rng, 4, V_D), sampled=1, topk=4, mtp=True)]
        _pass(c, om, mh, jobs)
        jobs = [dict(slot=0, past=9, n=6, ids=_ids(rng, 6, V_D), sampled=1, topk=4, mtp=True)]
        vals, ids, out = _pass(c, om, mh, jobs)
        _check(vals, ids, out, c)
        t = int(np.argmax(out[0]["logits"][0])) % V_D
        got = c.mtp_draft(0, 5, t, 15, 6)
        assert _same_drafts(got, mh.draft(0, out[0]["hidden"][5], t, 15, 6)) >= 3
        # the other session drafts from its own kept row (-1: keep what it has)
        got = c.mtp_draft(1, -1, 7, 4, 2)
        assert _same_drafts(got, mh.draft(1, None, 7, 4, 2)) >= 1
    finally:
        c.close()


def test_mtp_qwen38_widths_match_oracle(gpu):
    """The MTP head at Qwen3.8-27B's widths (hidden 5120, its full-attention
    block of 24 / 4 heads of 256 with the hybrid extras, the 65536-row draft
    vocabulary of tools/convert_hf.py:225) over four trunk blocks: fill from a
    prefill, a 5-draft chain, a verify of the token and four drafts, and a
    chain from its third row, against the oracle."""
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import Context
    vd = configs.QWEN38["mtp_vocab"]
    d = dict(configs.QWEN38, n_layer=4, layer_types=configs.QWEN38["layer_types"][:4])
    c = Context(d, n_max=512, t_max=64, slots=2)
    om = Hy.HybridModel(d, n_slots=2, max_pages=8)
    om.w = HW.make(d, SEED)
    HW.upload(c, om.w, d)
    wm = HW.make_mtp(d, SEED, vd)
    HW.upload_mtp(c, wm, d)
    mh = Hy.MtpHead(om, wm, vd)
    rng = np.random.default_rng(33)
    try:
        job = dict(slot=0, past=0, n=12, ids=_ids(rng, 12, vd), sampled=1, topk=4, mtp=True)
        vals, ids, out = _pass(c, om, mh, [job])
        _check(vals, ids, out, c)
        t = int(np.argmax(out[0]["logits"][0])) % vd
        got = c.mtp_draft(0, 11, t, 12, 5)
        assert _same_drafts(got, mh.draft(0, out[0]["hidden"][11], t, 12, 5)) >= 3
        ver = np.array([t] + [int(g) for g in got[:4]], np.int32)
        job = dict(slot=0, past=12, n=5, ids=ver, sampled=5, topk=4, mtp=True)
        vals, ids, out = _pass(c, om, mh, [job])
        _check(vals, ids, out, c)
        t2 = int(np.argmax(out[0]["logits"][2])) % vd
        got = c.mtp_draft(0, 2, t2, 15, 4)
        assert _same_drafts(got, mh.draft(0, out[0]["hidden"][2], t2, 15, 4)) >= 3
    finally:
        c.close()

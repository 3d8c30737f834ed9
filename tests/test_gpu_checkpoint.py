"""A checkpoint in the reference's on-disk layout (q8 at the converter's group
64 with f32 scales, tools/convert_hf.py:493, :594-649) read into a cc_ctx by
chattorrent_amd/checkpoint.py, then a decode pass against the oracle holding
the same weights. f32 scales at group 64 (or a multiple) are kept exactly,
one per row and 64-wide unit of the weight records. The same codes written at
group 32 (each scale repeated; f16-exact values, kept as f16 per 32) give
bit-identical logits: both formats feed every 32-wide half-group the same
f32 scale."""
import numpy as np
import pytest

import ckpt_writer as W
from chattorrent_amd import checkpoint as C
from chattorrent_amd import configs
from test_gpu_pass import SEED, _check_head, _ids

pytestmark = pytest.mark.gpu


def _oracle_weights(om, written, d):
    from oracle import model as Mo
    names = {"q_proj": "q", "k_proj": "k", "v_proj": "v", "o_proj": "o", "gate_proj": "gate", "up_proj": "up",
             "down_proj": "down"}

    def g32(t):
        codes, scales, group = t
        K = codes.shape[1]
        return codes, np.repeat(scales, group // 32, axis=1)[:, :-(-K // 32)].astype(np.float32)

    om.w = {"layers": []}
    for i in range(d["n_layer"]):
        blk = written[C.block_file(i)]
        lw = {names[n]: g32(t) for n, t in blk.items() if n in names}
        lw["ln1"] = blk["input_layernorm"]
        lw["ln2"] = blk["post_attention_layernorm"]
        om.w["layers"].append(lw)
    om.w["wte"] = g32(written["client.bin"]["wte"])
    om.w["norm"] = written["client.bin"]["norm"]
    if "lm_head.bin" in written:
        om.w["lm_head"] = g32(written["lm_head.bin"]["lm_head"])
    assert set(om.w["layers"][0]) == set(Mo.TENSORS) | {"ln1", "ln2"}


@pytest.mark.parametrize("tied", [True, False])
def test_checkpoint_pass_matches_oracle(gpu, tmp_path, tied):
    from chattorrent_amd.ccdecode import Context
    from oracle import model as Mo
    d = dict(configs.with_layers(configs.SMOLLM2, 2), tied=tied)
    written = W.make(str(tmp_path / "g64"), d, group=64)
    ctxs = [17, 130, 300]
    c = Context(d, n_max=512, t_max=16, slots=4)
    om = Mo.Model(d, n_slots=4, max_pages=8)
    try:
        C.upload(c, str(tmp_path / "g64"))
        _oracle_weights(om, written, d)
        for s, T in enumerate(ctxs):
            c.fill_random_kv(s, T, SEED, s + 1)
            om.fill_random_kv(s, T, SEED, s + 1)
        jobs = [dict(slot=s, past=T, n=1, ids=_ids(1, d["vocab"], 700 + s), sampled=1, topk=4)
                for s, T in enumerate(ctxs)]
        vals, ids = c.step(jobs, topk=4)
        _check_head(d, vals, ids, om.pass_(jobs), ctx=c)
        logits64 = c.read_logits(len(jobs))
    finally:
        c.close()
    # the same codes at group 32: each group-64 scale written twice
    w32 = {fn: {n: ((t[0], np.repeat(t[1], 2, axis=1)[:, :-(-t[0].shape[1] // 32)], 32) if isinstance(t, tuple) else t)
                for n, t in ts.items()} for fn, ts in written.items()}
    p32 = tmp_path / "g32"
    p32.mkdir()
    m = C.load_manifest(str(tmp_path / "g64"))
    for fn, ts in w32.items():
        order = [e["name"] for e in m["files"][fn]]
        m["files"][fn] = W.pack_file(str(p32), fn, [(n, ts[n]) for n in order])
    import json
    with open(p32 / "manifest.json", "w") as f:
        json.dump(m, f)
    c = Context(d, n_max=512, t_max=16, slots=4)
    try:
        C.upload(c, str(p32))
        for s, T in enumerate(ctxs):
            c.fill_random_kv(s, T, SEED, s + 1)
        c.step(jobs, topk=4)
        assert np.array_equal(c.read_logits(len(jobs)).view(np.uint32), logits64.view(np.uint32))
    finally:
        c.close()


def _rounded(written):
    """The checkpoint's tensors with every q8 scale rounded to f16 (what an
    f16 scale format would keep of the converter's f32 scales)."""
    return {fn: {n: ((t[0], W.f16_exact(t[1]), t[2]) if isinstance(t, tuple) else t) for n, t in ts.items()}
            for fn, ts in written.items()}


@pytest.mark.parametrize("group", [64, 128])
def test_checkpoint_f32_scales_against_oracle_at_f32(gpu, tmp_path, group):
    """A checkpoint whose q8 scales are the converter's f32 values (amax/127,
    not f16 values; tools/convert_hf.py:483-495 writes one per 64 values),
    configs[0]'s model (SmolLM2 shape, all 30 layers, tied head), 4 chats x 8
    greedy passes. The device keeps each f32 scale exactly (one per row and
    64-wide unit of the weight records, the bytes f16 scales per 32 take), as
    the reference does (web/model/kernels.js:116-126), so every pass is held
    to the usual bar against the oracle at the checkpoint's own f32 scales:
    logits within 1e-2, greedy ids equal above a 1e-3 margin. The oracle at
    the scales rounded to f16 runs beside it, to report what keeping f16
    would have moved. Every pass feeds the device's sampled ids to both."""
    from chattorrent_amd.ccdecode import Context
    from oracle import model as Mo
    d = dict(configs.SMOLLM2)
    written = W.make(str(tmp_path), d, group=group, f32_scales=True)
    scales = np.concatenate([t[1].ravel() for ts in written.values() for t in ts.values() if isinstance(t, tuple)])
    moved = float(np.abs(W.f16_exact(scales) / scales - 1).max())
    assert 0 < moved <= 2.0 ** -11, moved
    ctxs = [17, 130, 511, 1024]
    n_max = 1024 + 64
    c = Context(d, n_max=n_max, t_max=8, slots=4)
    om32 = Mo.Model(d, n_slots=4, max_pages=-(-n_max // 64))
    om16 = Mo.Model(d, n_slots=4, max_pages=-(-n_max // 64))
    rec = {"group": group, "passes": 8, "rows": 0, "max_err_vs_f32": 0.0, "max_f32_vs_f16_oracles": 0.0,
           "max_err_vs_f16": 0.0, "scale_max_rel_change_at_f16": moved}
    try:
        C.upload(c, str(tmp_path))
        _oracle_weights(om32, written, d)
        _oracle_weights(om16, _rounded(written), d)
        for s, T in enumerate(ctxs):
            for x in (c, om32, om16):
                x.fill_random_kv(s, T, SEED, s + 1)
        toks = [int(_ids(1, d["vocab"], 720 + s)[0]) for s in range(4)]
        for k in range(rec["passes"]):
            jobs = [dict(slot=s, past=T + k, n=1, ids=[toks[s]], sampled=1, topk=2) for s, T in enumerate(ctxs)]
            vals, ids = c.step(jobs, topk=2)
            got = c.read_logits(len(jobs))
            w16 = np.concatenate([w["logits"] for w in om16.pass_(jobs)])
            w32 = np.concatenate([w["logits"] for w in om32.pass_(jobs)])
            _check_head(d, vals, ids, [{"logits": w32[r:r + 1]} for r in range(len(jobs))], ctx=c)
            rec["rows"] += len(jobs)
            rec["max_err_vs_f32"] = max(rec["max_err_vs_f32"], float(np.abs(got - w32).max()))
            rec["max_f32_vs_f16_oracles"] = max(rec["max_f32_vs_f16_oracles"], float(np.abs(w32 - w16).max()))
            rec["max_err_vs_f16"] = max(rec["max_err_vs_f16"], float(np.abs(got - w16).max()))
            toks = [int(i) for i in ids[:, 0]]
    finally:
        c.close()
    import json
    import warnings
    warnings.warn("checkpoint f32 scales: " + json.dumps(rec))


def test_fused_tensor_scale_formats_do_not_mix(gpu):
    """q, k and v share one record set (the fused q|k|v product), so its parts
    must share one scale format: after q is uploaded with f32 scales at
    group 64, k with f16 scales is refused with CC_EARG and a message; a
    synthetic fill resets every tensor, after which either format loads."""
    from chattorrent_amd import ccdecode as cc
    from chattorrent_amd.ccdecode import CCError, Context
    d = configs.with_layers(configs.SMOLLM2, 1)
    H, D = d["hidden"], d["head_dim"]
    rng = np.random.default_rng(3)
    q_codes = rng.integers(-127, 128, (d["n_heads"] * D, H)).astype(np.int8)
    k_codes = rng.integers(-127, 128, (d["n_kv_heads"] * D, H)).astype(np.int8)
    s64 = rng.uniform(1e-4, 4e-4, (q_codes.shape[0], -(-H // 64))).astype(np.float32)
    s16 = W.f16_exact(rng.uniform(1e-4, 4e-4, (k_codes.shape[0], -(-H // 32)))).astype(np.float16).view(np.uint16)
    c = Context(d, n_max=256, t_max=4, slots=1)
    try:
        c.upload_q8(0, cc.T_Q, q_codes, s64, 64)
        with pytest.raises(CCError) as e:
            c.upload_q8(0, cc.T_K, k_codes, s16, 32)
        assert e.value.status == 5 and "one scale format" in str(e.value)
        c.fill_random(SEED)
        c.upload_q8(0, cc.T_K, k_codes, s16, 32)
        c.upload_q8(0, cc.T_V, k_codes, s16, 32)
    finally:
        c.close()


def test_checkpoint_split_over_two_contexts(gpu, tmp_path):
    """Two peers over one checkpoint (positions [0, 2) and [2, 4) of a
    2-block model): each uploads only its own files' tensors, and the f16
    hand-off between them gives the single context's tokens."""
    from chattorrent_amd.ccdecode import Context
    d = configs.with_layers(configs.SMOLLM2, 2)
    W.make(str(tmp_path), d, group=64)
    jobs = [dict(slot=0, past=0, n=5, ids=_ids(5, d["vocab"], 710), sampled=1, topk=2)]
    whole = Context(d, n_max=256, t_max=8, slots=1)
    a = Context(d, n_max=256, t_max=8, slots=1, lo=0, hi=2)
    b = Context(d, n_max=256, t_max=8, slots=1, lo=2, hi=4)
    try:
        for c in (whole, a, b):
            C.upload(c, str(tmp_path))
        v1, i1 = whole.step(jobs, topk=2)
        rows = a.step([dict(jobs[0], sampled=0)], at=0, to=2)
        v2, i2 = b.step([dict(jobs[0], ids=None, hidden=rows)], at=2, to=4, topk=2)
        assert np.array_equal(i1, i2) and np.array_equal(v1.view(np.uint32), v2.view(np.uint32))
    finally:
        for c in (whole, a, b):
            c.close()


def test_hybrid_checkpoint_equals_direct_upload(gpu, tmp_path):
    """A hybrid checkpoint with an MTP head (Gated DeltaNet blocks, full blocks
    with attn_gate / q_norm / k_norm, mtp.bin) read by checkpoint.py gives the
    same logits and drafts, bit for bit, as the same weights uploaded
    directly (tests/hybrid_weights.py), which the oracle tests pin."""
    import hybrid_weights as HW
    from chattorrent_amd.ccdecode import Context
    d = dict(HW.D256, mtp_vocab=64)
    w = HW.make(d, 3)
    wm = HW.make_mtp(d, 3, 64)
    W.make_hybrid(str(tmp_path), d, w, wm)
    m = C.load_manifest(str(tmp_path))
    dd = C.dims_from_manifest(m)
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, 64, 11).astype(np.int32)
    got = []
    for how in ("direct", "checkpoint"):
        c = Context(d if how == "direct" else dd, n_max=512, t_max=16, slots=1)
        try:
            if how == "direct":
                HW.upload(c, w, d)
                HW.upload_mtp(c, wm, d)
            else:
                C.upload(c, str(tmp_path))
            vals, ids = c.step([dict(slot=0, past=0, n=11, ids=prompt, sampled=1, mtp=True)], topk=2)
            drafts = c.mtp_draft(0, 10, int(ids[0, 0]) % 64, 11, 4)
            got.append((c.read_logits(1).copy(), drafts))
        finally:
            c.close()
    assert np.array_equal(got[0][0].view(np.uint32), got[1][0].view(np.uint32))
    assert np.array_equal(got[0][1], got[1][1])

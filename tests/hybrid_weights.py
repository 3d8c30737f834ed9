"""Random weights for a small hybrid (Qwen3.5-architecture) model, uploaded to
a Context through cc_upload and handed to the oracle's HybridModel, so both
start from identical values: q8 codes with f16-exact scales at group 32, and
f32 norms, conv weights and gate parameters."""
import numpy as np

# The reference's spike shape (oracle/qwen3.8-27b-spike/spike_config.json):
# three linear_attention blocks, then a full_attention block with q_norm,
# k_norm, the output gate and partial rotary.
SPIKE = dict(hidden=384, n_layer=4, n_heads=6, n_kv_heads=1, head_dim=64, ffn=512, vocab=256, rms_eps=1e-6,
             rope_theta=1e7, rot_dim=16, tied=False, hybrid=True,
             layer_types=["linear_attention"] * 3 + ["full_attention"],
             lin_nk=4, lin_nv=12, lin_dk=16, lin_dv=16, lin_conv=4)

# Qwen3.8-27B's Gated DeltaNet head widths (Dk = Dv = 128, value heads a
# multiple of key heads) at a small width, with full-attention heads of 128.
WIDE = dict(hidden=1024, n_layer=4, n_heads=8, n_kv_heads=2, head_dim=128, ffn=1536, vocab=512, rms_eps=1e-6,
            rope_theta=1e7, rot_dim=32, tied=True, hybrid=True,
            layer_types=["linear_attention", "full_attention", "linear_attention", "linear_attention"],
            lin_nk=2, lin_nv=6, lin_dk=128, lin_dv=128, lin_conv=4)

# Qwen3.8-27B's full-attention heads (head_dim 256, a quarter of it rotary,
# four query heads per kv head) and its Gated DeltaNet widths, small hidden
D256 = dict(hidden=512, n_layer=4, n_heads=4, n_kv_heads=1, head_dim=256, ffn=1024, vocab=384, rms_eps=1e-6,
            rope_theta=1e7, rot_dim=64, tied=False, hybrid=True,
            layer_types=["linear_attention"] * 3 + ["full_attention"],
            lin_nk=2, lin_nv=4, lin_dk=128, lin_dv=128, lin_conv=4)


def q8(rng, N, K, out_std=1.0):
    """int8 codes in ±127 and per-32 scales (exact in f16) sized so that a
    unit-RMS input row gives outputs of about `out_std`."""
    codes = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    s = out_std / (73.3 * np.sqrt(K))
    scales = (s * (0.75 + 0.5 * rng.random((N, -(-K // 32))))).astype(np.float16).astype(np.float32)
    return codes, scales


def make(d, seed):
    """The oracle's weight dict for `d` (HybridModel.w)."""
    rng = np.random.default_rng(seed)
    H, F, D = d["hidden"], d["ffn"], d["head_dim"]
    qd, kvd = d["n_heads"] * D, d["n_kv_heads"] * D
    kd, vd, nV = d["lin_nk"] * d["lin_dk"], d["lin_nv"] * d["lin_dv"], d["lin_nv"]
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)   # noqa: E731
    w = {"layers": []}
    for kind in d["layer_types"]:
        lw = {"ln1": norm(H), "ln2": norm(H), "gate": q8(rng, F, H), "up": q8(rng, F, H), "down": q8(rng, H, F)}
        if kind == "linear_attention":
            lw.update(kind="linear", in_q=q8(rng, kd, H), in_k=q8(rng, kd, H), in_v=q8(rng, vd, H),
                      in_z=q8(rng, vd, H), in_b=q8(rng, nV, H), in_a=q8(rng, nV, H), out=q8(rng, H, vd),
                      conv=(0.4 * rng.standard_normal((2 * kd + vd, d["lin_conv"]))).astype(np.float32),
                      gate_params=np.concatenate([0.5 * rng.standard_normal(nV) - 1.0,
                                                  0.5 * rng.standard_normal(nV)]).astype(np.float32),
                      gated_norm=norm(d["lin_dv"]))
        else:
            lw.update(kind="full", q=q8(rng, qd, H), k=q8(rng, kvd, H), v=q8(rng, kvd, H),
                      attn_gate=q8(rng, qd, H), o=q8(rng, H, qd), q_norm=norm(D), k_norm=norm(D))
        w["layers"].append(lw)
    # embedding rows of unit RMS when untied; a tied table is also the head,
    # so its rows are kept at the head's scale (logits of order one)
    w["wte"] = q8(rng, d["vocab"], H, out_std=1.0 if d.get("tied", True) else np.sqrt(H))
    w["norm"] = norm(H)
    if not d.get("tied", True):
        w["lm_head"] = q8(rng, d["vocab"], H)
    return w


def upload(ctx, w, d, lo=0, hi=None):
    """cc_upload of every tensor the context holds (positions [lo, hi))."""
    from chattorrent_amd import ccdecode as cc
    n = d["n_layer"]
    hi = n + 2 if hi is None else hi
    kd = d["lin_nk"] * d["lin_dk"]
    if lo == 0 or (hi == n + 2 and d.get("tied", True)):
        ctx.upload_q8(-1, cc.T_WTE, *w["wte"])
    if hi == n + 2:
        ctx.upload_norm(-1, cc.T_NORM, w["norm"])
        if not d.get("tied", True):
            ctx.upload_q8(-1, cc.T_LM_HEAD, *w["lm_head"])
    for i in range(max(lo, 1) - 1, min(hi, n + 1) - 1):
        lw = w["layers"][i]
        ctx.upload_norm(i, cc.T_LN1, lw["ln1"])
        ctx.upload_norm(i, cc.T_LN2, lw["ln2"])
        for t, name in ((cc.T_GATE, "gate"), (cc.T_UP, "up"), (cc.T_DOWN, "down")):
            ctx.upload_q8(i, t, *lw[name])
        if lw["kind"] == "linear":
            for t, name in ((cc.T_IN_Q, "in_q"), (cc.T_IN_K, "in_k"), (cc.T_IN_V, "in_v"), (cc.T_IN_Z, "in_z"),
                            (cc.T_IN_B, "in_b"), (cc.T_IN_A, "in_a"), (cc.T_OUT_PROJ, "out")):
                ctx.upload_q8(i, t, *lw[name])
            ctx.upload_norm(i, cc.T_CONV_Q, lw["conv"][:kd])
            ctx.upload_norm(i, cc.T_CONV_K, lw["conv"][kd:2 * kd])
            ctx.upload_norm(i, cc.T_CONV_V, lw["conv"][2 * kd:])
            ctx.upload_norm(i, cc.T_GATE_PARAMS, lw["gate_params"])
            ctx.upload_norm(i, cc.T_GATED_NORM, lw["gated_norm"])
        else:
            for t, name in ((cc.T_Q, "q"), (cc.T_K, "k"), (cc.T_V, "v"), (cc.T_O, "o"),
                            (cc.T_ATTN_GATE, "attn_gate")):
                ctx.upload_q8(i, t, *lw[name])
            ctx.upload_norm(i, cc.T_Q_NORM, lw["q_norm"])
            ctx.upload_norm(i, cc.T_K_NORM, lw["k_norm"])


def make_mtp(d, seed, draft_vocab):
    """The MTP head's weights (loader.js:633-634): the norms, fc_e / fc_h,
    the draft embedding and head over the first `draft_vocab` rows, and one
    full-attention block (with the hybrid extras on a hybrid model)."""
    rng = np.random.default_rng(seed + 1000)
    H, F, D = d["hidden"], d["ffn"], d["head_dim"]
    qd, kvd = d["n_heads"] * D, d["n_kv_heads"] * D
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)   # noqa: E731
    blk = {"kind": "full", "ln1": norm(H), "ln2": norm(H), "gate": q8(rng, F, H), "up": q8(rng, F, H),
           "down": q8(rng, H, F), "q": q8(rng, qd, H), "k": q8(rng, kvd, H), "v": q8(rng, kvd, H), "o": q8(rng, H, qd)}
    if d.get("hybrid"):
        blk.update(attn_gate=q8(rng, qd, H), q_norm=norm(D), k_norm=norm(D))
    return {"enorm": norm(H), "hnorm": norm(H), "mtp_norm": norm(H), "fc_e": q8(rng, H, H), "fc_h": q8(rng, H, H),
            "embed_draft": q8(rng, draft_vocab, H, out_std=np.sqrt(H)), "head_draft": q8(rng, draft_vocab, H),
            "block": blk}


def upload_mtp(ctx, wm, d):
    from chattorrent_amd import ccdecode as cc
    for t, name in ((cc.T_MTP_ENORM, "enorm"), (cc.T_MTP_HNORM, "hnorm"), (cc.T_MTP_NORM, "mtp_norm")):
        ctx.upload_norm(-1, t, wm[name])
    for t, name in ((cc.T_MTP_FC_E, "fc_e"), (cc.T_MTP_FC_H, "fc_h"), (cc.T_MTP_EMBED, "embed_draft"),
                    (cc.T_MTP_HEAD, "head_draft")):
        ctx.upload_q8(-1, t, *wm[name])
    b, L = wm["block"], cc.LAYER_MTP
    ctx.upload_norm(L, cc.T_LN1, b["ln1"])
    ctx.upload_norm(L, cc.T_LN2, b["ln2"])
    for t, name in ((cc.T_Q, "q"), (cc.T_K, "k"), (cc.T_V, "v"), (cc.T_O, "o"), (cc.T_GATE, "gate"),
                    (cc.T_UP, "up"), (cc.T_DOWN, "down")):
        ctx.upload_q8(L, t, *b[name])
    if d.get("hybrid"):
        ctx.upload_q8(L, cc.T_ATTN_GATE, *b["attn_gate"])
        ctx.upload_norm(L, cc.T_Q_NORM, b["q_norm"])
        ctx.upload_norm(L, cc.T_K_NORM, b["k_norm"])

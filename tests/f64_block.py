"""One full-attention block in float64 (test infrastructure, no GPU): the
oracle's block (oracle.model.Model.block, after web/model/model.js:368-409
fullBlockSegs and :307-316 ffnBlock: rmsnorm -> q, k, v -> RoPE -> attention
over the session's paged int8 cache -> o_proj -> residual -> rmsnorm -> SwiGLU
-> down -> residual) with every stored input taken as the oracle holds it:
the q8 codes and scales, the norm weights, the RoPE table's f32 values, and
the K/V cache rows, including the rows the job itself appended (their int8
codes are a discrete function of f32 inputs, so the f64 block reads the
oracle's). Rounded once to f16, its output is the block's exact result for
those inputs, against which the oracle's f32 arithmetic and the GPU's are
each measured in f16 steps."""
import numpy as np


def _deq(codes, scales, group=32):
    K = codes.shape[1]
    return codes.astype(np.float64) * np.repeat(np.asarray(scales, np.float64), group, axis=1)[:, :K]


def _rmsnorm(x, w, eps):
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * np.asarray(w, np.float64)


def _rope(x, past, tbl, rot):
    """Split-half RoPE on x [n, heads, D] (f64) at positions past.. from the
    oracle's table ([position][pair] interleaved cos, sin)."""
    half = rot // 2
    n = x.shape[0]
    t = np.asarray(tbl, np.float64).reshape(-1, half, 2)[past + np.arange(n)]
    c, s = t[..., 0][:, None, :], t[..., 1][:, None, :]
    a, b = x[..., :half].copy(), x[..., half:rot].copy()
    x[..., :half] = a * c - b * s
    x[..., half:rot] = b * c + a * s
    return x


def _kv64(words, D):
    codes = np.ascontiguousarray(words[:, :D // 4]).view(np.int8).astype(np.float64)
    sc = np.ascontiguousarray(words[:, D // 4:]).view(np.float32).astype(np.float64)
    return codes * np.repeat(sc, 32 if D >= 32 else D, axis=1)[:, :D]


def block_f64(om, layer, x, segs):
    """The block's residual output rows (before the f16 round) for input
    rows x [T, H] (f64): `om` holds the layer's weights and K/V (for a
    StreamedModel, after _load(layer)); segs: (slot, past, n, row) per job,
    rows packed in job order."""
    d = om.d
    lw = om.w["layers"][layer]
    D, nH, nKV = d["head_dim"], d["n_heads"], d["n_kv_heads"]
    group = nH // nKV
    g = om.group
    x = np.asarray(x, np.float64)
    y = _rmsnorm(x, lw["ln1"], d["rms_eps"])
    q = y @ _deq(*lw["q"], g).T
    ctx = np.zeros_like(q)
    for slot, past, n, row in segs:
        qh = _rope(q[row:row + n].reshape(n, nH, D).copy(), past, om.tbl, om.rot)
        T = past + n
        keep = np.arange(T)[None, :] <= (past + np.arange(n))[:, None]
        for hk in range(nKV):
            Kd = _kv64(om.kv_rows(layer, 0, slot, 0, T, hk), D)
            Vd = _kv64(om.kv_rows(layer, 1, slot, 0, T, hk), D)
            for h in range(hk * group, (hk + 1) * group):
                s = (qh[:, h, :] @ Kd.T) / np.sqrt(D)
                s = np.where(keep, s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                ctx[row:row + n, h * D:(h + 1) * D] = p @ Vd
    x1 = x + ctx @ _deq(*lw["o"], g).T
    y2 = _rmsnorm(x1, lw["ln2"], d["rms_eps"])
    gt = y2 @ _deq(*lw["gate"], g).T
    up = y2 @ _deq(*lw["up"], g).T
    act = gt / (1.0 + np.exp(-gt)) * up
    return x1 + act @ _deq(*lw["down"], g).T


def f16_bits(x64):
    """Round-to-nearest-even of f64 values to f16 bits, in one rounding."""
    return np.asarray(x64, np.float64).astype(np.float16).view(np.uint16)


def steps_from_exact(got_bits, exact_bits):
    """|got - exact| in f16 steps of the exact value (the step of the f16
    binade holding it; the subnormal step below 2^-14)."""
    g = np.asarray(got_bits, np.uint16).view(np.float16).astype(np.float64)
    e = np.asarray(exact_bits, np.uint16).view(np.float16).astype(np.float64)
    step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(e), 2.0 ** -14))) - 10)
    return np.abs(g - e) / step


def summary(steps):
    s = np.asarray(steps).ravel()
    return {"max": float(s.max()), "within_0": float((s == 0).mean()), "within_1": float((s <= 1).mean()),
            "within_2": float((s <= 2).mean()), "beyond_2": int((s > 2).sum()), "elements": int(s.size)}

"""The oracle, pinned before it is trusted (CPU only).

Each oracle function is checked against what fixes it independently of its
own formula: the reference's golden vectors (tests/golden/, copied from the
reference's oracle/ dumps), the reference tests' known-answer cases and
closed forms (web/dev/kernels.test.js:334-449, tools/f16.test.mjs:14-57,
tools/sampling.test.mjs:135-197), f64 brute force on small inputs, and
invariants (row independence, paging, batch invariance)."""
import json
import os

import numpy as np
import pytest

from oracle import lib as L
from oracle import model as Mo

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------- f16 ---
def test_every_half_round_trips():
    """tools/f16.test.mjs:14-25: every finite half survives half -> f32 -> half."""
    h = np.arange(65536, dtype=np.uint16)
    finite = ((h >> 10) & 0x1F) != 0x1F
    back = L.to_f16(L.from_f16(h))
    assert np.array_equal(back[finite], h[finite])
    v = L.from_f16(np.array([1, 0x7BFF], np.uint16))
    assert v[0] == 2.0 ** -24 and v[1] == 65504.0


def test_half_ties_to_even_and_clamps():
    """tools/f16.test.mjs:27-57: ties go to the even mantissa (both signs,
    across the subnormal boundary); past the range clamps to ±65504; NaN stays
    NaN; -0 keeps its sign; below half the smallest subnormal is zero."""
    for sign in (0, 0x8000):
        i = np.arange(0x7BFF, dtype=np.uint32)
        a = L.from_f16((sign | i).astype(np.uint16)).astype(np.float64)
        b = L.from_f16((sign | (i + 1)).astype(np.uint16)).astype(np.float64)
        mid = ((a + b) / 2).astype(np.float32)
        keep = (mid != a.astype(np.float32)) & (mid != b.astype(np.float32))
        want = (sign | np.where(i % 2 == 1, i + 1, i)).astype(np.uint16)
        assert np.array_equal(L.to_f16(mid[keep]), want[keep])
    big = L.from_f16(L.to_f16(np.array([1e6, -1e6, np.inf, -np.inf, 65520], np.float32)))
    assert list(big) == [65504, -65504, 65504, -65504, 65504]
    assert np.isnan(L.from_f16(L.to_f16(np.array([np.nan], np.float32))))[0]
    z = L.from_f16(L.to_f16(np.array([-0.0], np.float32)))
    assert z[0] == 0 and np.signbit(z[0])
    assert L.from_f16(L.to_f16(np.array([2.0 ** -26], np.float32)))[0] == 0


def test_round_f16_equals_f16js_rounding():
    """web/model/kernels.js:1356-1383 round_f16 must give web/f16.js's values
    bit for bit (web/dev/kernels.test.js:840-865): every tie between
    neighbouring halves, subnormals, clamps, wide-range noise."""
    halves = L.from_f16(np.arange(0x7C00, dtype=np.uint16)).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(23)
    noise = ((rng.random(50000) - 0.5) * 2.0 ** (rng.random(50000) * 40 - 25)).astype(np.float32)
    special = np.array([0, -0.0, np.inf, -np.inf, 65504, 65519, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25,
                        3 * 2 ** -25, 2 ** -14, 2 ** -15, 1, -1, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)
    x = np.concatenate([special, mids, -mids, noise])
    got = L.round_f16(x)
    want = L.from_f16(L.to_f16(x))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    n = np.array([np.nan], np.float32)
    assert np.isnan(L.round_f16(n)[0])


# ------------------------------------------------------------------ RoPE ---
def _params():
    with open(os.path.join(GOLD, "rope_params.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["smollm2", "llama31"])
def test_rope_matches_reference_goldens(name):
    """The reference's oracle dumps (tools/dump_*_oracle.py: f64 split-half
    RoPE of HF's q/k, llama3-scaled for Llama 3.1) at positions 0..4. The
    oracle's f32 table + f32 rotation (kernels.js:1093-1129, :2016-2045) agrees
    to f32 rounding."""
    p = _params()[name]
    D = p["head_dim"]
    for which, heads in (("q", p["n_heads"]), ("k", p["n_kv_heads"])):
        x = np.load(os.path.join(GOLD, f"{name}_{which}.npy"), allow_pickle=False)
        want = np.load(os.path.join(GOLD, f"{name}_{which}_rope.npy"), allow_pickle=False)
        T = x.shape[0]
        tbl = L.rope_table(p["rot"], p["theta"], T + 1, p.get("scaling"))
        h = np.ascontiguousarray(x.reshape(T, heads, D).transpose(1, 0, 2))
        L.rope(h, p["rot"], 0, tbl)
        assert np.abs(h - want).max() <= 4e-7 * np.abs(want).max()
        if p.get("scaling"):
            # the scaling matters: without it the same check fails
            plain = np.ascontiguousarray(x.reshape(T, heads, D).transpose(1, 0, 2))
            L.rope(plain, p["rot"], 0, L.rope_table(p["rot"], p["theta"], T + 1, None))
            assert np.abs(plain - want).max() > 1e-3


def test_rope_table_matches_qwen_spike_cos_sin():
    """oracle/qwen3.8-27b-spike/rope_cos.npy, rope_sin.npy (theta 1e7, rot 16),
    HF's [pos, rot] layout with the half duplicated."""
    p = _params()["qwen_spike"]
    c = np.load(os.path.join(GOLD, "qwen_spike_rope_cos.npy"), allow_pickle=False)
    s = np.load(os.path.join(GOLD, "qwen_spike_rope_sin.npy"), allow_pickle=False)
    half = p["rot"] // 2
    tbl = L.rope_table(p["rot"], p["theta"], c.shape[0]).reshape(c.shape[0], half, 2)
    for lo in (0, half):
        assert np.abs(tbl[:, :, 0] - c[:, lo:lo + half]).max() <= 1.2e-7
        assert np.abs(tbl[:, :, 1] - s[:, lo:lo + half]).max() <= 1.2e-7


def test_rope_closed_forms():
    """web/dev/kernels.test.js:376-407: a rotation keeps pair magnitudes, is the
    identity at position 0, and split-half differs from interleaved."""
    rng = np.random.default_rng(99)
    nH, T, D = 2, 3, 8
    q = (rng.random((nH, T, D)) * 2 - 1).astype(np.float32)
    tbl = L.rope_table(D, 1e5, 16)
    r = L.rope(q.copy(), D, 4, tbl)
    half = D // 2
    m0 = np.hypot(q[..., :half], q[..., half:])
    m1 = np.hypot(r[..., :half], r[..., half:])
    assert np.abs(m0 - m1).max() < 1e-6
    z = L.rope(q.copy(), D, 0, tbl)
    assert np.array_equal(z[:, 0], q[:, 0])
    inter = q.copy()
    for h in range(nH):
        for t in range(T):
            for i in range(half):
                k = ((4 + t) * half + i) * 2
                cs, sn = tbl[k], tbl[k + 1]
                a, b = q[h, t, 2 * i], q[h, t, 2 * i + 1]
                inter[h, t, 2 * i], inter[h, t, 2 * i + 1] = a * cs - b * sn, b * cs + a * sn
    assert np.abs(inter - r).max() > 1e-3


# ---------------------------------------------------------------- matmul ---
def test_matmul_hand_computed():
    """web/dev/kernels.test.js:344-351: the [out, in] weight convention, here
    with q8 codes and unit scales."""
    X = np.array([[1, 2, 3, 4, 0, 0, 0, 0], [5, 6, 7, 8, 0, 0, 0, 0]], np.float32)
    W = np.zeros((4, 8), np.int8)
    W[0, 0] = 1
    W[1, 1] = 1
    W[2, :4] = 1
    W[3, 0], W[3, 3] = 2, 1
    S = np.ones((4, 1), np.float32)
    Y = L.matmul_q8(X, W, S, group=32)
    assert np.array_equal(Y, np.array([[1, 2, 10, 6], [5, 6, 26, 18]], np.float32))


@pytest.mark.parametrize("M,K,N,g", [(1, 64, 5, 32), (3, 100, 7, 32), (4, 256 + 32, 9, 64), (2, 36, 3, 32)])
def test_matmul_vs_f64_brute_force(M, K, N, g):
    """f64 brute force on small shapes with partial last groups: the GEMV
    order is a valid f32 summation of exactly these terms."""
    rng = np.random.default_rng(M * K * N)
    X = (rng.random((M, K)) * 2 - 1).astype(np.float32)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    ng = -(-K // g)
    S = (rng.random((N, ng)) * 2 - 1).astype(np.float32)
    Y = L.matmul_q8(X, W, S, group=g)
    Sf = np.repeat(S, g, axis=1)[:, :K].astype(np.float64)
    exact = X.astype(np.float64) @ (W.astype(np.float64) * Sf).T
    bound = np.abs(X).astype(np.float64) @ (np.abs(W.astype(np.float64)) * np.abs(Sf)).T
    assert np.all(np.abs(Y - exact) <= K * 2.0 ** -23 * bound + 1e-30)
    # every row is a function of that row alone (the batch-invariance contract)
    for i in range(M):
        assert np.array_equal(L.matmul_q8(X[i:i + 1], W, S, group=g), Y[i:i + 1])


def test_gather_embed_is_exact_product():
    """gather_embed_nopos_q8: out[t, h] = q * S[v, h/32], one rounding."""
    rng = np.random.default_rng(2)
    wte = rng.integers(-127, 128, (13, 70 * 4)).astype(np.int8)
    S = (rng.random((13, 9)) * 2 - 1).astype(np.float32)
    ids = np.array([7, 0, 12], np.int32)
    out = L.gather_embed_q8(ids, wte, S)
    want = (wte[ids].astype(np.float64) * np.repeat(S[ids], 32, axis=1)[:, :280]).astype(np.float32)
    assert np.array_equal(out, want)


# --------------------------------------------------------------- rmsnorm ---
def test_rmsnorm_unit_mean_square():
    """web/dev/kernels.test.js:361-374."""
    rng = np.random.default_rng(99)
    x = (rng.random((2, 40)) * 2 - 1).astype(np.float32)
    y = L.rmsnorm(x, np.ones(40, np.float32), 1e-5)
    assert np.abs((y.astype(np.float64) ** 2).mean(axis=1) - 1).max() < 1e-4


# ------------------------------------------------------------- store_kv ---
def _dequant(words, D, RW):
    codes = words[:, :D // 4].copy().view(np.int8).astype(np.float64)
    sc = words[:, D // 4:].copy().view(np.float32).astype(np.float64)
    return codes * np.repeat(sc, 32 if D >= 32 else D, axis=1)[:, :D], sc


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("rot", [0, "D"])
def test_store_kv_invariants(D, rot):
    """web/dev/kernels.test.js:733-799: every value within half a step of its
    block's scale; scale = max|x|/127; a zero block gives scale 0 and codes 0;
    rows outside the job untouched."""
    rot = D if rot == "D" else 0
    nKV, T_new, T_past, N_max = 3, 3, 2, 11
    RW = Mo.kv_row_words(D)
    rng = np.random.default_rng(5)
    src = (rng.random((T_new, nKV * D)) * 2 - 1).astype(np.float32)
    src[0, :D] = 0
    cache = np.full(nKV * N_max * RW, 0xDEADBEEF, np.uint32)
    tbl = L.rope_table(D, 1e5, 32)
    L.store_kv(src, cache, T_past, N_max, nKV, D, rot, np.zeros(1, np.uint32), tbl if rot else None)
    dense = src.reshape(T_new, nKV, D).transpose(1, 0, 2).copy()
    want = L.rope(dense, rot, T_past, tbl) if rot else dense
    c = cache.reshape(nKV, N_max, RW)
    for n in range(nKV):
        rows = c[n, T_past:T_past + T_new]
        deq, sc = _dequant(rows, D, RW)
        for t in range(T_new):
            for b in range(D // 32):
                blk = want[n, t, 32 * b:32 * b + 32].astype(np.float64)
                amax = np.abs(blk).max()
                s = sc[t, b]
                assert abs(s - np.float32(amax) / np.float32(127)) <= 1e-7 * max(amax, 1e-30)
                err = np.abs(deq[t, 32 * b:32 * b + 32] - blk)
                assert np.all(err <= (0.5 + 1e-3) * (amax / 127) + 0.0) if amax else np.all(err == 0)
        untouched = np.concatenate([c[n, :T_past], c[n, T_past + T_new:]])
        assert np.all(untouched == 0xDEADBEEF)
    assert c[0, T_past, D // 4] == 0 and not c[0, T_past, :D // 4].any()


def test_store_kv_row_independent_and_paged():
    """web/dev/kernels.test.js:801-834: one T=5 job writes the bits of five T=1
    jobs, and a paged cache holds the rows of a contiguous one."""
    D, nKV, T, page, N = 64, 3, 5, 4, 8
    RW = Mo.kv_row_words(D)
    rng = np.random.default_rng(5)
    src = (rng.random((T, nKV * D)) * 2 - 1).astype(np.float32)
    tbl = L.rope_table(16, 1e5, 16)
    whole = np.zeros(nKV * N * RW, np.uint32)
    steps = np.zeros(nKV * N * RW, np.uint32)
    L.store_kv(src, whole, 1, N, nKV, D, 16, np.zeros(1, np.uint32), tbl)
    for t in range(T):
        L.store_kv(src[t:t + 1], steps, 1 + t, N, nKV, D, 16, np.zeros(1, np.uint32), tbl)
    assert np.array_equal(whole, steps)
    table = np.array([1, 0], np.uint32)
    paged = np.zeros(2 * nKV * page * RW, np.uint32)
    L.store_kv(src, paged, 1, page, nKV, D, 16, table, tbl)
    for n in range(nKV):
        for t in range(1, 1 + T):
            at = ((table[t // page] * nKV + n) * page + t % page) * RW
            assert np.array_equal(paged[at:at + RW], whole[(n * N + t) * RW:(n * N + t + 1) * RW])


# ------------------------------------------------------------- attention ---
def test_softmax_rows_sum_to_one_and_mask():
    """web/dev/kernels.test.js:409-428."""
    rng = np.random.default_rng(99)
    s = (rng.random((2, 3, 5)) * 2 - 1).astype(np.float32)
    p = L.causal_softmax(s, 2)
    assert np.abs(p.sum(-1) - 1).max() < 1e-6
    for i in range(3):
        assert np.all(p[:, i, 2 + i + 1:] == 0)


def _softmax64(s, T_past, exp=np.exp, shift=0):
    """Masked softmax in f64: row i sees keys 0..T_past+i (+ shift)."""
    s = np.asarray(s, np.float64)
    _, T_new, T_act = s.shape
    keep = np.arange(T_act)[None, :] <= (T_past + shift + np.arange(T_new))[:, None]
    m = np.where(keep, s, -np.inf).max(-1, keepdims=True)
    e = np.where(keep, exp(s - m), 0.0)
    return e / e.sum(-1, keepdims=True)


def test_softmax_values_vs_f64():
    """causal_softmax (kernels.js:1180-1253) against an f64 softmax with the
    same mask, over scores spread wide enough that exp's base matters. The
    same bar rejects an exp2 in place of exp and a causal limit one off."""
    rng = np.random.default_rng(123)
    T_past, T_new = 9, 4
    s = (rng.random((3, T_new, T_past + T_new)) * 16 - 8).astype(np.float32)
    p = L.causal_softmax(s, T_past)
    want = _softmax64(s, T_past)
    tol = 2e-6
    assert np.abs(p - want).max() < tol
    assert np.all(p[want == 0] == 0)
    # planted mistakes in the f64 statement: each must exceed the bar
    assert np.abs(p - _softmax64(s, T_past, exp=np.exp2)).max() > 100 * tol
    assert np.abs(p - _softmax64(s, T_past, shift=1)).max() > 100 * tol
    assert np.abs(p - _softmax64(s, T_past, shift=-1)).max() > 100 * tol


def _attend64(Qr, Kd, Vd, past, group, kv_of=None, shift=0):
    """f64 attention of Qr [nH, n, D] over dequantised rows Kd/Vd [nKV, T, D]:
    scores / sqrt(D), causal (row i sees 0..past+i), softmax, P.V."""
    nH, n, D = Qr.shape
    kv_of = kv_of or (lambda h: h // group)
    out = np.empty((nH, n, D))
    for h in range(nH):
        k, v = Kd[kv_of(h)], Vd[kv_of(h)]
        s = (Qr[h].astype(np.float64) @ k.T) / np.sqrt(D)
        out[h] = _softmax64(s[None], past, shift=shift)[0] @ v
    return out


def test_model_attend_vs_f64_paged_ragged_verify():
    """Model.attend (model.js:321-351: store K/V into the paged int8 cache,
    RoPE on Q, qk, exact causal softmax, P.V) for a verify job of 5 rows that
    crosses a page boundary through a non-monotone page table, against f64
    attention over the dequantised rows read back from the pool. The same bar
    rejects a wrong GQA head mapping and a causal limit one off."""
    d = dict(hidden=64, n_layer=1, n_heads=6, n_kv_heads=2, head_dim=64, ffn=64, vocab=64,
             rms_eps=1e-5, rope_theta=1e4, tied=True, group_q8=32)
    nH, nKV, D = 6, 2, 64
    group = nH // nKV
    om = Mo.Model(d, n_slots=3, max_pages=4)
    om.fill_random_kv(0, 64, 5, 1)
    om.fill_random_kv(1, 62, 5, 2)
    om.fill_random_kv(2, 64, 5, 3)
    past, n = 62, 5
    assert om.pool.ensure(om.frames[1], past + n)
    assert list(om.frames[1]["pages"][:2]) == [1, 3]          # non-monotone
    rng = np.random.default_rng(8)
    q = (rng.standard_normal((n, nH * D))).astype(np.float32)
    k = (rng.standard_normal((n, nKV * D))).astype(np.float32)
    v = (rng.standard_normal((n, nKV * D))).astype(np.float32)
    got = om.attend(0, 1, q, k, v, past).reshape(n, nH, D).transpose(1, 0, 2)
    Qr = L.rope(np.ascontiguousarray(q.reshape(n, nH, D).transpose(1, 0, 2)), D, past, om.tbl)
    RW = om.rw
    Kd = np.stack([_dequant(om.kv_rows(0, 0, 1, 0, past + n, h), D, RW)[0] for h in range(nKV)])
    Vd = np.stack([_dequant(om.kv_rows(0, 1, 1, 0, past + n, h), D, RW)[0] for h in range(nKV)])
    want = _attend64(Qr, Kd, Vd, past, group)
    scale = np.abs(want).max()
    tol = 2e-6 * scale
    assert np.abs(got - want).max() < tol
    assert np.abs(got - _attend64(Qr, Kd, Vd, past, group, kv_of=lambda h: h % nKV)).max() > 100 * tol
    assert np.abs(got - _attend64(Qr, Kd, Vd, past, group, shift=1)).max() > 100 * tol
    assert np.abs(got - _attend64(Qr, Kd, Vd, past, group, shift=-1)).max() > 100 * tol
    # the new rows are the job's own K (after RoPE) and V, quantised
    Kn = L.rope(np.ascontiguousarray(k.reshape(n, nKV, D).transpose(1, 0, 2)), D, past, om.tbl)
    assert np.abs(Kd[:, past:] - Kn).max() <= 0.5 * np.abs(Kn).max(-1, keepdims=True).max() / 127 + 1e-6
    assert np.abs(Vd[:, past:] - v.reshape(n, nKV, D).transpose(1, 0, 2)).max() <= np.abs(v).max() / 254 + 1e-6


def _contiguous_cache(vals, D, page_words=None):
    """Rows [n_kv][N_max][D] -> quantised words via the oracle's store (V)."""
    nKV, N, _ = vals.shape
    RW = Mo.kv_row_words(D)
    cache = np.zeros(nKV * N * RW, np.uint32)
    src = vals.transpose(1, 0, 2).reshape(N, nKV * D)
    L.store_kv(src, cache, 0, N, nKV, D, 0, np.zeros(1, np.uint32), None)
    deq = np.stack([_dequant(cache.reshape(nKV, N, RW)[n], D, RW)[0] for n in range(nKV)])
    return cache, deq


def test_attn_av_one_hot_selects_row():
    """web/dev/kernels.test.js:430-446: one-hot scores return that (dequantised)
    V row exactly — checks the GQA mapping and the cache stride."""
    D, nH, group, N = 32, 6, 3, 9
    nKV = nH // group
    rng = np.random.default_rng(1)
    cache, deq = _contiguous_cache((rng.random((nKV, N, D)) * 2 - 1).astype(np.float32), D)
    scores = np.zeros((nH, 1, 4), np.float32)
    scores[:, 0, 2] = 1
    out = L.attn_av(scores, cache, D, N, group, np.zeros(1, np.uint32))
    for h in range(nH):
        assert np.array_equal(out[h, 0], deq[h // group, 2].astype(np.float32))


def test_qk_scores_vs_f64():
    D, nH, group, N, T_new, T_act = 64, 6, 3, 12, 3, 10
    nKV = nH // group
    rng = np.random.default_rng(7)
    cache, deq = _contiguous_cache((rng.random((nKV, N, D)) * 2 - 1).astype(np.float32), D)
    Q = (rng.random((nH, T_new, D)) * 2 - 1).astype(np.float32)
    s = L.qk_scores(Q, cache, T_new, T_act, N, D, nH, group, np.zeros(1, np.uint32))
    want = np.einsum("htd,hsd->hts", Q.astype(np.float64),
                     np.repeat(deq, group, axis=0)[:, :T_act]) / np.sqrt(D)
    assert np.abs(s - want).max() < 1e-5


def test_silu_mul_vs_f64():
    rng = np.random.default_rng(3)
    g = (rng.random(1000) * 20 - 10).astype(np.float32)
    u = (rng.random(1000) * 2 - 1).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.abs(L.silu_mul(g, u) - want).max() < 1e-5


# ------------------------------------------------------------------ top-k ---
def test_topk_equals_sort_with_ties():
    """web/dev/kernels.test.js:1115-1149 and tools/sampling.test.mjs: larger
    value first, ties to the lower index; M = 1 is greedy's first max."""
    rng = np.random.default_rng(11)
    for V, M in [(1000, 1), (1000, 17), (5000, 256)]:
        row = rng.standard_normal(V).astype(np.float32)
        row[5::37] = row[3]
        vals, ids = L.topk(row, M)
        order = np.lexsort((np.arange(V), -row))[:M]
        assert np.array_equal(ids, order.astype(np.uint32))
        assert np.array_equal(vals, row[order])
        assert ids[0] == int(np.argmax(row))


# -------------------------------------------------------------- page pool ---
def test_page_pool_semantics():
    """web/model/model.js:132-211 (tools/stage.test.mjs:626-674): the lowest
    index pops first, pages follow logical order, release pushes them back so
    the frame's first page is the next to pop."""
    pool = Mo.PagePool(6, 4)
    a = {"pages": np.zeros(4, np.uint32), "owned": [], "max_pages": 4}
    b = {"pages": np.zeros(4, np.uint32), "owned": [], "max_pages": 4}
    assert pool.ensure(a, 9) and a["owned"] == [0, 1, 2]
    assert pool.ensure(b, 4) and b["owned"] == [3]
    assert not pool.ensure(b, 17)            # more than max_pages
    assert pool.release(a) == 3 and pool.free[-1] == 0
    assert pool.ensure(b, 12) and b["owned"] == [3, 0, 1]
    assert not pool.ensure(a, 16) or len(a["owned"]) == 4


# -------------------------------------------------------------- generators ---
def test_generator_prefix_is_stable():
    """The synthetic inputs are this build's own definition, shared with the
    device generator: pin their first values so neither side drifts."""
    codes, sc = L.gen_q8(7, 17, 2, 64, 32)
    assert codes.dtype == np.int8 and np.abs(codes.astype(int)).max() <= 127
    assert list(codes[0, :8]) == list(L.gen_q8(7, 17, 1, 64, 32)[0][0, :8])
    big, bsc = L.gen_q8(1, 16, 512, 512, 32)
    assert abs(big.astype(np.float64).std() - 40) < 1.0 and abs(big.astype(np.float64).mean()) < 0.5
    v = L.from_f16(bsc)
    assert v.min() >= 9.9e-5 and v.max() <= 4.01e-4
    kc, ks = L.gen_kv(3, 0x4B560000, 5, 0, 64, 2, 64)
    assert np.abs(kc.astype(int)).max() <= 127 and ks.min() >= 0.0049 and ks.max() <= 0.0201
    h = L.gen_normal_f16(1, 2, 20000)
    x = L.from_f16(h).astype(np.float64)
    assert abs(x.std() - 1) < 0.02 and abs(x.mean()) < 0.03


# ---------------------------------------------------------- oracle model ---
def test_oracle_batched_pass_equals_alone():
    """web/dev/batch.test.js:163-228 on the oracle itself: a batched pass gives
    each session the bits it gets alone; a swapped cache gives different bits
    (the control)."""
    d = dict(hidden=64, n_layer=2, n_heads=4, n_kv_heads=2, head_dim=16 * 4, ffn=96, vocab=300,
             rms_eps=1e-5, rope_theta=1e4, tied=True)
    d["n_heads"], d["head_dim"] = 1, 64
    d["n_kv_heads"] = 1
    m = Mo.Model(d, n_slots=3, max_pages=4)
    m.gen_weights(3)
    m.fill_random_kv(0, 40, 3, 1)
    m.fill_random_kv(1, 70, 3, 2)
    jobs = [dict(slot=0, past=40, n=1, ids=[5], sampled=1, topk=3),
            dict(slot=1, past=70, n=3, ids=[1, 2, 3], sampled=3, topk=3)]
    both = m.pass_(jobs)
    for j, r in zip(jobs, both):
        alone = m.pass_([j])[0]
        assert np.array_equal(alone["logits"].view(np.uint32), r["logits"].view(np.uint32))
    swapped = m.pass_([dict(jobs[0], slot=1, past=40)])[0]
    assert not np.array_equal(swapped["logits"], both[0]["logits"])


# ------------------------------------------------- block composition pins ---
def _gold(name, part):
    return np.load(os.path.join(GOLD, f"{name}_{part}.npy"), allow_pickle=False)


def _norm_fit(norm_out, unit):
    """How far `norm_out` is from `unit` (an rmsnorm output with unit
    weights) times one weight per channel: the weight is fitted by least
    squares over the tokens (the dumps carry no weights), and the worst
    residual is returned relative to max |norm_out|. The right input fits to
    f32 rounding; any other tensor leaves a residual of order one."""
    u = unit.astype(np.float64)
    y = norm_out.astype(np.float64)
    w = (y * u).sum(axis=0) / np.maximum((u * u).sum(axis=0), 1e-300)
    return float(np.abs(y - u * w).max() / np.abs(y).max())


def _composition_errors(name, compose):
    """Runs `compose` (compose_block's signature) on the reference's block-0
    embedding rows with the dumped attention and MLP outputs in place of the
    sublayers and unit norm weights, and measures, against the dumps:
    ln1 - what the attention sublayer was given, up to a per-channel weight;
    ln2 - what the MLP was given, up to a per-channel weight (this pins its
          input as the residual after attention);
    out - the block's output before the f16 round (block_00_out)."""
    eps = _params()[name]["rms_eps"]
    emb = _gold(name, "embeddings")
    seen = {}

    def attention(h):
        seen["h1"] = np.array(h)
        return _gold(name, "attn_out")

    def mlp(h):
        seen["h2"] = np.array(h)
        return _gold(name, "mlp_out")

    ones = np.ones(emb.shape[1], np.float32)
    x = np.ascontiguousarray(emb.copy())
    out = compose(x, ones, ones, eps, attention, mlp)
    want = _gold(name, "block_out")
    return {
        "ln1": _norm_fit(_gold(name, "ln1"), seen["h1"]),
        "ln2": _norm_fit(_gold(name, "ln2"), seen["h2"]),
        "out": float(np.abs(out.astype(np.float64) - want).max() / np.abs(want).max()),
    }


@pytest.mark.parametrize("name", ["smollm2", "llama31"])
def test_block_composition_matches_reference_dumps(name):
    """oracle/model.py compose_block (model.js:368-409, :307-316) against the
    reference's own HF dumps of block 0 (oracle/<model>/block00_*.npy,
    block_00_out.npy): rmsnorm of the block input feeds attention, the
    attention output is added to the residual, rmsnorm of that residual feeds
    the MLP, and the MLP output is added to it. The dumps agree with these
    relations to f32 rounding; the f16 round after the block (pinned by the
    f16 tests above) is the reference's own addition, absent from HF."""
    # the dumps themselves: the residual adds hold as sums of the dumped parts
    emb, att, mid = _gold(name, "embeddings"), _gold(name, "attn_out"), _gold(name, "after_attn_resid")
    assert np.abs(mid.astype(np.float64) - emb - att).max() <= 1e-7 * np.abs(mid).max()
    err = _composition_errors(name, Mo.compose_block)
    assert err["ln1"] <= 2e-7 and err["ln2"] <= 2e-7 and err["out"] <= 2e-7, err


def test_block_composition_check_catches_misplaced_parts():
    """The check above has teeth: compositions with a plausible mistake
    planted (the MLP's norm reading the block input, a dropped attention
    residual, the MLP output added to the block input, the MLP norm's input
    taken after the MLP residual) each fail it by orders of magnitude."""
    def ln2_from_input(x, ln1, ln2, eps, attention, mlp):
        x0 = x.copy()
        L.add_inplace(x, attention(L.rmsnorm(x, ln1, eps)))
        L.add_inplace(x, mlp(L.rmsnorm(x0, ln2, eps)))
        return x

    def no_attn_residual(x, ln1, ln2, eps, attention, mlp):
        x[:] = attention(L.rmsnorm(x, ln1, eps))
        L.add_inplace(x, mlp(L.rmsnorm(x, ln2, eps)))
        return x

    def mlp_on_entry(x, ln1, ln2, eps, attention, mlp):
        a = attention(L.rmsnorm(x, ln1, eps))
        h = L.rmsnorm(x + a, ln2, eps)
        L.add_inplace(x, mlp(h))
        return x

    def attn_norm_of_nothing(x, ln1, ln2, eps, attention, mlp):
        L.add_inplace(x, attention(L.rmsnorm(x * x, ln1, eps)))
        L.add_inplace(x, mlp(L.rmsnorm(x, ln2, eps)))
        return x

    for name in ("smollm2", "llama31"):
        for wrong in (ln2_from_input, no_attn_residual, mlp_on_entry, attn_norm_of_nothing):
            err = _composition_errors(name, wrong)
            assert max(err.values()) > 1e-3, (name, wrong.__name__, err)


def test_streamed_model_equals_model_over_passes():
    """Model.StreamedModel (weights and random KV regenerated per block, only
    the appended K/V rows kept) gives Model's bits: two consecutive passes,
    the second over the rows the first appended, logits and ids equal bitwise;
    and the paged KV fill writes the same words as Model.fill_random_kv."""
    d = dict(hidden=128, n_layer=3, n_heads=4, n_kv_heads=2, head_dim=32, ffn=192, vocab=500,
             rms_eps=1e-5, rope_theta=1e4, tied=True)
    ctxs = [(40, 1), (0, 2), (130, 3)]
    extra = 8
    sm = Mo.StreamedModel(d, 5, ctxs, extra)
    m = Mo.Model(d, n_slots=3, max_pages=sm.max_pages, n_pages=sm.pool.n_pages)
    m.gen_weights(5)
    for s, (T, key) in enumerate(ctxs):
        m.pool.ensure(m.frames[s], T + extra)
        if T:
            m.fill_random_kv(s, T, 5, key)
    assert all(np.array_equal(a["pages"], b["pages"]) for a, b in zip(m.frames, sm.frames))
    # the paged fill against the row-by-row copy: layer 2's whole K and V pools
    sm._load(2)
    for which in (0, 1):
        assert np.array_equal(sm._kv[which], (m.K, m.V)[which][2])
    jobs = [dict(slot=0, past=40, n=1, ids=[7], sampled=1, topk=3),
            dict(slot=1, past=0, n=5, ids=[1, 2, 3, 4, 5], sampled=1, topk=3),
            dict(slot=2, past=130, n=2, ids=[9, 8], sampled=2, topk=3)]
    for _ in range(2):
        a, b = m.pass_(jobs), sm.pass_(jobs)
        for ra, rb in zip(a, b):
            assert np.array_equal(ra["logits"].view(np.uint32), rb["logits"].view(np.uint32))
            assert np.array_equal(ra["ids"], rb["ids"])
        jobs = [dict(j, past=j["past"] + j["n"], n=1, ids=[int(r["ids"][-1][0])], sampled=1) for j, r in zip(jobs, a)]


def test_oracle_multi_row_job_equals_sequential_one_row_jobs():
    """The full-depth parity test checks k greedy steps with one oracle pass of
    k rows per chat fed the same ids: the oracle's rows are computed one by
    one (each row's matmuls, its own causal attention limit, its own K/V
    rows), so row i of a k-row job gives the bits of the i-th of k one-row
    passes."""
    d = dict(hidden=128, n_layer=2, n_heads=4, n_kv_heads=2, head_dim=32, ffn=192, vocab=500,
             rms_eps=1e-5, rope_theta=1e4, tied=True)
    a = Mo.Model(d, n_slots=2, max_pages=4)
    b = Mo.Model(d, n_slots=2, max_pages=4)
    for m in (a, b):
        m.gen_weights(9)
        m.fill_random_kv(0, 70, 9, 1)
        m.fill_random_kv(1, 20, 9, 2)
    ids = [[3, 17, 250], [8, 9, 10]]
    seq = []
    for i in range(3):
        seq.append(a.pass_([dict(slot=s, past=p + i, n=1, ids=[ids[s][i]], sampled=1, topk=2)
                            for s, p in ((0, 70), (1, 20))]))
    multi = b.pass_([dict(slot=s, past=p, n=3, ids=ids[s], sampled=3, topk=2) for s, p in ((0, 70), (1, 20))])
    for s in range(2):
        for i in range(3):
            assert np.array_equal(multi[s]["logits"][i].view(np.uint32), seq[i][s]["logits"][0].view(np.uint32))

"""Kernel-level parity: each HIP kernel against the oracle's restatement of the
reference kernel, on the same seeded inputs (web/dev/kernels.test.js is the
model: awkward dims, bitwise row invariance, closed-form checks).

Bars: bit-exact for round_f16, the KV quantiser's codes and scales, top-k ids
and values; tolerance for float reductions (stated per test)."""
import numpy as np
import pytest

from chattorrent_amd import configs

pytestmark = pytest.mark.gpu


def _ctx(gpu, d=None, n_max=1024, t_max=64, slots=4):
    from chattorrent_amd.ccdecode import Context
    return Context(d or configs.with_layers(configs.SMOLLM2, 2), n_max=n_max, t_max=t_max, slots=slots)


@pytest.fixture(scope="module")
def ctx(gpu):
    c = _ctx(gpu)
    yield c
    c.close()


def test_round_f16_bit_exact(ctx):
    """web/model/kernels.js:1356-1383 against web/f16.js semantics (the oracle
    restates both): every tie between neighbouring halves, subnormals, clamps."""
    from oracle import lib as L
    halves = L.from_f16(np.arange(0x7c00, dtype=np.uint16))
    mids = ((halves[:-1].astype(np.float64) + halves[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(23)
    noise = ((rng.random(50000) - 0.5) * 2.0 ** (rng.random(50000) * 40 - 25)).astype(np.float32)
    special = np.array([0, -0.0, np.inf, -np.inf, 65504, 65519, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25,
                        3 * 2 ** -25, 2 ** -14, 2 ** -15, 1, -1, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)
    x = np.concatenate([special, mids, -mids, noise])
    got = ctx.op_round_f16(x)
    want = L.round_f16(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the result equals fromF16(toF16(x)) (web/f16.js), NaN aside
    assert np.array_equal(got, L.from_f16(L.to_f16(x)))


@pytest.mark.parametrize("M,K,N", [(1, 576, 70), (5, 1000, 77), (12, 5120, 256), (17, 576, 1024),
                                   (32, 1536, 96), (33, 576, 64), (64, 320, 48), (100, 5120, 512),
                                   (130, 1536, 2048)])
def test_matmul_q8_vs_oracle(ctx, M, K, N):
    """matmul_gemv_q8 family (web/model/kernels.js:449-751): within a bound of
    2^-20 of the sum of |terms| (the MFMA path sums in a different order; the
    f16 hi/lo activation split keeps ~22 significant bits)."""
    from oracle import lib as L
    rng = np.random.default_rng(M * 1000 + K + N)
    X = (rng.random((M, K), np.float32) * 2 - 1).astype(np.float32)
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    S16 = L.to_f16((rng.random((N, (K + 31) // 32)) * 2 - 1).astype(np.float32))
    S = L.from_f16(S16)
    got = ctx.op_matmul_q8(X, W, S16)
    want = L.matmul_q8(X, W, S)
    Sfull = np.repeat(S, 32, axis=1)[:, :K]
    bound = np.abs(X).astype(np.float64) @ (np.abs(W.astype(np.float64)) * np.abs(Sfull)).T
    exact = X.astype(np.float64) @ (W.astype(np.float64) * Sfull).T
    assert np.all(np.abs(got - exact) <= 2.0 ** -20 * bound + 1e-30)
    assert np.all(np.abs(got - want) <= 2.0 ** -19 * bound + 1e-30)


def test_matmul_rows_match_one_row_bitwise(ctx):
    """A row's bits do not depend on its batch-mates (web/dev/kernels.test.js:
    578-650; docs/model.md 'Matching plain decoding row by row')."""
    from oracle import lib as L
    rng = np.random.default_rng(31)
    K, N = 6 * 32 + 32, 70
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    S16 = L.to_f16((rng.random((N, K // 32)) * 2 - 1).astype(np.float32))
    for M in [2, 3, 8, 15, 16, 17, 31, 32, 33, 48]:
        X = (rng.random((M, K), np.float32) * 2 - 1).astype(np.float32)
        rows = ctx.op_matmul_q8(X, W, S16)
        for i in range(M):
            one = ctx.op_matmul_q8(X[i:i + 1], W, S16)
            assert np.array_equal(one.view(np.uint32), rows[i:i + 1].view(np.uint32)), (M, i)


def test_matmul_many_rows_bitwise(ctx):
    """Above 32 rows the weights are reused across 64-row blocks (a different
    kernel), and every row still has the bits of the one-row call: the same
    K planes and the same partial-sum segments (at K 5120 a pair's 20 units
    are cut at varying points between the 32-row kernel's waves)."""
    from oracle import lib as L
    rng = np.random.default_rng(37)
    K, N = 5120, 3072
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    S16 = L.to_f16((rng.random((N, K // 32)) * 2 - 1).astype(np.float32))
    for M in [33, 70, 129]:
        X = (rng.random((M, K), np.float32) * 2 - 1).astype(np.float32)
        rows = ctx.op_matmul_q8(X, W, S16)
        for i in sorted({0, 1, M // 2, M - 2, M - 1}):
            one = ctx.op_matmul_q8(X[i:i + 1], W, S16)
            assert np.array_equal(one.view(np.uint32), rows[i:i + 1].view(np.uint32)), (M, i)
        few = ctx.op_matmul_q8(X[:32], W, S16)
        assert np.array_equal(few.view(np.uint32), rows[:32].view(np.uint32)), M


def test_matmul_many_rows_twelve_waves_bitwise(ctx):
    """The many-row matmul runs twelve waves a workgroup (folded segments in
    LDS) where that takes fewer rounds of workgroups over the CUs, else
    eight (folds in registers). At N 8240, K 5120 on 256 CUs that is twelve
    at 70 and 200 rows and eight at 129. Either way every row keeps the bits
    of the one-row call, so each call equals the first rows of the larger
    one. N 8240 ends in a partial pair group and a partial tile."""
    from oracle import lib as L
    rng = np.random.default_rng(43)
    K, N = 5120, 8240
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    S16 = L.to_f16((rng.random((N, K // 32)) * 2 - 1).astype(np.float32))
    X = (rng.random((200, K), np.float32) * 2 - 1).astype(np.float32)
    got = {M: ctx.op_matmul_q8(X[:M], W, S16) for M in (70, 129, 200)}
    for M, rows in got.items():
        for i in sorted({0, 1, M // 2, M - 2, M - 1}):
            one = ctx.op_matmul_q8(X[i:i + 1], W, S16)
            assert np.array_equal(one.view(np.uint32), rows[i:i + 1].view(np.uint32)), (M, i)
    assert np.array_equal(got[70].view(np.uint32), got[129][:70].view(np.uint32))
    assert np.array_equal(got[129].view(np.uint32), got[200][:129].view(np.uint32))


@pytest.mark.parametrize("K,N", [(2560, 8192), (5120, 8192), (4160, 8240), (2112, 4144)])
def test_matmul_summed_planes_bitwise(ctx, K, N):
    """With rows enough to fill the GPU without the K split (2048 rows: 32
    blocks of 64 rows times N/256 pair groups is two workgroups a CU or more),
    the many-row matmul adds its K planes itself and writes one: the rows keep
    the bits of the one-row, 32-row and 200-row calls, which write the planes
    separately. K 2560: 2 planes of 20 units; K 5120: 4, with the 32-row
    kernel's cut points inside them; K 4160: planes of 16, 16, 16 and 17
    units; K 2112: 16 and 17. N 8240 and 4144 end in a partial pair group and
    a partial tile."""
    from oracle import lib as L
    rng = np.random.default_rng(41 + K)
    M = 2048
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    S16 = L.to_f16((rng.random((N, K // 32)) * 2 - 1).astype(np.float32))
    X = (rng.random((M, K), np.float32) * 2 - 1).astype(np.float32)
    rows = ctx.op_matmul_q8(X, W, S16)
    for i in (0, 1, 777, M - 1):
        one = ctx.op_matmul_q8(X[i:i + 1], W, S16)
        assert np.array_equal(one.view(np.uint32), rows[i:i + 1].view(np.uint32)), i
    for a, n in ((0, 32), (1000, 200)):
        part = ctx.op_matmul_q8(X[a:a + n], W, S16)
        assert np.array_equal(part.view(np.uint32), rows[a:a + n].view(np.uint32)), (a, n)


@pytest.mark.parametrize("V,M", [(1000, 1), (1000, 5), (49152, 40), (151936, 1), (151936, 256)])
def test_topk_exact(ctx, V, M):
    """topk_stage/topkRows (web/model/kernels.js:1453-1507, :2129-2144): best M
    pairs, larger value first, ties to the lower index — exact."""
    from oracle import lib as L
    rng = np.random.default_rng(V + M)
    rows = 3
    logits = rng.standard_normal((rows, V)).astype(np.float32)
    logits[:, 7::97] = logits[0, 3]          # planted ties
    logits[1, 11] = logits[1].max() + 1      # a clear winner
    vals, ids = ctx.op_topk(logits, M)
    for r in range(rows):
        wv, wi = L.topk(logits[r], M)
        assert np.array_equal(ids[r], wi)
        assert np.array_equal(vals[r].view(np.uint32), wv.view(np.uint32))


def test_rmsnorm_vs_oracle(ctx):
    """rmsnorm (web/model/kernels.js:930-976). The GPU sums squares four
    columns a thread, across each 64-lane wave (butterfly) and then over the
    waves in order, instead of 256 strided lanes, so the scale differs by a few
    f32 ulp: within 1e-6 relative. Rows up to the 8192-column limit."""
    from oracle import lib as L
    rng = np.random.default_rng(4)
    for T, H in [(3, 576), (5, 5120), (2, 70 * 8), (2, 8192)]:
        x = rng.standard_normal((T, H)).astype(np.float32)
        w = (rng.random(H) + 0.5).astype(np.float32)
        got = ctx.op_rmsnorm(x, w)
        want = L.rmsnorm(x, w, ctx.d["rms_eps"])
        assert np.allclose(got, want, rtol=1e-6, atol=0)


def _oracle_cache(d, n_pages, page=64):
    from oracle import model as Mo
    rw = Mo.kv_row_words(d["head_dim"])
    return np.zeros(n_pages * d["n_kv_heads"] * page * rw, np.uint32)


# head_dim 256 (Qwen3.8-27B's full-attention heads) on a plain model shape
D256 = dict(hidden=1024, n_layer=1, n_heads=4, n_kv_heads=1, head_dim=256, ffn=1024, vocab=512, rms_eps=1e-6,
            rope_theta=1e7, tied=True)


@pytest.mark.parametrize("dims", ["smol", "27b", "d256"])
def test_store_kv_bit_exact(gpu, dims):
    """store_kv (web/model/kernels.js:1024-1073): RoPE'd K and plain V quantised
    per 32 values — codes and scales bit-exact with the oracle given the same
    input, including a zero block (scale 0, codes 0) and rows that cross a
    page boundary; rows outside the job are untouched."""
    from oracle import lib as L
    from oracle import model as Mo
    d = D256 if dims == "d256" else configs.with_layers(configs.SMOLLM2 if dims == "smol" else configs.M27B, 1)
    c = _ctx(gpu, d, n_max=512, t_max=16, slots=2)
    try:
        D, nKV = d["head_dim"], d["n_kv_heads"]
        rng = np.random.default_rng(5)
        T_past, T_new = 60, 9                 # crosses the first page boundary
        for which in (0, 1):
            src = rng.standard_normal((T_new, nKV * D)).astype(np.float32)
            src[0, :D] = 0.0                  # head 0 of row 0 all zero: zero blocks after RoPE too
            c.op_store_kv(0, which, 1, src, T_past)
            pages = c.pages(1)
            cache = _oracle_cache(d, 16)
            tbl = L.rope_table(D, d["rope_theta"], 1024)
            L.store_kv(src, cache, T_past, 64, nKV, D, D if which == 0 else 0, pages, tbl if which == 0 else None)
            rw = Mo.kv_row_words(D)
            for h in range(nKV):
                got = c.read_kv(0, which, 1, h, T_past, T_past + T_new)
                t = np.arange(T_past, T_past + T_new)
                rows = ((pages[t // 64].astype(np.int64) * nKV + h) * 64 + t % 64) * rw
                want = cache[rows[:, None] + np.arange(rw)[None, :]]
                assert np.array_equal(got, want), (which, h)
            z = c.read_kv(0, which, 1, 0, T_past, T_past + 1)
            assert z[0, D // 4] == 0 and not z[0, :8].any()
    finally:
        c.close()


def test_attend_vs_oracle(gpu):
    """qk_scores_gqa + causal_softmax + attn_av_gqa (web/model/kernels.js:
    1140-1310) over random int8 pages: decode rows, a causal verify run, and a
    ragged last page. The GPU softmax is online (max, sum merged per page and
    chunk); equal to the exact three-pass one within 2e-5 of max |out|. The
    causal mask runs only on pages past the first new position, so the cases
    put that position at a page's last token (63), at a page's first (64,
    128) and one before a page boundary with rows across it (127)."""
    from oracle import lib as L
    from oracle import model as Mo
    for base, tokens, n in [(configs.SMOLLM2, 130, 1), (configs.M27B, 700, 1), (configs.M27B, 300, 8),
                            (configs.SMOLLM2, 64, 37), (D256, 200, 1), (D256, 520, 6),
                            (configs.M27B, 63, 1), (configs.M27B, 128, 1), (configs.SMOLLM2, 127, 3)]:
        d = configs.with_layers(base, 1)
        c = _ctx(gpu, d, n_max=1024, t_max=64, slots=2)
        try:
            om = Mo.Model(d, n_slots=2, max_pages=16)
            c.fill_random_kv(1, tokens + n, 11, 3)
            om.fill_random_kv(1, tokens + n, 11, 3)
            D, nH = d["head_dim"], d["n_heads"]
            rng = np.random.default_rng(tokens + n)
            q = rng.standard_normal((n, nH * D)).astype(np.float32)
            got = c.op_attend(0, 1, q, tokens)
            # oracle: RoPE on Q, scores, exact softmax, P.V over the same rows
            pages = om.frames[1]["pages"]
            Qh = np.ascontiguousarray(q.reshape(n, nH, D).transpose(1, 0, 2))
            L.rope(Qh, D, tokens, om.tbl)
            group = nH // d["n_kv_heads"]
            s = L.qk_scores(Qh, om.K[0], n, tokens + n, 64, D, nH, group, pages)
            p = L.causal_softmax(s, tokens)
            ctxh = L.attn_av(p, om.V[0], D, 64, group, pages)
            want = ctxh.transpose(1, 0, 2).reshape(n, nH * D)
            err = np.abs(got - want).max()
            assert err <= 2e-5 * max(1.0, np.abs(want).max()), (base["hidden"], tokens, n, err)
        finally:
            c.close()


@pytest.mark.parametrize("shape", ["27b", "d256"])
def test_attend_verify_rows_equal_one_row_bitwise(gpu, shape):
    """A verify job's rows (several Q m-tiles: the workgroup's four waves share
    each page's dequantised fragments) give the bits of the same rows attended
    one at a time (one m-tile: each wave dequantises for itself), across a
    page and chunk boundary (positions 505..512)."""
    base = configs.M27B if shape == "27b" else D256
    d = configs.with_layers(base, 1)
    c = _ctx(gpu, d, n_max=1024, t_max=64, slots=2)
    try:
        P, n = 505, 8
        c.fill_random_kv(1, P + n, 5, 9)
        D, nH = d["head_dim"], d["n_heads"]
        q = np.random.default_rng(P).standard_normal((n, nH * D)).astype(np.float32)
        many = c.op_attend(0, 1, q, P)
        for i in range(n):
            one = c.op_attend(0, 1, q[i:i + 1], P + i)
            assert np.array_equal(one.view(np.uint32), many[i:i + 1].view(np.uint32)), (shape, i)
    finally:
        c.close()


@pytest.mark.parametrize("shape", ["27b", "d256"])
def test_attend_block_with_empty_slot_equals_full_block(gpu, shape):
    """A verify job of 8 rows (three m-tiles at a GQA group of 5, two at 4)
    leaves its block's last slot empty, and that idle wave loads and
    dequantises every page alone; in a job of four m-tiles each wave loads a
    quarter. The first 8 rows of a four-m-tile job give the bits of the 8-row
    job at the same position (rows past them only add masked tokens), across
    a page and chunk boundary (positions 505..)."""
    base = configs.M27B if shape == "27b" else D256
    d = configs.with_layers(base, 1)
    c = _ctx(gpu, d, n_max=1024, t_max=64, slots=2)
    try:
        D, nH, nKV = d["head_dim"], d["n_heads"], d["n_kv_heads"]
        group = nH // nKV
        full_n, part_n = 64 // group, 8
        assert -(-full_n * group // 16) == 4 and -(-part_n * group // 16) < 4, (full_n, group)
        P = 505
        c.fill_random_kv(1, P + full_n, 5, 9)
        q = np.random.default_rng(P + 1).standard_normal((full_n, nH * D)).astype(np.float32)
        full = c.op_attend(0, 1, q, P)
        part = c.op_attend(0, 1, q[:part_n], P)
        assert np.array_equal(full[:part_n].view(np.uint32), part.view(np.uint32)), shape
    finally:
        c.close()


def test_attend_ignores_stale_rows_past_the_context(gpu):
    """The pool rows past a job's tokens hold whatever an earlier session left
    there, NaN and inf included (web/model/kernels.js:1140-1310 never reads
    them: its loops stop at the context length). Poisoning every K and V
    row after the attended tokens, codes and scales, leaves the output
    bitwise unchanged: decode rows and a causal verify run whose last page
    is partly filled."""
    for base, tokens, n in [(configs.M27B, 700, 1), (configs.M27B, 300, 8), (D256, 520, 6)]:
        d = configs.with_layers(base, 1)
        c = _ctx(gpu, d, n_max=1024, t_max=64, slots=2)
        try:
            end = (tokens + n + 63) // 64 * 64 + 40          # rows into the next page too
            c.fill_random_kv(1, end, 11, 3)
            D, nH, nKV = d["head_dim"], d["n_heads"], d["n_kv_heads"]
            q = np.random.default_rng(tokens + n).standard_normal((n, nH * D)).astype(np.float32)
            clean = c.op_attend(0, 1, q, tokens)
            bad = np.empty((end - tokens - n, D // 4 + D // 32), np.uint32)
            bad[:, :D // 4] = 0x7f7f7f7f                    # codes at their largest
            bad[:, D // 4:] = np.array([0x7fc00000, 0x7f800000, 0xff800000, 0x7f7fffff] * D, np.uint32)[:D // 32]
            for which in (0, 1):
                for h in range(nKV):
                    c.write_kv(0, which, 1, h, tokens + n, bad)
            poisoned = c.op_attend(0, 1, q, tokens)
            assert np.isfinite(poisoned).all()
            assert np.array_equal(clean.view(np.uint32), poisoned.view(np.uint32)), (tokens, n)
        finally:
            c.close()


def test_attend_beyond_the_shifted_split(gpu):
    """The P.V operand is p * s_v with p carried times 2^8 through the softmax,
    so that its f16 lo half stays normal; a page holding a V scale above 255
    (|V| > 32385 in its 32-channel group) would overflow that f16, and the
    wave drops the shift from that page on. V scales of 300-5000 put on
    tokens of a page in the middle of a work item (page 1), on the first page
    of the next item (page 8) and on a later one (page 10): the output still
    matches the oracle (web/model/kernels.js:1255-1310 attn_av_gqa, f32 for
    any scale) within 2e-5 of max |out|, decode rows through each wave's own
    dequantisation and verify rows through the shared-page blocks, and each
    verify row keeps the bits of the same row attended alone. Then the other
    bound of the shift: rows whose scores reach past 4096 in log2 units
    (queries times 5000) drop it on their own, so they stay finite and near
    the oracle (within 1e-2 of max |out|: at such scores the softmax is one
    token, and the f32 rounding of the scores themselves moves the rest),
    while the rows beside them in the same verify job keep 2e-5 and every
    row keeps the bits of the same row alone."""
    from oracle import lib as L
    from oracle import model as Mo
    for base in (configs.M27B, D256):
        d = configs.with_layers(base, 1)
        D, nH, nKV = d["head_dim"], d["n_heads"], d["n_kv_heads"]
        group = nH // nKV
        tokens, nv = 700, 8
        c = _ctx(gpu, d, n_max=1024, t_max=64, slots=2)
        try:
            om = Mo.Model(d, n_slots=2, max_pages=16)
            c.fill_random_kv(1, tokens + nv, 11, 3)
            om.fill_random_kv(1, tokens + nv, 11, 3)
            big = {100: 300.0, 101: 5000.0, 103: 1000.0, 512: 700.0, 650: 2000.0}
            for h in range(nKV):
                rows = c.read_kv(0, 1, 1, h, 0, tokens + nv)
                assert np.array_equal(rows, om.kv_rows(0, 1, 1, 0, tokens + nv, h))
                for t, s in big.items():
                    sc = rows[t, D // 4:].view(np.float32)
                    sc[h % (D // 32)] = np.float32(s)
                c.write_kv(0, 1, 1, h, 0, rows)
                pg = om.frames[1]["pages"]
                t = np.arange(tokens + nv)
                at = ((pg[t // 64].astype(np.int64) * nKV + h) * 64 + t % 64) * om.rw
                om.V[0][at[:, None] + np.arange(om.rw)[None, :]] = rows
            pages = om.frames[1]["pages"]
            for n in (1, nv):
                q = np.random.default_rng(tokens + n).standard_normal((n, nH * D)).astype(np.float32)
                got = c.op_attend(0, 1, q, tokens)
                Qh = np.ascontiguousarray(q.reshape(n, nH, D).transpose(1, 0, 2))
                L.rope(Qh, D, tokens, om.tbl)
                s = L.qk_scores(Qh, om.K[0], n, tokens + n, 64, D, nH, group, pages)
                p = L.causal_softmax(s, tokens)
                want = L.attn_av(p, om.V[0], D, 64, group, pages).transpose(1, 0, 2).reshape(n, nH * D)
                assert np.isfinite(got).all(), (base["hidden"], n)
                err = np.abs(got - want).max()
                assert err <= 2e-5 * max(1.0, np.abs(want).max()), (base["hidden"], n, err)
                if n > 1:
                    for i in range(n):
                        one = c.op_attend(0, 1, q[i:i + 1], tokens + i)
                        assert np.array_equal(one.view(np.uint32), got[i:i + 1].view(np.uint32)), (base["hidden"], i)
            hot = [2, 5]
            q = np.random.default_rng(tokens + 99).standard_normal((nv, nH * D)).astype(np.float32)
            q[hot] *= 5000.0
            got = c.op_attend(0, 1, q, tokens)
            Qh = np.ascontiguousarray(q.reshape(nv, nH, D).transpose(1, 0, 2))
            L.rope(Qh, D, tokens, om.tbl)
            s = L.qk_scores(Qh, om.K[0], nv, tokens + nv, 64, D, nH, group, pages)
            assert np.abs(s[:, hot]).max() * 1.4426950408889634 > 2 * 4096, "scores short of the bound"
            p = L.causal_softmax(s, tokens)
            want = L.attn_av(p, om.V[0], D, 64, group, pages).transpose(1, 0, 2).reshape(nv, nH * D)
            assert np.isfinite(got).all(), base["hidden"]
            cold = [i for i in range(nv) if i not in hot]
            scale = max(1.0, np.abs(want).max())
            err_hot = np.abs(got[hot] - want[hot]).max()
            err_cold = np.abs(got[cold] - want[cold]).max()
            assert err_hot <= 1e-2 * scale, (base["hidden"], err_hot)
            assert err_cold <= 2e-5 * scale, (base["hidden"], err_cold)
            for i in range(nv):
                one = c.op_attend(0, 1, q[i:i + 1], tokens + i)
                assert np.array_equal(one.view(np.uint32), got[i:i + 1].view(np.uint32)), (base["hidden"], "hot", i)
        finally:
            c.close()

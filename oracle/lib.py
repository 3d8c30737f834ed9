"""ctypes bindings of oracle/ccoracle.c (test infrastructure only).

Each wrapper takes and returns numpy arrays. Build with ``make -C oracle``
(``__graft_entry__.build()`` does it).
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_PATH):
            raise RuntimeError(f"oracle library missing at {_PATH}: run `make -C oracle`")
        L = C.CDLL(_PATH)
        P = C.c_void_p
        i32, i64, u64, f32, f64 = C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_double
        sig = {
            "orc_half_bits": (C.c_uint16, [f32]),
            "orc_half_value": (f32, [C.c_uint16]),
            "orc_to_f16": (None, [P, P, i64]),
            "orc_from_f16": (None, [P, P, i64]),
            "orc_round_f16": (None, [P, i64]),
            "orc_rng": (u64, [u64, u64, u64]),
            "orc_gen_q8": (None, [u64, u64, i64, i64, i32, P, P]),
            "orc_gen_normal_f16": (None, [u64, u64, i64, P]),
            "orc_gen_ids": (None, [u64, u64, i64, i32, P]),
            "orc_gen_scale_f16": (C.c_uint16, [u64, u64, u64, f64, f64]),
            "orc_gen_kv": (None, [u64, u64, u64, i32, i32, i32, i32, P, P]),
            "orc_fill_kv_paged": (None, [u64, u64, u64, i32, i32, i32, i32, P, P]),
            "orc_matmul_q8": (None, [P, i32, i32, P, P, i32, i32, P]),
            "orc_gather_embed_q8": (None, [P, i32, i32, P, P, i32, P]),
            "orc_rmsnorm": (None, [P, P, P, i32, i32, f32]),
            "orc_rope_table": (None, [i32, f64, P, i32, P]),
            "orc_rope": (None, [P, i32, i32, i32, i32, i32, P]),
            "orc_store_kv": (None, [P, P, i32, i32, i32, i32, i32, i32, P, P]),
            "orc_qk_scores": (None, [P, P, P, i32, i32, i32, i32, i32, i32, P, i32, i32]),
            "orc_causal_softmax": (None, [P, i32, i32, i32, i32]),
            "orc_attn_av": (None, [P, P, P, i32, i32, i32, i32, i32, i32, P, i32, i32]),
            "orc_silu_mul": (None, [P, P, P, i64]),
            "orc_add_inplace": (None, [P, P, i64]),
            "orc_topk": (None, [P, i32, i32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --- f16 -------------------------------------------------------------------

def to_f16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_to_f16(_p(x), _p(out), x.size)
    return out


def from_f16(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_from_f16(_p(h), _p(out), h.size)
    return out


def round_f16(x):
    a = np.array(x, dtype=np.float32, copy=True)
    lib().orc_round_f16(_p(a), a.size)
    return a


# --- synthetic inputs ------------------------------------------------------

def rng(seed, stream, i):
    return lib().orc_rng(seed, stream, i)


def gen_q8(seed, stream, N, K, group=32):
    codes = np.empty((N, K), np.int8)
    ng = (K + group - 1) // group
    sc = np.empty((N, ng), np.uint16)
    lib().orc_gen_q8(seed, stream, N, K, group, _p(codes), _p(sc))
    return codes, sc


def gen_normal_f16(seed, stream, n):
    out = np.empty(n, np.uint16)
    lib().orc_gen_normal_f16(seed, stream, n, _p(out))
    return out


def gen_ids(seed, stream, n, vocab):
    out = np.empty(n, np.int32)
    lib().orc_gen_ids(seed, stream, n, vocab, _p(out))
    return out


def gen_scale_f16(seed, stream, i, lo, hi):
    return lib().orc_gen_scale_f16(seed, stream, i, lo, hi)


def gen_kv(seed, stream, key, t0, tokens, nKV, D):
    """Random KV rows: codes [tokens, nKV, D] int8, scales [tokens, nKV] f32."""
    codes = np.empty((tokens, nKV, D), np.int8)
    scales = np.empty((tokens, nKV), np.float32)
    lib().orc_gen_kv(seed, stream, key, t0, tokens, nKV, D, _p(codes), _p(scales))
    return codes, scales


def fill_kv_paged(seed, stream, key, tokens, nKV, D, page, pages, cache):
    """gen_kv's rows 0..tokens-1 written into a paged cache (u32 words,
    reference row layout) through the page table `pages`."""
    pages = _c(pages, np.uint32)
    assert cache.dtype == np.uint32 and cache.flags.c_contiguous
    assert len(pages) * page >= tokens
    lib().orc_fill_kv_paged(seed, stream, key, tokens, nKV, D, page, _p(pages), _p(cache))


# --- kernels ---------------------------------------------------------------

def matmul_q8(X, W, S, group=32):
    X = _c(X, np.float32)
    W = _c(W, np.int8)
    S = _c(S, np.float32)
    M, K = X.shape
    N = W.shape[0]
    assert W.shape[1] == K and K % 4 == 0
    Y = np.empty((M, N), np.float32)
    lib().orc_matmul_q8(_p(X), M, K, _p(W), _p(S), N, group, _p(Y))
    return Y


def gather_embed_q8(ids, wte, S, group=32):
    ids = _c(ids, np.int32)
    wte = _c(wte, np.int8)
    S = _c(S, np.float32)
    T, H = ids.size, wte.shape[1]
    out = np.empty((T, H), np.float32)
    lib().orc_gather_embed_q8(_p(ids), T, H, _p(wte), _p(S), group, _p(out))
    return out


def rmsnorm(x, w, eps):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    T, H = x.shape
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), _p(y), T, H, eps)
    return y


def rope_table(rot, theta, cap, scaling=None):
    tbl = np.empty(cap * rot, np.float32)
    s = None
    if scaling is not None:
        s = np.array([scaling["factor"], scaling["low_freq_factor"], scaling["high_freq_factor"],
                      scaling["original_max_position_embeddings"]], np.float64)
    lib().orc_rope_table(rot, theta, _p(s) if s is not None else None, cap, _p(tbl))
    return tbl


def rope(buf, rot, T_past, tbl):
    """In-place split-half RoPE on a dense [nH, T, D] buffer (returns it)."""
    assert buf.dtype == np.float32 and buf.flags.c_contiguous
    nH, T, D = buf.shape
    lib().orc_rope(_p(buf), nH, T, rot, D, T_past, _p(tbl))
    return buf


def store_kv(src, cache, T_past, page, nKV, D, rot, pages, tbl):
    src = _c(src, np.float32)
    pages = _c(pages, np.uint32)
    assert cache.dtype == np.uint32 and cache.flags.c_contiguous
    T_new = src.shape[0]
    t = tbl if tbl is not None else np.zeros(2, np.float32)
    lib().orc_store_kv(_p(src), _p(cache), T_new, T_past, page, nKV, D, rot, _p(pages), _p(t))


def qk_scores(Q, K, T_new, T_act, page, D, nH, group, pages, r0=0, T_q=None):
    Q = _c(Q, np.float32)
    T_q = T_new if T_q is None else T_q
    pages = _c(pages, np.uint32)
    out = np.empty((nH, T_new, T_act), np.float32)
    lib().orc_qk_scores(_p(Q), _p(K), _p(out), T_new, T_act, page, D, nH, group, _p(pages), r0, T_q)
    return out


def causal_softmax(scores, T_past):
    s = np.array(scores, dtype=np.float32, copy=True)
    nH, T_new, T_act = s.shape
    lib().orc_causal_softmax(_p(s), T_new, T_act, T_past, nH)
    return s


def attn_av(scores, V, D, page, group, pages, out=None, r0=0, T_q=None):
    scores = _c(scores, np.float32)
    nH, T_new, T_act = scores.shape
    T_q = T_new if T_q is None else T_q
    pages = _c(pages, np.uint32)
    if out is None:
        out = np.zeros((nH, T_q, D), np.float32)
    lib().orc_attn_av(_p(scores), _p(V), _p(out), T_new, T_act, page, D, nH, group, _p(pages), r0, T_q)
    return out


def silu_mul(g, u):
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    out = np.empty_like(g)
    lib().orc_silu_mul(_p(g), _p(u), _p(out), g.size)
    return out


def add_inplace(a, b):
    b = _c(b, np.float32)
    assert a.dtype == np.float32 and a.flags.c_contiguous and a.size == b.size
    lib().orc_add_inplace(_p(a), _p(b), a.size)
    return a


def topk(row, M):
    row = _c(row, np.float32)
    vals = np.empty(M, np.float32)
    ids = np.empty(M, np.uint32)
    lib().orc_topk(_p(row), row.size, M, _p(vals), _p(ids))
    return vals, ids

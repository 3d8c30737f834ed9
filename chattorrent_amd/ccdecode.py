"""ctypes binding of the C ABI (include/ccdecode.h) of libccdecode.so.

This is the Python host over the MI355X library: the tests and bench.py use
it; the JS Runner shim (node/runner.js) uses the N-API addon over the same
ABI. There is no CPU fallback: if the HIP library is missing, loading fails.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libccdecode.so")

CC_OK, CC_BUSY, CC_COLD, CC_STALE, CC_NOSPEC, CC_EARG, CC_EPOOL, CC_EOOM, CC_EDEVICE = range(9)
STATUS_NAMES = ["ok", "busy", "cold", "stale", "nospec", "bad-job", "pool-too-small", "out-of-memory",
                "device"]
(T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_LN1, T_LN2, T_WTE, T_NORM, T_LM_HEAD) = range(12)
# a hybrid checkpoint's full_attention extras and linear_attention tensors
(T_ATTN_GATE, T_Q_NORM, T_K_NORM, T_IN_Q, T_IN_K, T_IN_V, T_IN_Z, T_IN_B, T_IN_A, T_CONV_Q, T_CONV_K, T_CONV_V,
 T_GATE_PARAMS, T_GATED_NORM, T_OUT_PROJ) = range(12, 27)
# the MTP draft head; its block's tensors are the block ids at LAYER_MTP
(T_MTP_ENORM, T_MTP_HNORM, T_MTP_FC_E, T_MTP_FC_H, T_MTP_NORM, T_MTP_EMBED, T_MTP_HEAD) = range(27, 34)
LAYER_MTP = -2
FULL_ATTENTION, LINEAR_ATTENTION = 0, 1
EXPORTS = [
    "cc_create", "cc_destroy", "cc_last_error", "cc_upload", "cc_fill_random", "cc_step", "cc_release",
    "cc_slot_pages", "cc_free_pages", "cc_fill_random_kv", "cc_read_kv", "cc_write_kv", "cc_read_pages",
    "cc_stats_get", "cc_op_matmul_q8", "cc_op_store_kv", "cc_op_round_f16", "cc_op_topk", "cc_op_rmsnorm",
    "cc_op_attend", "cc_profile", "cc_profile_read", "cc_read_logits", "cc_mtp_draft", "cc_topk_noalloc",
    "cc_decode_steps",
]


class Dims(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("n_layer", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32), ("vocab", C.c_int32),
                ("q8_group", C.c_int32), ("rms_eps", C.c_float), ("rope_theta", C.c_double),
                ("rope_scaling", C.c_int32), ("rs_factor", C.c_double), ("rs_low_freq", C.c_double),
                ("rs_high_freq", C.c_double), ("rs_orig_max_pos", C.c_double), ("tied", C.c_int32),
                ("rot_dim", C.c_int32), ("hybrid", C.c_int32), ("layer_kinds", C.POINTER(C.c_uint8)),
                ("lin_nk", C.c_int32), ("lin_nv", C.c_int32), ("lin_dk", C.c_int32), ("lin_dv", C.c_int32),
                ("lin_conv", C.c_int32), ("mtp_vocab", C.c_int32)]


class Opts(C.Structure):
    _fields_ = [("lo", C.c_int32), ("hi", C.c_int32), ("n_max", C.c_int32), ("t_max", C.c_int32),
                ("slots", C.c_int32), ("sessions", C.c_int32), ("page_tokens", C.c_int32),
                ("max_jobs", C.c_int32), ("device", C.c_int32)]


class Job(C.Structure):
    _fields_ = [("slot", C.c_int32), ("past", C.c_int32), ("n", C.c_int32), ("sampled", C.c_int32),
                ("ids", C.POINTER(C.c_int32)), ("hidden", C.POINTER(C.c_uint16)), ("snap", C.c_int32),
                ("rollback", C.c_int32), ("keep", C.c_int32), ("mtp", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("vram_bytes", C.c_uint64), ("weight_bytes", C.c_uint64), ("kv_bytes", C.c_uint64),
                ("scratch_bytes", C.c_uint64), ("passes", C.c_int64), ("rows", C.c_int64),
                ("last_pass_ms", C.c_double)]


_lib = None


def load():
    """Loads libccdecode.so; raises if it is not built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m chattorrent_amd.build`")
    L = C.CDLL(LIB_PATH)
    P = C.c_void_p
    i32, i64, u64 = C.c_int32, C.c_int64, C.c_uint64
    sig = {
        "cc_create": (i32, [C.POINTER(Dims), C.POINTER(Opts), C.POINTER(P)]),
        "cc_destroy": (None, [P]),
        "cc_last_error": (C.c_char_p, [P]),
        "cc_upload": (i32, [P, i32, i32, P, C.c_size_t, P, C.c_size_t, i32, i32]),
        "cc_fill_random": (i32, [P, u64]),
        "cc_step": (i32, [P, C.POINTER(Job), i32, i32, i32, i32, P, P, P, P]),
        "cc_release": (i32, [P, i32]),
        "cc_slot_pages": (i32, [P, i32]),
        "cc_free_pages": (i32, [P]),
        "cc_fill_random_kv": (i32, [P, i32, i32, u64, u64]),
        "cc_read_kv": (i32, [P, i32, i32, i32, i32, i32, i32, P]),
        "cc_write_kv": (i32, [P, i32, i32, i32, i32, i32, i32, P]),
        "cc_read_pages": (i32, [P, i32, P, i32]),
        "cc_stats_get": (i32, [P, C.POINTER(Stats)]),
        "cc_op_matmul_q8": (i32, [P, P, i32, i32, P, P, i32, P]),
        "cc_op_store_kv": (i32, [P, i32, i32, i32, P, i32, i32]),
        "cc_op_round_f16": (i32, [P, P, i64]),
        "cc_op_topk": (i32, [P, P, i32, i32, i32, P, P]),
        "cc_op_rmsnorm": (i32, [P, P, P, i32, i32, P]),
        "cc_op_attend": (i32, [P, i32, i32, P, i32, i32, P]),
        "cc_read_logits": (i32, [P, i32, P]),
        "cc_mtp_draft": (i32, [P, i32, i32, i32, i32, i32, P]),
        "cc_decode_steps": (i32, [P, C.POINTER(Job), i32, i32, i32, P, P]),
        "cc_profile": (i32, [P, i32]),
        "cc_profile_read": (i32, [P, i32, C.POINTER(C.c_double), C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class CCError(RuntimeError):
    """A failed call; `.status` is the cc_status, `.kind` its name."""

    def __init__(self, status, msg):
        super().__init__(msg)
        self.status = status
        self.kind = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)


def layer_kinds(d):
    """Block kinds from `layer_types` (the manifest's strings), or None (all full)."""
    lt = d.get("layer_types")
    if not lt:
        return None
    return [LINEAR_ATTENTION if t == "linear_attention" else FULL_ATTENTION for t in lt]


def make_dims(d):
    sc = d.get("rope_scaling")
    dims = Dims(hidden=d["hidden"], n_layer=d["n_layer"], n_heads=d["n_heads"], n_kv_heads=d["n_kv_heads"],
                head_dim=d["head_dim"], ffn=d["ffn"], vocab=d["vocab"], q8_group=d.get("group_q8", 32),
                rms_eps=d["rms_eps"], rope_theta=d["rope_theta"], rope_scaling=1 if sc else 0,
                rs_factor=sc["factor"] if sc else 0.0, rs_low_freq=sc["low_freq_factor"] if sc else 0.0,
                rs_high_freq=sc["high_freq_factor"] if sc else 0.0,
                rs_orig_max_pos=sc["original_max_position_embeddings"] if sc else 0.0,
                tied=1 if d.get("tied", True) else 0, rot_dim=d.get("rot_dim", 0) or 0,
                hybrid=1 if d.get("hybrid") else 0, lin_nk=d.get("lin_nk", 0), lin_nv=d.get("lin_nv", 0),
                lin_dk=d.get("lin_dk", 0), lin_dv=d.get("lin_dv", 0), lin_conv=d.get("lin_conv", 0),
                mtp_vocab=d.get("mtp_vocab", 0) or 0)
    kinds = layer_kinds(d)
    if kinds is not None:
        arr = (C.c_uint8 * len(kinds))(*kinds)
        dims._kinds = arr   # kept alive with the struct; cc_create copies it
        dims.layer_kinds = C.cast(arr, C.POINTER(C.c_uint8))
    return dims


class Context:
    """One cc_ctx: a Runner's GPU half over positions [lo, hi)."""

    def __init__(self, d, n_max, t_max, slots, sessions=None, max_jobs=None, lo=0, hi=None, device=0):
        self.lib = load()
        self.d = dict(d)
        positions = d["n_layer"] + 2
        self.opts = Opts(lo=lo, hi=positions if hi is None else hi, n_max=n_max, t_max=t_max, slots=slots,
                         sessions=sessions or slots, page_tokens=64, max_jobs=max_jobs or (sessions or slots),
                         device=device)
        dims = make_dims(d)
        h = C.c_void_p()
        st = self.lib.cc_create(C.byref(dims), C.byref(self.opts), C.byref(h))
        self.h = h
        if st != CC_OK:
            msg = self.lib.cc_last_error(h).decode() if h else "cc_create failed"
            if h:
                self.lib.cc_destroy(h)
            self.h = None
            raise CCError(st, msg)

    def close(self):
        if self.h:
            self.lib.cc_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _chk(self, st):
        if st != CC_OK:
            raise CCError(st, self.lib.cc_last_error(self.h).decode())

    # --- weights ---------------------------------------------------------------
    def fill_random(self, seed):
        self._chk(self.lib.cc_fill_random(self.h, seed))

    def upload_q8(self, layer, tensor, codes, scales, group=32):
        """int8 codes [N, K] and scales [N, ceil(K/group)]: uint16 arrays are
        f16 bits, float32 arrays are f32 (rounded to f16 on the device side)."""
        codes = np.ascontiguousarray(codes, np.int8)
        if np.asarray(scales).dtype == np.float32:
            sc, kind = np.ascontiguousarray(scales, np.float32), 1
        else:
            sc, kind = np.ascontiguousarray(scales, np.uint16), 0
        self._chk(self.lib.cc_upload(self.h, layer, tensor, _p(codes), codes.size, _p(sc), sc.size, kind,
                                     int(group)))

    def upload_norm(self, layer, tensor, w):
        """An f32 tensor: a norm weight, or a hybrid block's q_norm, k_norm,
        conv1d_q/k/v ([channels, 4]), gate_params or gated_norm."""
        w = np.ascontiguousarray(w, np.float32)
        self._chk(self.lib.cc_upload(self.h, layer, tensor, _p(w), w.size, None, 0, 0, 32))

    # --- KV / pages --------------------------------------------------------------
    def fill_random_kv(self, slot, tokens, seed, key):
        self._chk(self.lib.cc_fill_random_kv(self.h, slot, tokens, seed, key))

    def read_kv(self, layer, which, slot, head, t0, t1):
        D = self.d["head_dim"]
        out = np.empty((t1 - t0, D // 4 + D // 32), np.uint32)
        self._chk(self.lib.cc_read_kv(self.h, layer, which, slot, head, t0, t1, _p(out)))
        return out

    def write_kv(self, layer, which, slot, head, t0, rows):
        rows = np.ascontiguousarray(rows, np.uint32)
        self._chk(self.lib.cc_write_kv(self.h, layer, which, slot, head, t0, t0 + rows.shape[0], _p(rows)))

    def pages(self, slot):
        n = self.lib.cc_slot_pages(self.h, slot)
        out = np.empty(max(n, 1), np.uint32)
        self._chk(self.lib.cc_read_pages(self.h, slot, _p(out), n))
        return out[:n]

    def read_logits(self, rows):
        out = np.empty((rows, self.d["vocab"]), np.float32)
        self._chk(self.lib.cc_read_logits(self.h, rows, _p(out)))
        return out

    def free_pages(self):
        return self.lib.cc_free_pages(self.h)

    def mtp_draft(self, slot, row, token, pos, k):
        """cc_mtp_draft: keep row `row` of the last pass (-1: the kept one) and
        chain `k` drafts after `token` at positions pos.. (uint32 [k])."""
        out = np.zeros(max(k, 1), np.uint32)
        self._chk(self.lib.cc_mtp_draft(self.h, slot, row, token, pos, k, _p(out)))
        return out[:k]

    def release(self, slot):
        self._chk(self.lib.cc_release(self.h, slot))

    def stats(self):
        s = Stats()
        self._chk(self.lib.cc_stats_get(self.h, C.byref(s)))
        return {k: getattr(s, k) for k, _ in Stats._fields_}

    KINDS = ("qkv", "o", "gate_up", "down", "head", "attn")

    def profile(self, enable=True):
        self._chk(self.lib.cc_profile(self.h, 1 if enable else 0))

    def profile_read(self):
        """{kind: (ms_total, launches, algorithmic_bytes)} since profile(True)."""
        out = {}
        for k, name in enumerate(self.KINDS):
            ms, n, b = C.c_double(), C.c_int64(), C.c_double()
            self._chk(self.lib.cc_profile_read(self.h, k, C.byref(ms), C.byref(n), C.byref(b)))
            out[name] = (ms.value, n.value, b.value)
        return out

    # --- the pass -----------------------------------------------------------------
    def step(self, jobs, at=0, to=None, topk=1):
        """jobs: dicts with slot, past, n, sampled and ids (or hidden f16 bits
        [n, H]), optionally snap (a verify) and keep (a rollback). Returns (vals [S, topk], ids [S, topk]) at the head, else the
        f16 bits of every row [T, H]. Raises CCError; `.statuses` holds the
        per-job statuses."""
        positions = self.d["n_layer"] + 2
        to = positions if to is None else to
        arr = (Job * len(jobs))()
        keep = []
        T = S = 0
        for i, j in enumerate(jobs):
            arr[i].slot, arr[i].past, arr[i].n = j["slot"], j["past"], j["n"]
            arr[i].sampled = j.get("sampled", 1 if to == positions else 0)
            if j.get("ids") is not None:
                a = np.ascontiguousarray(j["ids"], np.int32)
                keep.append(a)
                arr[i].ids = a.ctypes.data_as(C.POINTER(C.c_int32))
            if j.get("hidden") is not None:
                a = np.ascontiguousarray(j["hidden"], np.uint16)
                keep.append(a)
                arr[i].hidden = a.ctypes.data_as(C.POINTER(C.c_uint16))
            # speculation through linear_attention blocks: `snap` marks a
            # verify, `keep` (not None) rolls back to before the last verify
            arr[i].snap = 1 if j.get("snap") else 0
            arr[i].mtp = 1 if j.get("mtp") else 0
            if j.get("keep") is not None:
                arr[i].rollback, arr[i].keep = 1, int(j["keep"])
            T += j["n"]
            S += arr[i].sampled
        status = np.zeros(len(jobs), np.int32)
        if to == positions:
            vals = np.empty((max(S, 1), topk), np.float32)
            ids = np.empty((max(S, 1), topk), np.uint32)
            st = self.lib.cc_step(self.h, arr, len(jobs), at, to, topk, _p(vals), _p(ids), None, _p(status))
            if st != CC_OK:
                e = CCError(st, self.lib.cc_last_error(self.h).decode())
                e.statuses = status
                raise e
            return vals[:S], ids[:S]
        hid = np.empty((T, self.d["hidden"]), np.uint16)
        st = self.lib.cc_step(self.h, arr, len(jobs), at, to, 0, None, None, _p(hid), _p(status))
        if st != CC_OK:
            e = CCError(st, self.lib.cc_last_error(self.h).decode())
            e.statuses = status
            raise e
        return hid

    def decode_steps(self, slots, pasts, ids, steps, topk=1):
        """cc_decode_steps: `steps` greedy passes on the device for one-row
        jobs (slot, past, first id); returns (vals, ids) [steps, jobs, topk]."""
        n = len(slots)
        arr = (Job * n)()
        keep = []
        for i in range(n):
            a = np.array([int(ids[i])], np.int32)
            keep.append(a)
            arr[i].slot, arr[i].past, arr[i].n, arr[i].sampled = int(slots[i]), int(pasts[i]), 1, 1
            arr[i].ids = a.ctypes.data_as(C.POINTER(C.c_int32))
        vals = np.empty((steps, n, topk), np.float32)
        out = np.empty((steps, n, topk), np.uint32)
        self._chk(self.lib.cc_decode_steps(self.h, arr, n, steps, topk, _p(vals), _p(out)))
        return vals, out

    # --- kernel-level ops (parity tests) ---------------------------------------------
    def op_matmul_q8(self, X, W, scales_f16):
        X = np.ascontiguousarray(X, np.float32)
        W = np.ascontiguousarray(W, np.int8)
        S = np.ascontiguousarray(scales_f16, np.uint16)
        M, K = X.shape
        N = W.shape[0]
        Y = np.empty((M, N), np.float32)
        self._chk(self.lib.cc_op_matmul_q8(self.h, _p(X), M, K, _p(W), _p(S), N, _p(Y)))
        return Y

    def op_store_kv(self, layer, which, slot, src, past):
        src = np.ascontiguousarray(src, np.float32)
        self._chk(self.lib.cc_op_store_kv(self.h, layer, which, slot, _p(src), src.shape[0], past))

    def op_round_f16(self, a):
        a = np.array(a, dtype=np.float32, copy=True)
        self._chk(self.lib.cc_op_round_f16(self.h, _p(a), a.size))
        return a

    def op_topk(self, logits, M):
        logits = np.ascontiguousarray(logits, np.float32)
        rows, V = logits.shape
        vals = np.empty((rows, M), np.float32)
        ids = np.empty((rows, M), np.uint32)
        self._chk(self.lib.cc_op_topk(self.h, _p(logits), rows, V, M, _p(vals), _p(ids)))
        return vals, ids

    def op_rmsnorm(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        T, H = x.shape
        y = np.empty_like(x)
        self._chk(self.lib.cc_op_rmsnorm(self.h, _p(x), _p(w), T, H, _p(y)))
        return y

    def op_attend(self, layer, slot, q, past):
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty_like(q)
        self._chk(self.lib.cc_op_attend(self.h, layer, slot, _p(q), q.shape[0], past, _p(out)))
        return out

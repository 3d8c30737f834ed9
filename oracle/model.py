"""Oracle restatement of the batched ragged decode pass (test infrastructure only).

Follows, step for step:

* ``web/model/model.js:619-624`` blockSegs and ``:368-409`` fullBlockSegs — one
  block over packed segments: rmsnorm, q/k/v, per-segment attention over the
  session's own pages, o_proj, residual, SwiGLU MLP, residual, then
  ``round_f16`` of the residual stream;
* ``web/model/model.js:321-351`` attend — store K (RoPE'd) and V into the
  paged int8 cache, RoPE on Q, scores, exact causal softmax, P·V;
* ``web/model/model.js:664-679`` forward and ``web/model/stage.js:1314-1440``
  #pass — embedding gather + round, blocks, head on the sampled rows
  (rmsnorm, LM head, top-M);
* ``web/model/model.js:132-211`` the page pool: a free stack initialised so
  the lowest index pops first, ``ensurePages`` pops in logical order,
  ``freePages`` pushes a frame's pages back in reverse.

Synthetic weights come from the same counter-based generator the device uses
(stream numbering below), so host and device start from identical bits.
"""
import math

import numpy as np

from . import lib as L

# Generator streams, shared with chattorrent_amd/csrc (synth.hip).
STREAM_WTE = 1
STREAM_LM_HEAD = 2
TENSORS = ("q", "k", "v", "o", "gate", "up", "down")


def layer_stream(layer, name):
    return (layer + 1) * 16 + TENSORS.index(name)


def kv_stream(layer, which):
    """Stream of a layer's random KV fill; which = 0 for K, 1 for V."""
    return 0x4B560000 + layer * 2 + which


PAGE_TOKENS = 64  # web/split.js:75


def kv_row_words(D):
    """web/model/kernels.js:1955-1958 kvRowWords: D/4 code words + D/QB scales."""
    return D // 4 + D // min(32, D)


def tensor_shapes(d):
    H, D, F = d["hidden"], d["head_dim"], d["ffn"]
    return {
        "q": (d["n_heads"] * D, H), "k": (d["n_kv_heads"] * D, H), "v": (d["n_kv_heads"] * D, H),
        "o": (H, d["n_heads"] * D), "gate": (F, H), "up": (F, H), "down": (H, F),
    }


class PagePool:
    """web/model/model.js:132-147 makePagePool + :191-211 ensurePages/freePages."""

    def __init__(self, n_pages, page_tokens=PAGE_TOKENS):
        self.n_pages = n_pages
        self.page_tokens = page_tokens
        self.free = list(range(n_pages - 1, -1, -1))  # pops lowest index first

    def ensure(self, frame, tokens):
        need = -(-tokens // self.page_tokens)
        if need > frame["max_pages"]:
            return False
        while len(frame["owned"]) < need:
            if not self.free:
                return False
            phys = self.free.pop()
            frame["pages"][len(frame["owned"])] = phys
            frame["owned"].append(phys)
        return True

    def release(self, frame):
        n = len(frame["owned"])
        while frame["owned"]:
            self.free.append(frame["owned"].pop())
        return n


def compose_block(x, ln1, ln2, eps, attention, mlp):
    """One full-attention block's residual stream, in place on x [T, H] f32,
    before the block's f16 round: web/model/model.js:368-409 fullBlockSegs
    (rmsnorm(x) with ln1 -> the attention sublayer -> x += its output) and
    :307-316 ffnBlock (rmsnorm(x) with ln2 -> the MLP -> x += its output).
    `attention(h)` and `mlp(h)` return their sublayer's [T, H] output; the
    parity tests also run this with the reference's dumped sublayer outputs
    in their place, which pins the order of norms and residual adds."""
    L.add_inplace(x, attention(L.rmsnorm(x, ln1, eps)))
    L.add_inplace(x, mlp(L.rmsnorm(x, ln2, eps)))
    return x


class Model:
    """A full-attention Llama-style model with q8 weights and an int8 paged KV pool."""

    def __init__(self, d, n_slots, max_pages, n_pages=None, page_tokens=PAGE_TOKENS):
        self.d = d
        self.group = d.get("group_q8", 32)
        self.page = page_tokens
        self.max_pages = max_pages
        self.pool = PagePool(n_pages if n_pages is not None else n_slots * max_pages, page_tokens)
        D, nKV = d["head_dim"], d["n_kv_heads"]
        self.rw = kv_row_words(D)
        words = self.pool.n_pages * nKV * page_tokens * self.rw
        self.K = [np.zeros(words, np.uint32) for _ in range(d["n_layer"])]
        self.V = [np.zeros(words, np.uint32) for _ in range(d["n_layer"])]
        self.frames = [{"pages": np.zeros(max_pages, np.uint32), "owned": [], "max_pages": max_pages}
                       for _ in range(n_slots)]
        self.rot = d.get("rot_dim", D)
        self.tbl = L.rope_table(self.rot, d["rope_theta"], max_pages * page_tokens + 64,
                                d.get("rope_scaling"))
        self.w = None

    # --- weights -------------------------------------------------------------
    def gen_weights(self, seed):
        d, g = self.d, self.group
        self.w = {"layers": []}
        for layer in range(d["n_layer"]):
            lw = {}
            for name, (N, K) in tensor_shapes(d).items():
                codes, sc = L.gen_q8(seed, layer_stream(layer, name), N, K, g)
                lw[name] = (codes, L.from_f16(sc))
            lw["ln1"] = np.ones(d["hidden"], np.float32)
            lw["ln2"] = np.ones(d["hidden"], np.float32)
            self.w["layers"].append(lw)
        codes, sc = L.gen_q8(seed, STREAM_WTE, d["vocab"], d["hidden"], g)
        self.w["wte"] = (codes, L.from_f16(sc))
        self.w["norm"] = np.ones(d["hidden"], np.float32)
        if not d.get("tied", True):
            codes, sc = L.gen_q8(seed, STREAM_LM_HEAD, d["vocab"], d["hidden"], g)
            self.w["lm_head"] = (codes, L.from_f16(sc))

    def head_weight(self):
        return self.w.get("lm_head", self.w["wte"])

    # --- KV ------------------------------------------------------------------
    def fill_random_kv(self, slot, tokens, seed, key):
        """Random KV rows 0..tokens-1 for `slot` (web/model/model.js:191-202
        ensurePages takes the pages): codes uniform in [-127, 127], one f16
        scale ~U(0.005, 0.02) per (token, kv head), widened and replicated into
        each 32-block. `key` names the chat in the generator index, so the
        device fill reproduces the same rows."""
        d = self.d
        D, nKV, page = d["head_dim"], d["n_kv_heads"], self.page
        frame = self.frames[slot]
        if not self.pool.ensure(frame, tokens):
            raise RuntimeError("the KV pool cannot fit the fill")
        nb = D // min(32, D)
        t = np.arange(tokens)
        for layer in range(d["n_layer"]):
            for which, cache in ((0, self.K[layer]), (1, self.V[layer])):
                codes, scales = L.gen_kv(seed, kv_stream(layer, which), key, 0, tokens, nKV, D)
                for n in range(nKV):
                    rows = ((frame["pages"][t // page].astype(np.int64) * nKV + n) * page + t % page) * self.rw
                    cw = np.ascontiguousarray(codes[:, n, :]).view(np.uint32)
                    for w in range(D // 4):
                        cache[rows + w] = cw[:, w]
                    sbits = np.ascontiguousarray(scales[:, n]).view(np.uint32)
                    for b in range(nb):
                        cache[rows + D // 4 + b] = sbits
        return frame

    def kv_rows(self, layer, which, slot, t0, t1, head):
        """Reference-layout words of rows t0..t1-1 of one kv head: [t, RW] u32."""
        d = self.d
        nKV, page = d["n_kv_heads"], self.page
        frame = self.frames[slot]
        cache = (self.K if which == 0 else self.V)[layer]
        t = np.arange(t0, t1)
        rows = ((frame["pages"][t // page].astype(np.int64) * nKV + head) * page + t % page) * self.rw
        return cache[rows[:, None] + np.arange(self.rw)[None, :]]

    # --- the pass --------------------------------------------------------------
    def attend(self, layer, slot, q, k, v, past):
        d = self.d
        D, nH, nKV, group = d["head_dim"], d["n_heads"], d["n_kv_heads"], d["n_heads"] // d["n_kv_heads"]
        n = q.shape[0]
        pages = self.frames[slot]["pages"]
        Qh = np.ascontiguousarray(q.reshape(n, nH, D).transpose(1, 0, 2))
        L.store_kv(k, self.K[layer], past, self.page, nKV, D, self.rot, pages, self.tbl)
        L.store_kv(v, self.V[layer], past, self.page, nKV, D, 0, pages, None)
        L.rope(Qh, self.rot, past, self.tbl)
        T_act = past + n
        scores = L.qk_scores(Qh, self.K[layer], n, T_act, self.page, D, nH, group, pages)
        p = L.causal_softmax(scores, past)
        ctx = L.attn_av(p, self.V[layer], D, self.page, group, pages)
        return np.ascontiguousarray(ctx.transpose(1, 0, 2).reshape(n, nH * D))

    def block(self, layer, x, segs):
        d, g = self.d, self.group
        lw = self.w["layers"][layer]

        seen = {}

        def attention(h):
            q = L.matmul_q8(h, *lw["q"], group=g)
            k = L.matmul_q8(h, *lw["k"], group=g)
            v = L.matmul_q8(h, *lw["v"], group=g)
            merged = np.empty_like(q)
            for s in segs:
                a, b = s["row"], s["row"] + s["n"]
                merged[a:b] = self.attend(layer, s["slot"], q[a:b], k[a:b], v[a:b], s["past"])
            seen["attn"] = L.matmul_q8(merged, *lw["o"], group=g)
            return seen["attn"]

        def mlp(h):
            act = L.silu_mul(L.matmul_q8(h, *lw["gate"], group=g), L.matmul_q8(h, *lw["up"], group=g))
            seen["mlp"] = L.matmul_q8(act, *lw["down"], group=g)
            return seen["mlp"]

        compose_block(x, lw["ln1"], lw["ln2"], d["rms_eps"], attention, mlp)
        if getattr(self, "on_sublayers", None) is not None:
            self.on_sublayers(layer, seen["attn"], seen["mlp"])
        L.lib().orc_round_f16(L._p(x), x.size)
        return x

    def _run_block(self, layer, x, segs):
        self.block(layer, x, segs)

    def pass_(self, jobs, layers=None, head=True, capture=None):
        """One packed pass. `jobs`: dicts with slot, past, n, and ids [n] (or
        hidden [n, H] f32 holding f16 values), `sampled` (rows the head samples:
        the last one, or all n for a verify) and `topk` (M). Returns per job
        {"hidden": [n,H] f32, "logits": [sampled, V], "vals", "ids"}.
        `capture(layer, x)` is called with the residual after each block."""
        d = self.d
        H = d["hidden"]
        segs, row = [], 0
        for j in jobs:
            frame = self.frames[j["slot"]]
            if not self.pool.ensure(frame, j["past"] + j["n"]):
                raise RuntimeError("the KV pool cannot fit the job")
            segs.append({"slot": j["slot"], "past": j["past"], "n": j["n"], "row": row,
                         "snap": bool(j.get("snap")), "keep": j.get("keep")})
            row += j["n"]
        T = row
        if "ids" in jobs[0] and jobs[0]["ids"] is not None:
            ids = np.concatenate([np.asarray(j["ids"], np.int32) for j in jobs])
            codes, sc = self.w["wte"]
            x = L.gather_embed_q8(ids, codes, sc, self.group)
            L.lib().orc_round_f16(L._p(x), x.size)
        else:
            x = np.ascontiguousarray(np.concatenate([np.asarray(j["hidden"], np.float32) for j in jobs]))
        assert x.shape == (T, H)
        for layer in (range(d["n_layer"]) if layers is None else layers):
            self._run_block(layer, x, segs)
            if capture is not None:
                capture(layer, x)
        out = []
        for j, s in zip(jobs, segs):
            r = {"hidden": x[s["row"]:s["row"] + s["n"]].copy()}
            out.append(r)
        if head:
            rows = []
            for j, s in zip(jobs, segs):
                ns = j.get("sampled", 1)
                rows.extend(range(s["row"] + s["n"] - ns, s["row"] + s["n"]))
            if rows:
                hs = L.rmsnorm(x[rows], self.w["norm"], d["rms_eps"])
                logits = L.matmul_q8(hs, *self.head_weight(), group=self.group)
                at = 0
                for j, r in zip(jobs, out):
                    ns = j.get("sampled", 1)
                    M = j.get("topk", 1)
                    r["logits"] = logits[at:at + ns]
                    vals, ids = [], []
                    for i in range(ns):
                        v, ix = L.topk(logits[at + i], M)
                        vals.append(v)
                        ids.append(ix)
                    r["vals"], r["ids"] = np.array(vals), np.array(ids)
                    at += ns
        return out




class StreamedModel(Model):
    """Model at a full model's depth with bounded host memory, for the
    full-size parity tests: a block's q8 weights and
    its random KV rows are regenerated from the counter-based generator each
    time the block runs, into one layer's worth of buffers, and only the K/V
    rows the passes append are kept between passes. The arithmetic is
    Model's: the same block, attention and head, in the same order.

    `contexts`: per slot, (tokens of random KV, generator key), filled as
    Model.fill_random_kv fills them; every frame takes the pages for
    tokens + `extra` up front, in slot order."""

    def __init__(self, d, seed, contexts, extra, page_tokens=PAGE_TOKENS):
        self.d = d
        self.seed = seed
        self.group = d.get("group_q8", 32)
        self.page = page_tokens
        n_max = max(T for T, _ in contexts) + extra
        self.max_pages = -(-n_max // page_tokens)
        need = [-(-(T + extra) // page_tokens) for T, _ in contexts]
        self.pool = PagePool(sum(need), page_tokens)
        D, nKV = d["head_dim"], d["n_kv_heads"]
        self.rw = kv_row_words(D)
        words = self.pool.n_pages * nKV * page_tokens * self.rw
        self._kv = (np.zeros(words, np.uint32), np.zeros(words, np.uint32))
        self.K = [None] * d["n_layer"]
        self.V = [None] * d["n_layer"]
        self.frames = [{"pages": np.zeros(self.max_pages, np.uint32), "owned": [], "max_pages": self.max_pages}
                       for _ in contexts]
        for frame, (T, _) in zip(self.frames, contexts):
            self.pool.ensure(frame, T + extra)
        self.contexts = list(contexts)
        self.rot = d.get("rot_dim", D)
        self.tbl = L.rope_table(self.rot, d["rope_theta"], self.max_pages * page_tokens + 64, d.get("rope_scaling"))
        g = self.group
        self.w = {"layers": [None] * d["n_layer"], "norm": np.ones(d["hidden"], np.float32)}
        codes, sc = L.gen_q8(seed, STREAM_WTE, d["vocab"], d["hidden"], g)
        self.w["wte"] = (codes, L.from_f16(sc))
        if not d.get("tied", True):
            codes, sc = L.gen_q8(seed, STREAM_LM_HEAD, d["vocab"], d["hidden"], g)
            self.w["lm_head"] = (codes, L.from_f16(sc))
        # layer -> {(slot, t): (K words [nKV, RW], V words [nKV, RW])}
        self.kept = [dict() for _ in range(d["n_layer"])]
        self.on_layer = None   # called with each block index once it has run

    def _rows(self, slot, t):
        nKV = self.d["n_kv_heads"]
        page = self.frames[slot]["pages"][t // self.page].astype(np.int64)
        return (((page * nKV + np.arange(nKV)) * self.page + t % self.page) * self.rw)[:, None] + np.arange(self.rw)

    def _load(self, layer):
        d, g = self.d, self.group
        lw = {}
        for name, (N, K) in tensor_shapes(d).items():
            codes, sc = L.gen_q8(self.seed, layer_stream(layer, name), N, K, g)
            lw[name] = (codes, L.from_f16(sc))
        lw["ln1"] = np.ones(d["hidden"], np.float32)
        lw["ln2"] = np.ones(d["hidden"], np.float32)
        self.w["layers"][layer] = lw
        for which, buf in enumerate(self._kv):
            for slot, (T, key) in enumerate(self.contexts):
                if T:
                    L.fill_kv_paged(self.seed, kv_stream(layer, which), key, T, d["n_kv_heads"], d["head_dim"],
                                    self.page, self.frames[slot]["pages"], buf)
            for (slot, t), rows in self.kept[layer].items():
                buf[self._rows(slot, t)] = rows[which]
        self.K[layer], self.V[layer] = self._kv

    def _run_block(self, layer, x, segs):
        self._load(layer)
        self.block(layer, x, segs)
        for s in segs:
            for t in range(s["past"], s["past"] + s["n"]):
                r = self._rows(s["slot"], t)
                self.kept[layer][(s["slot"], t)] = (self._kv[0][r].copy(), self._kv[1][r].copy())
        self.w["layers"][layer] = None
        self.K[layer] = self.V[layer] = None
        if self.on_layer is not None:
            self.on_layer(layer)

    def fill_random_kv(self, slot, tokens, seed, key):
        raise NotImplementedError("a StreamedModel's KV is given at construction")

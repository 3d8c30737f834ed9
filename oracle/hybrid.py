"""Oracle restatement of the hybrid (Qwen3.5-architecture) blocks — test
infrastructure only: the parity tests compare the HIP path with these
functions; nothing in the product imports them.

Follows:

* ``web/model/kernels.js:1538-1580`` causal_conv1d (depthwise, SiLU fused,
  the job's window reaching before row 0 reads the history ring);
* ``web/model/kernels.js:1582-1620`` update_conv_history;
* ``web/model/kernels.js:1622-1670`` l2norm_heads (sum of squares + 1e-6,
  repeat_interleave by ``group``);
* ``web/model/kernels.js:1672-1805`` gated_delta_net_step (gates from the raw
  projections and the packed A_log / dt_bias, one pass over the old state per
  token with the readout ``qScale·(Σ(g·S)q + delta·(k·q))``);
* ``web/model/kernels.js:1822-1839`` sigmoid_mul;
* ``web/model/model.js:418-444`` linearCore and ``:472-527`` linearBlockSegs
  (the per-session recurrence, gated rmsnorm, out_proj);
* ``web/model/model.js:368-410`` fullBlockSegs's hybrid extras: attn_gate,
  q_norm / k_norm over head_dim, partial rotary, the output gate before
  o_proj.

All arithmetic is float32, in the reference's order where it fixes one.

Parity pins (``tests/test_oracle_hybrid.py``): every function is checked
against the reference's own dumps of a small Qwen3.5 model
(``oracle/qwen3.8-27b-spike`` of the reference: f32 weights of one
linear_attention and one full_attention layer with every intermediate), the
recurrence also against the textbook delta rule in float64, and the conv
history against a sliding window over the whole sequence.
"""
import numpy as np

from . import lib as L

F32 = np.float32


def silu(x):
    """x·sigmoid(x) as causal_conv1d and silu_mul write it: s = 1/(1+exp(-x)), x·s."""
    x = np.asarray(x, F32)
    s = (F32(1.0) / (F32(1.0) + np.exp(-x))).astype(F32)
    return (x * s).astype(F32)


def sigmoid_mul(gate, a):
    """kernels.js:1822-1839: sigmoid(gate)·a."""
    s = (F32(1.0) / (F32(1.0) + np.exp(-np.asarray(gate, F32)))).astype(F32)
    return (s * np.asarray(a, F32)).astype(F32)


def causal_conv1d(x, w, hist=None):
    """kernels.js:1538-1580. x [T, C] (this job's rows), w [C, K]; hist
    [K-1, C] holds the K-1 rows before x's row 0 (zeros for a new session).
    out[t, c] = silu(Σ_k w[c, k]·x[t-(K-1)+k, c]), k in order."""
    x = np.asarray(x, F32)
    T, C = x.shape
    K = w.shape[1]
    if hist is None:
        hist = np.zeros((K - 1, C), F32)
    full = np.concatenate([hist.astype(F32), x], axis=0)   # row K-1 is x's row 0
    acc = np.zeros((T, C), F32)
    for k in range(K):
        acc = (acc + w[:, k].astype(F32)[None, :] * full[k:k + T]).astype(F32)
    return silu(acc)


def update_conv_history(hist, new):
    """kernels.js:1582-1620: the ring after a chunk of rows `new` [T, C]: the
    last K-1 rows of old ++ new."""
    Kh = hist.shape[0]
    return np.ascontiguousarray(np.concatenate([hist, np.asarray(new, F32)], axis=0)[-Kh:]) if Kh else hist


def l2norm_heads(x, src_heads, D, group=1):
    """kernels.js:1622-1670: per (row, source head) x·(1/sqrt(Σx² + 1e-6)),
    written to heads src*group + g for g < group. x [T, src_heads*D] ->
    [T, src_heads*group, D]."""
    x = np.asarray(x, F32).reshape(-1, src_heads, D)
    ss = np.sum((x * x).astype(F32), axis=2, dtype=F32)
    scale = (F32(1.0) / np.sqrt(ss + F32(1e-6))).astype(F32)
    y = (x * scale[:, :, None]).astype(F32)
    return np.repeat(y, group, axis=1)


def gdn_gates(a_raw, b_raw, params, heads):
    """kernels.js:1736-1741: a = a_raw + dt_bias; softplus (a > 20 form for
    large a); g = exp(-exp(A_log)·sp); beta = sigmoid(b_raw)."""
    a = (np.asarray(a_raw, F32) + params[heads:2 * heads].astype(F32)).astype(F32)
    with np.errstate(over="ignore"):
        sp_small = np.log(F32(1.0) + np.exp(a)).astype(F32)
    sp_big = (a + np.log(F32(1.0) + np.exp(-a))).astype(F32)
    sp = np.where(a > 20.0, sp_big, sp_small).astype(F32)
    g = np.exp(-np.exp(params[:heads].astype(F32)) * sp).astype(F32)
    beta = (F32(1.0) / (F32(1.0) + np.exp(-np.asarray(b_raw, F32)))).astype(F32)
    return g, beta


def gdn_step(q, k, v, a_raw, b_raw, params, S):
    """kernels.js:1672-1805 over the rows of one session, in place on S
    [heads, Dk, Dv]. q, k [T, heads, Dk] (l2-normed, repeated), v [T, heads,
    Dv], a_raw / b_raw [T, heads]. Returns out [T, heads, Dv]."""
    T, heads, Dk = q.shape
    Dv = v.shape[2]
    q_scale = F32(1.0) / np.sqrt(F32(Dk))
    out = np.zeros((T, heads, Dv), F32)
    g, beta = gdn_gates(a_raw, b_raw, params, heads)
    for t in range(T):
        for h in range(heads):
            s = (S[h] * g[t, h]).astype(F32)                       # decay
            kv = (s * k[t, h][:, None]).astype(F32).sum(axis=0, dtype=F32)
            qo = (s * q[t, h][:, None]).astype(F32).sum(axis=0, dtype=F32)
            kq = np.sum((k[t, h] * q[t, h]).astype(F32), dtype=F32)
            delta = ((v[t, h] - kv) * beta[t, h]).astype(F32)
            S[h] = (s + (k[t, h][:, None] * delta[None, :]).astype(F32)).astype(F32)
            out[t, h] = ((qo + delta * kq) * q_scale).astype(F32)
    return out


def gated_rmsnorm(core, w, z, eps):
    """model.js:523-524: rmsnorm over each head's Dv values with gated_norm,
    then silu(z)·normed (RMSNormGated). core, z [T, nV*Dv]."""
    T = core.shape[0]
    Dv = w.shape[0]
    rows = np.ascontiguousarray(core.reshape(-1, Dv), F32)
    normed = L.rmsnorm(rows, np.asarray(w, F32), eps).reshape(T, -1)
    return L.silu_mul(np.ascontiguousarray(z, F32), np.ascontiguousarray(normed, F32))


class LinearState:
    """One session's recurrent state for one linear_attention layer
    (model.js:46-58 makeRecurrentState): S [nV, Dk, Dv] and the conv rings
    of the q, k and v channels (kept here as one [K-1, convDim] ring; the
    conv is depthwise, so the channel split changes nothing)."""

    def __init__(self, lin):
        self.S = np.zeros((lin["nV"], lin["Dk"], lin["Dv"]), F32)
        self.hist = np.zeros((lin["K4"] - 1, 2 * lin["keyDim"] + lin["valueDim"]), F32)

    def copy(self):
        c = LinearState.__new__(LinearState)
        c.S = self.S.copy()
        c.hist = self.hist.copy()
        return c


def lin_dims(d):
    nK, nV, Dk, Dv = d["lin_nk"], d["lin_nv"], d["lin_dk"], d["lin_dv"]
    return {"nK": nK, "nV": nV, "Dk": Dk, "Dv": Dv, "K4": d["lin_conv"], "keyDim": nK * Dk,
            "valueDim": nV * Dv, "group": nV // nK}


def linear_core(lin, lw, state, q, k, v, a, b):
    """model.js:418-444 linearCore for one session's rows: conv (with the
    ring), l2norm with the value-head repeat, the recurrence, then the ring
    advanced by the raw projections. Returns core [T, nV*Dv]."""
    T = q.shape[0]
    raw = np.concatenate([q, k, v], axis=1).astype(F32)
    conv = causal_conv1d(raw, lw["conv"], state.hist)
    kd = lin["keyDim"]
    cq, ck, cv = conv[:, :kd], conv[:, kd:2 * kd], conv[:, 2 * kd:]
    ql = l2norm_heads(cq, lin["nK"], lin["Dk"], lin["group"])
    kl = l2norm_heads(ck, lin["nK"], lin["Dk"], lin["group"])
    vv = cv.reshape(T, lin["nV"], lin["Dv"])
    out = gdn_step(ql, kl, vv, a, b, lw["gate_params"], state.S)
    state.hist = update_conv_history(state.hist, raw)
    return out.reshape(T, lin["nV"] * lin["Dv"])


def linear_block(d, lw, x, segs, states, matmul, rms_eps, spec=None):
    """model.js:472-526 linearBlockSegs, its attention half: x [T, H] gets
    out_proj's rows added in place (the SwiGLU MLP and the f16 round follow
    as in every block). `matmul(h, name)` gives the projection of rows h by
    weight `name`; `states[s]` is segment s's LinearState. `spec(s, st, rows)`
    (optional) runs before segment s's recurrence with its projections
    (q, k, v, a, b) and returns the state to use: restoreSpec / snapSpec
    (model.js:447-470)."""
    lin = lin_dims(d)
    h = L.rmsnorm(x, lw["ln1"], rms_eps)
    q, k, v = matmul(h, "in_q"), matmul(h, "in_k"), matmul(h, "in_v")
    z, bb, aa = matmul(h, "in_z"), matmul(h, "in_b"), matmul(h, "in_a")
    core = np.zeros((x.shape[0], lin["valueDim"]), F32)
    for i, (s, st) in enumerate(zip(segs, states)):
        r0, r1 = s["row"], s["row"] + s["n"]
        rows = (q[r0:r1], k[r0:r1], v[r0:r1], aa[r0:r1], bb[r0:r1])
        if spec is not None:
            st = spec(i, st, rows)
        core[r0:r1] = linear_core(lin, lw, st, *rows)
    gated = gated_rmsnorm(core, lw["gated_norm"], z, rms_eps)
    L.add_inplace(x, matmul(gated, "out"))
    return x


def qk_norm_rope(q, k, qn, kn, nH, nKV, D, eps):
    """fullBlockSegs's q_norm / k_norm (model.js:388-394): rmsnorm over each
    head's D values. RoPE is applied afterwards by attend as for any model."""
    T = q.shape[0]
    qo = L.rmsnorm(np.ascontiguousarray(q.reshape(T * nH, D), F32), qn, eps).reshape(T, nH * D)
    ko = L.rmsnorm(np.ascontiguousarray(k.reshape(T * nKV, D), F32), kn, eps).reshape(T, nKV * D)
    return np.ascontiguousarray(qo), np.ascontiguousarray(ko)


def full_block_extras(model, layer, lw, x, segs):
    """fullBlockSegs (model.js:368-410) on a hybrid checkpoint: attn_gate,
    q_norm / k_norm before RoPE, the output gate before o_proj."""
    d, g = model.d, model.group
    nH, nKV, D = d["n_heads"], d["n_kv_heads"], d["head_dim"]
    h = L.rmsnorm(x, lw["ln1"], d["rms_eps"])
    q = L.matmul_q8(h, *lw["q"], group=g)
    k = L.matmul_q8(h, *lw["k"], group=g)
    v = L.matmul_q8(h, *lw["v"], group=g)
    gate = L.matmul_q8(h, *lw["attn_gate"], group=g)
    qn, kn = qk_norm_rope(q, k, lw["q_norm"], lw["k_norm"], nH, nKV, D, d["rms_eps"])
    merged = np.empty_like(q)
    for s in segs:
        a, b = s["row"], s["row"] + s["n"]
        merged[a:b] = model.attend(layer, s["slot"], qn[a:b], kn[a:b], v[a:b], s["past"])
    attn = L.matmul_q8(sigmoid_mul(gate, merged), *lw["o"], group=g)
    L.add_inplace(x, attn)


class HybridModel:
    """The oracle pass over a hybrid model: model.js:619-624 blockSegs picks
    fullBlockSegs or linearBlockSegs per block. Wraps oracle.model.Model (the
    paged KV pool, attention, embedding and head) and keeps one LinearState
    per (session slot, linear block), started from zero by a job at position
    0 (a new session, model.js:46-58)."""

    def __init__(self, d, n_slots, max_pages):
        from . import model as Mo

        self.d = d
        self.base = Mo.Model(d, n_slots=n_slots, max_pages=max_pages)
        self.base.block = self.block
        self.lin = lin_dims(d) if d.get("lin_nk") else None
        self.states = {}
        self.spec = {}   # (slot, layer) -> (state before the last verify, its projections)

    @property
    def w(self):
        return self.base.w

    @w.setter
    def w(self, value):
        self.base.w = value

    def state(self, slot, layer, past):
        key = (slot, layer)
        if past == 0 or key not in self.states:
            self.states[key] = LinearState(self.lin)
        return self.states[key]

    def _ffn(self, lw, x):
        d, g = self.d, self.base.group
        h = L.rmsnorm(x, lw["ln2"], d["rms_eps"])
        act = L.silu_mul(L.matmul_q8(h, *lw["gate"], group=g), L.matmul_q8(h, *lw["up"], group=g))
        L.add_inplace(x, L.matmul_q8(act, *lw["down"], group=g))
        L.lib().orc_round_f16(L._p(x), x.size)

    def block(self, layer, x, segs):
        lw = self.w["layers"][layer]
        if lw.get("kind") == "linear":
            states = [self.state(s["slot"], layer, s["past"]) for s in segs]
            g = self.base.group

            def mm(h, name):
                return L.matmul_q8(h, *lw[name], group=g)

            def spec(i, st, rows):
                # restoreSpec: the state from before the last verify, then its
                # first `keep` rows again from their stored projections;
                # snapSpec: a verify keeps the state it starts from and its rows
                s = segs[i]
                key = (s["slot"], layer)
                if s.get("keep") is not None:
                    snap, saved = self.spec[key]
                    st = snap.copy()
                    kk = s["keep"]
                    if kk > 0:
                        linear_core(self.lin, lw, st, *(r[:kk] for r in saved))
                    self.states[key] = st
                if s.get("snap"):
                    self.spec[key] = (st.copy(), tuple(np.array(r) for r in rows))
                return st
            linear_block(self.d, lw, x, segs, states, mm, self.d["rms_eps"], spec)
        else:
            full_block_extras(self.base, layer, lw, x, segs)
        self._ffn(lw, x)
        return x

    def pass_(self, jobs, **kw):
        return self.base.pass_(jobs, **kw)


class MtpHead:
    """The MTP draft head (model.js:529-576 mtpBlock / mtpDraft / mtpChain,
    stage.js:296-320 #mtpAfter and :1404-1421 the fill). Its one
    full-attention block keeps its own int8 KV in a pool layer addressed by
    the trunk's page tables; each session keeps the trunk row its next MTP
    row pairs with (`kept`, zero until set). `trunk` is the oracle model
    (HybridModel or model.Model) whose frames and pool it shares."""

    def __init__(self, trunk, w, draft_vocab):
        from . import model as Mo

        base = trunk.base if isinstance(trunk, HybridModel) else trunk
        self.d = base.d
        d1 = dict(self.d, n_layer=1, layer_types=["full_attention"])
        self.m = Mo.Model(d1, n_slots=len(base.frames), max_pages=base.max_pages, n_pages=base.pool.n_pages)
        self.m.frames, self.m.pool = base.frames, base.pool
        self.w, self.V = w, draft_vocab
        self.kept = {}
        self.hybrid = bool(self.d.get("hybrid"))

    def _mm(self, h, t):
        return L.matmul_q8(np.ascontiguousarray(h, F32), *t, group=self.m.group)

    def block(self, hin, ids, slot, past):
        """mtpBlock: x = fc_e·enorm(embed_draft[ids]) + fc_h·hnorm(h), then the
        layer (no f16 round: it is not a trunk block)."""
        d, w = self.d, self.w
        codes, sc = w["embed_draft"]
        e = L.gather_embed_q8(np.asarray(ids, np.int32), codes, sc, self.m.group)
        x = self._mm(L.rmsnorm(e, w["enorm"], d["rms_eps"]), w["fc_e"])
        L.add_inplace(x, self._mm(L.rmsnorm(np.asarray(hin, F32), w["hnorm"], d["rms_eps"]), w["fc_h"]))
        lw = w["block"]
        segs = [{"slot": slot, "past": past, "n": len(ids), "row": 0}]
        if self.hybrid:
            full_block_extras(self.m, 0, lw, x, segs)
        else:
            h = L.rmsnorm(x, lw["ln1"], d["rms_eps"])
            qkv = [self._mm(h, lw[n]) for n in ("q", "k", "v")]
            L.add_inplace(x, self._mm(self.m.attend(0, slot, *qkv, past), lw["o"]))
        h = L.rmsnorm(x, lw["ln2"], d["rms_eps"])
        act = L.silu_mul(self._mm(h, lw["gate"]), self._mm(h, lw["up"]))
        L.add_inplace(x, self._mm(act, lw["down"]))
        return x

    def kept_row(self, slot):
        return self.kept.get(slot, np.zeros(self.d["hidden"], F32))

    def fill(self, job, hidden):
        """The MTP layer's KV for a job's rows: token past + r with the trunk
        row of past + r - 1 (the kept row for r = 0). `hidden`: the job's rows
        after the last block. A job that samples nothing keeps its last row."""
        n = job["n"]
        hin = np.concatenate([self.kept_row(job["slot"])[None, :], hidden[:n - 1]], axis=0)
        self.block(hin, job["ids"], job["slot"], job["past"])
        if job.get("sampled", 1) == 0:
            self.kept[job["slot"]] = np.array(hidden[n - 1], F32)

    def draft(self, slot, row, token, pos, k):
        """#mtpAfter + mtpChain: keep `row` (None: the kept one), then k drafts,
        each the argmax of head_draft·mtp_norm(x) over the draft rows, lowest
        id on a tie (argmax_rows, kernels.js:1405-1440)."""
        if row is not None:
            self.kept[slot] = np.array(row, F32)
        if k > 0 and not self.m.pool.ensure(self.m.frames[slot], pos + k):
            raise RuntimeError("the KV pool cannot fit the drafts")
        h, t, out = self.kept_row(slot)[None, :], token, []
        for i in range(k):
            x = self.block(h, [t], slot, pos + i)
            logits = self._mm(L.rmsnorm(x, self.w["mtp_norm"], self.d["rms_eps"]), self.w["head_draft"])[0]
            t = int(np.argmax(logits))   # the first maximum: the lowest id on a tie
            out.append((t, logits))
            h = x
        return out

"""Pins oracle/hybrid.py (the Gated DeltaNet block and the hybrid full-attention
extras) against the reference's own dump of a small Qwen3.5 model
(tests/golden/hybrid_spike.npz, from the reference's oracle/qwen3.8-27b-spike:
HF's float32 forward with every intermediate), against the textbook delta rule
in float64, and against whole-sequence forms of the chunked paths. No GPU."""
import json
import os

import numpy as np
import pytest

from oracle import hybrid as Hy
from oracle import lib as L

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def spike():
    z = np.load(os.path.join(HERE, "golden", "hybrid_spike.npz"), allow_pickle=False)
    a = {k: z[k] for k in z.files}
    a["cfg"] = json.loads(bytes(a.pop("config_json")).decode())
    return a


def _dims(cfg):
    nK, nV = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    Dk, Dv = cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
    return dict(nK=nK, nV=nV, Dk=Dk, Dv=Dv, K4=cfg["linear_conv_kernel_dim"], keyDim=nK * Dk, valueDim=nV * Dv,
                group=nV // nK)


def _close(got, want, rtol, atol_frac=1e-6):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want).max()
    assert err <= rtol * np.abs(want).max() + atol_frac, (err, np.abs(want).max())


def test_conv_matches_hf(spike):
    """causal_conv1d over the whole prompt (no history) = HF's causal_conv1d_fn with SiLU."""
    x, w = spike["layer00_conv_pre"][0] if spike["layer00_conv_pre"].ndim == 3 else spike["layer00_conv_pre"], \
        spike["weight_layer00_conv1d"]
    want = spike["layer00_conv_post"]
    want = want[0] if want.ndim == 3 else want
    _close(Hy.causal_conv1d(x, w), want, 1e-5)


def test_conv_chunks_with_history_equal_whole(spike):
    """Chunks carried through the ring give the whole sequence's conv, bit for
    bit (update_conv_history keeps exactly the rows the next window needs),
    for chunks shorter and longer than K-1."""
    x = spike["layer00_conv_pre"]
    x = x[0] if x.ndim == 3 else x
    w = spike["weight_layer00_conv1d"]
    whole = Hy.causal_conv1d(x, w)
    for cuts in ([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11], [5], [2, 7], [3, 4, 9]):
        hist = np.zeros((w.shape[1] - 1, x.shape[1]), np.float32)
        parts, a = [], 0
        for b in cuts + [x.shape[0]]:
            parts.append(Hy.causal_conv1d(x[a:b], w, hist))
            hist = Hy.update_conv_history(hist, x[a:b])
            a = b
        assert np.array_equal(np.concatenate(parts), whole), cuts


def test_qkv_split_l2norm_and_repeat(spike):
    """The conv output's q|k|v channel ranges, l2norm_heads with the value-head
    repeat (repeat_interleave: source head h feeds heads h*group..), = HF."""
    lin = _dims(spike["cfg"])
    conv = spike["layer00_conv_post"]
    conv = conv[0] if conv.ndim == 3 else conv
    kd = lin["keyDim"]
    T = conv.shape[0]
    rq = spike["layer00_query_raw"].reshape(T, lin["nV"], lin["Dk"])
    # the raw query HF hands the recurrence is the repeated conv output
    assert np.array_equal(np.repeat(conv[:, :kd].reshape(T, lin["nK"], lin["Dk"]), lin["group"], axis=1), rq)
    _close(Hy.l2norm_heads(conv[:, :kd], lin["nK"], lin["Dk"], lin["group"]),
           spike["layer00_query_l2norm"].reshape(T, lin["nV"], lin["Dk"]), 1e-6)
    _close(Hy.l2norm_heads(conv[:, kd:2 * kd], lin["nK"], lin["Dk"], lin["group"]),
           spike["layer00_key_l2norm"].reshape(T, lin["nV"], lin["Dk"]), 1e-6)
    assert np.array_equal(conv[:, 2 * kd:].reshape(T, lin["nV"], lin["Dv"]),
                          spike["layer00_value"].reshape(T, lin["nV"], lin["Dv"]))


def test_gates_match_hf(spike):
    """g = exp(-exp(A_log)·softplus(a + dt_bias)) (HF dumps the log, exp'd in
    its recurrence) and beta = sigmoid(b)."""
    nV = spike["layer00_A_log"].size
    params = np.concatenate([spike["layer00_A_log"], spike["layer00_dt_bias"]]).astype(np.float32)
    T = spike["layer00_a_raw"].shape[-2]
    g, beta = Hy.gdn_gates(spike["layer00_a_raw"].reshape(T, nV), spike["layer00_b_raw"].reshape(T, nV), params, nV)
    _close(g, np.exp(spike["layer00_g"].reshape(T, nV).astype(np.float64)), 1e-6)
    _close(beta, spike["layer00_beta"].reshape(T, nV), 1e-6)
    # the a > 20 branch of softplus agrees with the direct form where both are finite
    a = np.array([[19.0, 20.5, 25.0]], np.float32)
    g2, _ = Hy.gdn_gates(a, np.zeros_like(a), np.array([0, 0, 0, 0, 0, 0], np.float32), 3)
    _close(g2, np.exp(-np.log1p(np.exp(a.astype(np.float64)))), 1e-6)


def _delta_rule_f64(q, k, v, g, beta):
    """The textbook gated delta rule (HF torch_recurrent_gated_delta_rule), in
    float64: S = g·S; S += k ⊗ beta·(v − Sᵀk); out = Sᵀq / sqrt(Dk)."""
    T, H, Dk = q.shape
    Dv = v.shape[2]
    S = np.zeros((H, Dk, Dv))
    out = np.zeros((T, H, Dv))
    states = [S.copy()]
    for t in range(T):
        for h in range(H):
            S[h] *= g[t, h]
            kv = S[h].T @ k[t, h]
            S[h] += np.outer(k[t, h], beta[t, h] * (v[t, h] - kv))
            out[t, h] = S[h].T @ q[t, h] / np.sqrt(Dk)
        states.append(S.copy())
    return out, states


def test_recurrence_matches_hf_and_the_delta_rule(spike):
    """gdn_step's one-pass readout over the old state = HF's per-token
    recurrence (output and every state), and = the textbook rule in f64."""
    lin = _dims(spike["cfg"])
    T = spike["layer00_a_raw"].shape[-2]
    q = spike["layer00_query_l2norm"].reshape(T, lin["nV"], lin["Dk"]).astype(np.float32)
    k = spike["layer00_key_l2norm"].reshape(T, lin["nV"], lin["Dk"]).astype(np.float32)
    v = spike["layer00_value"].reshape(T, lin["nV"], lin["Dv"]).astype(np.float32)
    a = spike["layer00_a_raw"].reshape(T, lin["nV"])
    b = spike["layer00_b_raw"].reshape(T, lin["nV"])
    params = np.concatenate([spike["layer00_A_log"], spike["layer00_dt_bias"]]).astype(np.float32)
    states = spike["layer00_recurrent_states"].reshape(T + 1, lin["nV"], lin["Dk"], lin["Dv"])
    want = spike["layer00_recurrent_core_out_seq"].reshape(T, lin["nV"], lin["Dv"])
    S = np.zeros((lin["nV"], lin["Dk"], lin["Dv"]), np.float32)
    outs = []
    for t in range(T):
        outs.append(Hy.gdn_step(q[t:t + 1], k[t:t + 1], v[t:t + 1], a[t:t + 1], b[t:t + 1], params, S)[0])
        _close(S, states[t + 1], 1e-5)
    _close(np.stack(outs), want, 1e-5)
    # all rows in one call = one call per row, bit for bit
    S2 = np.zeros_like(S)
    assert np.array_equal(Hy.gdn_step(q, k, v, a, b, params, S2), np.stack(outs))
    assert np.array_equal(S2, S)
    g, beta = Hy.gdn_gates(a, b, params, lin["nV"])
    o64, st64 = _delta_rule_f64(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                                g.astype(np.float64), beta.astype(np.float64))
    _close(np.stack(outs), o64, 1e-5)
    _close(S, st64[-1], 1e-5)


def test_recurrence_beta_zero_reads_zero():
    """beta ≈ 0 and a zero state leave the readout at zero (the reference's own
    check, kernels.test.js:1388-1398), which a dropped beta would fail."""
    rng = np.random.default_rng(5)
    T, H, Dk, Dv = 5, 3, 5, 7
    q, k = rng.standard_normal((T, H, Dk)).astype(np.float32), rng.standard_normal((T, H, Dk)).astype(np.float32)
    v = rng.standard_normal((T, H, Dv)).astype(np.float32)
    a = rng.standard_normal((T, H)).astype(np.float32)
    params = np.concatenate([rng.standard_normal(H) - 1, rng.standard_normal(H)]).astype(np.float32)
    S = np.zeros((H, Dk, Dv), np.float32)
    out = Hy.gdn_step(q, k, v, a, np.full((T, H), -30.0, np.float32), params, S)
    assert np.abs(out).max() < 1e-3


def test_gated_norm_and_out_proj_match_hf(spike):
    """RMSNormGated over each head (gated_norm weight as is, eps 1e-6) times
    silu(z), then out_proj: HF's norm output and the linear_attn output."""
    lin = _dims(spike["cfg"])
    T = spike["layer00_z_raw"].shape[-2]
    core = spike["layer00_recurrent_core_out_seq"].reshape(T, lin["valueDim"])
    z = spike["layer00_z_raw"].reshape(T, lin["valueDim"])
    got = Hy.gated_rmsnorm(core, spike["weight_layer00_gated_norm"], z, spike["cfg"]["rms_norm_eps"])
    _close(got, spike["layer00_gated_norm_out"].reshape(T, lin["valueDim"]), 1e-5)
    out = got @ spike["weight_layer00_out_proj"].T
    _close(out, spike["layer00_linear_attn_out"].reshape(T, -1), 1e-5)


def test_full_attention_extras_match_hf(spike):
    """The hybrid full-attention layer: q_proj's per-head q|gate halves
    (tools/convert_hf.py:150-160 split_q_gate), q_norm/k_norm with the
    converter's +1, partial rotary (rot 16 of 64, theta 1e7), and the output
    gate sigmoid(gate)·attention before o_proj."""
    cfg = spike["cfg"]
    nH, nKV, D, rot = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["rot_dim"]
    eps = cfg["rms_norm_eps"]
    T = spike["layer03_q_proj_raw"].shape[-2]
    qg = spike["layer03_q_proj_raw"].reshape(T, nH, 2, D)
    q, gate = qg[:, :, 0].reshape(T, nH * D), qg[:, :, 1].reshape(T, nH * D)
    assert np.array_equal(gate, spike["layer03_gate_raw"].reshape(T, nH * D))
    k = spike["layer03_k_proj_raw"].reshape(T, nKV * D)
    qn, kn = Hy.qk_norm_rope(q, k, spike["weight_layer03_q_norm"] + 1.0, spike["weight_layer03_k_norm"] + 1.0,
                             nH, nKV, D, eps)
    _close(qn, spike["layer03_q_norm_out"].reshape(T, nH * D), 1e-5)
    _close(kn, spike["layer03_k_norm_out"].reshape(T, nKV * D), 1e-5)
    tbl = L.rope_table(rot, cfg["rope_theta"], T + 8)
    Qh = np.ascontiguousarray(qn.reshape(T, nH, D).transpose(1, 0, 2))
    L.rope(Qh, rot, 0, tbl)
    _close(Qh.transpose(1, 0, 2), spike["layer03_q_rope"].reshape(T, nH, D), 1e-5)
    Kh = np.ascontiguousarray(kn.reshape(T, nKV, D).transpose(1, 0, 2))
    L.rope(Kh, rot, 0, tbl)
    _close(Kh.transpose(1, 0, 2), spike["layer03_k_rope"].reshape(T, nKV, D), 1e-5)
    # channels past rot_dim are not rotated
    assert np.array_equal(Qh.transpose(1, 0, 2)[:, :, rot:], qn.reshape(T, nH, D)[:, :, rot:])
    # f32 causal attention on the rotated q/k, the gate, o_proj
    v = spike["layer03_v"].reshape(T, nKV, D).astype(np.float64)
    Q, K = Qh.transpose(1, 0, 2).astype(np.float64), Kh.transpose(1, 0, 2).astype(np.float64)
    grp = nH // nKV
    ctx = np.zeros((T, nH, D))
    for h in range(nH):
        s = Q[:, h] @ K[:, h // grp].T / np.sqrt(D)
        s[np.triu_indices(T, 1)] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ctx[:, h] = p @ v[:, h // grp]
    gated = Hy.sigmoid_mul(gate, ctx.reshape(T, nH * D).astype(np.float32))
    _close(gated @ spike["weight_layer03_o_proj"].T, spike["layer03_attn_out"].reshape(T, -1), 1e-5)

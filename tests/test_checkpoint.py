"""The on-disk checkpoint reader (chattorrent_amd/checkpoint.py) against a
checkpoint written in the reference's layout (tests/ckpt_writer.py): the
manifest's dims (web/model/loader.js:146-201), its checks (:206-240), and
the tensor reads with uploadTensors' shape/alignment/size checks and error
messages (:455-525). No GPU: the upload itself is in test_gpu_checkpoint.py."""
import json
import os

import numpy as np
import pytest

import ckpt_writer as W
from chattorrent_amd import checkpoint as C

D_SMALL = dict(hidden=128, n_layer=2, n_heads=2, n_kv_heads=1, head_dim=64, ffn=256, vocab=300, rms_eps=1e-5,
               rope_theta=10000.0, tied=False)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("ckpt"))
    written = W.make(path, D_SMALL, group=64)
    return path, written


def test_dims_and_checks(ckpt):
    path, _ = ckpt
    m = C.load_manifest(path)
    d = C.dims_from_manifest(m)
    for k in ("hidden", "n_layer", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "rms_eps", "rope_theta"):
        assert d[k] == D_SMALL[k], k
    assert d["tied"] is False and d["dtype"] == "q8" and not d["hybrid"]
    assert C.check_manifest(m, d) == []
    bad = dict(m, weight_layout="in_out", dtype="f32", act="gelu")
    probs = C.check_manifest(bad)
    assert any("weight_layout in_out" in p for p in probs)
    assert any("act gelu" in p for p in probs)
    assert any("dtype f32" in p for p in probs)
    with pytest.raises(ValueError, match="manifest is missing vocab"):
        C.dims_from_manifest({k: v for k, v in m.items() if k != "vocab"})
    # defaults of dimsFromManifest
    d2 = C.dims_from_manifest({k: v for k, v in m.items() if k not in ("rms_eps", "rope_theta", "tied_lm_head")})
    assert d2["rms_eps"] == 1e-5 and d2["rope_theta"] == 10000.0 and d2["tied"] is True


def test_tensors_read_back(ckpt):
    path, written = ckpt
    m = C.load_manifest(path)
    d = C.dims_from_manifest(m)
    for i in range(d["n_layer"]):
        got = C.load_block(path, m, d, i)
        want = written[C.block_file(i)]
        assert set(got) == set(want)
        for name, t in want.items():
            if isinstance(t, tuple):
                codes, scales, group = got[name]
                assert group == 64 and np.array_equal(codes, t[0]) and np.array_equal(scales, t[1])
            else:
                assert np.array_equal(got[name], t)
    client = C.load_client(path, m, d)
    assert np.array_equal(client["wte"][0], written["client.bin"]["wte"][0])
    assert np.array_equal(client["lm_head"][1], written["lm_head.bin"]["lm_head"][1])
    assert np.array_equal(client["norm"], written["client.bin"]["norm"])


def test_read_errors(ckpt):
    path, _ = ckpt
    m = C.load_manifest(path)
    d = C.dims_from_manifest(m)
    fn = C.block_file(0)
    entries = m["files"][fn]
    shapes = C.block_shapes(d)
    with pytest.raises(ValueError, match=r"block_00.bin: no tensor named q_proj"):
        C.read_tensors(path, fn, [e for e in entries if e["name"] != "q_proj"], shapes)
    wrong = dict(shapes, q_proj=[64, 128])
    with pytest.raises(ValueError, match=r"block_00.bin:q_proj shape \[128, 128\], expected \[64, 128\]"):
        C.read_tensors(path, fn, entries, wrong)
    with pytest.raises(ValueError, match="unexpected tensor"):
        C.read_tensors(path, fn, entries + [dict(entries[0], name="extra")], shapes)
    odd = [dict(e, scales_size=e["scales_size"] + 4) if e["name"] == "k_proj" else e for e in entries]
    with pytest.raises(ValueError, match="k_proj scales are"):
        C.read_tensors(path, fn, odd, shapes)
    mis = [dict(e, offset=e["offset"] + 2) if e["name"] == "v_proj" else e for e in entries]
    with pytest.raises(ValueError, match="not 4-byte aligned"):
        C.read_tensors(path, fn, mis, shapes)
    # strict off: a subset of the file
    got = C.read_tensors(path, fn, entries, {"q_proj": shapes["q_proj"]}, strict=False)
    assert list(got) == ["q_proj"]


def test_manifest_is_json_the_reference_reads(ckpt):
    """The fields loader.js reads, with their types."""
    path, _ = ckpt
    with open(os.path.join(path, "manifest.json")) as f:
        m = json.load(f)
    for e in m["files"]["block_00.bin"]:
        assert {"name", "shape", "offset", "size", "dtype"} <= set(e)
        if e["dtype"] == "q8":
            assert {"group", "scales_offset", "scales_size"} <= set(e)


def test_hybrid_checkpoint_reads_back(tmp_path):
    """A hybrid checkpoint (Gated DeltaNet and full blocks with the Qwen3.5
    extras, an MTP file): dims, per-kind shapes and every tensor read back."""
    import hybrid_weights as HW
    d = dict(HW.SPIKE)
    w = HW.make(d, 5)
    wm = HW.make_mtp(d, 5, 64)
    W.make_hybrid(str(tmp_path), d, w, wm)
    m = C.load_manifest(str(tmp_path))
    dd = C.dims_from_manifest(m)
    assert C.check_manifest(m, dd) == []
    for k in ("hybrid", "rot_dim", "lin_nk", "lin_nv", "lin_dk", "lin_dv", "lin_conv", "layer_types"):
        assert dd[k] == d[k], k
    assert dd["mtp_vocab"] == 64
    blk = C.load_block(str(tmp_path), m, dd, 0)
    assert set(blk) == set(C.block_shapes(dd, "linear_attention"))
    kd = d["lin_nk"] * d["lin_dk"]
    assert np.array_equal(blk["conv1d_k"], w["layers"][0]["conv"][kd:2 * kd])
    assert np.array_equal(blk["in_proj_b"][0], w["layers"][0]["in_b"][0])
    full = C.load_block(str(tmp_path), m, dd, 3)
    assert {"attn_gate", "q_norm", "k_norm"} <= set(full)
    mt = C.load_mtp(str(tmp_path), m, dd)
    assert np.array_equal(mt["head_draft"][1], wm["head_draft"][1]) and mt["head_draft"][2] == 32
    bad = dict(m, linear_num_value_heads=7)
    assert any("not divisible" in p for p in C.check_manifest(bad))

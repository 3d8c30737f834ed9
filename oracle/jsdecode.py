"""Test infrastructure: the inputs and the runner of oracle/js/decode.js, the
single-threaded JavaScript restatement of the decode pass (the CPU "JS path"
baseline). Only tests/ and bench.py's cpu_baseline use it.

write_inputs() writes what Model.gen_weights and Model.fill_random_kv build
(the same counter-based generator, oracle/model.py), as flat files:
  <tensor>.i8 / <tensor>.f32   q8 codes [N, K] and f32 scales [N, K/32]
  L<l>_ln1.f32, L<l>_ln2.f32, norm.f32, rope.f32 (oracle rope table)
  L<l>_K<s>.u32 / L<l>_V<s>.u32   slot s's rows 0..T-1, [T][nKV] rows of the
                                   reference layout (D/4 code words, then the
                                   row's f32 scale once per 32 values)
  model.json                       dims, contexts, first ids
run() executes node on them and returns its JSON line."""
import json
import os
import shutil
import subprocess

import numpy as np

from . import lib as L
from . import model as Mo

HERE = os.path.dirname(os.path.abspath(__file__))
SCRIPT = os.path.join(HERE, "js", "decode.js")


def node_binary():
    return shutil.which("node") or shutil.which("nodejs")


def write_inputs(path, d, seed, contexts, first_ids, steps, logits_out=None):
    os.makedirs(path, exist_ok=True)
    H, D, nKV = d["hidden"], d["head_dim"], d["n_kv_heads"]
    assert d.get("rot_dim", D) == D and H % 32 == 0 and d["ffn"] % 32 == 0, "dense full-rotary shapes only"

    def q8(name, stream, N, K):
        codes, sc = L.gen_q8(seed, stream, N, K, 32)
        codes.tofile(os.path.join(path, name + ".i8"))
        L.from_f16(sc).astype(np.float32).tofile(os.path.join(path, name + ".f32"))

    q8("wte", Mo.STREAM_WTE, d["vocab"], H)
    if not d.get("tied", True):
        q8("lm_head", Mo.STREAM_LM_HEAD, d["vocab"], H)
    np.ones(H, np.float32).tofile(os.path.join(path, "norm.f32"))
    cap = max(contexts) + steps + 64
    L.rope_table(D, d["rope_theta"], cap, d.get("rope_scaling")).tofile(os.path.join(path, "rope.f32"))
    rw = Mo.kv_row_words(D)
    for layer in range(d["n_layer"]):
        for name, (N, K) in Mo.tensor_shapes(d).items():
            q8(f"L{layer}_{name}", Mo.layer_stream(layer, name), N, K)
        for ln in ("ln1", "ln2"):
            np.ones(H, np.float32).tofile(os.path.join(path, f"L{layer}_{ln}.f32"))
        for which, tag in ((0, "K"), (1, "V")):
            for s, T in enumerate(contexts):
                rows = np.zeros((T, nKV, rw), np.uint32)
                if T:
                    codes, scales = L.gen_kv(seed, Mo.kv_stream(layer, which), s + 1, 0, T, nKV, D)
                    rows[:, :, :D // 4] = codes.reshape(T, nKV, D).view(np.uint32)
                    rows[:, :, D // 4:] = scales.view(np.uint32)[:, :, None]
                rows.tofile(os.path.join(path, f"L{layer}_{tag}{s}.u32"))
    meta = {"dims": {k: d[k] for k in ("hidden", "head_dim", "n_heads", "n_kv_heads", "ffn", "vocab", "n_layer",
                                       "rms_eps")},
            "tied": bool(d.get("tied", True)), "contexts": [int(T) for T in contexts],
            "first_ids": [int(i) for i in first_ids], "logits_out": logits_out}
    with open(os.path.join(path, "model.json"), "w") as f:
        json.dump(meta, f)


def run(path, steps, timeout=600):
    node = node_binary()
    if node is None:
        raise RuntimeError("node is not installed")
    r = subprocess.run([node, SCRIPT, path, str(steps)], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                       text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"decode.js failed: {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])

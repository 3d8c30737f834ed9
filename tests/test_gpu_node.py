"""The Node host on the GPU: the JS Runner over the N-API addon decodes the
same greedy tokens as the C ABI driven directly, whole and split across two
Runners at a block boundary (f16 hand-off)."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from chattorrent_amd import configs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")


@pytest.mark.gpu
@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_node_runner_matches_c_abi(gpu):
    from chattorrent_amd.ccdecode import Context
    d = configs.with_layers(configs.SMOLLM2, 4)
    rng = np.random.default_rng(7)
    chats = [rng.integers(0, d["vocab"], n).tolist() for n in (5, 9, 3)]
    cfg = {"dims": d, "seed": 11, "nMax": 256, "tMax": 32, "chats": chats, "steps": 4, "cut": 3}
    print("[node] running tests/node/native_pass.js", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "native_pass.js"), json.dumps(cfg)], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    # The same decode through the C ABI from Python, every chat in one pass.
    c = Context(d, n_max=256, t_max=32, slots=3)
    c.fill_random(11)
    _, ids = c.step([{"slot": i, "past": 0, "n": len(p), "ids": p, "sampled": 1} for i, p in enumerate(chats)])
    hist = [[int(ids[i, 0])] for i in range(len(chats))]
    past = [len(p) for p in chats]
    for _ in range(cfg["steps"]):
        _, ids = c.step([{"slot": i, "past": past[i], "n": 1, "ids": [hist[i][-1]], "sampled": 1}
                         for i in range(len(chats))])
        for i in range(len(chats)):
            hist[i].append(int(ids[i, 0]))
            past[i] += 1
    assert out["whole"] == hist
    assert out["split"] == hist
    assert out["batched"] >= 1


@pytest.mark.gpu
@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_node_runner_loads_checkpoint(gpu, tmp_path):
    """Runner.append over node/loader.js: a q8 checkpoint in the reference's
    layout (group 64, f32 scales) loaded position by position, whole and split
    at a block with the rows crossing in the peers' message format
    (node/wire.js); the tokens equal the C ABI's with the same checkpoint
    loaded by chattorrent_amd/checkpoint.py."""
    import ckpt_writer as W
    from chattorrent_amd import checkpoint as C
    from chattorrent_amd.ccdecode import Context
    d = configs.with_layers(configs.SMOLLM2, 3)
    W.make(str(tmp_path), d, group=64)
    rng = np.random.default_rng(8)
    chats = [rng.integers(0, d["vocab"], n).tolist() for n in (4, 7)]
    cfg = {"dims": d, "seed": 0, "nMax": 256, "tMax": 32, "chats": chats, "steps": 3, "cut": 2,
           "checkpoint": str(tmp_path), "wire": True}
    print("[node] running tests/node/native_pass.js with a checkpoint", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "native_pass.js"), json.dumps(cfg)], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    c = Context(d, n_max=256, t_max=32, slots=2)
    try:
        C.upload(c, str(tmp_path))
        _, ids = c.step([{"slot": i, "past": 0, "n": len(p), "ids": p, "sampled": 1} for i, p in enumerate(chats)])
        hist = [[int(ids[i, 0])] for i in range(len(chats))]
        past = [len(p) for p in chats]
        for _ in range(cfg["steps"]):
            _, ids = c.step([{"slot": i, "past": past[i], "n": 1, "ids": [hist[i][-1]], "sampled": 1}
                             for i in range(len(chats))])
            for i in range(len(chats)):
                hist[i].append(int(ids[i, 0]))
                past[i] += 1
    finally:
        c.close()
    assert out["whole"] == hist
    assert out["split"] == hist


@pytest.mark.gpu
def test_node_speculative_decoding_equals_greedy(gpu, tmp_path):
    """The JS Runner on a hybrid checkpoint with an MTP head: greedy decoding
    with the head's drafts verified in one pass (rejected drafts rolled back
    through the Gated DeltaNet blocks) emits exactly the tokens of plain
    greedy decoding, for three chats at once."""
    import ckpt_writer as W
    import hybrid_weights as HW
    d = dict(HW.D256)
    w = HW.make(d, 4)
    wm = HW.make_mtp(d, 4, d["vocab"])
    W.make_hybrid(str(tmp_path), d, w, wm)
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, d["vocab"], n).tolist() for n in (5, 9, 3)]
    cfg = {"checkpoint": str(tmp_path), "nMax": 256, "tMax": 32, "prompts": prompts, "steps": 24}
    print("[node] running tests/node/spec_pass.js", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "spec_pass.js"), json.dumps(cfg)], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print("[node] verifies", out["verifies"], "accepted drafts", out["accepted"], "| known drafts: verifies",
          out["verifies2"], "accepted", out["accepted2"], flush=True)
    assert out["spec"] == out["plain"]
    assert out["verifies"] > 0 and out["nospec"] == 0
    # drafts from the plain run itself (some wrong): partly and wholly accepted verifies
    assert out["known"] == out["plain"]
    assert out["accepted2"] > out["verifies2"]

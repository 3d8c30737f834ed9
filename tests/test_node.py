"""The Node host (chattorrent_amd/node): the JS Runner's policy on the CPU stub
backend (tests/node/runner.test.js), the addon's load and exports."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "chattorrent_amd", "node", "ccdecode.node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def test_runner_policy_on_stub_backend():
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "runner.test.js")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("passed")


@pytest.mark.skipif(not os.path.exists(ADDON), reason="addon not built")
def test_addon_exports_every_binding():
    code = "const a = require(process.argv[1]); console.log(Object.keys(a).sort().join(','))"
    r = subprocess.run([NODE, "-e", code, ADDON], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=60)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().split(",") == sorted(
        ["create", "destroy", "fillRandom", "fillRandomKV", "upload", "step", "release", "slotPages", "freePages",
         "readLogits", "stats", "lastError", "mtpDraft"])


def test_loader_reads_reference_checkpoint(tmp_path):
    """node/loader.js (web/model/loader.js's dims, checks and tensor reads over
    the filesystem) on a checkpoint in the reference's layout: every tensor's
    length, group and exact sums equal what was written."""
    import json
    import numpy as np
    import ckpt_writer as W
    d = dict(hidden=128, n_layer=2, n_heads=2, n_kv_heads=1, head_dim=64, ffn=256, vocab=300, rms_eps=1e-5,
             rope_theta=10000.0, tied=False)
    written = W.make(str(tmp_path), d, group=64)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "loader.test.js"), str(tmp_path)], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0, r.stdout
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["dims"]["n_heads"] == 2 and out["dims"]["tied_lm_head"] is False
    files = dict(written)
    files["client"] = dict(written["client.bin"], **written["lm_head.bin"])
    for fn, ts in files.items():
        if fn in ("client.bin", "lm_head.bin"):
            continue
        for name, t in ts.items():
            got = out["files"][fn][name]
            if isinstance(t, tuple):
                assert got["kind"] == "q8" and got["n"] == t[0].size and got["ns"] == t[1].size and got["group"] == 64
                assert got["codes"] == int(t[0].astype(np.int64).sum())
                assert abs(got["scales"] - float(t[1].astype(np.float64).sum())) <= 1e-9 * t[1].size
            else:
                assert got["kind"] == "f32" and got["n"] == t.size
                assert abs(got["sum"] - float(t.astype(np.float64).sum())) <= 1e-9 * t.size


def test_wire_format():
    """node/wire.js: the peers' message framing and fragmentation (web/net.js:73-207)."""
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "wire.test.js")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("passed")

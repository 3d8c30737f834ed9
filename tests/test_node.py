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
         "readLogits", "stats", "lastError"])

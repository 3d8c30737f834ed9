"""The C ABI boundary on the CPU: the built library loads and exports every
function include/ccdecode.h declares, the Python binding names the same set,
and a context refuses cleanly without a GPU (no CPU fallback)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ccdecode.h")
LIB = os.path.join(ROOT, "chattorrent_amd", "libccdecode.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for must in ["cc_create", "cc_destroy", "cc_step", "cc_release", "cc_upload", "cc_last_error",
                 "cc_op_matmul_q8", "cc_op_store_kv", "cc_op_attend", "cc_op_topk"]:
        assert must in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = C.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_python_binding_matches_header():
    from chattorrent_amd import ccdecode
    assert sorted(ccdecode.EXPORTS) == declared()


@pytest.mark.skipif(not os.path.exists(LIB) or os.path.exists("/dev/kfd"), reason="needs a host without a GPU")
def test_no_gpu_is_an_error_not_a_fallback():
    from chattorrent_amd import configs
    from chattorrent_amd.ccdecode import CCError, Context
    with pytest.raises(CCError) as e:
        Context(configs.with_layers(configs.SMOLLM2, 1), n_max=128, t_max=4, slots=1)
    assert e.value.status == 8   # CC_EDEVICE


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one MI355X: asked for more GPUs it exits with a
    message (status 2) before touching any device, rather than reporting a
    one-GPU figure under an N-GPU label."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stderr)
    assert r.stdout == ""
    assert "one MI355X" in r.stderr

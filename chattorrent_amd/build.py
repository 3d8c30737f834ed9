"""Builds the HIP library (libccdecode.so, gfx950) and the N-API addon in-tree.

    python -m chattorrent_amd.build [--no-addon]

The library is the product: every kernel of the pass is hand-written HIP for
gfx950, compiled here with hipcc (it cross-compiles without a GPU). Flags:
  -ffp-contract=off   no implicit a*b+c fusion: the KV quantiser, RoPE and the
                      residual round must reproduce the reference's f32 steps;
  -packed-fp32-ops    disabled: no packed FP32 instructions are generated.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libccdecode.so")
PROBE = os.path.join(HERE, "libccprobe.so")
ADDON_DIR = os.path.join(HERE, "node")
ADDON = os.path.join(ADDON_DIR, "ccdecode.node")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the scale FMA reads them without copies
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]
SOURCES = ["kernels.hip", "api.hip"]


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that note is harmless.
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build failed: {' '.join(cmd)}")
    return out


def build_lib():
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *HIP_FLAGS, *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp]
    _run(cmd)
    os.replace(tmp, LIB)
    return LIB


def build_probe():
    """The bandwidth probes the benchmark reports beside its roofline
    (csrc/probe.hip): a library of their own, so the decode library carries
    no measurement code."""
    tmp = PROBE + ".tmp"
    _run([HIPCC, *HIP_FLAGS, os.path.join(CSRC, "probe.hip"), "-o", tmp])
    os.replace(tmp, PROBE)
    return PROBE


def build_addon():
    """The N-API addon (node/ccdecode_napi.cc) linked against libccdecode.so.
    Needs the Node headers (/usr/include/node); skipped when they are absent."""
    inc = "/usr/include/node"
    src = os.path.join(ADDON_DIR, "ccdecode_napi.cc")
    if not (os.path.isdir(inc) and os.path.exists(src)):
        return None
    cxx = shutil.which("g++") or "g++"
    tmp = ADDON + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-I", inc, "-I", os.path.join(ROOT, "include"),
           src, "-o", tmp, "-L", HERE, "-lccdecode", "-Wl,-rpath,$ORIGIN/..",
           "-Wl,--unresolved-symbols=ignore-in-object-files"]
    _run(cmd)
    os.replace(tmp, ADDON)
    return ADDON


def build_oracle():
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")])


def main():
    build_lib()
    build_probe()
    if "--no-addon" not in sys.argv:
        build_addon()
    print(LIB)


if __name__ == "__main__":
    main()

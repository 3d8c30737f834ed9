"""ccdecode: an MI355X-native batched ragged decode pass (l-wn/ChatTorrent's Runner pass).

* ``csrc/`` — the HIP kernels for gfx950 and the C ABI (include/ccdecode.h),
  built into ``libccdecode.so``;
* ``ccdecode`` — the ctypes host binding (Python);
* ``node/`` — the N-API addon and the JS Runner shim that keeps the
  reference's Runner API (web/model/stage.js);
* ``configs`` — the benchmark model shapes.
"""
from . import configs  # noqa: F401

__all__ = ["configs", "ccdecode"]

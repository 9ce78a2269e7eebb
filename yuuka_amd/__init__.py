"""yuuka_amd — MI355X (gfx950) implementation of yuuka's speculative verify path.

The product is the C-ABI library libyuuka_hip.so (include/yuuka_hip.h). This
package holds its sources (csrc/), the in-tree build (build.py), a ctypes
binding mirroring the reference Go binding (hip.py), the synthetic workload
generators of the benchmark configurations (synth.py) and the host-side
verify engine (engine.py).
"""
from . import hip  # noqa: F401

__all__ = ["hip"]

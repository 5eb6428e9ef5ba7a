"""42-Berlin-Engine decode hot path on MI355X (gfx950).

csrc/        HIP kernels and the C ABI (built into lib42be_hip.so)
be42.py      ctypes host mirror used by tests, smoke() and bench.py

The directory name is not a Python identifier; load it by path, e.g.
``sys.path.insert(0, "<repo>/42-berlin-engine_amd"); import be42``.
"""
import os
import sys

_here = os.path.dirname(os.path.abspath(__file__))
if _here not in sys.path:
    sys.path.insert(0, _here)

import be42  # noqa: E402,F401

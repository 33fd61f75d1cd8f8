"""cppnet_amd — MI355X (gfx950) training backend for CppNet.

Native pieces (built in-tree by ``python -m cppnet_amd.build``):
  _lib/libcnhip.so   hand-written HIP kernels + the C ABI of include/cnhip.h
  _lib/libcppnet.so  C++17 CppNet-compatible layer classes (device "gpu") and
                     the trainer C ABI of include/cppnet_train.h

Python here is a thin ctypes front end used by tests and bench.py.
"""
from pathlib import Path

__version__ = "0.1.0"
PACKAGE_DIR = Path(__file__).resolve().parent
LIB_DIR = PACKAGE_DIR / "_lib"

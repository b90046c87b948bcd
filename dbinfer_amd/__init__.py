"""MI355X-native KV-cache + GQA attention hot path of dbinfer.

The product is ``libdbi_kv.so`` (hand-written gfx950 HIP kernels behind the
C-ABI in ``include/dbi_kv.h``). This package holds its sources (``csrc/``),
the C++ host mirror of the reference's KV-cache call sites (``host/``) and a
thin Python handle (``kv.HipKV``) used by tests and ``bench.py``.
"""
from ._lib import LIB_PATH, load  # noqa: F401

__all__ = ["LIB_PATH", "load"]

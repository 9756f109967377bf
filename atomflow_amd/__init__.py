"""atomflow_amd — MI355X-native KV-cache hot path of AtomFlow.

The product is ``libatomflow_kv.so`` (hand-written gfx950 HIP kernels behind the
C ABI in ``include/af_kv.h``). This package loads it with ctypes and mirrors the
reference's operator interface for Python callers (``atomflow_amd.kv``). There
is no CPU fallback: every entry point raises when the library is missing or a
call fails.
"""
import ctypes
import os
import subprocess

from . import _abi

_HERE = os.path.dirname(os.path.abspath(__file__))
# ATOMFLOW_KV_LIB selects another build of the same library (the host sanitizer
# build of tests/test_host_sanitizers.py); the default is the in-tree build.
LIB_PATH = os.environ.get("ATOMFLOW_KV_LIB") or os.path.join(_HERE, "libatomflow_kv.so")
_lib = None

# af_kv.h status codes
AF_OK = 0
AF_ERR_POOL_EXHAUSTED = -1
AF_ERR_INVALID_ARG = -2
AF_ERR_UNSUPPORTED = -3
AF_ERR_OUT_OF_RANGE = -4
AF_ERR_BAD_BLOCK = -5
AF_ERR_WORKSPACE = -6
AF_ERR_BAD_SEQUENCE = -7
AF_ERR_BAD_FILE = -9
AF_ERR_TIMEOUT = -10
AF_KV_FP16 = 1
AF_KV_FP8_E4M3 = 3
AF_KV_POOL_SHARED_BLOCKS = 1


class AfError(RuntimeError):
    def __init__(self, status, what=""):
        self.status = status
        msg = lib().af_status_string(status).decode()
        super().__init__(f"{what}: status {status} ({msg})" if what else f"status {status} ({msg})")


def build(force=True, jobs=8):
    """Compiles libatomflow_kv.so for gfx950 in-tree (hipcc cross-compiles without a GPU)."""
    csrc = os.path.join(_HERE, "csrc")
    if force:
        subprocess.run(["make", "-C", csrc, "clean"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(["make", "-C", csrc, f"-j{jobs}"], check=True)


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
        _lib = _abi.bind(ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL))
    return _lib


def check(status, what=""):
    if status != AF_OK:
        raise AfError(status, what)
    return status

"""ctypes binding of libwebyiq_q4q8.so (include/webyiq_q4q8.h).

The library is built in-tree by webyiq_amd.build (or __graft_entry__.build()).
There is no fallback: if the library is missing, loading raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwebyiq_q4q8.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "webyiq_q4q8.h")

WQ_OK = 0
WQ_EINVAL = -1
WQ_ESHAPE = -2
WQ_EALIGN = -3
WQ_EHIP = -4
WQ_EWORKSPACE = -5

MODE_STORE, MODE_ACCUMULATE, MODE_SILU_MUL = 0, 1, 2
PATH_DECODE, PATH_SPEC, PATH_PREFILL = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_LINEAR = [_P, _P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _I32, _I32, _P]

PROTOTYPES = {
    "wq_last_error": ([], ctypes.c_char_p),
    "wq_abi_version": ([], ctypes.c_int),
    "wq_quant_act": ([_P, _P, _P, _F, _I64, _I64, _I32, _I32, _P, _P, _P], ctypes.c_int),
    "wq_gemv": (_LINEAR, ctypes.c_int),
    "wq_quant_gemv": ([_P, _P, _P, _F, _P, _P, _I64, _I64, _I32, _I64, _I32, _P, _P, _P, _P], ctypes.c_int),
    "wq_gemm": (_LINEAR + [_P, _P, _SZ], ctypes.c_int),
    "wq_gemm_workspace_bytes": ([_I64, _I64, _I32, _I64, _I32, _I32], _SZ),
    "wq_gemv_debug_acc": (_LINEAR + [_P], ctypes.c_int),
    "wq_gemm_debug_acc": (_LINEAR + [_P], ctypes.c_int),
    "wq_matmul": ([_P, _I32] + _LINEAR[1:] + [_P], ctypes.c_int),
    "wq_argmax": ([_P, _P, _I64, _I64, _P, _P], ctypes.c_int),
    "wq_lm_head_argmax": ([_P, _P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _SZ],
                          ctypes.c_int),
    "wq_lm_head_argmax_noalloc": ([_P, _P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _I32, _P, _P, _P],
                                  ctypes.c_int),
    "wq_lm_head_noalloc_reset": ([_P], ctypes.c_int),
    "wq_lm_head_workspace_bytes": ([], _SZ),
    "wq_workspace_clear": ([_P, _P, _SZ], ctypes.c_int),
    "wq_embed": ([_P, _P, _P, _I64, _I64, _I32, _P, _I64, _P], ctypes.c_int),
    "wq_gather_rows": ([_P, _P, _P, _I64, _I64, _I32, _P, _I64, _P, _P], ctypes.c_int),
    "wq_mtp_in": ([_P, _P, _P, _P, _P, _P, _F, _I64, _I64, _P, _P, _P], ctypes.c_int),
    "wq_attn_combine": ([_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P], ctypes.c_int),
}


class WqError(RuntimeError):
    """A failed C-ABI call: .code is the WQ_E* status, the message is wq_last_error()."""

    def __init__(self, code, message):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


_lib = None


def _hip_runtimes():
    """Paths of the libamdhip64 images mapped into this process."""
    try:
        with open("/proc/self/maps") as f:
            return sorted({l.split()[-1] for l in f if "libamdhip64" in l})
    except OSError:
        return []


def load():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m webyiq_amd.build` "
                "(the int4 x int8 path has no CPU fallback)")
        # torch bundles its own libamdhip64.so (soname libamdhip64.so.7).  Loading
        # it first makes this library bind to that same runtime instance; loading
        # ours first would map /opt/rocm's copy too, and a second HIP runtime in
        # one process finds no device.
        import torch  # noqa: F401
        lib = ctypes.CDLL(LIB_PATH)
        runtimes = _hip_runtimes()
        if len(runtimes) > 1:
            raise RuntimeError(f"two HIP runtimes mapped in this process: {runtimes}")
        for name, (args, res) in PROTOTYPES.items():
            f = getattr(lib, name)
            f.argtypes = args
            f.restype = res
        _lib = lib
    return _lib


def check(rc):
    if rc != WQ_OK:
        raise WqError(rc, load().wq_last_error().decode())
    return rc


def call(name, *args):
    return check(getattr(load(), name)(*args))

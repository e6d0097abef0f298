"""ctypes binding of ``libfra.so`` (declared in ``include/fra.h``).

The library is loaded from the package directory.  There is no fallback:
when it is missing, every call raises, so a GPU run can never silently take
another path.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfra.so")

FRA_DTYPE_BF16 = 0
FRA_DTYPE_F16 = 1
FRA_DTYPE_F32 = 2

FRA_OK = 0
FRA_EINVAL = -1
FRA_EUNSUPPORTED = -2
FRA_EHIP = -3

FRA_KERNEL_NONE = 0
FRA_KERNEL_WINDOW = 1
FRA_KERNEL_LONG = 2

ABI_VERSION = 3


class FwdArgs(ctypes.Structure):
    """Mirror of ``struct fra_fwd_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("q_stride_seq", ctypes.c_int64),
        ("q_stride_head", ctypes.c_int64),
        ("k_stride_seq", ctypes.c_int64),
        ("k_stride_head", ctypes.c_int64),
        ("v_stride_seq", ctypes.c_int64),
        ("v_stride_head", ctypes.c_int64),
        ("out_stride_seq", ctypes.c_int64),
        ("out_stride_head", ctypes.c_int64),
        ("rope_stride_seq", ctypes.c_int64),
        ("total_seq", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_seqs", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("rope_width", ctypes.c_int32),
        ("qkv_dtype", ctypes.c_int32),
        ("rope_dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("flags", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
    ]


class BwdArgs(ctypes.Structure):
    """Mirror of ``struct fra_bwd_args``."""

    _fields_ = [(n, ctypes.c_void_p) for n in
                ("q", "k", "v", "cos", "sin", "out", "dout", "lse", "cu_seqlens", "dq", "dk", "dv")] + \
               [(f"{t}_stride_{ax}", ctypes.c_int64) for t in ("q", "k", "v", "out", "dout", "dq", "dk", "dv")
                for ax in ("seq", "head")] + \
               [("rope_stride_seq", ctypes.c_int64)] + \
               [(n, ctypes.c_int32) for n in ("total_seq", "num_heads", "head_dim", "num_seqs", "max_seqlen",
                                              "rope_width", "qkv_dtype", "rope_dtype")] + \
               [("softmax_scale", ctypes.c_float), ("flags", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64)]


class Plan(ctypes.Structure):
    """Mirror of ``struct fra_plan``."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("grid", ctypes.c_int32),
        ("block", ctypes.c_int32),
        ("block_q", ctypes.c_int32),
        ("block_kv", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("split_units", ctypes.c_int32),
        ("split_parts", ctypes.c_int32),
        ("name", ctypes.c_char * 64),
    ]


class RopePositions(ctypes.Structure):
    """Mirror of ``struct fra_rope_positions``."""

    _fields_ = [
        ("pos", ctypes.c_void_p),
        ("inv_freq", ctypes.c_void_p),
    ]


# Every symbol include/fra.h declares, with its ctypes signature.
SIGNATURES = {
    "fra_fwd_varlen": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "fra_fwd_varlen_static": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "fra_query_plan": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(Plan)]),
    "fra_fwd_varlen_pos": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(RopePositions), ctypes.c_void_p]),
    "fra_fwd_varlen_gather": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(RopePositions), ctypes.c_void_p,
                                             ctypes.c_void_p]),
    "fra_workspace_bytes_pos": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(RopePositions),
                                               ctypes.POINTER(ctypes.c_int64)]),
    "fra_query_plan_pos": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(RopePositions),
                                          ctypes.POINTER(Plan)]),
    "fra_workspace_bytes": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.POINTER(ctypes.c_int64)]),
    "fra_supports_head_dim": (ctypes.c_int, [ctypes.c_int32]),
    "fra_last_error": (ctypes.c_char_p, []),
    "fra_version": (ctypes.c_char_p, []),
    "fra_abi_version": (ctypes.c_int32, []),
    "fra_sizeof_args": (ctypes.c_int32, []),
    "fra_sizeof_plan": (ctypes.c_int32, []),
    "fra_bwd_varlen": (ctypes.c_int, [ctypes.POINTER(BwdArgs), ctypes.c_void_p]),
    "fra_bwd_query_plan": (ctypes.c_int, [ctypes.POINTER(BwdArgs), ctypes.POINTER(Plan)]),
    "fra_bwd_workspace_bytes": (ctypes.c_int, [ctypes.POINTER(BwdArgs), ctypes.POINTER(ctypes.c_int64)]),
    "fra_sizeof_bwd_args": (ctypes.c_int32, []),
}

_lib = None
_lock = threading.Lock()


class FraError(RuntimeError):
    """A failing status from libfra.so."""

    def __init__(self, code: int, message: str):
        super().__init__(f"libfra error {code}: {message}")
        self.code = code


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build it with `python -m fused_rope_attn_amd.build` "
                "(there is no fallback path)")
        # torch first: its HIP runtime (soname libamdhip64.so.7) is then the
        # one libfra.so binds to, so both share device contexts and streams.
        import torch  # noqa: F401
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.fra_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libfra ABI {lib.fra_abi_version()} != expected {ABI_VERSION}")
        if (lib.fra_sizeof_args() != ctypes.sizeof(FwdArgs) or lib.fra_sizeof_plan() != ctypes.sizeof(Plan)
                or lib.fra_sizeof_bwd_args() != ctypes.sizeof(BwdArgs)):
            raise RuntimeError("libfra struct layout does not match the ctypes mirror")
        _lib = lib
        return lib


def last_error() -> str:
    return load().fra_last_error().decode()


def check(code: int) -> None:
    if code != FRA_OK:
        raise FraError(code, last_error())

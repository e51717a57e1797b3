"""ctypes binding of ``libchia_attn.so`` (declared in include/chia_attn.h).

The shared library is loaded once, lazily, from the package directory.  There
is no fallback: if the library is missing the call raises, so a GPU run can
never silently take another code path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libchia_attn.so"

NORM_SOFTMAX = 0
NORM_SIGMOID = 1
NORM_RELU = 2
NORMS = {"softmax": NORM_SOFTMAX, "sigmoid": NORM_SIGMOID, "relu": NORM_RELU}

ABI_VERSION = 4

# Entry points declared in include/chia_attn.h (checked by the CPU tests).
EXPORTS = (
    "chia_attn_fwd",
    "chia_attn_fwd_lse",
    "chia_attn_fwd_fp8",
    "chia_attn_bwd",
    "chia_attn_bwd_noalloc",
    "chia_attn_bwd_workspace_size",
    "chia_attn_plan",
    "chia_attn_tile_map",
    "chia_attn_query_intervals",
    "chia_attn_status_string",
    "chia_attn_abi_version",
)

_i64x3 = ctypes.c_int64 * 3


class AttnArgs(ctypes.Structure):
    """Mirror of ``chia_attn_args``."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("norm", ctypes.c_uint32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", _i64x3),
        ("k_stride", _i64x3),
        ("v_stride", _i64x3),
        ("o_stride", _i64x3),
        ("causal", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("dilation", ctypes.c_int32),
        ("block", ctypes.c_int32),
        ("prefix", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("bias", ctypes.c_float),
        ("post_scale", ctypes.c_float),
        ("head_scale", ctypes.c_void_p),
        ("alibi_slopes", ctypes.c_void_p),
        ("kv_heads", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("cu_seqlens", ctypes.c_void_p),
        ("seq_order", ctypes.c_void_p),
        ("reserved", ctypes.c_int32 * 2),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(AttnArgs)
        self.dilation = 1
        self.post_scale = 1.0
        for key, val in kw.items():
            setattr(self, key, val)


class BwdArgs(ctypes.Structure):
    """Mirror of ``chia_attn_bwd_args``."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("reserved0", ctypes.c_uint32),
        ("fwd", ctypes.POINTER(AttnArgs)),
        ("dout", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("dout_stride", _i64x3),
        ("dq_stride", _i64x3),
        ("dk_stride", _i64x3),
        ("dv_stride", _i64x3),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("reserved", ctypes.c_int32 * 8),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(BwdArgs)
        for key, val in kw.items():
            setattr(self, key, val)


FP8_E4M3 = 0  # chia_attn_fp8_args.format: CHIA_ATTN_FP8_E4M3
FP8_E5M2 = 1  # CHIA_ATTN_FP8_E5M2


class Fp8Args(ctypes.Structure):
    """Mirror of ``chia_attn_fp8_args``."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("format", ctypes.c_uint32),
        ("attn", ctypes.POINTER(AttnArgs)),
        ("q_descale", ctypes.c_float),
        ("k_descale", ctypes.c_float),
        ("v_descale", ctypes.c_float),
        ("reserved", ctypes.c_int32 * 5),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(Fp8Args)
        self.q_descale = self.k_descale = self.v_descale = 1.0
        for key, val in kw.items():
            setattr(self, key, val)


class PlanInfo(ctypes.Structure):
    """Mirror of ``chia_attn_plan_info``."""

    _fields_ = [
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("wave_m", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("workgroups", ctypes.c_int64),
        ("tiles_total", ctypes.c_int64),
        ("tiles_visited", ctypes.c_int64),
        ("wave_tiles_visited", ctypes.c_int64),
        ("wave_tiles_partial", ctypes.c_int64),
        ("pairs_visible", ctypes.c_int64),
        ("residues", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 7),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_ if name != "reserved"}


class ChiaAttnError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: status {status}: {status_string(status)}")


_lib = None
_lock = threading.Lock()


def _load():
    global _lib
    if _lib is not None:  # loaded: no lock on the launch path
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built ({LIB_PATH}); run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python -m chia_proj_amd._build` first"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.chia_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p]
        lib.chia_attn_fwd.restype = ctypes.c_int
        lib.chia_attn_fwd_lse.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_void_p, ctypes.c_void_p]
        lib.chia_attn_fwd_lse.restype = ctypes.c_int
        lib.chia_attn_fwd_fp8.argtypes = [ctypes.POINTER(Fp8Args), ctypes.c_void_p]
        lib.chia_attn_fwd_fp8.restype = ctypes.c_int
        lib.chia_attn_bwd.argtypes = [ctypes.POINTER(BwdArgs), ctypes.c_void_p]
        lib.chia_attn_bwd.restype = ctypes.c_int
        lib.chia_attn_bwd_noalloc.argtypes = [ctypes.POINTER(BwdArgs), ctypes.c_void_p]
        lib.chia_attn_bwd_noalloc.restype = ctypes.c_int
        lib.chia_attn_bwd_workspace_size.argtypes = [ctypes.POINTER(AttnArgs)]
        lib.chia_attn_bwd_workspace_size.restype = ctypes.c_int64
        lib.chia_attn_plan.argtypes = [ctypes.POINTER(AttnArgs), ctypes.POINTER(PlanInfo)]
        lib.chia_attn_plan.restype = ctypes.c_int
        lib.chia_attn_tile_map.argtypes = [
            ctypes.POINTER(AttnArgs), ctypes.c_int32, ctypes.c_int32,
            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
            ctypes.c_void_p, ctypes.c_int64,
        ]
        lib.chia_attn_tile_map.restype = ctypes.c_int
        lib.chia_attn_query_intervals.argtypes = [
            ctypes.POINTER(AttnArgs), ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(ctypes.c_int32), ctypes.c_int64,
        ]
        lib.chia_attn_query_intervals.restype = ctypes.c_int
        lib.chia_attn_status_string.argtypes = [ctypes.c_int]
        lib.chia_attn_status_string.restype = ctypes.c_char_p
        lib.chia_attn_abi_version.argtypes = []
        lib.chia_attn_abi_version.restype = ctypes.c_int
        if lib.chia_attn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {lib.chia_attn_abi_version()} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def lib():
    return _load()


def status_string(status: int) -> str:
    return _load().chia_attn_status_string(int(status)).decode()


def fwd(args: AttnArgs, stream: int) -> None:
    st = _load().chia_attn_fwd(args, stream)  # argtypes pass the struct by reference
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_fwd")


def fwd_lse(args: AttnArgs, lse_ptr: int, stream: int) -> None:
    st = _load().chia_attn_fwd_lse(ctypes.byref(args), ctypes.c_void_p(lse_ptr), ctypes.c_void_p(stream))
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_fwd_lse")


def fwd_fp8(args: Fp8Args, stream: int) -> None:
    st = _load().chia_attn_fwd_fp8(args, stream)  # argtypes pass the struct by reference
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_fwd_fp8")


def bwd_workspace_size(args: AttnArgs) -> int:
    n = _load().chia_attn_bwd_workspace_size(ctypes.byref(args))
    if n < 0:
        raise ChiaAttnError(int(n), "chia_attn_bwd_workspace_size")
    return int(n)


def bwd(args: BwdArgs, stream: int) -> None:
    st = _load().chia_attn_bwd(ctypes.byref(args), ctypes.c_void_p(stream))
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_bwd")


def bwd_noalloc(args: BwdArgs, stream: int) -> None:
    """chia_attn_bwd without the workspace: the row statistics go to the library's
    static per-GPU scratch (calls on one GPU must not overlap)."""
    st = _load().chia_attn_bwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream))
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_bwd_noalloc")


def plan(args: AttnArgs) -> dict:
    info = PlanInfo()
    st = _load().chia_attn_plan(ctypes.byref(args), ctypes.byref(info))
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_plan")
    return info.as_dict()


def tile_map(args: AttnArgs, residue: int, rows_per_block: int):
    import numpy as np

    n_qb = ctypes.c_int32()
    n_kt = ctypes.c_int32()
    lib_ = _load()
    st = lib_.chia_attn_tile_map(ctypes.byref(args), residue, rows_per_block, ctypes.byref(n_qb),
                                 ctypes.byref(n_kt), None, 0)
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_tile_map")
    out = np.zeros((n_qb.value, n_kt.value), dtype=np.int8)
    st = lib_.chia_attn_tile_map(ctypes.byref(args), residue, rows_per_block, ctypes.byref(n_qb),
                                 ctypes.byref(n_kt), out.ctypes.data, out.size)
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_tile_map")
    return out


def query_intervals(args: AttnArgs, residue: int, length: int):
    import numpy as np

    jlo = np.zeros(max(length, 1), dtype=np.int32)
    jhi = np.zeros(max(length, 1), dtype=np.int32)
    pre = ctypes.c_int32()
    st = _load().chia_attn_query_intervals(ctypes.byref(args), residue, jlo.ctypes.data, jhi.ctypes.data,
                                           ctypes.byref(pre), jlo.size)
    if st != 0:
        raise ChiaAttnError(st, "chia_attn_query_intervals")
    return jlo[:length], jhi[:length], pre.value

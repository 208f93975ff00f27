"""ctypes binding of librmoe.so (the C ABI declared in include/rmoe.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
runnel_amd/csrc``).  There is no fallback: if the shared library is missing
every entry point raises, so a GPU run can never silently take another path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librmoe.so"

RMOE_OK = 0
RMOE_EINVAL = -1
RMOE_EBITS = -2
RMOE_EALIGN = -3
RMOE_EWS = -4
RMOE_EHIP = -5
RMOE_ENULL = -6
RMOE_ETIMEOUT = -7
RMOE_EPLACEMENT = -8

ABI_VERSION = 5

EXPORTED = (
    "rmoe_abi_version", "rmoe_last_error", "rmoe_status_string",
    "rmoe_validate_layer", "rmoe_workspace_bytes", "rmoe_router",
    "rmoe_switch_glu", "rmoe_switch_workspace_bytes", "rmoe_gather_qmm",
    "rmoe_moe_block", "rmoe_quantize", "rmoe_dequantize", "rmoe_stream_read",
    "rmoe_router_workspace_bytes", "rmoe_chain_table_bytes", "rmoe_chain_table_pack",
    "rmoe_moe_chain", "rmoe_workspace_status_offset", "rmoe_router_q",
    "rmoe_switch_combine", "rmoe_switch_combine_workspace_bytes", "rmoe_rms_norm",
    "rmoe_set_cooperative_launch", "rmoe_moe_block_noalloc",
)

# rmoe_moe_block_noalloc's static scratch per GPU (RMOE_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 16 << 20


class RmoeError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


class QWeight(ctypes.Structure):
    """rmoe_qweight"""
    _fields_ = [
        ("w", ctypes.c_void_p), ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p), ("experts", ctypes.c_int32),
        ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
        ("bits", ctypes.c_int32), ("group_size", ctypes.c_int32),
    ]


class Layer(ctypes.Structure):
    """rmoe_layer"""
    _fields_ = [
        ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32), ("experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32), ("norm_topk_prob", ctypes.c_int32),
        ("router_w", ctypes.c_void_p), ("shared_gate_w", ctypes.c_void_p),
        ("gate_up", QWeight), ("down", QWeight),
        ("shared_gate_up", QWeight), ("shared_down", QWeight),
        ("router_q", QWeight), ("shared_gate_q", QWeight),
        ("post_norm_w", ctypes.c_void_p), ("norm_eps", ctypes.c_float),
    ]


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load librmoe.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import "
                "__graft_entry__ as g; g.build()'` or `make -C runnel_amd/csrc`")
        lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I32 = ctypes.c_int32
        I64 = ctypes.c_int64
        SZ = ctypes.c_size_t
        LP = ctypes.POINTER(Layer)
        QP = ctypes.POINTER(QWeight)
        lib.rmoe_abi_version.restype = ctypes.c_int
        lib.rmoe_abi_version.argtypes = []
        lib.rmoe_last_error.restype = ctypes.c_char_p
        lib.rmoe_last_error.argtypes = []
        lib.rmoe_status_string.restype = ctypes.c_char_p
        lib.rmoe_status_string.argtypes = [ctypes.c_int]
        lib.rmoe_validate_layer.argtypes = [LP]
        lib.rmoe_workspace_bytes.restype = SZ
        lib.rmoe_workspace_bytes.argtypes = [LP, I32]
        lib.rmoe_switch_workspace_bytes.restype = SZ
        lib.rmoe_switch_workspace_bytes.argtypes = [QP, QP, I32, I32]
        lib.rmoe_router.argtypes = [P, I32, I32, I32, I32, P, I32, P, P, P, SZ, P]
        lib.rmoe_router_q.argtypes = [QP, I32, I32, P, I32, P, P, P, SZ, P]
        lib.rmoe_rms_norm.argtypes = [P, P, I32, I32, ctypes.c_float, P, P]
        lib.rmoe_router_workspace_bytes.restype = SZ
        lib.rmoe_router_workspace_bytes.argtypes = [I32, I32, I32]
        lib.rmoe_switch_glu.argtypes = [QP, QP, P, I32, P, I32, P, P, SZ, P]
        lib.rmoe_switch_combine.argtypes = [QP, QP, P, I32, P, P, I32, P, P, P, SZ, P]
        lib.rmoe_switch_combine_workspace_bytes.restype = SZ
        lib.rmoe_switch_combine_workspace_bytes.argtypes = [QP, QP, I32, I32]
        lib.rmoe_gather_qmm.argtypes = [P, I32, P, P, I32, QP, P, P, P]
        lib.rmoe_moe_block.argtypes = [LP, P, I32, P, P, P, P, P, SZ, P]
        lib.rmoe_moe_block_noalloc.argtypes = [LP, P, I32, P, P, P, P, P, P]
        lib.rmoe_quantize.argtypes = [P, I64, I32, I32, I32, P, P, P, P]
        lib.rmoe_dequantize.argtypes = [QP, I64, I64, P, P, P]
        lib.rmoe_stream_read.argtypes = [P, SZ, P, I32, P]
        lib.rmoe_chain_table_bytes.restype = SZ
        lib.rmoe_chain_table_bytes.argtypes = [I32]
        lib.rmoe_chain_table_pack.argtypes = [LP, I32, P]
        lib.rmoe_moe_chain.argtypes = [LP, P, I32, P, P, P, SZ, P]
        lib.rmoe_workspace_status_offset.restype = SZ
        lib.rmoe_workspace_status_offset.argtypes = []
        lib.rmoe_set_cooperative_launch.argtypes = [I32]
        for name in EXPORTED:
            if name not in ("rmoe_last_error", "rmoe_status_string",
                            "rmoe_workspace_bytes", "rmoe_switch_workspace_bytes",
                            "rmoe_switch_combine_workspace_bytes",
                            "rmoe_router_workspace_bytes", "rmoe_chain_table_bytes",
                            "rmoe_workspace_status_offset"):
                getattr(lib, name).restype = ctypes.c_int
        if lib.rmoe_abi_version() != ABI_VERSION:
            raise RuntimeError("librmoe.so ABI version mismatch; rebuild it")
        _lib = lib
        return lib


def check(status: int) -> None:
    if status != RMOE_OK:
        lib = load()
        msg = lib.rmoe_last_error().decode() or lib.rmoe_status_string(status).decode()
        if status in (RMOE_EINVAL, RMOE_EBITS, RMOE_EALIGN, RMOE_ENULL, RMOE_EWS):
            raise ValueError(f"{msg} (status {status})")
        raise RmoeError(status, msg)


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor, None for None."""
    return None if t is None else t.data_ptr()


def stream_handle(device=None) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream

"""ctypes view of include/voidinfer_sampling.h (the C ABI of libvoidinfer_sampling.so).

Struct layouts are mirrored twice: as numpy dtypes (for building device arrays of
parameters / reading outputs) and as ctypes structures (for by-pointer host
arguments).  ``load()`` raises ImportError when the built library is missing, so
no caller can silently fall back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

import os

# VOIDINFER_AMD_LIB selects another build of the same library (e.g. an instrumented one).
LIB_PATH = Path(os.environ.get("VOIDINFER_AMD_LIB", Path(__file__).resolve().parent / "libvoidinfer_sampling.so"))

BF16, F16, F32 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH, ERR_DEVICE = range(6)
FLAG_NONFINITE, FLAG_EMPTY, FLAG_ZERO_Q, FLAG_NO_RESIDUAL, FLAG_BAD_HISTORY = 1, 2, 4, 8, 16
FLAG_ERROR = 0x80000000
VERIFY_GREEDY, VERIFY_SAMPLED, VERIFY_SAMPLED_TOPK = 0, 1, 2
ROUTE_TOPK, ROUTE_FULL, ROUTE_ALL = 1, 2, 3
ABSENT_OCCURRENCE = 0x7F7F7F7F

GREEDY_ROW = np.dtype([("serial", "<u8"), ("token", "<i4"), ("nonfinite", "<u4")])
ROW_PARAMS = np.dtype([
    ("temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"),
    ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"), ("frequency_penalty", "<f4"),
    ("top_k", "<i4"), ("lane", "<u4"), ("seed", "<u8"), ("position", "<i4"), ("reserved", "<u4"),
])
SAMPLE_STATS = np.dtype([
    ("flags", "<u4"), ("support", "<u4"), ("finite", "<u4"), ("reserved", "<u4"),
    ("support_mass", "<f8"), ("uniform", "<f8"),
])
assert GREEDY_ROW.itemsize == 16 and ROW_PARAMS.itemsize == 48 and SAMPLE_STATS.itemsize == 32


DRAFT_SAMPLING = np.dtype([   # vi_draft_sampling == DraftSelectSampling (dflash2_draft.cu:2562-2572)
    ("inv_temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"), ("top_k", "<i4"), ("seed", "<u8"),
    ("key_base", "<i4"), ("reserved", "<i4"), ("presence_penalty", "<f4"), ("reserved2", "<i4"),
    ("first_occurrence", "<u8"),
])
assert DRAFT_SAMPLING.itemsize == 48


class DeviceSampling(C.Structure):
    """vi_device_sampling == Exl3DeviceSampling (src/exl3/sampled_select.h:17-28)."""
    _fields_ = [
        ("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
        ("seed", C.c_uint64), ("presence_penalty", C.c_float), ("reserved", C.c_int32),
        ("first_occurrence", C.c_void_p),
    ]


assert C.sizeof(DeviceSampling) == 40

_vp, _i, _i64, _u64, _sz, _u32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_size_t, C.c_uint32

SIGNATURES = {
    "vi_init": ([], _i),
    "vi_status_string": ([_i], C.c_char_p),
    "vi_abi_version": ([], _u32),
    "vi_greedy_workspace_bytes": ([_i, _i], _sz),
    "vi_greedy_rows": ([_vp, _i, _i, _i, _i64, _u64, _vp, _vp, _sz, _vp], _i),
    "vi_greedy_rows_noalloc": ([_vp, _i, _i, _i, _i64, _u64, _vp, _vp], _i),
    "vi_topk_workspace_bytes": ([_i, _i, _i], _sz),
    "vi_topk_rows": ([_vp, _i, _i, _i, _i64, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp], _i),
    "vi_topk16_for_test": ([_vp, _i, _i, _vp, _vp, _vp, _vp], _i),
    "vi_sampled_packet_workspace_bytes": ([_i, _i], _sz),
    "vi_sampled_packet": ([_vp, _i, _i, _i, _i64, C.POINTER(DeviceSampling), _i, _vp, _i, _vp, _i, _u64,
                           _vp, _vp, _sz, _vp], _i),
    "vi_row_scores_workspace_bytes": ([_i, _i], _sz),
    "vi_row_scores": ([_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _vp, _sz, _vp], _i),
    "vi_sampled_scores_workspace_bytes": ([_i, _i], _sz),
    "vi_sampled_scores": ([_vp, _i, _i, _i, _i64, C.POINTER(DeviceSampling), _i, C.c_float, _vp, _vp, _vp, _vp,
                           _sz, _vp], _i),
    "vi_draft_choice": ([_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "vi_selector_chain": ([_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "vi_build_verification_tree": ([_vp, _i, _vp, _vp, _i, _i, C.c_float, _vp, _vp, _vp, _vp], _i),
    "vi_penalty_state_bytes": ([_i, _i], _sz),
    "vi_penalty_state_reset": ([_vp, _i, _i, _i, _vp], _i),
    "vi_penalty_state_update": ([_vp, _i, _i, _i, _vp, _vp, _i, _vp], _i),
    "vi_sample_rows_state": ([_vp, _i, _i, _i, _i64, _vp, _vp, _i, _i, _vp, _vp, _vp, _i64, _vp, _u32, _vp, _sz,
                              _vp], _i),
    "vi_packet_transport_create": ([_i, _i, C.POINTER(C.c_void_p)], _i),
    "vi_packet_transport_destroy": ([_vp], _i),
    "vi_packet_submit": ([_vp, _vp, _i, _vp, C.POINTER(C.c_int)], _i),
    "vi_packet_query": ([_vp, _i, C.POINTER(C.c_int)], _i),
    "vi_packet_finish": ([_vp, _i, _vp, _i], _i),
    "vi_presence_reset": ([_vp, _i, _vp], _i),
    "vi_presence_truncate": ([_vp, _i, _i, _vp], _i),
    "vi_presence_record": ([_vp, _i, _i, _vp, _sz, _vp], _i),
    "vi_sample_workspace_bytes": ([_i, _i, _i64], _sz),
    "vi_sample_rows": ([_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _u32, _vp, _sz,
                        _vp], _i),
    "vi_verify_workspace_bytes": ([_i, _i, _i], _sz),
    "vi_verify_rows": ([_i, _vp, _i, _i64, _i, _vp, _i, _i64, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                        _vp, _sz, _vp], _i),
    "vi_probe_read": ([_vp, _sz, _vp, _vp], _i),
    "vi_probe_copy": ([_vp, _vp, _sz, _vp], _i),
}

_lib = None


def load() -> C.CDLL:
    """Load the in-tree library (ImportError if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python voidinfer_amd/build.py` "
                "(there is no CPU fallback)")
        lib = C.CDLL(str(LIB_PATH))
        for name, (args, res) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as e:
                raise ImportError(f"{LIB_PATH} lacks {name}: it is older than its sources, rebuild it with "
                                  "`python voidinfer_amd/build.py`") from e
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


class VIError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = load().vi_status_string(status).decode()
        super().__init__(f"{what}: {msg} (status {status})")


def check(status: int, what: str) -> None:
    if status != OK:
        if status == ERR_INVALID:
            raise ValueError(f"{what}: invalid argument")
        raise VIError(status, what)

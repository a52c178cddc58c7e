"""ctypes binding of libfsamp.so (the C ABI in include/fsamp.h).

The library is loaded from this package directory; there is no fallback: a missing or
unloadable library raises, so nothing can silently run another implementation.
"""

from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libfsamp.so")

DTYPE_F16 = 0
DTYPE_BF16 = 1
K_MAX = 1024

# every function the header declares, with (restype, argtypes)
_vp, _i32, _i64, _u64, _dbl, _sz = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                    ctypes.c_uint64, ctypes.c_double, ctypes.c_size_t)


class Plan(ctypes.Structure):
    _fields_ = [("batch", _i64), ("vocab", _i64), ("k", _i64), ("splits", _i32),
                ("slice", _i32), ("threads", _i32), ("chunks", _i32), ("vec", _i32),
                ("reserved", _i32), ("workspace_bytes", _sz)]


class RowParams(ctypes.Structure):
    """fsamp_row_params: per-row controls and the graph-safe offset counter (device pointers)."""
    _fields_ = [("top_k", _vp), ("top_p", _vp), ("temperature", _vp), ("offset_counter", _vp)]


class Call(ctypes.Structure):
    """fsamp_call (include/fsamp.h), field for field."""
    _fields_ = [("struct_bytes", _sz), ("logits", _vp), ("dtype", _i32),
                ("threads_override", _i32), ("batch", _i64), ("vocab", _i64), ("ld", _i64),
                ("top_k", _i64), ("top_p", _dbl), ("splits_override", _i64), ("u", _vp),
                ("seed", _u64), ("offset", _u64), ("seed_ptr", _vp), ("offset_ptr", _vp),
                ("top_k_row", _vp), ("top_p_row", _vp), ("temperature_row", _vp),
                ("out", _vp), ("keep", _vp), ("renormed", _vp), ("ids", _vp), ("words", _vp),
                ("id_offset", _i64), ("counters", _vp), ("counter_bytes", _sz),
                ("scratch", _vp), ("scratch_bytes", _sz)]

    def __init__(self, **kw):
        super().__init__(struct_bytes=ctypes.sizeof(Call), **kw)


class AttrRow(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("threads", _i32), ("chunks", _i32),
                ("vgprs", _i32), ("scratch_bytes", _i32), ("lds_bytes", _i32),
                ("blocks_per_cu", _i32)]


SIGNATURES = {
    "fsamp_error_string": (ctypes.c_char_p, [_i32]),
    "fsamp_make_plan": (_i32, [_vp, _i64, _i64, _i64, _i64, ctypes.POINTER(Plan)]),
    "fsamp_workspace_bytes": (_sz, [_vp, _i64, _i64, _i64, _i64]),
    "fsamp_workspace_init": (_i32, [_vp, _sz, _vp]),
    "fsamp_sample": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _u64, _u64, _vp, _vp, _sz,
                            _i64, _vp]),
    "fsamp_stages": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _u64, _u64, _vp, _vp, _vp,
                            _vp, _sz, _i64, _vp]),
    "fsamp_sample_ex": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _u64, _u64,
                               ctypes.POINTER(RowParams), _vp, _vp, _vp, _vp, _sz, _i64, _vp]),
    "fsamp_topk": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _sz, _i64, _vp]),
    "fsamp_probe_phase": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _i64, _vp, _vp, _sz, _i64,
                                 _vp]),
    "fsamp_probe_noop": (_i32, [_i64, _vp, _vp]),
    "fsamp_probe_scan_rowblock": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp]),
    "fsamp_probe_scan_split": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "fsamp_probe_load": (_i32, [_vp, _i32, _i64, _i64, _vp, _vp]),
    "fsamp_probe_stream_words": (_i64, [_i64, _i64]),
    "fsamp_probe_stream": (_i32, [_vp, _i32, _i64, _i64, _vp, _i64, _vp]),
    "fsamp_kernel_attrs": (_i32, [ctypes.POINTER(AttrRow), _i32, ctypes.POINTER(_i32)]),
    "fsamp_counter_bytes": (_sz, [_i64]),
    "fsamp_scratch_bytes": (_sz, [_vp, _i64, _i64, _i64, _i64]),
    "fsamp_run": (_i32, [ctypes.c_void_p, _vp]),
    "fsamp_sample_noalloc": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _u64, _u64, _vp,
                                    _i64, _vp]),
    "fsamp_topk_shard": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _sz, _vp, _sz,
                                _i64, _vp]),
    "fsamp_merge_sample": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _u64, _u64, _vp, _vp,
                                  _vp, _vp, _vp]),
    "fsamp_debug_wave_selftest": (_i32, [_vp, _vp]),
    "fsamp_debug_sample_traced": (_i32, [_vp, _i32, _i64, _i64, _i64, _dbl, _vp, _vp, _vp, _sz,
                                         _i64, _vp, _vp]),
}

_lib = None


def load():
    """Load libfsamp.so and declare every entry point; raises if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python -m llm_sampling_kernel_amd.build` "
                "(the sampler has no non-HIP fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class FsampError(RuntimeError):
    def __init__(self, status: int):
        self.status = status
        super().__init__(load().fsamp_error_string(status).decode())


def check(status: int) -> None:
    if status != 0:
        raise FsampError(status)

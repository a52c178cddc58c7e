"""ctypes front end of the CPU oracle in fsamp_oracle.c.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package.  The oracle restates
benchmarks/reference.py:29-81 (stable sort -> top-k -> softmax -> cumsum -> exclusive-prefix
cut -> renorm -> draw) with an explicit per-row uniform ``u`` in place of torch.multinomial.
Inputs are numpy arrays of raw 16-bit patterns (dtype "float16" / "bfloat16") or float32.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

DTYPES = {"float16": 0, "bfloat16": 1, "float32": 2}
ERRORS = {1: "logits contain NaN", 2: "logits contain +inf",
          3: "logits contain a row that is entirely -inf"}

_lib = None


def build() -> None:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run oracle.build() or make -C oracle")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, dbl, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int
        L.oracle_sample.argtypes = [vp, i32, i64, i64, i64, dbl, vp, vp, vp, vp, vp, vp, vp, vp,
                                    vp, i32]
        L.oracle_sample.restype = i32
        L.oracle_sample_rows.argtypes = [vp, i32, i64, i64, i64, dbl, vp, vp, vp, vp, vp, vp, vp,
                                         vp, vp, vp, vp, vp, i32]
        L.oracle_sample_rows.restype = i32
        L.oracle_sample_fullsort.argtypes = [vp, i32, i64, i64, i64, dbl, vp, vp, vp, i32]
        L.oracle_sample_fullsort.restype = i32
        L.oracle_stages_f64.argtypes = [vp, i32, i64, i64, i64, dbl, vp, vp, vp, vp]
        L.oracle_stages_f64.restype = i32
        L.oracle_stages_f64_t.argtypes = [vp, i32, i64, i64, i64, dbl, dbl, vp, vp, vp, vp]
        L.oracle_stages_f64_t.restype = i32
        L.oracle_validate.argtypes = [vp, i32, i64, i64]
        L.oracle_validate.restype = i32
        L.oracle_expf_array.argtypes = [vp, vp, i64]
        L.oracle_key16_array.argtypes = [vp, vp, i64]
        L.oracle_rng_uniform_rows.argtypes = [ctypes.c_uint64, ctypes.c_uint64, i64, vp]
        L.oracle_splitmix64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.oracle_splitmix64_next.restype = ctypes.c_uint64
        L.oracle_to_float.argtypes = [ctypes.c_uint16, i32]
        L.oracle_to_float.restype = ctypes.c_float
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _logits(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype not in DTYPES:
        raise ValueError(f"unknown dtype {dtype}")
    want = np.float32 if dtype == "float32" else np.uint16
    x = np.ascontiguousarray(x)
    if x.dtype != want:
        raise TypeError(f"{dtype} logits must be passed as {np.dtype(want).name} bit patterns")
    if x.ndim != 2:
        raise ValueError(f"logits must be [B, V], got shape {tuple(x.shape)}")
    return x


@dataclass(frozen=True)
class Stages:
    """Per-rank stage outputs, mirroring benchmarks/reference.py:8-17 (arrays, not tensors)."""

    topk_ids: np.ndarray   # [B,K] int64, descending value, ties by ascending id
    topk_vals: np.ndarray  # [B,K] float32
    probs: np.ndarray      # [B,K] float32 softmax over the K survivors
    cumsum: np.ndarray     # [B,K] float32 inclusive prefix of probs
    keep: np.ndarray       # [B,K] bool
    cutoff: np.ndarray     # [B] int32, number of kept ranks
    renormed: np.ndarray   # [B,K] float32, probs / Z_p on kept ranks, 0 elsewhere
    token_ids: np.ndarray  # [B] int64


def validate(x: np.ndarray, dtype: str) -> None:
    """reference.py:20-26: raise ValueError on NaN, +inf or an all -inf row."""
    x = _logits(x, dtype)
    rc = lib().oracle_validate(_ptr(x), DTYPES[dtype], x.shape[0], x.shape[1])
    if rc in ERRORS:
        raise ValueError(ERRORS[rc])
    if rc != 0:
        raise ValueError(f"oracle_validate failed ({rc})")


def sample(x: np.ndarray, dtype: str, top_k: int, top_p: float, u: np.ndarray, *,
           check_inputs: bool = True, return_stages: bool = False, nthreads: int = 1,
           top_k_row=None, top_p_row=None, temperature=None):
    """The restated sampler: [B,V] logits + u[B] -> token ids [B] (or Stages).

    top_k_row (int32 [B]), top_p_row (float32 [B]) and temperature (float32 [B]) are the
    per-row controls of fsamp_sample_ex (oracle_sample_rows)."""
    x = _logits(x, dtype)
    if top_k < 1:
        raise ValueError(f"top_k must be >= 1, got {top_k}")
    if not 0.0 < top_p <= 1.0:
        raise ValueError(f"top_p must be in (0, 1], got {top_p}")
    if check_inputs:
        validate(x, dtype)
    B, V = x.shape
    K = min(int(top_k), V)
    u = np.ascontiguousarray(u, dtype=np.float32).reshape(B)
    tok = np.empty(B, np.int64)
    if return_stages:
        ids = np.empty((B, K), np.int64)
        vals, probs, cum, ren = (np.empty((B, K), np.float32) for _ in range(4))
        keep = np.empty((B, K), np.uint8)
        cutoff = np.empty(B, np.int32)
    else:
        ids = vals = probs = cum = ren = keep = cutoff = None
    rows = [None if a is None else np.ascontiguousarray(a, dtype=t).reshape(B)
            for a, t in ((top_k_row, np.int32), (top_p_row, np.float32),
                         (temperature, np.float32))]
    rc = lib().oracle_sample_rows(_ptr(x), DTYPES[dtype], B, V, int(top_k), float(top_p),
                                  _ptr(u), _ptr(rows[0]), _ptr(rows[1]), _ptr(rows[2]),
                                  _ptr(tok), _ptr(ids), _ptr(vals), _ptr(probs), _ptr(cum),
                                  _ptr(keep), _ptr(ren), _ptr(cutoff), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle_sample failed ({rc})")
    if not return_stages:
        return tok
    return Stages(ids, vals, probs, cum, keep.astype(bool), cutoff, ren, tok)


def sample_fullsort(x: np.ndarray, dtype: str, top_k: int, top_p: float, u: np.ndarray, *,
                    nthreads: int = 1):
    """sample() with the selection in the reference's own form (reference.py:48-54): each row
    converted to fp32 and fully sorted by a stable merge sort, O(V log V), instead of the
    counting sort.  Returns (token_ids [B], topk_ids [B,K]); no input validation."""
    x = _logits(x, dtype)
    if top_k < 1 or not 0.0 < top_p <= 1.0:
        raise ValueError("top_k must be >= 1 and top_p in (0, 1]")
    B, V = x.shape
    K = min(int(top_k), V)
    u = np.ascontiguousarray(u, dtype=np.float32).reshape(B)
    tok = np.empty(B, np.int64)
    ids = np.empty((B, K), np.int64)
    rc = lib().oracle_sample_fullsort(_ptr(x), DTYPES[dtype], B, V, int(top_k), float(top_p),
                                      _ptr(u), _ptr(tok), _ptr(ids), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle_sample_fullsort failed ({rc})")
    return tok, ids


def stages_f64(x: np.ndarray, dtype: str, top_k: int, top_p: float, temperature: float = 1.0):
    """fp64 restatement of softmax/cumsum/cut/renorm over the same top-k candidates, with the
    softmax taken over (x - max) / temperature.

    Returns (probs, cumsum, renormed, cutoff) as float64 [B,K] arrays and int32 [B].
    """
    x = _logits(x, dtype)
    B, V = x.shape
    K = min(int(top_k), V)
    probs, cum, ren = (np.empty((B, K), np.float64) for _ in range(3))
    cutoff = np.empty(B, np.int32)
    rc = lib().oracle_stages_f64_t(_ptr(x), DTYPES[dtype], B, V, int(top_k), float(top_p),
                                   float(temperature), _ptr(probs), _ptr(cum), _ptr(ren),
                                   _ptr(cutoff))
    if rc != 0:
        raise RuntimeError(f"oracle_stages_f64 failed ({rc})")
    return probs, cum, ren, cutoff


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_expf_array(_ptr(x), _ptr(y), x.size)
    return y


def key16(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    k = np.empty(b.shape, np.uint32)
    lib().oracle_key16_array(_ptr(b), _ptr(k), b.size)
    return k


def rng_uniform(seed: int, offset: int, rows: int) -> np.ndarray:
    """Per-row uniforms of the (seed, offset) API (csrc/fused_sampling.cuh:65-71)."""
    u = np.empty(rows, np.float32)
    lib().oracle_rng_uniform_rows(ctypes.c_uint64(seed & (2**64 - 1)),
                                  ctypes.c_uint64(offset & (2**64 - 1)), rows, _ptr(u))
    return u


def splitmix64_sequence(seed: int, n: int) -> list[int]:
    st = ctypes.c_uint64(seed)
    return [int(lib().oracle_splitmix64_next(ctypes.byref(st))) for _ in range(n)]


def to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Decode 16-bit patterns to float32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    if dtype == "bfloat16":
        return (b.astype(np.uint32) << 16).view(np.float32)
    if dtype == "float16":
        return b.view(np.float16).astype(np.float32)
    raise ValueError(dtype)

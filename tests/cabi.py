"""Helpers for tests that call libfsamp.so's C ABI directly (ctypes), beside the torch module.

Every helper allocates its own device buffers with torch and passes raw pointers and torch's
current HIP stream, the way a C caller of include/fsamp.h would.
"""

from __future__ import annotations

import ctypes

import torch

from llm_sampling_kernel_amd import _lib


def stream_ptr(device=None) -> int:
    idx = torch.cuda.current_device() if device is None else torch.device(device).index or 0
    return torch.cuda.current_stream(idx).cuda_stream


def vp(t) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dtype_code(x: torch.Tensor) -> int:
    return _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F16


def classic_workspace(x: torch.Tensor, top_k: int, splits: int = 0):
    """A zeroed single-buffer workspace of fsamp_workspace_bytes() for this call."""
    B, V = x.shape
    n = _lib.load().fsamp_workspace_bytes(vp(x), B, V, top_k, splits)
    assert n > 0
    return torch.zeros(n, dtype=torch.uint8, device=x.device)


def split_workspace(x: torch.Tensor, B: int, V: int, top_k: int, splits: int = 0,
                    any_plan: bool = False):
    """(counters, scratch) for fsamp_run: zeroed counters, uninitialised scratch.  any_plan
    sizes the scratch for any split count (at most 16), as a forced workgroup size may need."""
    lib = _lib.load()
    cb = lib.fsamp_counter_bytes(B)
    sb = lib.fsamp_scratch_bytes(vp(x), B, V, top_k, splits)
    if any_plan:
        sb = max(sb, B * 16 * min(top_k, V) * 8)
    counters = torch.zeros(max(cb, 1), dtype=torch.uint8, device=x.device)
    scratch = torch.empty(max(sb, 1), dtype=torch.uint8, device=x.device)
    return counters, cb, scratch, sb


def run(x: torch.Tensor, top_k: int, top_p: float, *, u=None, seed=0, offset=0, seed_ptr=None,
        offset_ptr=None, splits=0, threads=0, stages=False, ids=False, ld=None, vocab=None,
        counters=None):
    """fsamp_run on [B, vocab] logits at x (row stride ld).  Returns token ids (or
    [ids, keep, renormed] with stages, or the [B, k] candidate ids with ids=True) as tensors."""
    lib = _lib.load()
    B = x.shape[0]
    V = x.shape[1] if vocab is None else vocab
    K = min(top_k, V)
    cnt, cb, scr, sb = split_workspace(x, B, V, top_k, splits, any_plan=threads != 0)
    if counters is not None:
        cnt, cb = counters, counters.numel()
    c = _lib.Call(logits=x.data_ptr(), dtype=dtype_code(x), threads_override=threads, batch=B,
                  vocab=V, ld=0 if ld is None else ld, top_k=top_k, top_p=top_p,
                  splits_override=splits, seed=seed & (2**64 - 1), offset=offset & (2**64 - 1),
                  counters=cnt.data_ptr(), counter_bytes=cb, scratch=scr.data_ptr(),
                  scratch_bytes=sb)
    if u is not None:
        c.u = u.data_ptr()
    if seed_ptr is not None:
        c.seed_ptr = seed_ptr.data_ptr()
    if offset_ptr is not None:
        c.offset_ptr = offset_ptr.data_ptr()
    if ids:
        out = torch.empty((B, K), dtype=torch.int64, device=x.device)
        c.ids = out.data_ptr()
    else:
        out = torch.empty(B, dtype=torch.int64, device=x.device)
        c.out = out.data_ptr()
    keep = ren = None
    if stages:
        keep = torch.empty((B, K), dtype=torch.bool, device=x.device)
        ren = torch.empty((B, K), dtype=torch.float32, device=x.device)
        c.keep, c.renormed = keep.data_ptr(), ren.data_ptr()
    _lib.check(lib.fsamp_run(ctypes.byref(c), ctypes.c_void_p(stream_ptr(x.device))))
    torch.cuda.synchronize()
    return [out, keep, ren] if stages else out

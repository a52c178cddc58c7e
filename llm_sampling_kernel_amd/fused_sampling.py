"""Torch-facing mirror of the reference's extension module ``fused_sampling``.

Same function names, argument order and meaning as csrc/bindings.cpp:16-25, the same
``RuntimeError`` messages for the checks the reference makes (csrc/fused_sampling.cu:341-357,
:422-424), plus ``sample_fused_u`` for the explicit per-row uniform the C ABI takes.  Every call
forwards device pointers and torch's current HIP stream to libfsamp.so (include/fsamp.h);
there is no other implementation behind these functions.

Deliberate differences from the reference:
  - top_k may be up to 1024 (reference: 128), so the "top_k must be <= ..." message names 1024;
  - ``offset < 0`` (torch-generator path, csrc/fused_sampling.cu:441-447) takes the seed and
    offset from torch's default generator of the logits' device on the host and advances that
    generator's offset by 4 per call, as the reference's philox_cuda_state(4) does; the device
    stream is splitmix64(seed, offset, row) like the explicit-offset path.  Under HIP-graph
    capture this path raises: pass an explicit offset or ``u`` there.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_WORKSPACES: dict = {}


def _stream_ptr(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    try:
        return torch._C._cuda_getCurrentRawStream(idx)
    except AttributeError:  # pragma: no cover - older torch
        return torch.cuda.current_stream(idx).cuda_stream


def _check_logits(logits: torch.Tensor) -> int:
    if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dim() == 2
            and logits.is_contiguous()):
        raise RuntimeError("logits must be a contiguous cuda [B, V] tensor")
    if logits.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if logits.dtype == torch.float16:
        return _lib.DTYPE_F16
    raise RuntimeError("logits must be float16 or bfloat16")


def _check_top_k(top_k: int, vocab: int) -> None:
    if top_k < 1:
        raise RuntimeError("top_k must be >= 1")
    if min(top_k, vocab) > _lib.K_MAX:
        raise RuntimeError(f"top_k must be <= {_lib.K_MAX}")


def _check_top_p(top_p: float) -> None:
    if not (top_p > 0.0 and top_p <= 1.0):
        raise RuntimeError("top_p must be in (0, 1]")


def make_plan(logits: torch.Tensor, top_k: int, splits_override: int = 0) -> _lib.Plan:
    plan = _lib.Plan()
    _lib.check(_lib.load().fsamp_make_plan(ctypes.c_void_p(logits.data_ptr()), logits.shape[0],
                                           logits.shape[1], int(top_k), int(splits_override),
                                           ctypes.byref(plan)))
    return plan


def _workspace(logits: torch.Tensor, top_k: int, splits_override: int, stream: int):
    """Cached per (device, stream) workspace whose per-row counters are zero.

    Layout (include/fsamp.h): [counters: round_up(128*B, 256) bytes][per-split candidates].
    A call with S > 1 leaves its counters zero and candidates behind them; a later call with a
    larger B would read those candidates as counters, so the buffer is zeroed again whenever
    the counter region grows past what is known to be clean.
    """
    lib = _lib.load()
    B, V = logits.shape
    need = lib.fsamp_workspace_bytes(ctypes.c_void_p(logits.data_ptr()), B, V, int(top_k),
                                     int(splits_override))
    if need == 0:
        return None, 0
    key = (logits.device.index, stream)
    entry = _WORKSPACES.get(key)
    counter_bytes = ((128 * B + 255) // 256) * 256
    if entry is None or entry["buf"].numel() < need:
        buf = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=logits.device)
        _lib.check(lib.fsamp_workspace_init(ctypes.c_void_p(buf.data_ptr()), buf.numel(),
                                            ctypes.c_void_p(stream)))
        entry = {"buf": buf, "clean": buf.numel()}
        _WORKSPACES[key] = entry
    elif entry["clean"] < counter_bytes:
        buf = entry["buf"]
        _lib.check(lib.fsamp_workspace_init(ctypes.c_void_p(buf.data_ptr()), buf.numel(),
                                            ctypes.c_void_p(stream)))
        entry["clean"] = buf.numel()
    entry["clean"] = min(entry["clean"], counter_bytes)
    return entry["buf"], entry["buf"].numel()


def _ws_args(logits, top_k, splits_override, stream):
    buf, nbytes = _workspace(logits, top_k, splits_override, stream)
    return (ctypes.c_void_p(buf.data_ptr()) if buf is not None else None), nbytes


def _generator_seed_offset(device: torch.device) -> tuple[int, int]:
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("the torch-generator draw (offset < 0) cannot be captured in a HIP "
                           "graph; pass an explicit offset or per-row u")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    gen = torch.cuda.default_generators[idx]
    seed, off = gen.initial_seed(), gen.get_offset()
    gen.set_offset(off + 4)
    return seed, off


def _u_ptr(u: torch.Tensor | None, B: int, device: torch.device):
    if u is None:
        return None
    if not (u.is_cuda and u.dtype == torch.float32 and u.is_contiguous() and u.numel() == B
            and u.device == device):
        raise RuntimeError("u must be a contiguous float32 cuda tensor with one value per row")
    return ctypes.c_void_p(u.data_ptr())


def _sample(logits, top_k, top_p, seed, offset, splits_override, u, stages):
    dtype = _check_logits(logits)
    B, V = logits.shape
    _check_top_k(int(top_k), V)
    _check_top_p(float(top_p))
    if u is None and offset < 0:
        seed, offset = _generator_seed_offset(logits.device)
    stream = _stream_ptr(logits.device)
    ws, ws_bytes = _ws_args(logits, top_k, splits_override, stream)
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    uptr = _u_ptr(u, B, logits.device)
    lib = _lib.load()
    seed64, off64 = int(seed) & (2**64 - 1), int(offset) & (2**64 - 1)
    if stages:
        K = min(int(top_k), V)
        keep = torch.empty((B, K), dtype=torch.bool, device=logits.device)
        renormed = torch.empty((B, K), dtype=torch.float32, device=logits.device)
        _lib.check(lib.fsamp_stages(ctypes.c_void_p(logits.data_ptr()), dtype, B, V, int(top_k),
                                    float(top_p), uptr, seed64, off64,
                                    ctypes.c_void_p(out.data_ptr()),
                                    ctypes.c_void_p(keep.data_ptr()),
                                    ctypes.c_void_p(renormed.data_ptr()), ws, ws_bytes,
                                    int(splits_override), ctypes.c_void_p(stream)))
        return [out, keep, renormed]
    _lib.check(lib.fsamp_sample(ctypes.c_void_p(logits.data_ptr()), dtype, B, V, int(top_k),
                                float(top_p), uptr, seed64, off64,
                                ctypes.c_void_p(out.data_ptr()), ws, ws_bytes,
                                int(splits_override), ctypes.c_void_p(stream)))
    return out


def sample_fused(logits: torch.Tensor, top_k: int, top_p: float, seed: int, offset: int,
                 splits_override: int) -> torch.Tensor:
    """[B, V] logits -> [B] int64 token ids (csrc/fused_sampling.cu:449-458).

    offset >= 0: row b's uniform is splitmix64(seed, offset, b); offset < 0: seed and offset
    come from torch's default generator, which is advanced.
    """
    return _sample(logits, top_k, top_p, seed, offset, splits_override, None, False)


def sample_fused_u(logits: torch.Tensor, top_k: int, top_p: float, u: torch.Tensor,
                   splits_override: int = 0) -> torch.Tensor:
    """[B, V] logits and one fp32 uniform per row u[B] in [0, 1) -> [B] int64 token ids."""
    return _sample(logits, top_k, top_p, 0, 0, splits_override, u, False)


def stages_fused(logits: torch.Tensor, top_k: int, top_p: float, seed: int, offset: int,
                 splits_override: int) -> list:
    """[token_ids [B], keep bool [B,K], renormed f32 [B,K]] (csrc/fused_sampling.cu:503-513)."""
    if offset < 0:
        raise RuntimeError("stages_fused takes an explicit offset >= 0")
    return _sample(logits, top_k, top_p, seed, offset, splits_override, None, True)


def stages_fused_u(logits: torch.Tensor, top_k: int, top_p: float, u: torch.Tensor,
                   splits_override: int = 0) -> list:
    """stages_fused with explicit per-row uniforms."""
    return _sample(logits, top_k, top_p, 0, 0, splits_override, u, True)


def topk_fused(logits: torch.Tensor, top_k: int, splits_override: int) -> torch.Tensor:
    """[B, K] candidate ids, descending value, ties by ascending id (:460-473)."""
    dtype = _check_logits(logits)
    B, V = logits.shape
    _check_top_k(int(top_k), V)
    stream = _stream_ptr(logits.device)
    ws, ws_bytes = _ws_args(logits, top_k, splits_override, stream)
    ids = torch.empty((B, min(int(top_k), V)), dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().fsamp_topk(ctypes.c_void_p(logits.data_ptr()), dtype, B, V,
                                      int(top_k), ctypes.c_void_p(ids.data_ptr()), ws, ws_bytes,
                                      int(splits_override), ctypes.c_void_p(stream)))
    return ids


def probe_phase(logits: torch.Tensor, top_k: int, top_p: float, phase: int,
                splits_override: int) -> torch.Tensor:
    """Run phases 1..phase of the pipeline and stop (:475-501); phase 7 == sample_fused with
    seed = offset = 0."""
    dtype = _check_logits(logits)
    B, V = logits.shape
    _check_top_k(int(top_k), V)
    _check_top_p(float(top_p))
    if not 1 <= int(phase) <= 7:
        raise RuntimeError("phase must be in [1, 7]")
    stream = _stream_ptr(logits.device)
    ws, ws_bytes = _ws_args(logits, top_k, splits_override, stream)
    out = torch.zeros(B, dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().fsamp_probe_phase(ctypes.c_void_p(logits.data_ptr()), dtype, B, V,
                                             int(top_k), float(top_p), int(phase),
                                             ctypes.c_void_p(out.data_ptr()), ws, ws_bytes,
                                             int(splits_override), ctypes.c_void_p(stream)))
    return out


def probe_noop(logits: torch.Tensor) -> torch.Tensor:
    """Launch floor: allocate [B] and write it (csrc/probes.cu:86-94)."""
    _check_logits(logits)
    B = logits.shape[0]
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().fsamp_probe_noop(B, ctypes.c_void_p(out.data_ptr()),
                                            ctypes.c_void_p(_stream_ptr(logits.device))))
    return out


def probe_scan_rowblock(logits: torch.Tensor) -> torch.Tensor:
    """One full pass (argmax), one workgroup per row (csrc/probes.cu:96-106)."""
    dtype = _check_logits(logits)
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().fsamp_probe_scan_rowblock(ctypes.c_void_p(logits.data_ptr()), dtype,
                                                     B, V, ctypes.c_void_p(out.data_ptr()),
                                                     ctypes.c_void_p(_stream_ptr(logits.device))))
    return out


def probe_scan_split(logits: torch.Tensor, splits: int) -> torch.Tensor:
    """One full pass split over `splits` workgroups per row, then a merge (:108-125)."""
    dtype = _check_logits(logits)
    B, V = logits.shape
    if splits < 1:
        raise RuntimeError("splits must be >= 1")
    partial = torch.empty((B, int(splits)), dtype=torch.int64, device=logits.device)
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    _lib.check(_lib.load().fsamp_probe_scan_split(ctypes.c_void_p(logits.data_ptr()), dtype, B,
                                                  V, int(splits),
                                                  ctypes.c_void_p(out.data_ptr()),
                                                  ctypes.c_void_p(partial.data_ptr()),
                                                  partial.numel() * 8,
                                                  ctypes.c_void_p(_stream_ptr(logits.device))))
    return out


def kernel_attrs() -> list:
    """[(name, chunks, threads, vgprs, scratch_bytes, lds_bytes, blocks_per_cu)] per compiled
    sampler kernel (:515-540; chunks stands where the reference reports its merge width P)."""
    lib = _lib.load()
    n = ctypes.c_int32(0)
    _lib.check(lib.fsamp_kernel_attrs(None, 0, ctypes.byref(n)))
    rows = (_lib.AttrRow * n.value)()
    _lib.check(lib.fsamp_kernel_attrs(rows, n.value, ctypes.byref(n)))
    return [(r.name.decode(), r.chunks, r.threads, r.vgprs, r.scratch_bytes, r.lds_bytes,
             r.blocks_per_cu) for r in rows]

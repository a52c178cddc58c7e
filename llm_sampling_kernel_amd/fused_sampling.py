"""Torch-facing mirror of the reference's extension module ``fused_sampling``.

Same function names, argument order and meaning as csrc/bindings.cpp:16-25, the same
``RuntimeError`` messages for the checks the reference makes (csrc/fused_sampling.cu:341-357,
:422-424), plus ``sample_fused_u`` for the explicit per-row uniform the C ABI takes.  Every call
forwards device pointers and torch's current HIP stream to libfsamp.so (include/fsamp.h);
there is no other implementation behind these functions.

Deliberate differences from the reference:
  - top_k may be up to 1024 (reference: 128), so the "top_k must be <= ..." message names 1024;
  - ``offset < 0`` (torch-generator path, csrc/fused_sampling.cu:441-447): outside graph
    capture the seed and offset come from torch's default generator of the logits' device, on
    the host, and the generator's offset advances by 4 per call, as the reference's
    philox_cuda_state(4) does.  Under HIP-graph capture the offset comes from a device counter
    that the kernel itself advances by 4 per call, so every replay draws fresh uniforms (the
    reference reads a graph-safe device offset for the same purpose, :112-118).  The counter is
    created, from the generator's offset, by the first generator-path call made outside
    capture (a warm-up call, as graph capture needs anyway).  Either way the row uniform is
    splitmix64(seed, offset, row) like the explicit-offset path.

Extensions with no counterpart in the reference (SEMANTICS.md lists them as open):
``sample_fused_ex`` with per-row top_k / top_p / temperature.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_WORKSPACES: dict = {}
_OFFSET_COUNTERS: dict = {}  # device index -> int64[1] device tensor (graph-safe draw offset)


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
    """Cached per (device, stream) workspace whose counters are zero.

    Layout (include/fsamp.h): [row counters: round_up(128*B, 256) bytes][grid counter: 256]
    [per-split candidates].  A call leaves its counters zero and candidates behind them; a
    later call with a larger B would read those candidates as counters, so the buffer is zeroed
    again whenever the counter region grows past what is known to be clean.
    """
    lib = _lib.load()
    B, V = logits.shape
    need = lib.fsamp_workspace_bytes(ctypes.c_void_p(logits.data_ptr()), B, V, int(top_k),
                                     int(splits_override))
    if need == 0:
        return None, 0
    key = (logits.device.index, stream)
    entry = _WORKSPACES.get(key)
    counter_bytes = ((128 * B + 255) // 256) * 256 + 256
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


def _generator(device: torch.device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return idx, torch.cuda.default_generators[idx]


def offset_counter(device: torch.device) -> torch.Tensor:
    """The device's graph-safe offset counter (int64[1]); created from torch's generator offset
    on first use, which must happen outside graph capture."""
    idx, gen = _generator(device)
    ctr = _OFFSET_COUNTERS.get(idx)
    if ctr is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("call sample_fused with offset=None once outside graph capture "
                               "before capturing it (that creates its device offset counter)")
        ctr = torch.tensor([gen.get_offset()], dtype=torch.int64, device=torch.device("cuda", idx))
        _OFFSET_COUNTERS[idx] = ctr
    return ctr


def _generator_draw(device: torch.device):
    """(seed, offset, counter): outside capture the host generator's offset (advanced by 4) and
    no counter; under capture the device counter, which the kernel advances."""
    idx, gen = _generator(device)
    if torch.cuda.is_current_stream_capturing():
        return gen.initial_seed(), 0, offset_counter(device)
    offset_counter(device)  # make sure a later capture finds it
    seed, off = gen.initial_seed(), gen.get_offset()
    gen.set_offset(off + 4)
    return seed, off, None


def _u_ptr(u: torch.Tensor | None, B: int, device: torch.device):
    if u is None:
        return None
    if not (u.is_cuda and u.dtype == torch.float32 and u.is_contiguous() and u.numel() == B
            and u.device == device):
        raise RuntimeError("u must be a contiguous float32 cuda tensor with one value per row")
    return ctypes.c_void_p(u.data_ptr())


def _row_array(a, B: int, dtype: torch.dtype, device: torch.device, name: str):
    if a is None:
        return None
    if not (isinstance(a, torch.Tensor) and a.is_cuda and a.dtype == dtype and a.is_contiguous()
            and a.numel() == B and a.device == device):
        raise RuntimeError(f"{name} must be a contiguous {dtype} cuda tensor with one value per "
                           "row")
    return a


def _sample(logits, top_k, top_p, seed, offset, splits_override, u, stages, top_k_row=None,
            top_p_row=None, temperature=None):
    dtype = _check_logits(logits)
    B, V = logits.shape
    _check_top_k(int(top_k), V)
    _check_top_p(float(top_p))
    counter = None
    if u is None and offset < 0:
        seed, offset, counter = _generator_draw(logits.device)
    dev = logits.device
    kr = _row_array(top_k_row, B, torch.int32, dev, "top_k_row")
    pr = _row_array(top_p_row, B, torch.float32, dev, "top_p_row")
    tr = _row_array(temperature, B, torch.float32, dev, "temperature")
    rows = _lib.RowParams(kr.data_ptr() if kr is not None else None,
                          pr.data_ptr() if pr is not None else None,
                          tr.data_ptr() if tr is not None else None,
                          counter.data_ptr() if counter is not None else None)
    stream = _stream_ptr(dev)
    ws, ws_bytes = _ws_args(logits, top_k, splits_override, stream)
    out = torch.empty(B, dtype=torch.int64, device=dev)
    uptr = _u_ptr(u, B, dev)
    seed64, off64 = int(seed) & (2**64 - 1), int(offset) & (2**64 - 1)
    keep = renormed = None
    if stages:
        K = min(int(top_k), V)
        keep = torch.empty((B, K), dtype=torch.bool, device=dev)
        renormed = torch.empty((B, K), dtype=torch.float32, device=dev)
    _lib.check(_lib.load().fsamp_sample_ex(
        ctypes.c_void_p(logits.data_ptr()), dtype, B, V, int(top_k), float(top_p), uptr, seed64,
        off64, ctypes.byref(rows), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(keep.data_ptr()) if stages else None,
        ctypes.c_void_p(renormed.data_ptr()) if stages else None, ws, ws_bytes,
        int(splits_override), ctypes.c_void_p(stream)))
    return [out, keep, renormed] if stages else out


def sample_fused(logits: torch.Tensor, top_k: int, top_p: float, seed: int, offset: int,
                 splits_override: int) -> torch.Tensor:
    """[B, V] logits -> [B] int64 token ids (csrc/fused_sampling.cu:449-458).

    offset >= 0: row b's uniform is splitmix64(seed, offset, b); offset < 0: seed and offset
    come from torch's default generator, which is advanced (a device counter under capture).
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


def sample_fused_ex(logits: torch.Tensor, top_k: int, top_p: float, *, u=None, seed: int = 0,
                    offset: int = -1, top_k_row=None, top_p_row=None, temperature=None,
                    splits_override: int = 0, stages: bool = False):
    """Sampling with per-row controls (fsamp_sample_ex): top_k_row int32[B] (row b samples from
    its top min(max(top_k_row[b], 1), top_k) ranks), top_p_row float32[B], temperature
    float32[B] (softmax of (x - max) / T; T <= 0 is greedy).  u, or seed / offset as in
    sample_fused.  Returns token ids, or [token ids, keep, renormed] with stages=True."""
    return _sample(logits, top_k, top_p, seed, offset, splits_override, u, stages,
                   top_k_row, top_p_row, temperature)


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


def probe_load(logits: torch.Tensor, wave_max: torch.Tensor | None = None) -> torch.Tensor:
    """Load-only floor in the sampler's B=256 launch shape: [B, 8] int32 per-wave maximum order
    keys (fsamp_probe_load).  No counterpart in the reference."""
    dtype = _check_logits(logits)
    B, V = logits.shape
    if wave_max is None:
        wave_max = torch.empty(B * 8, dtype=torch.int32, device=logits.device)
    if not (wave_max.is_cuda and wave_max.dtype == torch.int32 and wave_max.numel() >= B * 8
            and wave_max.is_contiguous()):
        raise RuntimeError("wave_max must be a contiguous int32 cuda tensor of B*8 entries")
    _lib.check(_lib.load().fsamp_probe_load(ctypes.c_void_p(logits.data_ptr()), dtype, B, V,
                                            ctypes.c_void_p(wave_max.data_ptr()),
                                            ctypes.c_void_p(_stream_ptr(logits.device))))
    return wave_max[:B * 8].view(B, 8)


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

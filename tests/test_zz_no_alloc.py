"""fsamp_sample_noalloc (the entry point that allocates nothing) against fsamp_sample.

Both are called through the C ABI with the same inputs; the no-allocation entry keeps its
split candidates and row tickets in the library's fixed device scratch, the classic one in a
caller workspace.  Two calls in a row, the second smaller, must both agree bit for bit (and with
the oracle); a call larger than the fixed scratch must be refused with its own status.
"""

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from llm_sampling_kernel_amd import _lib  # noqa: E402
from llm_sampling_kernel_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

import cabi  # noqa: E402

pytestmark = pytest.mark.gpu


def _bits(shape, seed, scale, dtype):
    x = np.random.Generator(np.random.PCG64(seed)).standard_normal(shape).astype(np.float32)
    return W.to_bits(x * scale, dtype)


def _dev(bits, dtype):
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(torch.bfloat16 if dtype == "bfloat16" else torch.float16).cuda()


def _classic(x, k, p, u, splits):
    lib = _lib.load()
    B, V = x.shape
    out = torch.empty(B, dtype=torch.int64, device="cuda")
    ws = cabi.classic_workspace(x, k, splits)
    _lib.check(lib.fsamp_sample(cabi.vp(x), cabi.dtype_code(x), B, V, k, p, cabi.vp(u), 0, 0,
                                cabi.vp(out), cabi.vp(ws), ws.numel(), splits,
                                ctypes.c_void_p(cabi.stream_ptr())))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _noalloc(x, k, p, u, splits, seed=0, offset=0):
    lib = _lib.load()
    B, V = x.shape
    out = torch.full((B,), -7, dtype=torch.int64, device="cuda")
    rc = lib.fsamp_sample_noalloc(cabi.vp(x), cabi.dtype_code(x), B, V, k, p, cabi.vp(u), seed,
                                  offset, cabi.vp(out), splits, ctypes.c_void_p(cabi.stream_ptr()))
    torch.cuda.synchronize()
    return rc, out.cpu().numpy()


def test_noalloc_matches_the_workspace_entry_on_two_calls_in_a_row():
    # first call: B=64 C2-like rows, 4 splits; second call smaller: B=8, 6 splits, other k
    cases = [(64, 128256, 50, 0.95, "float16", 0, 11), (8, 40000, 20, 0.9, "bfloat16", 6, 12)]
    for B, V, k, p, dtype, splits, seed in cases:
        bits = _bits((B, V), seed, 2.0, dtype)
        x = _dev(bits, dtype)
        un = np.random.Generator(np.random.PCG64(seed + 100)).random(B, dtype=np.float32)
        u = torch.from_numpy(un).cuda()
        want = _classic(x, k, p, u, splits)
        rc, got = _noalloc(x, k, p, u, splits)
        assert rc == 0, _lib.load().fsamp_error_string(rc)
        assert np.array_equal(got, want), (B, V, k)
        assert np.array_equal(got, O.sample(bits, dtype, k, p, un, nthreads=8)), (B, V, k)


def test_noalloc_repeats_and_follows_the_seed_offset_stream():
    bits = _bits((16, 151936), 21, 3.0, "bfloat16")
    x = _dev(bits, "bfloat16")
    first = None
    for _ in range(3):  # the scratch keeps the last call's contents; the answer must not move
        rc, got = _noalloc(x, 50, 0.9, None, 0, seed=99, offset=8)
        assert rc == 0
        first = got if first is None else first
        assert np.array_equal(got, first)
    want = O.sample(bits, "bfloat16", 50, 0.9, O.rng_uniform(99, 8, 16), nthreads=8)
    assert np.array_equal(first, want)


def test_noalloc_refuses_calls_larger_than_its_scratch():
    lib = _lib.load()
    # 2048 split rows need more tickets than the fixed scratch holds: refused before launch
    x = torch.zeros(2048, 4096, dtype=torch.bfloat16, device="cuda")
    rc, _ = _noalloc(x, 50, 0.9, None, 4)
    assert rc == 13 and b"fixed scratch" in lib.fsamp_error_string(rc)
    # split candidates past 4 MiB: 1000 rows x 4 splits x 256 words x 8 bytes = 8 MB
    x = torch.zeros(1000, 8192, dtype=torch.bfloat16, device="cuda")
    rc, _ = _noalloc(x, 256, 0.9, None, 4)
    assert rc == 13
    # a plan with one split per row needs no scratch at all, whatever its size
    x = torch.zeros(2048, 4096, dtype=torch.bfloat16, device="cuda")
    rc, got = _noalloc(x, 5, 0.9, None, 1)
    assert rc == 0 and ((got >= 0) & (got < 5)).all()  # five equal logits: ids 0..4 are kept

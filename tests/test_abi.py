"""CPU checks of the C ABI: the library loads, exports every entry point include/fsamp.h
declares, and its host-side planning and argument checks behave (no kernel is launched)."""

import ctypes
import os
import re

import pytest

from llm_sampling_kernel_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fsamp.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fsamp_[a-z_]+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    names = declared_functions()
    for want in ("fsamp_sample", "fsamp_topk", "fsamp_stages", "fsamp_probe_phase",
                 "fsamp_probe_noop", "fsamp_probe_scan_rowblock", "fsamp_probe_scan_split",
                 "fsamp_kernel_attrs"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def plan(B, V, k, splits=0, ptr=4096):
    p = _lib.Plan()
    rc = _lib.load().fsamp_make_plan(ctypes.c_void_p(ptr), B, V, k, splits, ctypes.byref(p))
    return rc, p


@pytest.mark.parametrize("B,V,k,S,threads", [
    (1, 151936, 50, 6, 512),      # C1: 6 splits of 25328 elements
    (16, 128256, 50, 4, 512),     # C2, B=16: 4 splits of 32064
    (64, 128256, 50, 2, 512),     # C2, B=64: 2 splits (128 workgroups)
    (128, 128256, 50, 1, 1024),   # a 32-chunk slice on a grid of <= 192 takes 1024 x 16
    (256, 128256, 50, 1, 512),    #   and beyond that the 512-thread streaming tiling
    (48, 151936, 50, 2, 512),     # B * S stays within 128 workgroups for k <= 128
    (96, 151936, 50, 1, 512),     #   (so that the grid runs in one wave of the 256 CUs)
    (8, 151936, 50, 6, 512),      # C3
    (16, 151936, 256, 4, 1024),   # C4 k=256: wide k takes 1024 threads, 4 splits
    (16, 151936, 1024, 4, 1024),  # C4 k=1024: 4 splits, 4096 merged words
    (256, 151936, 50, 1, 512),    # C5: one workgroup per row, slice in VGPRs
    (256, 151936, 256, 1, 512),   # wide k over a whole row: the 512-thread register tiling
    (1, 32000, 50, 1, 512),       # short rows are not split (V <= 65536)
    (1, 256000, 50, 8, 512),      # long rows take up to 8 splits (V > 196608)
    (16, 151936, 128, 4, 512),    # 64 < k <= 128: at most 4 splits
])
def test_plans_for_the_benchmark_shapes(B, V, k, S, threads):
    rc, p = plan(B, V, k)
    assert rc == 0 and p.splits == S and p.threads == threads
    assert p.threads * p.chunks * 8 >= p.slice and p.slice * p.splits >= V
    assert p.slice % 8 == 0 and p.vec == 1
    assert p.workspace_bytes == ((128 * B + 255) // 256) * 256 + 256 + (0 if S == 1 else B * S * k * 8)


@pytest.mark.parametrize("B,S", [(1, 8), (16, 8), (64, 4), (128, 2), (256, 1)])
def test_rows_read_by_element_split_up_to_eight_ways_within_256_workgroups(B, S):
    rc, p = plan(B, 50257, 50)
    assert rc == 0 and p.vec == 0 and p.splits == S
    assert p.threads * p.chunks * 8 >= p.slice and (S - 1) * p.slice < 50257 <= S * p.slice


def test_every_plan_tiles_its_slice_and_fits_the_merge_buffer():
    for B in (1, 2, 7, 16, 64, 127, 128, 300):
        for V in (1, 7, 8, 30, 1000, 4001, 32000, 128256, 151936, 262143, 262144):
            for k in (1, 20, 50, 256, 1024):
                for splits in (0, 1, 3, 64):
                    for ptr in (4096, 4098):
                        rc, p = plan(B, V, k, splits, ptr)
                        if min(k, V) > 1024:
                            continue
                        assert rc == 0, (B, V, k, splits, rc)
                        assert p.threads * p.chunks * 8 >= p.slice
                        assert p.splits * p.k <= 4096
                        assert (p.splits - 1) * p.slice < V <= p.splits * p.slice
                        assert p.vec == int(ptr % 16 == 0 and V % 8 == 0)


def test_stream_probe_sizes_and_refusals_before_any_launch():
    lib = _lib.load()
    # 256 x 151936 bf16 = 4,861,952 vectors = 4,748 workgroups of 1,024 vectors, 4 waves each
    assert lib.fsamp_probe_stream_words(256, 151936) == 4748 * 4
    assert lib.fsamp_probe_stream_words(3, 1000) == 4          # 375 vectors: one workgroup
    assert lib.fsamp_probe_stream_words(0, 1000) == 0
    buf = ctypes.c_void_p(4096)
    assert lib.fsamp_probe_stream(ctypes.c_void_p(4098), 1, 2, 64, buf, 64, None) == 10  # unaligned
    assert lib.fsamp_probe_stream(ctypes.c_void_p(4096), 1, 2, 60, buf, 64, None) == 10  # V % 8
    assert lib.fsamp_probe_stream(ctypes.c_void_p(4096), 1, 2, 64, buf, 3, None) == 6   # too few words
    assert lib.fsamp_probe_stream(ctypes.c_void_p(4096), 1, 2, 64, None, 64, None) == 7


def test_argument_checks_return_the_reference_messages():
    lib = _lib.load()
    assert plan(1, 100, 0)[0] == 3 and b"top_k must be >= 1" == lib.fsamp_error_string(3)
    assert plan(1, 5000, 2000)[0] == 4 and b"top_k must be <= 1024" == lib.fsamp_error_string(4)
    assert plan(0, 100, 5)[0] == 2
    assert lib.fsamp_error_string(1) == b"logits must be float16 or bfloat16"
    assert lib.fsamp_error_string(5) == b"top_p must be in (0, 1]"
    assert lib.fsamp_error_string(2) == b"logits must be a contiguous cuda [B, V] tensor"
    # the launch entry points check arguments before touching the device
    null = ctypes.c_void_p(0)
    assert lib.fsamp_sample(ctypes.c_void_p(4096), 2, 1, 100, 5, 0.9, None, 0, 0,
                            ctypes.c_void_p(4096), None, 0, 0, null) == 1
    assert lib.fsamp_sample(ctypes.c_void_p(4096), 1, 1, 100, 5, 1.5, None, 0, 0,
                            ctypes.c_void_p(4096), None, 0, 0, null) == 5
    assert lib.fsamp_sample(ctypes.c_void_p(4096), 1, 1, 151936, 50, 0.9, None, 0, 0,
                            ctypes.c_void_p(4096), None, 0, 0, null) == 6  # workspace needed
    assert lib.fsamp_probe_phase(ctypes.c_void_p(4096), 1, 1, 100, 5, 0.9, 8,
                                 ctypes.c_void_p(4096), None, 0, 0, null) == 8
    assert lib.fsamp_probe_scan_split(ctypes.c_void_p(4096), 1, 1, 100, 0,
                                      ctypes.c_void_p(4096), None, 0, null) == 9


def test_split_workspace_sizes_and_the_call_struct_checks():
    lib = _lib.load()
    assert lib.fsamp_counter_bytes(1) == 256 and lib.fsamp_counter_bytes(3) == 512
    assert lib.fsamp_counter_bytes(0) == 0
    p = ctypes.c_void_p(4096)
    assert lib.fsamp_scratch_bytes(p, 256, 151936, 50, 0) == 0  # one split per row
    assert lib.fsamp_scratch_bytes(p, 1, 151936, 50, 0) == 6 * 50 * 8
    assert lib.fsamp_scratch_bytes(p, 16, 151936, 1024, 0) == 16 * 4 * 1024 * 8
    # a struct of another size is refused before anything else is read
    c = _lib.Call(logits=4096, dtype=1, batch=1, vocab=100, top_k=5, top_p=0.9, out=4096)
    c.struct_bytes = ctypes.sizeof(_lib.Call) - 8
    assert lib.fsamp_run(ctypes.byref(c), None) == 12
    assert lib.fsamp_error_string(12).startswith(b"fsamp_call")
    c = _lib.Call(logits=4096, dtype=1, batch=1, vocab=100, top_k=5, top_p=0.9)
    assert lib.fsamp_run(ctypes.byref(c), None) == 7  # no output
    c.out, c.ids = 4096, 4096
    assert lib.fsamp_run(ctypes.byref(c), None) == 7  # two outputs
    c = _lib.Call(logits=4096, dtype=1, batch=1, vocab=100, ld=50, top_k=5, top_p=0.9, out=4096)
    assert lib.fsamp_run(ctypes.byref(c), None) == 2  # row stride below the row
    c = _lib.Call(logits=4096, dtype=1, batch=1, vocab=151936, top_k=50, top_p=0.9, out=4096)
    assert lib.fsamp_run(ctypes.byref(c), None) == 6  # split rows need counters and scratch
    c = _lib.Call(logits=4096, dtype=1, batch=1, vocab=100, top_k=5, top_p=0.9, out=4096,
                  threads_override=384)
    assert lib.fsamp_run(ctypes.byref(c), None) == 2


def test_shard_and_merge_entries_check_their_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(4096)
    # top_k larger than the shard
    assert lib.fsamp_topk_shard(p, 1, 2, 64, 64, 65, 0, p, None, 0, None, 0, 0, None) == 4
    # global ids past 2^32 - 2
    assert lib.fsamp_topk_shard(p, 1, 2, 64, 64, 8, 0xFFFFFFF0, p, None, 0, None, 0, 0,
                                None) == 2
    assert lib.fsamp_merge_sample(p, 3, 2, 4, 8, 0.9, None, 0, 0, p, None, None, None,
                                  None) == 1
    assert lib.fsamp_merge_sample(p, 1, 2, 4, 0, 0.9, None, 0, 0, p, None, None, None,
                                  None) == 3
    assert lib.fsamp_merge_sample(p, 1, 2, 4, 2000, 0.9, None, 0, 0, p, None, None, None,
                                  None) == 4
    assert lib.fsamp_merge_sample(p, 1, 2, 4, 8, 1.5, None, 0, 0, p, None, None, None,
                                  None) == 5
    # exactly one of out / ids
    assert lib.fsamp_merge_sample(p, 1, 2, 4, 8, 0.9, None, 0, 0, p, None, None, p,
                                  None) == 7
    assert lib.fsamp_merge_sample(p, 1, 2, 4, 8, 0.9, None, 0, 0, None, None, None, None,
                                  None) == 7


def test_the_torch_module_is_the_compiled_extension_with_the_reference_surface():
    torch = pytest.importorskip("torch")
    from llm_sampling_kernel_amd import _fsamp_torch, fused_sampling

    assert os.path.dirname(os.path.abspath(_fsamp_torch.__file__)) == \
        os.path.dirname(os.path.abspath(_lib.__file__))
    for name in ("sample_fused", "topk_fused", "stages_fused", "probe_phase", "probe_noop",
                 "probe_scan_rowblock", "probe_scan_split", "kernel_attrs", "probe_load",
                 "probe_stream"):
        assert getattr(fused_sampling, name) is getattr(_fsamp_torch, name)
    x = torch.zeros(2, 64, dtype=torch.bfloat16)  # a CPU tensor: refused before any launch
    with pytest.raises(RuntimeError, match="contiguous cuda"):
        fused_sampling.sample_fused(x, 5, 0.9, 0, 0, 0)
    with pytest.raises(RuntimeError, match="contiguous cuda"):
        fused_sampling.topk_fused(x, 5, 0)

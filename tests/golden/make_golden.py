"""Write the golden fixtures under tests/golden/.

known_answers.json -- the closed-form cases the reference's own tests assert (data only: the
    inputs and the expected outputs, each with the reference test it comes from).  They pin the
    oracle on the CPU and the HIP path on the GPU.
workloads.npz -- for each benchmark case (C1..C5 at full size): the sha256 prefix of the seeded
    input bytes, and the oracle's top-k ids, cutoff and token ids for the case's u.  The GPU
    tests regenerate the inputs (llm_sampling_kernel_amd.workloads), check the digest, and
    compare the kernel with these arrays.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from llm_sampling_kernel_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402


def spec(B: int, V: int, fill: float, runs=()) -> dict:
    """Compact [B, V] input: every element `fill`, then x[:, start:stop:step] = value per run."""
    return {"shape": [B, V], "fill": fill, "runs": [list(r) for r in runs]}


def expand(logits) -> list:
    """Dense rows from either a list of rows or a spec() dict."""
    if isinstance(logits, list):
        return logits
    B, V = logits["shape"]
    row = [logits["fill"]] * V
    for start, stop, step, value in logits["runs"]:
        for i in range(start, stop, step):
            row[i] = value
    return [list(row) for _ in range(B)]


def known_answers() -> list[dict]:
    """Inputs are rows of float values (or a spec() dict) plus a dtype; expected fields are exact."""
    L = []
    L.append(dict(
        name="cutoff_hand_example", ref="tests/test_reference.py:69-74", dtype="float32",
        logits=[[math.log(p) for p in (0.40, 0.30, 0.15, 0.10, 0.05)]], top_k=5, top_p=0.90,
        cutoff=[4], keep=[[True, True, True, True, False]]))
    L.append(dict(
        name="four_equal_logits", ref="tests/test_reference.py:77-83", dtype="float32",
        logits=[[0.0] * 4], top_k=4, top_p=0.5, cutoff=[2], cumsum=[[0.25, 0.5, 0.75, 1.0]]))
    for dtype in ("float16", "bfloat16"):
        for p, kept in ((0.25, 2), (0.5, 4), (0.75, 6), (0.875, 7)):
            L.append(dict(
                name=f"eight_equal_{dtype}_{p}", ref="tests/test_fused_kernel.py:244-257",
                dtype=dtype, logits=spec(4, 4000, -30.0, [(0, 8, 1, 10.0)]), top_k=8, top_p=p,
                cutoff=[kept] * 4))
    L.append(dict(
        name="ties_even_positions", ref="tests/test_reference.py:411-416", dtype="float32",
        logits=spec(1, 64, 0.0, [(0, 64, 2, 1.0)]), top_k=8, top_p=1.0,
        topk_ids=[[0, 2, 4, 6, 8, 10, 12, 14]]))
    L.append(dict(
        name="boundary_tie_group", ref="tests/test_reference.py:418-423", dtype="float32",
        logits=spec(1, 20, 0.0, [(3, 12, 1, 5.0)]), top_k=5, top_p=1.0,
        topk_ids=[[3, 4, 5, 6, 7]]))
    L.append(dict(
        name="full_tie_lowest_ids", ref="tests/test_reference.py:444-448", dtype="float32",
        logits=spec(4, 500, 0.0), top_k=50, top_p=1.0, topk_ids=[list(range(50))] * 4))
    for dtype in ("float16", "bfloat16"):
        L.append(dict(
            name=f"all_equal_{dtype}", ref="tests/test_fused_kernel.py:40-45", dtype=dtype,
            logits=spec(4, 4000, 0.0), top_k=50, top_p=0.9, topk_ids=[list(range(50))] * 4))
    L.append(dict(
        name="boundary_tie_keeps_value", ref="tests/test_reference.py:243-247", dtype="float32",
        logits=spec(1, 10, 0.0, [(0, 3, 1, 5.0)]), top_k=5, top_p=1.0,
        topk_vals=[[5.0, 5.0, 5.0, 0.0, 0.0]]))
    L.append(dict(
        name="top_p_one_saturated_cumsum", ref="tests/test_reference.py:182-188",
        dtype="float32", logits=spec(1, 100, -50.0, [(0, 1, 1, 50.0)]), top_k=100, top_p=1.0, cutoff=[100],
        cumsum0=[1.0]))
    L.append(dict(
        name="wide_dynamic_range", ref="tests/test_reference.py:290-294", dtype="float32",
        logits=[[1e30, 1.0, 0.0, -1.0, -1e30]], top_k=5, top_p=0.95, cutoff=[1]))
    for dtype in ("float16", "bfloat16"):
        L.append(dict(
            name=f"one_hot_spike_{dtype}", ref="tests/test_fused_kernel.py:69-73", dtype=dtype,
            logits=spec(8, 4000, -30.0, [(1234, 1235, 1, 30.0)]), top_k=50, top_p=0.9,
            token_any_u=[1234] * 8))
    return L


def workload_fixtures() -> dict:
    out = {}
    for c in W.all_cases():
        s = O.sample(c.logits, c.dtype, c.top_k, c.top_p, c.u, return_stages=True, nthreads=8)
        out[f"{c.name}/digest"] = np.frombuffer(c.digest().encode(), dtype=np.uint8)
        out[f"{c.name}/topk_ids"] = s.topk_ids.astype(np.int32)
        out[f"{c.name}/cutoff"] = s.cutoff.astype(np.int32)
        out[f"{c.name}/token_ids"] = s.token_ids.astype(np.int64)
    return out


def main() -> None:
    O.build()
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known_answers(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "workloads.npz"), **workload_fixtures())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()

"""Seeded synthetic inputs for the five benchmark configurations (C1-C5).

The shapes, value distributions and sampling parameters are those of the five benchmark
configurations listed below; the generators are numpy PCG64 streams with fixed seeds so that
the same bytes are produced on the build container and on the GPU box.  Logits are returned as raw 16-bit patterns (uint16) plus
their dtype name, because numpy has no bfloat16; ``to_bf16_bits`` rounds to nearest-even exactly
as ``torch.Tensor.to(torch.bfloat16)`` does.

  C1  B=1,   V=151936, bf16, N(0, 3^2),                               k=50,  p=0.90
  C2  B in {1,4,16,64}, V=128256, fp16, N(0, 2^2) + 16 positions per row boosted by U[4,10],
      k in {20,50}, p=0.95
  C3  B=8,   V=151936, bf16, values drawn from linspace(-8, 8, 64),   k=50,  p=0.90
  C4  B=16,  V=151936, bf16, N(0, 1.5^2),                             k in {256,1024}, p=0.99
  C5  B=256, V=151936, bf16, N(0, 3^2) + Zipf(1.1)-ranked bias: per row a random permutation
      pi of the vocabulary and bias[pi[r]] = 6 * (r+1)^-1.1,          k=50,  p=0.90

Every case also carries one fp32 uniform u per row (``u ~ U[0,1)`` from the same stream).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

SEED_BASE = 1000


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (NaN kept quiet)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    b = f.view(np.uint32)
    rounded = ((b.astype(np.uint64) + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return to_bf16_bits(x)
    if dtype == "float16":
        return to_f16_bits(x)
    raise ValueError(dtype)


@dataclass(frozen=True)
class Case:
    name: str
    config: str       # "C1".."C5"
    logits: np.ndarray  # [B,V] uint16 bit patterns
    dtype: str        # "bfloat16" | "float16"
    top_k: int
    top_p: float
    u: np.ndarray     # [B] float32

    @property
    def batch(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def digest(self) -> str:
        h = hashlib.sha256()
        h.update(self.logits.tobytes())
        h.update(self.u.tobytes())
        return h.hexdigest()[:16]


def _rng(index: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED_BASE + index))


def c1() -> Case:
    g = _rng(1)
    x = g.standard_normal((1, 151936), dtype=np.float32) * 3.0
    u = g.random(1, dtype=np.float32)
    return Case("C1", "C1", to_bf16_bits(x), "bfloat16", 50, 0.90, u)


def c2(batch: int, top_k: int) -> Case:
    assert batch in (1, 4, 16, 64) and top_k in (20, 50)
    g = _rng(2 * 1000 + batch)
    V = 128256
    x = g.standard_normal((batch, V), dtype=np.float32) * 2.0
    for r in range(batch):
        pos = g.choice(V, size=16, replace=False)
        x[r, pos] += g.uniform(4.0, 10.0, size=16).astype(np.float32)
    u = g.random(batch, dtype=np.float32)
    return Case(f"C2_B{batch}_k{top_k}", "C2", to_f16_bits(x), "float16", top_k, 0.95, u)


def c3() -> Case:
    g = _rng(3)
    grid = np.linspace(-8.0, 8.0, 64, dtype=np.float32)
    x = grid[g.integers(0, 64, size=(8, 151936))]
    u = g.random(8, dtype=np.float32)
    return Case("C3", "C3", to_bf16_bits(x), "bfloat16", 50, 0.90, u)


def c4(top_k: int) -> Case:
    assert top_k in (256, 1024)
    g = _rng(4)
    x = g.standard_normal((16, 151936), dtype=np.float32) * 1.5
    u = g.random(16, dtype=np.float32)
    return Case(f"C4_k{top_k}", "C4", to_bf16_bits(x), "bfloat16", top_k, 0.99, u)


def c5_bias(V: int, g: np.random.Generator) -> np.ndarray:
    """Zipf(1.1)-ranked bias of one row: bias[pi[r]] = 6 * (r+1)^-1.1 for a random pi."""
    ranks = np.arange(1, V + 1, dtype=np.float64)
    bias = np.empty(V, np.float32)
    bias[g.permutation(V)] = (6.0 * ranks ** -1.1).astype(np.float32)
    return bias


def c5(batch: int = 256) -> Case:
    g = _rng(5)
    V = 151936
    x = g.standard_normal((batch, V), dtype=np.float32) * 3.0
    for r in range(batch):
        x[r] += c5_bias(V, g)
    u = g.random(batch, dtype=np.float32)
    return Case("C5" if batch == 256 else f"C5_B{batch}", "C5", to_bf16_bits(x), "bfloat16",
                50, 0.90, u)


def all_cases() -> list[Case]:
    out = [c1()]
    out += [c2(b, k) for b in (1, 4, 16, 64) for k in (20, 50)]
    out += [c3(), c4(256), c4(1024), c5()]
    return out


CASE_NAMES = (["C1"] + [f"C2_B{b}_k{k}" for b in (1, 4, 16, 64) for k in (20, 50)]
              + ["C3", "C4_k256", "C4_k1024", "C5"])


def case(name: str) -> Case:
    if name == "C1":
        return c1()
    if name.startswith("C2_"):
        b, k = name[4:].split("_k")
        return c2(int(b), int(k))
    if name == "C3":
        return c3()
    if name.startswith("C4_k"):
        return c4(int(name[4:]))
    if name == "C5":
        return c5()
    raise KeyError(name)

"""Python front end mirroring the reference's benchmarks/fused.py:8-21.

``offset=None`` maps to -1, which draws the seed/offset from torch's default generator of the
logits' device; an explicit offset gives a reproducible stream.  ``sample_fused_u`` is the
explicit-uniform form (one fp32 u per row).
"""

from . import fused_sampling

DEFAULT_SEED = 0x5EED


def sample_fused(logits, top_k, top_p, seed=DEFAULT_SEED, offset=None, splits=0):
    off = -1 if offset is None else offset
    return fused_sampling.sample_fused(logits, int(top_k), float(top_p), int(seed), int(off),
                                       int(splits))


def topk_fused(logits, top_k, splits=0):
    return fused_sampling.topk_fused(logits, int(top_k), int(splits))


def sample_fused_u(logits, top_k, top_p, u, splits=0):
    return fused_sampling.sample_fused_u(logits, int(top_k), float(top_p), u, int(splits))

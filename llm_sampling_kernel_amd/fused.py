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


def sample_fused_ex(logits, top_k, top_p, u=None, seed=DEFAULT_SEED, offset=None, top_k_row=None,
                    top_p_row=None, temperature=None, splits=0):
    """Per-row top_k / top_p / temperature (int32 / float32 / float32 [B] cuda tensors)."""
    off = -1 if offset is None else offset
    return fused_sampling.sample_fused_ex(logits, int(top_k), float(top_p), u=u, seed=int(seed),
                                          offset=int(off), top_k_row=top_k_row,
                                          top_p_row=top_p_row, temperature=temperature,
                                          splits_override=int(splits))

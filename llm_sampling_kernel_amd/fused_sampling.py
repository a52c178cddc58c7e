"""The sampler's torch module: the reference's extension module ``fused_sampling``.

Same function names, argument order and meaning as csrc/bindings.cpp:16-25, and the same
``RuntimeError`` messages for the checks the reference makes (csrc/fused_sampling.cu:341-357,
:422-424).  Every function is the compiled extension ``_fsamp_torch`` (csrc/fsamp_torch.cpp),
which launches libfsamp.so's kernels through the C ABI of include/fsamp.h on torch's current
HIP stream.  There is no other implementation behind these names: if the extension is not
built, importing this module fails.

Deliberate differences from the reference:
  - top_k may be up to 1024 (reference: 128), so the "top_k must be <= ..." message names 1024;
  - ``stages_fused`` refuses a negative offset (the reference would use it as a huge unsigned
    offset).
``offset < 0`` (the generator path, csrc/fused_sampling.cu:441-447) takes the seed and offset
from torch's default generator of the logits' device with philox_cuda_state(4), as the
reference does, so eager calls and HIP-graph replays draw from one generator stream.

Additions with no counterpart in the reference:
  sample_fused_u / stages_fused_u   one explicit fp32 uniform per row;
  sample_fused_ex                   per-row top_k / top_p / temperature (SEMANTICS.md lists
                                    them as open);
  topk_shard / merge_sample         the vocabulary-parallel split of the sampler: per-shard
                                    sorted candidate words, then the merge and draw;
  probe_load                        the load-only floor of the large-batch launch shape;
  probe_stream                      the streaming-read floor of the whole batch, no row shape.
"""

from __future__ import annotations

import ctypes

import torch  # noqa: F401  (loads libtorch before the extension)

from . import _lib
from ._fsamp_torch import (  # noqa: F401
    kernel_attrs,
    merge_sample,
    probe_load,
    probe_noop,
    probe_phase,
    probe_scan_rowblock,
    probe_scan_split,
    probe_stream,
    sample_fused,
    sample_fused_ex,
    sample_fused_u,
    stages_fused,
    stages_fused_u,
    topk_fused,
    topk_shard,
)


def make_plan(logits: torch.Tensor, top_k: int, splits_override: int = 0) -> _lib.Plan:
    """The launch plan (split count, workgroup size, register tiling) for these logits."""
    plan = _lib.Plan()
    _lib.check(_lib.load().fsamp_make_plan(ctypes.c_void_p(logits.data_ptr()), logits.shape[0],
                                           logits.shape[1], int(top_k), int(splits_override),
                                           ctypes.byref(plan)))
    return plan

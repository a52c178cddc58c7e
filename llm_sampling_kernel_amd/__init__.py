"""MI355X-native fused top-k + top-p sampler (gfx950 HIP kernels behind a C ABI).

``fused_sampling`` mirrors the reference extension module, ``fused`` its Python front end.
The compute path is libfsamp.so (built by ``python -m llm_sampling_kernel_amd.build``).
"""

from . import fused, fused_sampling  # noqa: F401
from .fused import DEFAULT_SEED, sample_fused, sample_fused_u, topk_fused  # noqa: F401

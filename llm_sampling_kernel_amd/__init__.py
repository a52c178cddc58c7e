"""MI355X-native fused top-k + top-p sampler (gfx950 HIP kernels behind a C ABI).

``fused_sampling`` mirrors the reference extension module, ``fused`` its Python front end.
The compute path is libfsamp.so (built by ``python -m llm_sampling_kernel_amd.build``).

The package imports its submodules on first use, so that ``llm_sampling_kernel_amd.build``
can run in a fresh checkout where libfsamp.so and the torch extension are not built yet.
Using any sampler name without them fails at that point: there is no fallback.
"""

import importlib

_FROM_FUSED = ("DEFAULT_SEED", "sample_fused", "sample_fused_u", "topk_fused")


def __getattr__(name):
    if name in ("fused", "fused_sampling"):
        return importlib.import_module(f"{__name__}.{name}")
    if name in _FROM_FUSED:
        return getattr(importlib.import_module(f"{__name__}.fused"), name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")

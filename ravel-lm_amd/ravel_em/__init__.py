"""MI355X-native RAVEL event-memory operator.

Drop-in for the reference module ``ravel_lm/ravel_memory.py``: the public
functions below keep its names and signatures and run as hand-written HIP
kernels for gfx950 behind the C ABI in include/ravel_em.h.
"""
from .ravel_memory import (
    RavelLayerCache,
    _composite_key_dtype,
    causal_last_k_lookup,
    causal_last_k_sources,
    causal_sum_lookup,
    sort_order,
)

__all__ = [
    "RavelLayerCache",
    "_composite_key_dtype",
    "causal_last_k_lookup",
    "causal_last_k_sources",
    "causal_sum_lookup",
    "sort_order",
]

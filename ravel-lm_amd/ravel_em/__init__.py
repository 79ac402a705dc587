"""MI355X-native RAVEL event-memory operator.

Drop-in for the reference module ``ravel_lm/ravel_memory.py``: the public
functions below keep its names and signatures and run as hand-written HIP
kernels for gfx950 behind the C ABI in include/ravel_em.h.  ``fused_latest1_linear``
replaces the reference's fused arm ``triton_fused_latest1_linear``
(ravel_lm/triton_memory.py:477-485).  ``LayerAddresses`` lets the lookups
produce the memory layer's addresses (ravel_lm/model.py:195-231, :303-307)
inside their kernels.
"""
from .addressing import (LayerAddresses, literal_addresses_from_tokens, literal_addresses_step,
                         product_code_addresses)
from .fused import fused_latest1_linear
from .ravel_memory import (
    RavelLayerCache,
    _composite_key_dtype,
    causal_last_k_and_sum_lookup,
    causal_last_k_lookup,
    causal_last_k_sources,
    causal_sum_lookup,
    sort_order,
)

__all__ = [
    "LayerAddresses",
    "RavelLayerCache",
    "_composite_key_dtype",
    "causal_last_k_and_sum_lookup",
    "causal_last_k_lookup",
    "causal_last_k_sources",
    "causal_sum_lookup",
    "fused_latest1_linear",
    "literal_addresses_from_tokens",
    "literal_addresses_step",
    "product_code_addresses",
    "sort_order",
]

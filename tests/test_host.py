"""Host-side behaviour of the drop-in module that needs no GPU: the same
exceptions as the reference for bad arguments (ravel_lm/ravel_memory.py:87-97,
:140-141, :195-196, :274-275, :287-288), the key-dtype rule, and a loud error
instead of any CPU fallback when tensors are not on a ROCm device."""
import pytest
import torch

import ravel_em
from ravel_em import (RavelLayerCache, causal_last_k_and_sum_lookup, causal_last_k_lookup,
                      causal_sum_lookup)
from ravel_em.ravel_memory import _composite_key_dtype


def test_composite_key_dtype_uses_int32_only_when_safe():
    # tests/test_memory.py:11-13 of the reference
    assert _composite_key_dtype(1, 2048, 3, 1024) == torch.int32
    assert _composite_key_dtype(1024, 65536, 64, 65536) == torch.int64


def test_public_names_match_reference_module():
    for name in ["causal_last_k_lookup", "causal_sum_lookup", "RavelLayerCache", "_composite_key_dtype"]:
        assert hasattr(ravel_em.ravel_memory, name)
    import inspect

    sig = inspect.signature(causal_last_k_lookup)
    assert list(sig.parameters) == ["write_addresses", "payloads", "read_addresses", "address_space", "k", "write_mask"]
    assert sig.parameters["address_space"].kind is inspect.Parameter.KEYWORD_ONLY
    assert sig.parameters["k"].default == 1
    sig = inspect.signature(causal_sum_lookup)
    assert list(sig.parameters) == ["write_addresses", "payloads", "read_addresses", "address_space", "write_mask"]
    # the joint call takes causal_last_k_lookup's arguments
    sig = inspect.signature(causal_last_k_and_sum_lookup)
    assert list(sig.parameters) == ["write_addresses", "payloads", "read_addresses", "address_space", "k", "write_mask"]
    assert sig.parameters["address_space"].kind is inspect.Parameter.KEYWORD_ONLY


def test_shape_errors_match_reference():
    a = torch.zeros(2, 5, 3, dtype=torch.long)
    p = torch.zeros(2, 5, 3, 4)
    with pytest.raises(ValueError, match="same shape"):
        causal_last_k_lookup(a, p, torch.zeros(2, 5, 2, dtype=torch.long), address_space=8)
    with pytest.raises(ValueError, match=r"\[B, T, C\]"):
        causal_last_k_lookup(a[0], p, a[0], address_space=8)
    with pytest.raises(ValueError, match=r"\[B, T, C, D\]"):
        causal_last_k_lookup(a, p[0], address_space=8)
    with pytest.raises(ValueError, match="leading dimensions"):
        causal_last_k_lookup(a, torch.zeros(2, 4, 3, 4), address_space=8)
    with pytest.raises(ValueError, match="k must be positive"):
        causal_last_k_lookup(a, p, address_space=8, k=0)
    with pytest.raises(ValueError, match="write_mask"):
        causal_last_k_lookup(a, p, address_space=8, write_mask=torch.ones(2, 4, dtype=torch.bool))
    with pytest.raises(ValueError, match="expected write_addresses"):
        causal_sum_lookup(a[0], p, address_space=8)
    with pytest.raises(ValueError, match="same shape"):
        causal_last_k_and_sum_lookup(a, p, torch.zeros(2, 5, 2, dtype=torch.long), address_space=8)
    with pytest.raises(ValueError, match="k must be positive"):
        causal_last_k_and_sum_lookup(a, p, address_space=8, k=0)
    with pytest.raises(ValueError, match="write_mask"):
        causal_last_k_and_sum_lookup(a, p, address_space=8, write_mask=torch.ones(2, 4, dtype=torch.bool))


def test_cache_shape_errors_match_reference():
    cache = RavelLayerCache.empty(1, 2, 16, 3, device="cpu", dtype=torch.float32)
    assert cache.values.shape == (1, 2, 16, 3) and cache.filled.shape == (1, 2, 16)
    with pytest.raises(ValueError, match="does not match"):
        cache.read(torch.tensor([[5, 7, 1]]))
    with pytest.raises(ValueError, match="do not match"):
        cache.write(torch.tensor([[5, 7]]), torch.zeros(1, 2, 4))
    k4 = RavelLayerCache.empty(2, 3, 8, 5, device="cpu", dtype=torch.bfloat16, k=4)
    assert k4.values.shape == (2, 3, 8, 4, 5) and k4.filled.shape == (2, 3, 8, 4) and k4.k == 4


def test_cpu_tensors_raise_instead_of_falling_back():
    a = torch.zeros(1, 5, 1, dtype=torch.long)
    p = torch.zeros(1, 5, 1, 2)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        causal_last_k_lookup(a, p, address_space=8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        causal_sum_lookup(a, p, address_space=8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        causal_last_k_and_sum_lookup(a, p, address_space=8)
    cache = RavelLayerCache.empty(1, 2, 16, 3, device="cpu", dtype=torch.float32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        cache.read(torch.tensor([[5, 7]]))


def test_unsupported_payload_dtype_is_a_type_error():
    from ravel_em import _native as nat

    with pytest.raises(TypeError):
        nat.payload_code(torch.int32)


def test_fused_latest1_linear_errors_match_reference():
    # ravel_lm/triton_memory.py:390-395
    from ravel_em import fused_latest1_linear

    w = torch.zeros(2, 3, 4, dtype=torch.long)
    p = torch.zeros(2, 3, 4, 8)
    with pytest.raises(ValueError, match=r"expected write/read \[B,T,C\]"):
        fused_latest1_linear(w[0], p, None, torch.zeros(5, 32), address_space=9)
    with pytest.raises(ValueError, match=r"weight must have shape \[M, C \* P\]"):
        fused_latest1_linear(w, p, None, torch.zeros(5, 31), address_space=9)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        fused_latest1_linear(w, p, None, torch.zeros(5, 32), address_space=9)


def test_eager_fast_path_only_for_plain_tensors_outside_compile():
    """Plain tensors outside torch.compile may skip the dispatcher; a tensor
    subclass (as torch.compile's fake tensors are) or tracing keeps the op."""
    from ravel_em import _ops

    class Sub(torch.Tensor):
        pass

    t = torch.zeros(2, 3, 4)
    assert _ops.eager(t, None, t)
    assert not _ops.eager(t, t.as_subclass(Sub))
    compiled = torch.compile(lambda x: x + int(_ops.eager(x)), backend="eager", fullgraph=True)
    assert compiled(torch.zeros(1)).item() == 0.0

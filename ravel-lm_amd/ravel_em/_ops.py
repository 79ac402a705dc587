"""torch.library custom ops over the C ABI.

The ops carry fake (meta) implementations and autograd formulas so that
``torch.compile(fullgraph=True)`` can trace through them, following the
custom_op + register_fake + register_autograd pattern of the reference's MPS arm
(ravel_lm/mps_memory.py:109-187).  Every op launches on torch's current stream
and allocates its workspace from torch's caching allocator.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as nat

Tensor = torch.Tensor


def _call(fn, *args) -> None:
    nat.check(fn(*args))


def eager(*tensors: Optional[Tensor]) -> bool:
    """True when a call may run an op's implementation directly instead of
    through the dispatcher: nothing is tracing (no torch.compile) and every
    tensor is a plain tensor (no fake, meta-programming or other subclass).
    The callers also require that no autograd graph is recorded.  The
    dispatcher costs several microseconds a call, which short tapes notice."""
    if torch.compiler.is_compiling():
        return False
    return all(t is None or type(t) is torch.Tensor for t in tensors)


# ------------------------------------------------------------- latest-k --


def latest_k_impl(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
    k: int,
    want_src: bool,
) -> Tuple[Tensor, Tensor, Tensor]:
    """The body of ravel_em::latest_k (also called directly, see eager)."""
    lib = nat.library()
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    values = payloads.new_empty(B, T, C, k, D)
    mask = torch.empty(B, T, C, k, dtype=torch.bool, device=dev)
    src = torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev)
    has_read = read_addresses is not None
    has_mask = write_mask is not None
    nbytes = lib.ravel_em_latest_k_workspace(B, T, C, address_space, k, int(has_read), int(has_mask), int(want_src))
    ws = nat.workspace(nbytes, dev)
    _call(
        lib.ravel_em_latest_k_fwd,
        nat.ptr(write_addresses), nat.ptr(read_addresses), nat.addr_code(write_addresses.dtype),
        nat.ptr(write_mask), nat.ptr(payloads), nat.payload_code(payloads.dtype),
        B, T, C, D, address_space, k,
        nat.ptr(values), nat.ptr(mask), nat.ptr(src) if want_src else None,
        nat.ptr(ws), ws.numel(), nat.stream_of(payloads),
    )
    nat.after_call(ws)
    return values, mask, src


@torch.library.custom_op("ravel_em::latest_k", mutates_args=())
def latest_k(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
    k: int,
    want_src: bool,
) -> Tuple[Tensor, Tensor, Tensor]:
    return latest_k_impl(write_addresses, payloads, read_addresses, write_mask, address_space, k,
                         want_src)


@latest_k.register_fake
def _latest_k_fake(write_addresses, payloads, read_addresses, write_mask, address_space, k, want_src):
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    return (
        payloads.new_empty(B, T, C, k, D),
        torch.empty(B, T, C, k, dtype=torch.bool, device=dev),
        torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev),
    )


@torch.library.custom_op("ravel_em::latest_k_backward", mutates_args=())
def latest_k_backward(src: Tensor, grad_values: Tensor, chain: bool) -> Tensor:
    lib = nat.library()
    B, T, C, k, D = grad_values.shape
    grad_values = grad_values.contiguous()
    grad_payload = grad_values.new_empty(B, T, C, D)
    code = nat.payload_code(grad_values.dtype)
    nbytes = lib.ravel_em_latest_k_bwd_workspace(B, T, C, D, k, code, int(chain))
    ws = nat.workspace(nbytes, grad_values.device)
    _call(
        lib.ravel_em_latest_k_bwd,
        nat.ptr(src), nat.ptr(grad_values), code, B, T, C, D, k, int(chain),
        nat.ptr(grad_payload), nat.ptr(ws), ws.numel(), nat.stream_of(grad_values),
    )
    if not chain:  # the sorted form's workspace carries a status word
        nat.after_call(ws)
    return grad_payload


@latest_k_backward.register_fake
def _latest_k_backward_fake(src, grad_values, chain):
    B, T, C, k, D = grad_values.shape
    return grad_values.new_empty(B, T, C, D)


def _latest_k_setup(ctx, inputs, output):
    write_addresses, payloads, read_addresses, write_mask, address_space, k, want_src = inputs
    _, mask, src = output
    ctx.save_for_backward(src)
    ctx.chain = read_addresses is None and write_mask is None
    ctx.want_src = want_src
    ctx.mark_non_differentiable(mask, src)


def _latest_k_grad(ctx, grad_values, _grad_mask, _grad_src):
    (src,) = ctx.saved_tensors
    if not ctx.want_src:
        raise RuntimeError("ravel_em.latest_k was called without sources; cannot differentiate")
    grad_payload = latest_k_backward(src, grad_values, ctx.chain)
    return None, grad_payload, None, None, None, None, None


latest_k.register_autograd(_latest_k_grad, setup_context=_latest_k_setup)


# -------------------------------------------------------------- seg-sum --


def seg_sum_impl(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
) -> Tuple[Tensor, Tensor]:
    """The body of ravel_em::seg_sum (also called directly, see eager)."""
    lib = nat.library()
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    out = payloads.new_empty(B, T, C, D)
    mask = torch.empty(B, T, C, dtype=torch.bool, device=dev)
    code = nat.payload_code(payloads.dtype)
    nbytes = lib.ravel_em_seg_sum_workspace(
        B, T, C, D, address_space, int(read_addresses is not None), int(write_mask is not None), code
    )
    ws = nat.workspace(nbytes, dev)
    _call(
        lib.ravel_em_seg_sum_fwd,
        nat.ptr(write_addresses), nat.ptr(read_addresses), nat.addr_code(write_addresses.dtype),
        nat.ptr(write_mask), nat.ptr(payloads), code, B, T, C, D, address_space,
        nat.ptr(out), nat.ptr(mask), nat.ptr(ws), ws.numel(), nat.stream_of(payloads),
    )
    nat.after_call(ws)
    return out, mask


@torch.library.custom_op("ravel_em::seg_sum", mutates_args=())
def seg_sum(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
) -> Tuple[Tensor, Tensor]:
    return seg_sum_impl(write_addresses, payloads, read_addresses, write_mask, address_space)


@seg_sum.register_fake
def _seg_sum_fake(write_addresses, payloads, read_addresses, write_mask, address_space):
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    return payloads.new_empty(B, T, C, D), torch.empty(B, T, C, dtype=torch.bool, device=payloads.device)


@torch.library.custom_op("ravel_em::seg_sum_backward", mutates_args=())
def seg_sum_backward(
    write_addresses: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    grad_sum: Tensor,
    address_space: int,
) -> Tensor:
    lib = nat.library()
    B, T, C, D = grad_sum.shape
    grad_sum = grad_sum.contiguous()
    grad_payload = grad_sum.new_empty(B, T, C, D)
    code = nat.payload_code(grad_sum.dtype)
    nbytes = lib.ravel_em_seg_sum_bwd_workspace(
        B, T, C, D, address_space, int(read_addresses is not None), int(write_mask is not None), code
    )
    ws = nat.workspace(nbytes, grad_sum.device)
    _call(
        lib.ravel_em_seg_sum_bwd,
        nat.ptr(write_addresses), nat.ptr(read_addresses), nat.addr_code(write_addresses.dtype),
        nat.ptr(write_mask), nat.ptr(grad_sum), code, B, T, C, D, address_space,
        nat.ptr(grad_payload), nat.ptr(ws), ws.numel(), nat.stream_of(grad_sum),
    )
    nat.after_call(ws)
    return grad_payload


@seg_sum_backward.register_fake
def _seg_sum_backward_fake(write_addresses, read_addresses, write_mask, grad_sum, address_space):
    return grad_sum.new_empty(grad_sum.shape)


def _seg_sum_setup(ctx, inputs, output):
    write_addresses, payloads, read_addresses, write_mask, address_space = inputs
    ctx.save_for_backward(write_addresses, read_addresses, write_mask)
    ctx.address_space = address_space
    ctx.mark_non_differentiable(output[1])


def _seg_sum_grad(ctx, grad_sum, _grad_mask):
    write_addresses, read_addresses, write_mask = ctx.saved_tensors
    grad_payload = seg_sum_backward(write_addresses, read_addresses, write_mask, grad_sum, ctx.address_space)
    return None, grad_payload, None, None, None


seg_sum.register_autograd(_seg_sum_grad, setup_context=_seg_sum_setup)


# ------------------------------------------------------ latest-k + sum --


def latest_k_sum_impl(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
    k: int,
    want_src: bool,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The body of ravel_em::latest_k_sum (also called directly, see eager):
    (values, mask, src, sum, sum_mask) of one tape in one C call."""
    lib = nat.library()
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    values = payloads.new_empty(B, T, C, k, D)
    mask = torch.empty(B, T, C, k, dtype=torch.bool, device=dev)
    src = torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev)
    out = payloads.new_empty(B, T, C, D)
    smask = torch.empty(B, T, C, dtype=torch.bool, device=dev)
    code = nat.payload_code(payloads.dtype)
    nbytes = lib.ravel_em_latest_k_sum_workspace(
        B, T, C, D, address_space, k, int(read_addresses is not None), int(write_mask is not None),
        int(want_src), code)
    ws = nat.workspace(nbytes, dev)
    _call(
        lib.ravel_em_latest_k_sum_fwd,
        nat.ptr(write_addresses), nat.ptr(read_addresses), nat.addr_code(write_addresses.dtype),
        nat.ptr(write_mask), nat.ptr(payloads), code, B, T, C, D, address_space, k,
        nat.ptr(values), nat.ptr(mask), nat.ptr(src) if want_src else None, nat.ptr(out),
        nat.ptr(smask), nat.ptr(ws), ws.numel(), nat.stream_of(payloads),
    )
    nat.after_call(ws)
    return values, mask, src, out, smask


@torch.library.custom_op("ravel_em::latest_k_sum", mutates_args=())
def latest_k_sum(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    write_mask: Optional[Tensor],
    address_space: int,
    k: int,
    want_src: bool,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return latest_k_sum_impl(write_addresses, payloads, read_addresses, write_mask, address_space,
                             k, want_src)


@latest_k_sum.register_fake
def _latest_k_sum_fake(write_addresses, payloads, read_addresses, write_mask, address_space, k,
                       want_src):
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    return (
        payloads.new_empty(B, T, C, k, D),
        torch.empty(B, T, C, k, dtype=torch.bool, device=dev),
        torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev),
        payloads.new_empty(B, T, C, D),
        torch.empty(B, T, C, dtype=torch.bool, device=dev),
    )


def _latest_k_sum_setup(ctx, inputs, output):
    write_addresses, payloads, read_addresses, write_mask, address_space, k, want_src = inputs
    _, mask, src, _, smask = output
    ctx.save_for_backward(src, write_addresses, read_addresses, write_mask)
    ctx.chain = read_addresses is None and write_mask is None
    ctx.want_src = want_src
    ctx.address_space = address_space
    ctx.mark_non_differentiable(mask, src, smask)


def _latest_k_sum_grad(ctx, grad_values, _grad_mask, _grad_src, grad_sum, _grad_smask):
    src, write_addresses, read_addresses, write_mask = ctx.saved_tensors
    if not ctx.want_src:
        raise RuntimeError("ravel_em.latest_k_sum was called without sources; cannot differentiate")
    grad_payload = latest_k_backward(src, grad_values, ctx.chain)
    grad_payload = grad_payload + seg_sum_backward(write_addresses, read_addresses, write_mask,
                                                   grad_sum, ctx.address_space)
    return None, grad_payload, None, None, None, None, None


latest_k_sum.register_autograd(_latest_k_sum_grad, setup_context=_latest_k_sum_setup)


# ------------------------------------------------------- direct C calls --


def sort_order(write_addresses: Tensor, write_mask: Optional[Tensor], address_space: int,
               key_dtype: torch.dtype) -> Tuple[Tensor, Tensor]:
    """(sorted_keys, order) exactly as torch.sort of the reference's flat keys."""
    lib = nat.library()
    B, T, C = write_addresses.shape
    dev = write_addresses.device
    n_valid = B * T * C if write_mask is None else C * int(write_mask.sum().item())
    keys = torch.empty(n_valid, dtype=key_dtype, device=dev)
    order = torch.empty(n_valid, dtype=torch.int64, device=dev)
    if n_valid == 0:
        return keys, order
    nbytes = lib.ravel_em_sort_order_workspace(B, T, C, address_space, int(write_mask is not None))
    ws = nat.workspace(nbytes, dev)
    _call(
        lib.ravel_em_sort_order,
        nat.ptr(write_addresses), nat.addr_code(write_addresses.dtype), nat.ptr(write_mask),
        B, T, C, address_space, nat.ptr(keys), nat.ptr(order), nat.ptr(ws), ws.numel(),
        nat.stream_of(write_addresses),
    )
    nat.after_call(ws)
    return keys, order


def cache_read(values: Tensor, filled: Tensor, addresses: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    lib = nat.library()
    B, C, A = filled.shape[:3]
    D = values.shape[-1]
    out = values.new_empty(B, C, k, D)
    mask = torch.empty(B, C, k, dtype=torch.bool, device=values.device)
    _call(
        lib.ravel_em_cache_read,
        nat.ptr(values), nat.ptr(filled), nat.ptr(addresses), nat.addr_code(addresses.dtype),
        nat.payload_code(values.dtype), B, C, A, k, D, nat.ptr(out), nat.ptr(mask),
        nat.stream_of(values),
    )
    return out, mask


def cache_write(values: Tensor, filled: Tensor, addresses: Tensor, payloads: Tensor, k: int) -> None:
    lib = nat.library()
    B, C, A = filled.shape[:3]
    D = values.shape[-1]
    _call(
        lib.ravel_em_cache_write,
        nat.ptr(values), nat.ptr(filled), nat.ptr(addresses), nat.addr_code(addresses.dtype),
        nat.ptr(payloads), nat.payload_code(values.dtype), B, C, A, k, D, nat.stream_of(values),
    )


def cache_step(values: Tensor, filled: Tensor, read_addresses: Tensor, write_addresses: Tensor,
               payloads: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    lib = nat.library()
    B, C, A = filled.shape[:3]
    D = values.shape[-1]
    out = values.new_empty(B, C, k, D)
    mask = torch.empty(B, C, k, dtype=torch.bool, device=values.device)
    _call(
        lib.ravel_em_cache_step,
        nat.ptr(values), nat.ptr(filled), nat.ptr(read_addresses), nat.ptr(write_addresses),
        nat.addr_code(read_addresses.dtype), nat.ptr(payloads), nat.payload_code(values.dtype),
        B, C, A, k, D, nat.ptr(out), nat.ptr(mask), nat.stream_of(values),
    )
    return out, mask


def cache_prefill(write_addresses: Tensor, payloads: Tensor, write_mask: Optional[Tensor],
                  address_space: int, k: int, values: Tensor, filled: Tensor) -> None:
    lib = nat.library()
    B, T, C = write_addresses.shape
    D = payloads.shape[-1]
    dev = payloads.device
    nbytes = lib.ravel_em_cache_prefill_workspace(B, T, C, address_space, int(write_mask is not None))
    ws = nat.workspace(nbytes, dev)
    _call(
        lib.ravel_em_cache_prefill,
        nat.ptr(write_addresses), nat.addr_code(write_addresses.dtype), nat.ptr(write_mask),
        nat.ptr(payloads), nat.payload_code(payloads.dtype), B, T, C, D, address_space, k,
        nat.ptr(values), nat.ptr(filled), nat.ptr(ws), ws.numel(), nat.stream_of(payloads),
    )
    nat.after_call(ws)

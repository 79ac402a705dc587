"""The latest-1 lookup fused into the fuse layer's linear map.

Drop-in for the reference's fused arm ``triton_fused_latest1_linear``
(ravel_lm/triton_memory.py:477-485; forward and backward of its autograd
function :378-475), which ravel_lm/model.py:350-365 calls instead of
``causal_last_k_lookup`` + ``fast_linear`` when k == 1, no sum read and no write
mask:

    out[b, t, :] = weight @ concat_c(values[b, t, c, :])

with ``values`` the latest-1 lookup.  On the device the looked-up rows are
gathered straight into the MFMA tiles of the GEMM (``ravel_em_latest1_linear_fwd``)
and never stored: bf16/f16 payloads with P % 8 == 0 and f32 payloads with
P % 4 == 0 (the reference model runs fp32 when autocast is off), any M.  Other
shapes (f64 payloads, other P, a weight of another dtype) run the lookup kernels
followed by a library GEMM on the device.  There is no CPU path.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as nat
from . import _ops
from .addressing import LayerAddresses

Tensor = torch.Tensor


def _mfma_ok(payloads: Tensor, weight: Tensor) -> bool:
    """The MFMA kernel takes bf16/f16 payloads with P % 8 == 0 and f32 payloads
    with P % 4 == 0 (16-byte units of a head's row), weight of the payload
    dtype, both 16-byte aligned; any M."""
    P = payloads.shape[-1]
    aligned = all(t.data_ptr() % 16 == 0 for t in (payloads, weight))
    per_unit = {torch.bfloat16: 8, torch.float16: 8, torch.float32: 4}.get(payloads.dtype)
    return (per_unit is not None and P % per_unit == 0 and weight.dtype == payloads.dtype
            and weight.shape[0] >= 1 and aligned)


@torch.library.custom_op("ravel_em::latest1_linear", mutates_args=())
def _latest1_linear(write_addresses: Tensor, payloads: Tensor, read_addresses: Optional[Tensor],
                    weight: Tensor, address_space: int) -> Tuple[Tensor, Tensor]:
    B, T, C, P = payloads.shape
    M = weight.shape[0]
    dev = payloads.device
    src = torch.empty(B, T, C, dtype=torch.int32, device=dev)
    if _mfma_ok(payloads, weight):
        lib = nat.library()
        out = payloads.new_empty(B, T, M)
        nbytes = lib.ravel_em_latest1_linear_workspace(B, T, C, address_space,
                                                       int(read_addresses is not None), 1)
        ws = nat.workspace(nbytes, dev)
        nat.check(lib.ravel_em_latest1_linear_fwd(
            nat.ptr(write_addresses), nat.ptr(read_addresses), nat.addr_code(write_addresses.dtype),
            nat.ptr(payloads), nat.payload_code(payloads.dtype), nat.ptr(weight),
            B, T, C, P, M, address_space, nat.ptr(out), nat.ptr(src), nat.ptr(ws), ws.numel(),
            nat.stream_of(payloads)))
        nat.after_call(ws)
        return out, src
    values, _, s = _ops.latest_k(write_addresses, payloads, read_addresses, None, address_space, 1, True)
    out = torch.matmul(values.reshape(B * T, C * P), weight.t()).reshape(B, T, M)
    return out, s.view(B, T, C)


@_latest1_linear.register_fake
def _latest1_linear_fake(write_addresses, payloads, read_addresses, weight, address_space):
    B, T, C, P = payloads.shape
    return (payloads.new_empty(B, T, weight.shape[0]),
            torch.empty(B, T, C, dtype=torch.int32, device=payloads.device))


def _setup(ctx, inputs, output):
    write_addresses, payloads, read_addresses, weight, address_space = inputs
    _, src = output
    ctx.save_for_backward(src, payloads, weight)
    ctx.chain = read_addresses is None
    ctx.mark_non_differentiable(src)


def _grads(ctx, grad_out, need_payload: bool, need_weight: bool):
    """ravel_lm/triton_memory.py:428-475: grad_weight = grad^T @ read_flat,
    grad_payload = scatter of grad @ weight through the sources."""
    src, payloads, weight = ctx.saved_tensors
    B, T, C, P = payloads.shape
    M = weight.shape[0]
    grad2d = grad_out.reshape(B * T, M).to(payloads.dtype)
    grad_weight = grad_payload = None
    if need_weight:
        read_flat = gather_read_rows(payloads, src)
        grad_weight = torch.matmul(grad2d.t(), read_flat.reshape(B * T, C * P)).to(weight.dtype)
    if need_payload:
        grad_read = torch.matmul(grad2d, weight).reshape(B, T, C, 1, P).contiguous()
        grad_payload = _ops.latest_k_backward(src.view(B, T, C, 1), grad_read, ctx.chain)
    return grad_payload, grad_weight


def _backward(ctx, grad_out, _grad_src):
    gp, gw = _grads(ctx, grad_out, ctx.needs_input_grad[1], ctx.needs_input_grad[3])
    return None, gp, None, gw, None


_latest1_linear.register_autograd(_backward, setup_context=_setup)


@torch.library.custom_op("ravel_em::latest1_linear_gen", mutates_args=())
def _latest1_linear_gen(tokens: Optional[Tensor], history: Optional[Tensor],
                        write_logits: Optional[Tensor], read_logits: Optional[Tensor],
                        payloads: Tensor, weight: Tensor, n_literal: int, bos: int,
                        n_learned: int, ncb: int, cbs: int, position: int,
                        address_space: int) -> Tuple[Tensor, Tensor]:
    B, T, C, P = payloads.shape
    M = weight.shape[0]
    dev = payloads.device
    w = nat.addr_gen(tokens, n_literal, bos, write_logits, n_learned, ncb, cbs, history, position)
    r = None if read_logits is None else nat.addr_gen(tokens, n_literal, bos, read_logits,
                                                      n_learned, ncb, cbs, history, position)
    if _mfma_ok(payloads, weight):
        lib = nat.library()
        src = torch.empty(B, T, C, dtype=torch.int32, device=dev)
        out = payloads.new_empty(B, T, M)
        nbytes = lib.ravel_em_latest1_linear_workspace(B, T, C, address_space, int(r is not None), 1)
        ws = nat.workspace(nbytes, dev)
        nat.check(lib.ravel_em_latest1_linear_fwd(
            nat.ref(w), nat.ref(r), nat.ADDR_GEN, nat.ptr(payloads), nat.payload_code(payloads.dtype),
            nat.ptr(weight), B, T, C, P, M, address_space, nat.ptr(out), nat.ptr(src), nat.ptr(ws),
            ws.numel(), nat.stream_of(payloads)))
        nat.after_call(ws)
        return out, src
    from .addressing import latest_k_gen

    values, _, s = latest_k_gen(tokens, history, write_logits, read_logits, payloads, None,
                                n_literal, bos, n_learned, ncb, cbs, position, address_space, 1,
                                True)
    out = torch.matmul(values.reshape(B * T, C * P), weight.t()).reshape(B, T, M)
    return out, s.view(B, T, C)


@_latest1_linear_gen.register_fake
def _latest1_linear_gen_fake(tokens, history, write_logits, read_logits, payloads, weight,
                             n_literal, bos, n_learned, ncb, cbs, position, address_space):
    B, T, C, P = payloads.shape
    return (payloads.new_empty(B, T, weight.shape[0]),
            torch.empty(B, T, C, dtype=torch.int32, device=payloads.device))


def _setup_gen(ctx, inputs, output):
    payloads, weight = inputs[4], inputs[5]
    _, src = output
    ctx.save_for_backward(src, payloads, weight)
    ctx.chain = inputs[3] is None
    ctx.mark_non_differentiable(src)


def _backward_gen(ctx, grad_out, _grad_src):
    gp, gw = _grads(ctx, grad_out, ctx.needs_input_grad[4], ctx.needs_input_grad[5])
    return (None, None, None, None, gp, gw) + (None,) * 7


_latest1_linear_gen.register_autograd(_backward_gen, setup_context=_setup_gen)


def gather_read_rows(payloads: Tensor, src: Tensor) -> Tensor:
    """[B,T,C,P] rows payload[src] (zeros where src < 0), on the device."""
    lib = nat.library()
    B, T, C, P = payloads.shape
    out = payloads.new_empty(B, T, C, P)
    n = B * T * C
    nat.check(lib.ravel_em_gather_rows(nat.ptr(payloads), n, P * payloads.element_size(),
                                       nat.ptr(src), n, nat.ptr(out), None, nat.stream_of(payloads)))
    return out


def fused_latest1_linear(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor],
    weight: Tensor,
    *,
    address_space: int,
) -> Tensor:
    """``weight @ concat_c(latest-1 values)`` for every (b, t): [B, T, M].

    Same contract as the reference's ``triton_fused_latest1_linear``
    (ravel_lm/triton_memory.py:390-395): write/read addresses [B,T,C], payloads
    [B,T,C,P], weight [M, C*P]; ``read_addresses=None`` reads where it writes.
    ``write_addresses`` may be a LayerAddresses (then read_addresses is None):
    the addresses are produced inside the sort and the read search.
    """
    if isinstance(write_addresses, LayerAddresses):
        return _fused_gen(write_addresses, payloads, read_addresses, weight, address_space)
    if payloads.ndim != 4 or write_addresses.ndim != 3 or (
        read_addresses is not None and read_addresses.ndim != 3
    ):
        raise ValueError("expected write/read [B,T,C] and payloads [B,T,C,P]")
    B, T, C, P = payloads.shape
    M = weight.shape[0]
    if weight.ndim != 2 or weight.shape != (M, C * P):
        raise ValueError("weight must have shape [M, C * P]")
    if write_addresses.shape != (B, T, C) or (
        read_addresses is not None and read_addresses.shape != (B, T, C)
    ):
        raise ValueError("expected write/read [B,T,C] and payloads [B,T,C,P]")
    if address_space <= 0:
        raise ValueError("address_space must be positive")
    nat.require_device(write_addresses, payloads, weight, read_addresses)
    from .ravel_memory import _composite_key_dtype, _prepare

    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, r = _prepare(write_addresses, read_addresses, key_dtype)
    out, _ = _latest1_linear(w, payloads.contiguous(), r, weight.to(payloads.dtype).contiguous(),
                             int(address_space))
    return out


def _fused_gen(src: LayerAddresses, payloads: Tensor, read_addresses, weight: Tensor,
               address_space: int) -> Tensor:
    if read_addresses is not None:
        raise ValueError("with LayerAddresses the read addresses come from its read_logits; "
                         "read_addresses must be None")
    B, T = src._check()
    if payloads.ndim != 4 or payloads.shape[:3] != (B, T, src.heads):
        raise ValueError("expected payloads [B,T,C,P] with C = literal + learned heads")
    C, P = src.heads, payloads.shape[-1]
    M = weight.shape[0]
    if weight.ndim != 2 or weight.shape != (M, C * P):
        raise ValueError("weight must have shape [M, C * P]")
    if address_space <= 0:
        raise ValueError("address_space must be positive")
    tok, hist, wl, rl = src.tensors()
    nat.require_device(payloads, weight, tok, hist, wl, rl)
    out, _ = _latest1_linear_gen(tok, hist, wl, rl, payloads.contiguous(),
                                 weight.to(payloads.dtype).contiguous(), *src.cfg(),
                                 int(address_space))
    return out

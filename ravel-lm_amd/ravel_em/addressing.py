"""Address production of the memory layer, inside the kernels.

The reference's memory layer builds two int64 [B, T, C] address tensors with a
chain of elementwise torch ops before every lookup (RavelMemoryLayer.forward,
ravel_lm/model.py:325-346): the literal families of
``literal_addresses_from_tokens`` (model.py:195-231) and the product codes of
the learned addressors (``_decode_codes``, model.py:303-307; the same decode as
ProductCodeAddressor.forward, model.py:177-187), concatenated literal-first.

Here a :class:`LayerAddresses` describes those inputs (token ids, addressor
logits) and the lookups take it in place of the write address tensor: the key
build and the read search compute each record's address where they need it, so
no address tensor is written or read.  ``literal_addresses_from_tokens`` and
``product_code_addresses`` produce the same addresses as tensors (one kernel
each) for callers that want them.  All of it runs on the device only.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _native as nat
from . import _ops

Tensor = torch.Tensor


def _tokens(token_ids: Tensor) -> Tensor:
    # The reference hashes token_ids.long(); int32 ids are read as they are.
    return token_ids if token_ids.dtype in (torch.int32, torch.int64) else token_ids.long()


def _logits(logits: Tensor, B: int, T: int) -> Tensor:
    # [B, T, N] with a unit last stride, as the slice of the layer's packed
    # projection is (model.py:335, :339-341); other layouts are made so.
    x = logits.reshape(B, T, -1)
    if x.stride(-1) != 1:
        x = x.contiguous()
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.float()
    return x


@dataclass(frozen=True)
class LayerAddresses:
    """Where a memory layer's addresses come from.

    Heads ``0 .. n_literal_heads-1`` are the literal families of token_ids
    (ravel_lm/model.py:195-231); heads ``n_literal_heads ..`` are the product
    codes of the addressor logits (model.py:177-187, :303-307).  Writes use
    ``write_logits``, reads ``read_logits`` (None: reads use the write
    addresses), as model.py:338-346 concatenates them.

    token_ids:     [B, T] integer token ids (needed when n_literal_heads > 0)
    write_logits:  [B, T, n_learned_heads * n_codebooks * codebook_size]
    read_logits:   same shape, or None
    token_history: [B, h] tokens before t = 0, newest last (None: a sequence
                   start, bos_token_id before it), as the decode step's
                   token_history [prev2, prev1] (model.py:234-263)
    position:      position of t = 0 for the token/position heads (j >= 3)
    """

    token_ids: Optional[Tensor]
    n_literal_heads: int
    bos_token_id: int
    write_logits: Optional[Tensor] = None
    read_logits: Optional[Tensor] = None
    n_learned_heads: int = 0
    n_codebooks: int = 2
    codebook_size: int = 16
    token_history: Optional[Tensor] = None
    position: int = 0

    @property
    def heads(self) -> int:
        return int(self.n_literal_heads) + int(self.n_learned_heads)

    @property
    def same(self) -> bool:
        """Reads use the write addresses."""
        return self.n_learned_heads == 0 or self.read_logits is None

    def shape(self) -> Tuple[int, int]:
        src = self.token_ids if self.n_literal_heads > 0 else self.write_logits
        if src is None:
            raise ValueError("LayerAddresses needs token_ids for literal heads and write_logits for learned heads")
        return int(src.shape[0]), int(src.shape[1])

    def _check(self) -> Tuple[int, int]:
        if self.n_literal_heads < 0 or self.n_learned_heads < 0:
            raise ValueError("head counts must be non-negative")
        if self.n_literal_heads > 0 and (self.token_ids is None or self.token_ids.ndim != 2):
            raise ValueError("token_ids must have shape [B,T]")
        B, T = self.shape()
        if self.n_literal_heads >= 3 and T < 2 and self.token_history is None:
            # The reference's torch.stack of its heads fails for these lengths.
            raise RuntimeError("the trigram literal head needs T >= 2")
        if self.token_history is not None and (self.token_history.ndim != 2 or
                                               self.token_history.shape[0] != B):
            raise ValueError("token_history must have shape [B, h]")
        if self.n_learned_heads > 0:
            if self.n_codebooks <= 0 or self.codebook_size <= 0:
                raise ValueError("n_codebooks and codebook_size must be positive")
            n = self.n_learned_heads * self.n_codebooks * self.codebook_size
            for name, x in (("write_logits", self.write_logits), ("read_logits", self.read_logits)):
                if x is None:
                    if name == "write_logits":
                        raise ValueError("learned heads need write_logits")
                    continue
                if x.shape[:2] != (B, T) or math.prod(x.shape[2:]) != n:
                    raise ValueError(f"{name} must have shape [B, T, {n}]")
        return B, T

    def tensors(self) -> Tuple[Optional[Tensor], Optional[Tensor], Optional[Tensor], Optional[Tensor]]:
        """(tokens, history, write_logits, read_logits) as the kernels read them."""
        B, T = self._check()
        tok = hist = None
        if self.n_literal_heads > 0:
            tok = _tokens(self.token_ids)
            if self.token_history is not None and self.token_history.shape[1] > 0:
                hist = self.token_history.to(tok.dtype)
        wl = rl = None
        if self.n_learned_heads > 0:
            wl = _logits(self.write_logits, B, T)
            if not self.same:
                rl = _logits(self.read_logits, B, T)
        return tok, hist, wl, rl

    def cfg(self) -> Tuple[int, int, int, int, int, int]:
        """(n_literal, bos, n_learned, n_codebooks, codebook_size, position)."""
        return (int(self.n_literal_heads), int(self.bos_token_id), int(self.n_learned_heads),
                int(self.n_codebooks), int(self.codebook_size), int(self.position))

    def materialize(self, *, address_space: int) -> Tuple[Tensor, Tensor]:
        """(write, read) int64 [B, T, C] address tensors, as model.py:338-346
        builds them (read is the write tensor when reads use write addresses)."""
        B, T = self._check()
        tok, hist, wl, rl = self.tensors()
        w = _addresses(tok, hist, wl, B, T, *self.cfg(), int(address_space))
        r = w if self.same else _addresses(tok, hist, rl, B, T, *self.cfg(), int(address_space))
        return w, r


def _check_space(address_space: int) -> None:
    if int(address_space) <= 0:
        raise ValueError("address_space must be positive")


def literal_addresses_from_tokens(
    token_ids: Tensor,
    *,
    address_space: int,
    n_heads: int,
    bos_token_id: int,
) -> Tensor:
    """Literal address families of token ids, [B, T, n_heads] int64.

    Same result as ravel_lm/model.py:195-231 (heads: token id, rolling bigram
    hash, rolling trigram hash, then token/position hashes), in one kernel.
    """
    if token_ids.ndim != 2:
        raise ValueError("token_ids must have shape [B,T]")
    B, T = token_ids.shape
    if n_heads <= 0:
        return torch.empty(B, T, 0, device=token_ids.device, dtype=torch.long)
    _check_space(address_space)
    src = LayerAddresses(token_ids, int(n_heads), int(bos_token_id))
    nat.require_device(token_ids)
    return src.materialize(address_space=address_space)[0]


def literal_addresses_step(
    token_ids: Tensor,
    token_history: Tensor,
    *,
    address_space: int,
    n_heads: int,
    position: int,
    bos_token_id: int,
) -> Tensor:
    """Literal addresses of one decode step, [B, n_heads] int64.

    Same result as ravel_lm/model.py:234-263: token_ids [B], token_history
    [B, h] holding the previous tokens newest last ([prev2, prev1]); a history
    shorter than two tokens reads bos_token_id before it.  One kernel.
    """
    B = token_ids.shape[0]
    if n_heads <= 0:
        return torch.empty(B, 0, device=token_ids.device, dtype=torch.long)
    _check_space(address_space)
    hist = token_history if token_history.ndim == 2 else token_history.view(B, -1)
    src = LayerAddresses(token_ids.reshape(B, 1), int(n_heads), int(bos_token_id),
                         token_history=hist, position=int(position))
    nat.require_device(token_ids, token_history)
    return src.materialize(address_space=address_space)[0].view(B, int(n_heads))


def product_code_addresses(
    logits: Tensor,
    *,
    n_heads: int,
    n_codebooks: int,
    codebook_size: int,
    address_space: int,
) -> Tensor:
    """Product-code addresses of addressor logits, [..., n_heads] int64.

    ``logits`` is [..., n_heads * n_codebooks * codebook_size]; the result is
    ``_decode_codes`` of ravel_lm/model.py:303-307 (argmax per codebook, codes
    packed with powers of codebook_size, remainder by address_space), in one
    kernel.
    """
    lead = tuple(logits.shape[:-1])
    if n_heads <= 0:
        return torch.empty(*lead, 0, device=logits.device, dtype=torch.long)
    _check_space(address_space)
    if logits.shape[-1] != n_heads * n_codebooks * codebook_size:
        raise RuntimeError(
            f"logits of last size {logits.shape[-1]} do not reshape to "
            f"[{n_heads}, {n_codebooks}, {codebook_size}]")
    nat.require_device(logits)
    x = logits.unsqueeze(0) if logits.ndim == 2 else logits
    if x.ndim != 3:
        x = x.reshape(1, -1, x.shape[-1])
    src = LayerAddresses(None, 0, 0, x, None, int(n_heads), int(n_codebooks), int(codebook_size))
    out = src.materialize(address_space=address_space)[0]
    return out.reshape(*lead, int(n_heads))


# ------------------------------------------------------------ custom ops --


def _descs(tokens, history, write_logits, read_logits, n_literal, bos, n_learned, ncb, cbs,
           position):
    w = nat.addr_gen(tokens, n_literal, bos, write_logits, n_learned, ncb, cbs, history, position)
    r = None if read_logits is None else nat.addr_gen(tokens, n_literal, bos, read_logits,
                                                      n_learned, ncb, cbs, history, position)
    return w, r


def _device_of(*ts) -> torch.device:
    for t in ts:
        if t is not None:
            return t.device
    raise ValueError("no input tensor")


@torch.library.custom_op("ravel_em::addresses", mutates_args=())
def _addresses(tokens: Optional[Tensor], history: Optional[Tensor], logits: Optional[Tensor],
               B: int, T: int, n_literal: int, bos: int, n_learned: int, ncb: int, cbs: int,
               position: int, address_space: int) -> Tensor:
    dev = _device_of(tokens, logits)
    out = torch.empty(B, T, n_literal + n_learned, dtype=torch.int64, device=dev)
    g = nat.addr_gen(tokens, n_literal, bos, logits, n_learned, ncb, cbs, history, position)
    nat.check(nat.library().ravel_em_addresses(nat.ref(g), B, T, address_space, nat.INT64,
                                               nat.ptr(out), torch.cuda.current_stream(dev).cuda_stream))
    return out


@_addresses.register_fake
def _addresses_fake(tokens, history, logits, B, T, n_literal, bos, n_learned, ncb, cbs, position,
                    address_space):
    return torch.empty(B, T, n_literal + n_learned, dtype=torch.int64, device=_device_of(tokens, logits))


@torch.library.custom_op("ravel_em::latest_k_gen", mutates_args=())
def latest_k_gen(tokens: Optional[Tensor], history: Optional[Tensor],
                 write_logits: Optional[Tensor], read_logits: Optional[Tensor], payloads: Tensor,
                 write_mask: Optional[Tensor], n_literal: int, bos: int, n_learned: int, ncb: int,
                 cbs: int, position: int, address_space: int, k: int,
                 want_src: bool) -> Tuple[Tensor, Tensor, Tensor]:
    lib = nat.library()
    B, T, C, D = payloads.shape
    dev = payloads.device
    values = payloads.new_empty(B, T, C, k, D)
    mask = torch.empty(B, T, C, k, dtype=torch.bool, device=dev)
    src = torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev)
    w, r = _descs(tokens, history, write_logits, read_logits, n_literal, bos, n_learned, ncb, cbs,
                  position)
    nbytes = lib.ravel_em_latest_k_workspace(B, T, C, address_space, k, int(r is not None),
                                             int(write_mask is not None), int(want_src))
    ws = nat.workspace(nbytes, dev)
    nat.check(lib.ravel_em_latest_k_fwd(
        nat.ref(w), nat.ref(r), nat.ADDR_GEN, nat.ptr(write_mask), nat.ptr(payloads),
        nat.payload_code(payloads.dtype), B, T, C, D, address_space, k, nat.ptr(values),
        nat.ptr(mask), nat.ptr(src) if want_src else None, nat.ptr(ws), ws.numel(),
        nat.stream_of(payloads)))
    nat.after_call(ws)
    return values, mask, src


@latest_k_gen.register_fake
def _latest_k_gen_fake(tokens, history, write_logits, read_logits, payloads, write_mask, n_literal,
                       bos, n_learned, ncb, cbs, position, address_space, k, want_src):
    B, T, C, D = payloads.shape
    dev = payloads.device
    return (payloads.new_empty(B, T, C, k, D),
            torch.empty(B, T, C, k, dtype=torch.bool, device=dev),
            torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev))


def _latest_k_gen_setup(ctx, inputs, output):
    read_logits, write_mask, want_src = inputs[3], inputs[5], inputs[-1]
    _, mask, src = output
    ctx.save_for_backward(src)
    ctx.chain = read_logits is None and write_mask is None
    ctx.want_src = want_src
    ctx.mark_non_differentiable(mask, src)


def _latest_k_gen_grad(ctx, grad_values, _grad_mask, _grad_src):
    (src,) = ctx.saved_tensors
    if not ctx.want_src:
        raise RuntimeError("ravel_em.latest_k_gen was called without sources; cannot differentiate")
    grad_payload = _ops.latest_k_backward(src, grad_values, ctx.chain)
    return (None, None, None, None, grad_payload) + (None,) * 10


latest_k_gen.register_autograd(_latest_k_gen_grad, setup_context=_latest_k_gen_setup)


@torch.library.custom_op("ravel_em::seg_sum_gen", mutates_args=())
def seg_sum_gen(tokens: Optional[Tensor], history: Optional[Tensor],
                write_logits: Optional[Tensor], read_logits: Optional[Tensor], payloads: Tensor,
                write_mask: Optional[Tensor], n_literal: int, bos: int, n_learned: int, ncb: int,
                cbs: int, position: int, address_space: int) -> Tuple[Tensor, Tensor]:
    lib = nat.library()
    B, T, C, D = payloads.shape
    dev = payloads.device
    out = payloads.new_empty(B, T, C, D)
    mask = torch.empty(B, T, C, dtype=torch.bool, device=dev)
    code = nat.payload_code(payloads.dtype)
    w, r = _descs(tokens, history, write_logits, read_logits, n_literal, bos, n_learned, ncb, cbs,
                  position)
    nbytes = lib.ravel_em_seg_sum_workspace(B, T, C, D, address_space, int(r is not None),
                                            int(write_mask is not None), code)
    ws = nat.workspace(nbytes, dev)
    nat.check(lib.ravel_em_seg_sum_fwd(
        nat.ref(w), nat.ref(r), nat.ADDR_GEN, nat.ptr(write_mask), nat.ptr(payloads), code,
        B, T, C, D, address_space, nat.ptr(out), nat.ptr(mask), nat.ptr(ws), ws.numel(),
        nat.stream_of(payloads)))
    nat.after_call(ws)
    return out, mask


@seg_sum_gen.register_fake
def _seg_sum_gen_fake(tokens, history, write_logits, read_logits, payloads, write_mask, n_literal,
                      bos, n_learned, ncb, cbs, position, address_space):
    B, T, C, D = payloads.shape
    return payloads.new_empty(B, T, C, D), torch.empty(B, T, C, dtype=torch.bool, device=payloads.device)


@torch.library.custom_op("ravel_em::seg_sum_gen_backward", mutates_args=())
def seg_sum_gen_backward(tokens: Optional[Tensor], history: Optional[Tensor],
                         write_logits: Optional[Tensor], read_logits: Optional[Tensor],
                         write_mask: Optional[Tensor], grad_sum: Tensor, n_literal: int, bos: int,
                         n_learned: int, ncb: int, cbs: int, position: int,
                         address_space: int) -> Tensor:
    lib = nat.library()
    B, T, C, D = grad_sum.shape
    grad_sum = grad_sum.contiguous()
    grad_payload = grad_sum.new_empty(B, T, C, D)
    code = nat.payload_code(grad_sum.dtype)
    w, r = _descs(tokens, history, write_logits, read_logits, n_literal, bos, n_learned, ncb, cbs,
                  position)
    nbytes = lib.ravel_em_seg_sum_bwd_workspace(B, T, C, D, address_space, int(r is not None),
                                                int(write_mask is not None), code)
    ws = nat.workspace(nbytes, grad_sum.device)
    nat.check(lib.ravel_em_seg_sum_bwd(
        nat.ref(w), nat.ref(r), nat.ADDR_GEN, nat.ptr(write_mask), nat.ptr(grad_sum), code,
        B, T, C, D, address_space, nat.ptr(grad_payload), nat.ptr(ws), ws.numel(),
        nat.stream_of(grad_sum)))
    nat.after_call(ws)
    return grad_payload


@seg_sum_gen_backward.register_fake
def _seg_sum_gen_backward_fake(tokens, history, write_logits, read_logits, write_mask, grad_sum,
                               n_literal, bos, n_learned, ncb, cbs, position, address_space):
    return grad_sum.new_empty(grad_sum.shape)


def _seg_sum_gen_setup(ctx, inputs, output):
    tokens, history, write_logits, read_logits, _payloads, write_mask = inputs[:6]
    ctx.save_for_backward(tokens, history, write_logits, read_logits, write_mask)
    ctx.cfg = inputs[6:]
    ctx.mark_non_differentiable(output[1])


def _seg_sum_gen_grad(ctx, grad_sum, _grad_mask):
    tokens, history, write_logits, read_logits, write_mask = ctx.saved_tensors
    grad_payload = seg_sum_gen_backward(tokens, history, write_logits, read_logits, write_mask,
                                        grad_sum, *ctx.cfg)
    return (None, None, None, None, grad_payload) + (None,) * 8


seg_sum_gen.register_autograd(_seg_sum_gen_grad, setup_context=_seg_sum_gen_setup)


@torch.library.custom_op("ravel_em::latest_k_sum_gen", mutates_args=())
def latest_k_sum_gen(tokens: Optional[Tensor], history: Optional[Tensor],
                     write_logits: Optional[Tensor], read_logits: Optional[Tensor],
                     payloads: Tensor, write_mask: Optional[Tensor], n_literal: int, bos: int,
                     n_learned: int, ncb: int, cbs: int, position: int, address_space: int,
                     k: int, want_src: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    lib = nat.library()
    B, T, C, D = payloads.shape
    dev = payloads.device
    values = payloads.new_empty(B, T, C, k, D)
    mask = torch.empty(B, T, C, k, dtype=torch.bool, device=dev)
    src = torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev)
    out = payloads.new_empty(B, T, C, D)
    smask = torch.empty(B, T, C, dtype=torch.bool, device=dev)
    code = nat.payload_code(payloads.dtype)
    w, r = _descs(tokens, history, write_logits, read_logits, n_literal, bos, n_learned, ncb, cbs,
                  position)
    nbytes = lib.ravel_em_latest_k_sum_workspace(B, T, C, D, address_space, k, int(r is not None),
                                                 int(write_mask is not None), int(want_src), code)
    ws = nat.workspace(nbytes, dev)
    nat.check(lib.ravel_em_latest_k_sum_fwd(
        nat.ref(w), nat.ref(r), nat.ADDR_GEN, nat.ptr(write_mask), nat.ptr(payloads), code,
        B, T, C, D, address_space, k, nat.ptr(values), nat.ptr(mask),
        nat.ptr(src) if want_src else None, nat.ptr(out), nat.ptr(smask), nat.ptr(ws), ws.numel(),
        nat.stream_of(payloads)))
    nat.after_call(ws)
    return values, mask, src, out, smask


@latest_k_sum_gen.register_fake
def _latest_k_sum_gen_fake(tokens, history, write_logits, read_logits, payloads, write_mask,
                           n_literal, bos, n_learned, ncb, cbs, position, address_space, k,
                           want_src):
    B, T, C, D = payloads.shape
    dev = payloads.device
    return (payloads.new_empty(B, T, C, k, D),
            torch.empty(B, T, C, k, dtype=torch.bool, device=dev),
            torch.empty((B, T, C, k) if want_src else (0,), dtype=torch.int32, device=dev),
            payloads.new_empty(B, T, C, D),
            torch.empty(B, T, C, dtype=torch.bool, device=dev))


def _latest_k_sum_gen_setup(ctx, inputs, output):
    tokens, history, write_logits, read_logits, _payloads, write_mask = inputs[:6]
    _, mask, src, _, smask = output
    ctx.save_for_backward(src, tokens, history, write_logits, read_logits, write_mask)
    ctx.chain = read_logits is None and write_mask is None
    ctx.want_src = inputs[-1]
    ctx.cfg = inputs[6:13]
    ctx.mark_non_differentiable(mask, src, smask)


def _latest_k_sum_gen_grad(ctx, grad_values, _grad_mask, _grad_src, grad_sum, _grad_smask):
    src, tokens, history, write_logits, read_logits, write_mask = ctx.saved_tensors
    if not ctx.want_src:
        raise RuntimeError("ravel_em.latest_k_sum_gen was called without sources; "
                           "cannot differentiate")
    grad_payload = _ops.latest_k_backward(src, grad_values, ctx.chain)
    grad_payload = grad_payload + seg_sum_gen_backward(tokens, history, write_logits, read_logits,
                                                       write_mask, grad_sum, *ctx.cfg)
    return (None, None, None, None, grad_payload) + (None,) * 10


latest_k_sum_gen.register_autograd(_latest_k_sum_gen_grad, setup_context=_latest_k_sum_gen_setup)


# ------------------------------------------------------------ lookups --


def _check_payloads(src: LayerAddresses, payloads: Tensor, write_mask: Optional[Tensor]):
    B, T = src._check()
    if payloads.ndim != 4 or payloads.shape[:3] != (B, T, src.heads):
        raise ValueError("payloads must have shape [B, T, C, D] with C = literal + learned heads")
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    return B, T


def last_k_lookup(src: LayerAddresses, payloads: Tensor, *, address_space: int, k: int = 1,
                  write_mask: Optional[Tensor] = None,
                  want_src: Optional[bool] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """causal_last_k_lookup with the addresses of `src` produced in the kernels;
    returns (values, mask, src) like causal_last_k_sources (src empty when not
    wanted)."""
    _check_payloads(src, payloads, write_mask)
    if k <= 0:
        raise ValueError("k must be positive")
    _check_space(address_space)
    tok, hist, wl, rl = src.tensors()
    nat.require_device(payloads, tok, hist, wl, rl, write_mask)
    m = None if write_mask is None else write_mask.bool().contiguous()
    if want_src is None:
        want_src = torch.is_grad_enabled() and payloads.requires_grad
    return latest_k_gen(tok, hist, wl, rl, payloads.contiguous(), m, *src.cfg(),
                        int(address_space), int(k), bool(want_src))


def sum_lookup(src: LayerAddresses, payloads: Tensor, *, address_space: int,
               write_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """causal_sum_lookup with the addresses of `src` produced in the kernels."""
    _check_payloads(src, payloads, write_mask)
    _check_space(address_space)
    tok, hist, wl, rl = src.tensors()
    nat.require_device(payloads, tok, hist, wl, rl, write_mask)
    m = None if write_mask is None else write_mask.bool().contiguous()
    return seg_sum_gen(tok, hist, wl, rl, payloads.contiguous(), m, *src.cfg(),
                       int(address_space))


def last_k_and_sum_lookup(src: LayerAddresses, payloads: Tensor, *, address_space: int,
                          k: int = 1, write_mask: Optional[Tensor] = None
                          ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """causal_last_k_and_sum_lookup with the addresses of `src` produced in the
    kernels; returns (values, mask, summed, sum_mask)."""
    _check_payloads(src, payloads, write_mask)
    if k <= 0:
        raise ValueError("k must be positive")
    _check_space(address_space)
    tok, hist, wl, rl = src.tensors()
    nat.require_device(payloads, tok, hist, wl, rl, write_mask)
    m = None if write_mask is None else write_mask.bool().contiguous()
    want_src = torch.is_grad_enabled() and payloads.requires_grad
    values, mask, _, summed, sum_mask = latest_k_sum_gen(
        tok, hist, wl, rl, payloads.contiguous(), m, *src.cfg(), int(address_space), int(k),
        bool(want_src))
    return values, mask, summed, sum_mask


def cache_step(src: LayerAddresses, values: Tensor, filled: Tensor, payloads: Tensor,
               k: int) -> Tuple[Tensor, Tensor]:
    """One decode step of the cache with the addresses of `src` (T = 1: token
    ids [B] or [B, 1], logits [B, N] or [B, 1, N]) produced in the kernel:
    read at the read addresses, then shift-insert payloads at the write
    addresses (model.py:401-426)."""
    B, C, A = filled.shape[:3]
    D = values.shape[-1]
    tok = src.token_ids
    if tok is not None and tok.ndim == 1:
        tok = tok.view(-1, 1)

    def step_logits(x):
        return None if x is None else (x.view(x.shape[0], 1, -1) if x.ndim == 2 else x)

    one = LayerAddresses(tok, src.n_literal_heads, src.bos_token_id,
                         step_logits(src.write_logits), step_logits(src.read_logits),
                         src.n_learned_heads, src.n_codebooks, src.codebook_size,
                         src.token_history, src.position)
    Bs, T = one._check()
    if Bs != B or T != 1 or one.heads != C:
        raise ValueError(f"step addresses [{Bs}, {T}] x {one.heads} heads do not match the cache [{B}, {C}]")
    t, hist, wl, rl = one.tensors()
    nat.require_device(values, payloads, t, hist, wl, rl)
    w, r = _descs(t, hist, wl, rl, *one.cfg())
    r = w if r is None else r  # reads use the write addresses
    out = values.new_empty(B, C, k, D)
    mask = torch.empty(B, C, k, dtype=torch.bool, device=values.device)
    nat.check(nat.library().ravel_em_cache_step(
        nat.ptr(values), nat.ptr(filled), nat.ref(r), nat.ref(w), nat.ADDR_GEN,
        nat.ptr(payloads), nat.payload_code(values.dtype), B, C, A, k, D, nat.ptr(out),
        nat.ptr(mask), nat.stream_of(values)))
    return out, mask

"""Drop-in replacement of ``ravel_lm/ravel_memory.py`` on MI355X.

Same public names, signatures, argument meaning, return shapes/dtypes and
exceptions as the reference module; the work runs in hand-written HIP kernels
for gfx950 behind the C ABI of include/ravel_em.h.  Inputs must live on a ROCm
device: there is no CPU path and no fallback.

Reference interface (file:line in the reference tree):
  _composite_key_dtype   ravel_lm/ravel_memory.py:45-49
  causal_last_k_lookup   ravel_lm/ravel_memory.py:52-176
  causal_sum_lookup      ravel_lm/ravel_memory.py:179-241
  RavelLayerCache        ravel_lm/ravel_memory.py:244-292
  causal_last_k_and_sum_lookup  the pair of the two lookups that
                         ravel_lm/model.py:366-386 makes on one tape

Device-side waits.  The sorts and the long-tape sums coordinate blocks through
bounded waits; a wait that runs out of spins sets a bit in the call's status
word instead of hanging, and the call's outputs are then not valid.  The
functions here do not read that word by default (reading it synchronizes the
stream): set RAVEL_EM_CHECK_STATUS=1, or call
ravel_em._native.set_status_check(True), to have every call read it and raise
DeviceWaitError when a bit is set.  The tests run with the check on.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _native as nat
from . import _ops
from .addressing import LayerAddresses, last_k_and_sum_lookup, last_k_lookup, sum_lookup
from .addressing import cache_step as _addr_cache_step

Tensor = torch.Tensor


def _composite_key_dtype(B: int, T: int, C: int, address_space: int) -> torch.dtype:
    """int32 when every composite key ((b*C+c)*A+a)*(T+1)+t fits, else int64.

    Reference: ravel_lm/ravel_memory.py:45-49 (the T+1 radix leaves room for the
    read key t-1 at t=0).
    """
    bound = int(B) * int(C) * int(address_space) * (int(T) + 1)
    return torch.int32 if bound <= torch.iinfo(torch.int32).max else torch.int64


def _as_addresses(t: Tensor, key_dtype: torch.dtype) -> Tensor:
    """Address tensor handed to the kernels: int32 or int64, contiguous.

    The reference converts addresses with ``.to(key_dtype)`` before the
    remainder (ravel_memory.py:127-128); the kernels reproduce that conversion
    for int64 inputs, other integer dtypes widen to int64 exactly, and floating
    inputs take the reference's own conversion here.
    """
    if t.dtype in (torch.int32, torch.int64):
        return t.contiguous()
    if t.is_floating_point():
        return t.to(key_dtype).contiguous()
    return t.to(torch.int64).contiguous()


def _prepare(write_addresses: Tensor, read_addresses: Optional[Tensor], key_dtype: torch.dtype):
    w = _as_addresses(write_addresses, key_dtype)
    r = None if read_addresses is None else _as_addresses(read_addresses, key_dtype)
    if r is not None and r.dtype != w.dtype:
        w, r = w.to(torch.int64), r.to(torch.int64)
    return w, r


def _no_read(read_addresses) -> None:
    if read_addresses is not None:
        raise ValueError("with LayerAddresses the read addresses come from its read_logits; "
                         "read_addresses must be None")


def causal_last_k_lookup(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor] = None,
    *,
    address_space: int,
    k: int = 1,
    write_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """Exact causal last-k lookup over an event tape.

    For every read at time ``t`` returns the latest ``k`` payloads written to the
    same ``(batch, head, address)`` at times ``< t``; slot ``j`` is the
    ``(j+1)``-th most recent.  Reference: ravel_lm/ravel_memory.py:52-176.

    Args:
        write_addresses: [B, T, C] integer addresses for writes, or a
                         LayerAddresses whose write and read addresses the
                         kernels produce (then read_addresses must be None).
        payloads:        [B, T, C, D] payload tensor.
        read_addresses:  [B, T, C] integer read addresses. Defaults to writes.
        address_space:   number of legal addresses per memory head (addresses
                         are reduced with Python-style remainder).
        k:               number of latest records to return.
        write_mask:      optional [B, T] boolean mask; false entries do not write.

    Returns:
        values: [B, T, C, k, D] (missing slots are zero)
        mask:   [B, T, C, k] true where a causal record existed.
    """
    if isinstance(write_addresses, LayerAddresses):
        _no_read(read_addresses)
        values, mask, _ = last_k_lookup(write_addresses, payloads, address_space=address_space,
                                        k=k, write_mask=write_mask)
        return values, mask
    same = read_addresses is None or read_addresses is write_addresses
    if read_addresses is None:
        read_addresses = write_addresses
    if write_addresses.shape != read_addresses.shape:
        raise ValueError("write_addresses and read_addresses must have the same shape")
    if write_addresses.ndim != 3:
        raise ValueError("addresses must have shape [B, T, C]")
    if payloads.ndim != 4:
        raise ValueError("payloads must have shape [B, T, C, D]")
    B, T, C = write_addresses.shape
    if payloads.shape[:3] != (B, T, C):
        raise ValueError("payloads leading dimensions must match addresses")
    if k <= 0:
        raise ValueError("k must be positive")
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    nat.require_device(write_addresses, payloads, read_addresses, write_mask)
    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, r = _prepare(write_addresses, None if same else read_addresses, key_dtype)
    m = None if write_mask is None else write_mask.bool().contiguous()
    want_src = torch.is_grad_enabled() and payloads.requires_grad
    p = payloads.contiguous()
    op = _ops.latest_k_impl if not want_src and _ops.eager(w, p, r, m) else _ops.latest_k
    values, mask, _ = op(w, p, r, m, int(address_space), int(k), want_src)
    return values, mask


def causal_last_k_sources(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor] = None,
    *,
    address_space: int,
    k: int = 1,
    write_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor]:
    """``causal_last_k_lookup`` plus the source record of every slot.

    Returns ``(values, mask, src)`` where ``src [B, T, C, k]`` (int32) is the flat
    index ``(b*T + t_src)*C + c`` of the record each slot was copied from, or -1.
    The reference's MPS and Triton arms expose the same source index
    (ravel_lm/mps_memory.py:109-141, triton_latest1.py:60-63), which
    experiments/chime_arm.py:53-70 consumes.  ``write_addresses`` may be a
    LayerAddresses, as in causal_last_k_lookup.
    """
    if isinstance(write_addresses, LayerAddresses):
        _no_read(read_addresses)
        return last_k_lookup(write_addresses, payloads, address_space=address_space, k=k,
                             write_mask=write_mask, want_src=True)
    if read_addresses is None:
        read_addresses = write_addresses
    same = read_addresses is write_addresses
    if write_addresses.shape != read_addresses.shape or write_addresses.ndim != 3:
        raise ValueError("addresses must have shape [B, T, C]")
    B, T, C = write_addresses.shape
    if payloads.ndim != 4 or payloads.shape[:3] != (B, T, C):
        raise ValueError("payloads must have shape [B, T, C, D]")
    if k <= 0:
        raise ValueError("k must be positive")
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    nat.require_device(write_addresses, payloads, read_addresses, write_mask)
    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, r = _prepare(write_addresses, None if same else read_addresses, key_dtype)
    m = None if write_mask is None else write_mask.bool().contiguous()
    return _ops.latest_k(w, payloads.contiguous(), r, m, int(address_space), int(k), True)


def causal_sum_lookup(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor] = None,
    *,
    address_space: int,
    write_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """Exact causal segmented prefix-sum lookup over the event tape.

    For every read at time ``t`` returns the sum of all payloads with matching
    ``(batch, head, address)`` and time ``< t``, and whether any existed.
    Reference: ravel_lm/ravel_memory.py:179-241.  Sums accumulate in fp32 for
    16-bit payloads and fp64 for 32/64-bit payloads, rounded once to the payload
    dtype.  ``write_addresses`` may be a LayerAddresses, as in
    causal_last_k_lookup.
    """
    if isinstance(write_addresses, LayerAddresses):
        _no_read(read_addresses)
        return sum_lookup(write_addresses, payloads, address_space=address_space,
                          write_mask=write_mask)
    same = read_addresses is None or read_addresses is write_addresses
    if read_addresses is None:
        read_addresses = write_addresses
    if write_addresses.ndim != 3 or payloads.ndim != 4:
        raise ValueError("expected write_addresses [B,T,C] and payloads [B,T,C,D]")
    B, T, C = write_addresses.shape
    if read_addresses.shape != (B, T, C) or payloads.shape[:3] != (B, T, C):
        raise ValueError("expected write_addresses [B,T,C] and payloads [B,T,C,D]")
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    nat.require_device(write_addresses, payloads, read_addresses, write_mask)
    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, r = _prepare(write_addresses, None if same else read_addresses, key_dtype)
    m = None if write_mask is None else write_mask.bool().contiguous()
    p = payloads.contiguous()
    graph = torch.is_grad_enabled() and p.requires_grad
    op = _ops.seg_sum_impl if not graph and _ops.eager(w, p, r, m) else _ops.seg_sum
    return op(w, p, r, m, int(address_space))


def causal_last_k_and_sum_lookup(
    write_addresses: Tensor,
    payloads: Tensor,
    read_addresses: Optional[Tensor] = None,
    *,
    address_space: int,
    k: int = 1,
    write_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """``causal_last_k_lookup`` and ``causal_sum_lookup`` of one tape in one call.

    Returns ``(values, mask, summed, sum_mask)``: exactly the results of
    ``causal_last_k_lookup(write_addresses, payloads, read_addresses,
    address_space=address_space, k=k, write_mask=write_mask)`` followed by
    ``causal_sum_lookup(...)`` of the same tape, which is the pair of calls the
    reference memory layer makes when ``use_sum_read`` is set
    (ravel_lm/model.py:366-386; each call sorts the tape,
    ravel_lm/ravel_memory.py:151 and :216).  Here the tape is sorted once for
    both where one kernel can emit both results.  ``write_addresses`` may be a
    LayerAddresses, as in causal_last_k_lookup.
    """
    if isinstance(write_addresses, LayerAddresses):
        _no_read(read_addresses)
        return last_k_and_sum_lookup(write_addresses, payloads, address_space=address_space, k=k,
                                     write_mask=write_mask)
    same = read_addresses is None or read_addresses is write_addresses
    if read_addresses is None:
        read_addresses = write_addresses
    if write_addresses.shape != read_addresses.shape:
        raise ValueError("write_addresses and read_addresses must have the same shape")
    if write_addresses.ndim != 3:
        raise ValueError("addresses must have shape [B, T, C]")
    if payloads.ndim != 4:
        raise ValueError("payloads must have shape [B, T, C, D]")
    B, T, C = write_addresses.shape
    if payloads.shape[:3] != (B, T, C):
        raise ValueError("payloads leading dimensions must match addresses")
    if k <= 0:
        raise ValueError("k must be positive")
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    nat.require_device(write_addresses, payloads, read_addresses, write_mask)
    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, r = _prepare(write_addresses, None if same else read_addresses, key_dtype)
    m = None if write_mask is None else write_mask.bool().contiguous()
    p = payloads.contiguous()
    graph = torch.is_grad_enabled() and p.requires_grad
    op = _ops.latest_k_sum_impl if not graph and _ops.eager(w, p, r, m) else _ops.latest_k_sum
    values, mask, _, summed, sum_mask = op(w, p, r, m, int(address_space), int(k), graph)
    return values, mask, summed, sum_mask


def sort_order(
    write_addresses: Tensor,
    *,
    address_space: int,
    write_mask: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """``torch.sort`` of the reference's flat composite write keys.

    Returns ``(sorted_keys, order)`` exactly as ravel_lm/ravel_memory.py:133-151
    builds them (keys in the ``_composite_key_dtype``, order int64 indices into
    the flat tape with masked times removed).  Exposed so the sort itself can be
    checked bit-for-bit; with a write_mask the output length is read back from
    the device.
    """
    if write_addresses.ndim != 3:
        raise ValueError("addresses must have shape [B, T, C]")
    B, T, C = write_addresses.shape
    if write_mask is not None and write_mask.shape != (B, T):
        raise ValueError("write_mask must have shape [B, T]")
    nat.require_device(write_addresses, write_mask)
    key_dtype = _composite_key_dtype(B, T, C, address_space)
    w, _ = _prepare(write_addresses, None, key_dtype)
    m = None if write_mask is None else write_mask.bool().contiguous()
    return _ops.sort_order(w, m, int(address_space), key_dtype)


def _cache_addresses(addresses: Tensor) -> Tensor:
    # The cache clamps (ravel_memory.py:276, :289); the kernels clamp int32 and
    # int64 alike, other integer dtypes widen to int64 exactly.
    if addresses.dtype in (torch.int32, torch.int64):
        return addresses.contiguous()
    return addresses.long().contiguous()


@dataclass
class RavelLayerCache:
    """O(address_space * heads * payload_dim * k) latest-value cache for decoding.

    Same latest-record semantics as ``causal_last_k_lookup``: with ``k == 1``
    (the reference layout) ``values`` is [B, C, A, D] and ``filled`` [B, C, A];
    with ``k > 1`` they are [B, C, A, k, D] and [B, C, A, k], slot ``j`` holding
    the ``(j+1)``-th most recent write.  Reference: ravel_lm/ravel_memory.py:244-292.
    """

    values: Tensor
    filled: Tensor

    @property
    def k(self) -> int:
        return 1 if self.filled.ndim == 3 else int(self.filled.shape[3])

    @classmethod
    def empty(
        cls,
        batch_size: int,
        n_heads: int,
        address_space: int,
        payload_dim: int,
        *,
        device: torch.device | str,
        dtype: torch.dtype,
        k: int = 1,
    ) -> "RavelLayerCache":
        if k <= 0:
            raise ValueError("k must be positive")
        slots = () if k == 1 else (k,)
        values = torch.zeros(batch_size, n_heads, address_space, *slots, payload_dim, device=device, dtype=dtype)
        filled = torch.zeros(batch_size, n_heads, address_space, *slots, device=device, dtype=torch.bool)
        return cls(values=values, filled=filled)

    @classmethod
    def prefill(
        cls,
        write_addresses: Tensor,
        payloads: Tensor,
        *,
        address_space: int,
        k: int = 1,
        write_mask: Optional[Tensor] = None,
    ) -> "RavelLayerCache":
        """Cache state after writing ``write_addresses[:, t]`` / ``payloads[:, t]``
        for t = 0..T-1 in order, built in one pass over the sorted tape (the
        reference prefills token by token, ravel_lm/model.py:600-602)."""
        if write_addresses.ndim != 3 or payloads.ndim != 4:
            raise ValueError("expected write_addresses [B,T,C] and payloads [B,T,C,D]")
        B, T, C = write_addresses.shape
        if payloads.shape[:3] != (B, T, C):
            raise ValueError("payloads leading dimensions must match addresses")
        if k <= 0:
            raise ValueError("k must be positive")
        if write_mask is not None and write_mask.shape != (B, T):
            raise ValueError("write_mask must have shape [B, T]")
        nat.require_device(write_addresses, payloads, write_mask)
        D = payloads.shape[-1]
        slots = () if k == 1 else (k,)
        values = payloads.new_empty(B, C, address_space, *slots, D)
        filled = torch.empty(B, C, address_space, *slots, device=payloads.device, dtype=torch.bool)
        m = None if write_mask is None else write_mask.bool().contiguous()
        _ops.cache_prefill(_cache_addresses(write_addresses), payloads.contiguous(), m,
                           int(address_space), int(k), values, filled)
        return cls(values=values, filled=filled)

    def _squeeze(self, vals: Tensor, mask: Tensor) -> Tuple[Tensor, Tensor]:
        if self.k == 1:
            return vals.squeeze(2), mask.squeeze(2)
        return vals, mask

    def read(self, addresses: Tensor) -> Tuple[Tensor, Tensor]:
        """Read latest values for addresses [B, C].

        Returns ([B,C,D], [B,C]) for k == 1, ([B,C,k,D], [B,C,k]) otherwise."""
        B, C = addresses.shape
        if self.values.shape[:2] != (B, C):
            raise ValueError(f"cache shape {self.values.shape[:2]} does not match addresses {(B, C)}")
        nat.require_device(self.values, self.filled, addresses)
        vals, mask = _ops.cache_read(self.values, self.filled, _cache_addresses(addresses), self.k)
        return self._squeeze(vals, mask)

    def write(self, addresses: Tensor, payloads: Tensor) -> None:
        """Write latest payloads. addresses [B,C], payloads [B,C,D]."""
        B, C = addresses.shape
        D = payloads.shape[-1]
        if self.values.shape[:2] != (B, C) or self.values.shape[-1] != D:
            raise ValueError("cache and payload shapes do not match")
        nat.require_device(self.values, self.filled, addresses, payloads)
        _ops.cache_write(self.values, self.filled, _cache_addresses(addresses),
                         payloads.to(self.values.dtype).contiguous(), self.k)

    def step(self, read_addresses: Tensor, write_addresses: Optional[Tensor], payloads: Tensor) -> Tuple[Tensor, Tensor]:
        """``read(read_addresses)`` then ``write(write_addresses, payloads)`` in one launch.

        ``read_addresses`` may be a LayerAddresses of one decode step (token ids
        [B], token_history [B, h], position, logits [B, N]; write_addresses
        None): the kernel then produces both address sets itself, as
        RavelMemoryLayer.step does before its read and write
        (ravel_lm/model.py:401-426).
        """
        if isinstance(read_addresses, LayerAddresses):
            if write_addresses is not None:
                raise ValueError("with LayerAddresses the write addresses come from it; write_addresses must be None")
            D = payloads.shape[-1]
            if self.values.shape[-1] != D or payloads.shape[:2] != self.values.shape[:2]:
                raise ValueError("cache and payload shapes do not match")
            vals, mask = _addr_cache_step(read_addresses, self.values, self.filled,
                                          payloads.to(self.values.dtype).contiguous(), self.k)
            return self._squeeze(vals, mask)
        B, C = read_addresses.shape
        D = payloads.shape[-1]
        if write_addresses.shape != (B, C):
            raise ValueError("read and write addresses must have the same shape")
        if self.values.shape[:2] != (B, C) or self.values.shape[-1] != D:
            raise ValueError("cache and payload shapes do not match")
        nat.require_device(self.values, self.filled, read_addresses, write_addresses, payloads)
        r = _cache_addresses(read_addresses)
        w = _cache_addresses(write_addresses)
        if r.dtype != w.dtype:
            r, w = r.long(), w.long()
        vals, mask = _ops.cache_step(self.values, self.filled, r, w,
                                     payloads.to(self.values.dtype).contiguous(), self.k)
        return self._squeeze(vals, mask)

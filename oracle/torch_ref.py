"""The reference operator's own algorithm, restated with torch on the CPU.

TEST INFRASTRUCTURE ONLY (and the CPU baseline that bench.py times).  It
follows the step sequence of ravel_lm/ravel_memory.py so that its output,
including the rounding of the cumsum-based sum, is what the reference CPU path
produces:
  latest-k  composite keys -> torch.sort -> searchsorted(right) - 1 ->
            candidate/stream check -> gather            (:126-176)
  sum       sort -> permuted payload -> global cumsum -> minus the prefix
            before each stream's start -> searchsorted -> gather (:200-241)
  cache     clamp -> gather / scatter                    (:271-292)
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

Tensor = torch.Tensor


def key_dtype(B: int, T: int, C: int, A: int) -> torch.dtype:
    """ravel_memory.py:45-49."""
    return torch.int32 if B * C * A * (T + 1) <= 2**31 - 1 else torch.int64


def _stream_base(addr: Tensor, A: int) -> Tensor:
    """((b*C + c) * A + a) for addresses [B,T,C] already reduced (:26-38)."""
    B, T, C = addr.shape
    bc = torch.arange(B * C, dtype=addr.dtype).view(B, 1, C)
    return bc * A + addr


def _flat_keys(addr: Tensor, A: int, shift: int) -> Tuple[Tensor, Tensor]:
    B, T, C = addr.shape
    base = _stream_base(addr, A)
    times = torch.arange(T, dtype=addr.dtype).view(1, T, 1) + shift
    return base.reshape(-1), (base * (T + 1) + times).reshape(-1)


def _reduced(addr: Tensor, kd: torch.dtype, A: int) -> Tensor:
    return addr.to(kd).remainder(A)


def latest_k(write: Tensor, payload: Tensor, read: Optional[Tensor] = None, *, address_space: int,
             k: int = 1, write_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    if read is None:
        read = write
    B, T, C = write.shape
    D = payload.shape[-1]
    A = int(address_space)
    kd = key_dtype(B, T, C, A)
    _, wkeys = _flat_keys(_reduced(write, kd, A), A, 0)
    rows = payload.reshape(-1, D)
    if write_mask is not None:
        keep = write_mask.bool().view(B, T, 1).expand(B, T, C).reshape(-1)
        wkeys, rows = wkeys[keep], rows[keep]
    if wkeys.numel() == 0:
        return payload.new_zeros(B, T, C, k, D), torch.zeros(B, T, C, k, dtype=torch.bool)
    sorted_keys, order = torch.sort(wkeys)
    rbase, rkeys = _flat_keys(_reduced(read, kd, A), A, -1)
    last = torch.searchsorted(sorted_keys, rkeys, right=True) - 1
    cand = last.view(-1, 1) - torch.arange(k).view(1, k)
    inside = cand >= 0
    cand = cand.clamp_min(0)
    same_stream = sorted_keys[cand.reshape(-1)].view(-1, k) // (T + 1) == rbase.view(-1, 1)
    valid = inside & same_stream
    vals = rows.index_select(0, order.index_select(0, cand.reshape(-1))).view(-1, k, D)
    vals = vals * valid.unsqueeze(-1).to(vals.dtype)
    return vals.view(B, T, C, k, D), valid.view(B, T, C, k)


def seg_sum(write: Tensor, payload: Tensor, read: Optional[Tensor] = None, *, address_space: int,
            write_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    if read is None:
        read = write
    B, T, C = write.shape
    D = payload.shape[-1]
    A = int(address_space)
    kd = key_dtype(B, T, C, A)
    _, wkeys = _flat_keys(_reduced(write, kd, A), A, 0)
    rows = payload.reshape(-1, D)
    if write_mask is not None:
        keep = write_mask.bool().view(B, T, 1).expand(B, T, C).reshape(-1)
        wkeys, rows = wkeys[keep], rows[keep]
    if wkeys.numel() == 0:
        return payload.new_zeros(B, T, C, D), torch.zeros(B, T, C, dtype=torch.bool)
    sorted_keys, order = torch.sort(wkeys)
    sorted_rows = rows.index_select(0, order)
    stream = sorted_keys // (T + 1)
    starts = torch.ones_like(stream, dtype=torch.bool)
    starts[1:] = stream[1:] != stream[:-1]
    total = torch.cumsum(sorted_rows, dim=0)
    start_idx = torch.nonzero(starts).flatten()
    seg_id = torch.cumsum(starts.long(), dim=0) - 1
    before = total.new_zeros(start_idx.numel(), D)
    has_prev = start_idx > 0
    before[has_prev] = total.index_select(0, start_idx[has_prev] - 1)
    within = total - before.index_select(0, seg_id)
    rbase, rkeys = _flat_keys(_reduced(read, kd, A), A, -1)
    idx = torch.searchsorted(sorted_keys, rkeys, right=True) - 1
    valid = idx >= 0
    idx = idx.clamp_min(0)
    valid = valid & (stream.index_select(0, idx) == rbase)
    out = within.index_select(0, idx) * valid.unsqueeze(-1).to(payload.dtype)
    return out.view(B, T, C, D), valid.view(B, T, C)


def cache_read(values: Tensor, filled: Tensor, addresses: Tensor) -> Tuple[Tensor, Tensor]:
    """k=1 cache read, ravel_memory.py:271-281."""
    B, C = addresses.shape
    A, D = values.shape[2], values.shape[-1]
    idx = addresses.long().clamp(0, A - 1)
    vals = torch.gather(values, 2, idx.view(B, C, 1, 1).expand(B, C, 1, D)).squeeze(2)
    mask = torch.gather(filled, 2, idx.view(B, C, 1)).squeeze(2)
    return vals * mask.unsqueeze(-1).to(vals.dtype), mask


def cache_write(values: Tensor, filled: Tensor, addresses: Tensor, payload: Tensor) -> None:
    """k=1 cache write, ravel_memory.py:283-292."""
    B, C = addresses.shape
    A, D = values.shape[2], values.shape[-1]
    idx = addresses.long().clamp(0, A - 1)
    values.scatter_(2, idx.view(B, C, 1, 1).expand(B, C, 1, D), payload.unsqueeze(2))
    filled.scatter_(2, idx.view(B, C, 1), torch.ones(B, C, 1, dtype=torch.bool))


def literal_addresses(tokens: Tensor, *, address_space: int, n_heads: int, bos_token_id: int) -> Tensor:
    """literal_addresses_from_tokens, ravel_lm/model.py:195-231: the same torch
    op sequence (shifted copies padded with bos, int64 products, remainder,
    stack), for the CPU baseline of the layer's address production."""
    B, T = tokens.shape
    toks = tokens.long()
    A = int(address_space)
    pad = torch.full((B, 2), int(bos_token_id), dtype=torch.long)
    prev1 = torch.cat([pad[:, :1], toks[:, :-1]], dim=1)
    prev2 = torch.cat([pad, toks[:, :-2]], dim=1)
    heads = []
    for j in range(n_heads):
        if j == 0:
            h = toks
        elif j == 1:
            h = prev1 * 257 + toks * 131 + 17
        elif j == 2:
            h = prev2 * 65537 + prev1 * 257 + toks * 131 + 31
        else:
            pos = torch.arange(T, dtype=torch.long).view(1, T).expand(B, T)
            h = toks * (1009 + 2 * j) + pos * (9176 + j) + j * 97
        heads.append(h.remainder(A))
    return torch.stack(heads, dim=-1)


def product_codes(logits: Tensor, *, n_heads: int, n_codebooks: int, codebook_size: int,
                  address_space: int) -> Tensor:
    """_decode_codes, ravel_lm/model.py:303-307 (argmax per codebook, codes
    times powers of codebook_size, summed, remainder)."""
    codes = logits.reshape(*logits.shape[:-1], n_heads, n_codebooks, codebook_size).argmax(dim=-1)
    mult = torch.tensor([codebook_size ** q for q in range(n_codebooks)], dtype=torch.long)
    return (codes.long() * mult).sum(dim=-1).remainder(int(address_space))

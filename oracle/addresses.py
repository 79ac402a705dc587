"""Address production of the reference's memory layer, restated for the CPU.

TEST INFRASTRUCTURE ONLY.  Plain Python loops over small inputs, one function
per reference routine:

  literal_addresses   literal_addresses_from_tokens, ravel_lm/model.py:195-231
  literal_addresses_step  its decode-step form, ravel_lm/model.py:234-263
  product_codes       ProductCodeAddressor.forward's decode, model.py:177-187,
                      and RavelMemoryLayer._decode_codes, model.py:303-307
  layer_addresses     the write/read assembly of RavelMemoryLayer.forward,
                      model.py:333-346 (literal heads first, then learned)

Integer arithmetic is Python's (unbounded) reduced to two's-complement int64
before each remainder, which is what torch's int64 tensors compute; the
remainder is Python's (result in [0, A) for A > 0), as torch.remainder.
Argmax follows torch.argmax: the index of the first maximum, where a NaN counts
as larger than every number and the first NaN wins.
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple


def _i64(x: int) -> int:
    return ((x + 2**63) % 2**64) - 2**63


def literal_addresses(tokens: Sequence[Sequence[int]], *, address_space: int, n_heads: int,
                      bos_token_id: int) -> List[List[List[int]]]:
    """[B][T][n_heads] addresses of ravel_lm/model.py:195-231.

    Head 0 is the token, head 1 hashes (t-1, t), head 2 hashes (t-2, t-1, t),
    heads j >= 3 mix the token with its position t; tokens before the start of
    a row are bos_token_id (the reference pads with torch.full(bos) and shifts).
    """
    A = address_space
    out = []
    for row in tokens:
        T = len(row)
        orow = []
        for t in range(T):
            x = int(row[t])
            p1 = int(row[t - 1]) if t >= 1 else bos_token_id
            p2 = int(row[t - 2]) if t >= 2 else bos_token_id
            heads = []
            for j in range(n_heads):
                if j == 0:
                    h = x
                elif j == 1:
                    h = p1 * 257 + x * 131 + 17
                elif j == 2:
                    h = p2 * 65537 + p1 * 257 + x * 131 + 31
                else:
                    h = x * (1009 + 2 * j) + t * (9176 + j) + j * 97
                heads.append(_i64(h) % A)
            orow.append(heads)
        out.append(orow)
    return out


def literal_addresses_step(tokens: Sequence[int], history: Sequence[Sequence[int]], *,
                           address_space: int, n_heads: int, position: int,
                           bos_token_id: int) -> List[List[int]]:
    """[B][n_heads] addresses of ravel_lm/model.py:234-263 for one decode step:
    prev1 is the last history column (bos_token_id when the history is empty),
    prev2 the one before it (bos_token_id when there are fewer than two), and
    the token/position heads use `position`."""
    A = address_space
    out = []
    for b, x in enumerate(tokens):
        h = list(history[b]) if history else []
        p1 = int(h[-1]) if len(h) >= 1 else bos_token_id
        p2 = int(h[-2]) if len(h) >= 2 else bos_token_id
        x = int(x)
        heads = []
        for j in range(n_heads):
            if j == 0:
                v = x
            elif j == 1:
                v = p1 * 257 + x * 131 + 17
            elif j == 2:
                v = p2 * 65537 + p1 * 257 + x * 131 + 31
            else:
                v = x * (1009 + 2 * j) + int(position) * (9176 + j) + j * 97
            heads.append(_i64(v) % A)
        out.append(heads)
    return out


def _argmax(values: Sequence[float]) -> int:
    best_i = 0
    best = values[0]
    for i in range(1, len(values)):
        v = values[i]
        if math.isnan(best):
            break
        if math.isnan(v) or v > best:
            best, best_i = v, i
    return best_i


def product_codes(logits_rows: Sequence[Sequence[float]], *, n_heads: int, n_codebooks: int,
                  codebook_size: int, address_space: int) -> List[List[int]]:
    """Per row of n_heads * n_codebooks * codebook_size logits, the n_heads
    addresses sum_q argmax(codebook q) * codebook_size**q, remainder by A
    (ravel_lm/model.py:170-187: multipliers 1, cbs, cbs**2, ...)."""
    out = []
    per = n_codebooks * codebook_size
    for row in logits_rows:
        heads = []
        for h in range(n_heads):
            addr, mult = 0, 1
            for q in range(n_codebooks):
                lo = h * per + q * codebook_size
                addr += _argmax(list(row[lo:lo + codebook_size])) * mult
                mult *= codebook_size
            heads.append(_i64(addr) % address_space)
        out.append(heads)
    return out


def layer_addresses(tokens: Optional[Sequence[Sequence[int]]], write_logits, read_logits, *,
                    address_space: int, n_literal: int, bos_token_id: int, n_learned: int,
                    n_codebooks: int, codebook_size: int,
                    B: int, T: int) -> Tuple[list, list]:
    """(write, read) [B][T][C] of model.py:333-346: literal heads, then the
    learned heads of write_logits / read_logits ([B][T][N] nested lists;
    read_logits None = reads use the write addresses)."""
    lit = (literal_addresses(tokens, address_space=address_space, n_heads=n_literal,
                             bos_token_id=bos_token_id)
           if n_literal > 0 else [[[] for _ in range(T)] for _ in range(B)])

    def learned(lg):
        if n_learned == 0:
            return [[[] for _ in range(T)] for _ in range(B)]
        return [product_codes(lg[b], n_heads=n_learned, n_codebooks=n_codebooks,
                              codebook_size=codebook_size, address_space=address_space)
                for b in range(B)]

    lw = learned(write_logits)
    write = [[lit[b][t] + lw[b][t] for t in range(T)] for b in range(B)]
    if n_learned == 0 or read_logits is None:
        return write, write
    lr = learned(read_logits)
    read = [[lit[b][t] + lr[b][t] for t in range(T)] for b in range(B)]
    return write, read

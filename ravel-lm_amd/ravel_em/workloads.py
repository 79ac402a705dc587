"""Seeded synthetic inputs for the five benchmark configurations (cfg1-cfg5).

Inputs are drawn with a ``torch.Generator`` on the target device (fast at the
large configs; deterministic per seed and device type).  Addresses are int64,
which is what the reference model produces (ravel_lm/model.py:195-231).

  cfg1  ravel_200k_byte: B=8 T=256 H=4 literal heads over byte tokens, A=512,
        D=16 fp32, k=4 (variant "1b": all heads = raw byte, A=256)
  cfg2  BPE-1k: B=32 T=1024 H=8 literal heads over Zipf(1.1) tokens, A=1024,
        D=32 fp32 or bf16, k=8
  cfg3  product-code routing: B=64 T=4096 H=8, address = argmax of two 64-way
        N(0,1) codebooks (code0 + 64*code1, A=4096), separate read logits,
        D=64 bf16, k=4
  cfg4  long context: B=4 T=65536 H=16, addresses U{0..65535}, D=64 bf16, k=1;
        adversarial variant: 90% of records at address 0
  cfg5  decode cache [B=256, H=8, A=4096, k=4, D=64] bf16 prefilled from T=2048
        Zipf(1.1) addresses, then single-token steps
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .addressing import LayerAddresses

Tensor = torch.Tensor
BOS = 257  # RavelConfig.bos_token_id (ravel_lm/config.py)


@dataclass
class Workload:
    name: str
    write: Tensor
    read: Optional[Tensor]
    payload: Tensor
    address_space: int
    k: int
    # the layer inputs the addresses come from (token ids / addressor logits)
    source: Optional[LayerAddresses] = None

    @property
    def shape(self):
        B, T, C, D = self.payload.shape
        return B, T, C, D

    @property
    def tokens(self) -> int:
        B, T, _, _ = self.payload.shape
        return B * T


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def literal_addresses(tokens: Tensor, *, address_space: int, n_heads: int, bos: int = BOS) -> Tensor:
    """Literal address families of ravel_lm/model.py:195-231 (token id, rolling
    bigram and trigram hashes, then token/position hashes)."""
    B, T = tokens.shape
    toks = tokens.long()
    A = address_space
    pad1 = torch.full((B, 1), bos, device=toks.device, dtype=torch.long)
    prev1 = torch.cat([pad1, toks[:, :-1]], dim=1)
    prev2 = torch.cat([pad1, pad1, toks[:, :-2]], dim=1)[:, :T]
    pos = torch.arange(T, device=toks.device, dtype=torch.long).view(1, T).expand(B, T)
    heads = []
    for j in range(n_heads):
        if j == 0:
            h = toks
        elif j == 1:
            h = prev1 * 257 + toks * 131 + 17
        elif j == 2:
            h = prev2 * 65537 + prev1 * 257 + toks * 131 + 31
        else:
            h = toks * (1009 + 2 * j) + pos * (9176 + j) + j * 97
        heads.append(h.remainder(A))
    return torch.stack(heads, dim=-1)


def literal_addresses_step(tokens: Tensor, history: Tensor, *, address_space: int, n_heads: int,
                           position: int, bos: int = BOS) -> Tensor:
    """One decode step of the literal families (ravel_lm/model.py:234-263):
    tokens [B], history [B, 2] = [prev2, prev1]; torch ops on the device, the
    reference's own formulation (timed against the in-kernel production)."""
    toks = tokens.long()
    A = address_space
    prev1 = history[:, -1].long() if history.numel() else torch.full_like(toks, bos)
    prev2 = history[:, -2].long() if history.shape[1] >= 2 else torch.full_like(toks, bos)
    heads = []
    for j in range(n_heads):
        if j == 0:
            h = toks
        elif j == 1:
            h = prev1 * 257 + toks * 131 + 17
        elif j == 2:
            h = prev2 * 65537 + prev1 * 257 + toks * 131 + 31
        else:
            h = toks * (1009 + 2 * j) + int(position) * (9176 + j) + j * 97
        heads.append(h.remainder(A))
    return torch.stack(heads, dim=-1)


def zipf(shape, n: int, g: torch.Generator, s: float = 1.1) -> Tensor:
    """Draws from p(r) proportional to r^-s over ranks r = 1..n; returns r-1."""
    ranks = torch.arange(1, n + 1, device=g.device, dtype=torch.float64)
    p = ranks.pow(-s)
    p = (p / p.sum()).float()
    numel = 1
    for x in shape:
        numel *= x
    out = torch.multinomial(p, numel, replacement=True, generator=g)
    return out.view(*shape)


def _normal(shape, g: torch.Generator, dtype: torch.dtype) -> Tensor:
    return torch.randn(*shape, generator=g, device=g.device, dtype=torch.float32).to(dtype)


def cfg1(device="cuda", variant: str = "1") -> Workload:
    g = _gen(device, 1001)
    B, T, H, D = 8, 256, 4, 16
    toks = torch.randint(0, 256, (B, T), generator=g, device=g.device)
    if variant == "1b":
        A = 256
        addr = toks.view(B, T, 1).expand(B, T, H).contiguous()
    else:
        A = 512
        addr = literal_addresses(toks, address_space=A, n_heads=H)
    payload = _normal((B, T, H, D), g, torch.float32)
    src = LayerAddresses(toks, H, BOS) if variant != "1b" else None
    return Workload(f"cfg{variant}", addr, None, payload, A, 4, src)


def cfg2(device="cuda", dtype: torch.dtype = torch.float32) -> Workload:
    g = _gen(device, 1002)
    B, T, H, D, A = 32, 1024, 8, 32, 1024
    toks = zipf((B, T), 1024, g)
    addr = literal_addresses(toks, address_space=A, n_heads=H)
    payload = _normal((B, T, H, D), g, dtype)
    return Workload(f"cfg2_{str(dtype).split('.')[-1]}", addr, None, payload, A, 8,
                    LayerAddresses(toks, H, BOS))


def product_code_addresses(B: int, T: int, H: int, g: torch.Generator, codebook: int = 64) -> Tensor:
    """argmax over two `codebook`-way N(0,1) logit groups, packed as
    code0 + codebook*code1 (ravel_lm/model.py:170-187)."""
    out = torch.empty(B, T, H, dtype=torch.long, device=g.device)
    for b in range(B):
        logits = torch.randn(T, H, 2, codebook, generator=g, device=g.device)
        codes = logits.argmax(dim=-1)
        out[b] = codes[..., 0] + codebook * codes[..., 1]
    return out


def cfg3(device="cuda", B: int = 64, T: int = 4096) -> Workload:
    g = _gen(device, 1003)
    H, D = 8, 64
    write = product_code_addresses(B, T, H, g)
    read = product_code_addresses(B, T, H, g)
    payload = _normal((B, T, H, D), g, torch.bfloat16)
    return Workload("cfg3", write, read, payload, 4096, 4)


def cfg3_logits(device="cuda", B: int = 64, T: int = 4096) -> Workload:
    """cfg3 as the memory layer sees it: bf16 N(0,1) write and read addressor
    logits side by side in one packed projection row [B, T, 2 * H*2*64]
    (ravel_lm/model.py:325-341), decoded inside the lookup.  ``write``/``read``
    hold the same addresses decoded by torch.argmax on the device."""
    g = _gen(device, 1013)
    H, D, Q, S, A = 8, 64, 2, 64, 4096
    n = H * Q * S
    packed = torch.empty(B, T, 2 * n, dtype=torch.bfloat16, device=g.device)
    for b in range(B):
        packed[b] = torch.randn(T, 2 * n, generator=g, device=g.device).to(torch.bfloat16)
    wl, rl = packed[..., :n], packed[..., n:]
    mult = torch.tensor([1, S], device=g.device)
    write = (wl.reshape(B, T, H, Q, S).argmax(-1) * mult).sum(-1).remainder(A)
    read = (rl.reshape(B, T, H, Q, S).argmax(-1) * mult).sum(-1).remainder(A)
    payload = _normal((B, T, H, D), g, torch.bfloat16)
    src = LayerAddresses(None, 0, BOS, wl, rl, H, Q, S)
    return Workload("cfg3_logits", write, read, payload, A, 4, src)


def cfg4(device="cuda", adversarial: bool = False, B: int = 4, T: int = 65536) -> Workload:
    g = _gen(device, 1005 if adversarial else 1004)
    H, D, A = 16, 64, 65536
    addr = torch.randint(0, A, (B, T, H), generator=g, device=g.device)
    if adversarial:
        hot = torch.rand(B, T, H, generator=g, device=g.device) < 0.9
        addr = torch.where(hot, torch.zeros_like(addr), addr)
    payload = _normal((B, T, H, D), g, torch.bfloat16)
    return Workload("cfg4_adv" if adversarial else "cfg4", addr, None, payload, A, 1)


@dataclass
class DecodeWorkload:
    prefill_write: Tensor  # [B, T, H]
    prefill_payload: Tensor  # [B, T, H, D]
    step_read: Tensor  # [S, B, H]
    step_write: Tensor  # [S, B, H]
    step_payload: Tensor  # [S, B, H, D]
    address_space: int
    k: int


def cfg5(device="cuda", B: int = 256, T: int = 2048, steps: int = 1024) -> DecodeWorkload:
    g = _gen(device, 1006)
    H, D, A, k = 8, 64, 4096, 4
    pw = zipf((B, T, H), A, g)
    pp = _normal((B, T, H, D), g, torch.bfloat16)
    sr = zipf((steps, B, H), A, g)
    sw = zipf((steps, B, H), A, g)
    sp = _normal((steps, B, H, D), g, torch.bfloat16)
    return DecodeWorkload(pw, pp, sr, sw, sp, A, k)


def algorithmic_bytes_latest_k(w: Workload) -> int:
    """Inputs read once + outputs written once for one latest-k call."""
    B, T, C, D = w.shape
    N = B * T * C
    esz = w.payload.element_size()
    addr = N * w.write.element_size() * (1 if w.read is None else 2)
    return addr + N * D * esz + N * w.k * D * esz + N * w.k


def algorithmic_bytes_sum(w: Workload) -> int:
    """Extra bytes of the segmented-sum output on the same tape."""
    B, T, C, D = w.shape
    N = B * T * C
    return N * D * w.payload.element_size() + N


def algorithmic_bytes_latest_k_sum(w: Workload) -> int:
    """Latest-k and segmented sum of one tape: inputs read once, both outputs
    written once (the "latest-k + sum" bytes of the benchmark statement)."""
    return algorithmic_bytes_latest_k(w) + algorithmic_bytes_sum(w)

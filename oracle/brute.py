"""Pure-Python brute force of the event-memory operator for tiny inputs.

TEST INFRASTRUCTURE ONLY.  Per (b, c) stream a dictionary keeps each address's
write history in time order, the pattern of the reference's own test
(tests/test_memory.py:43-50).  Address reduction and the int32 key-dtype
conversion follow ravel_lm/ravel_memory.py:45-49, :127-128.
"""
from __future__ import annotations

from typing import List, Optional, Tuple


def key_is_int32(B: int, T: int, C: int, A: int) -> bool:
    return B * C * A * (T + 1) <= 2**31 - 1


def wrap(a: int, A: int, via_int32: bool) -> int:
    if via_int32:
        a = ((a + 2**31) % 2**32) - 2**31  # two's-complement truncation to int32
    return a % A  # Python remainder: result in [0, A)


def latest_k_src(write, read, A: int, k: int, mask=None) -> List:
    """write/read nested lists [B][T][C]; mask [B][T] or None.  Returns
    src[b][t][c][j] = flat record index (b*T + t_src)*C + c, or -1."""
    B, T, C = len(write), len(write[0]), len(write[0][0])
    via32 = key_is_int32(B, T, C, A)
    read = write if read is None else read
    out = [[[[-1] * k for _ in range(C)] for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for c in range(C):
            hist = {}
            for t in range(T):
                prior = hist.get(wrap(read[b][t][c], A, via32), [])
                for j, ts in enumerate(reversed(prior[-k:])):
                    out[b][t][c][j] = (b * T + ts) * C + c
                if mask is None or mask[b][t]:
                    hist.setdefault(wrap(write[b][t][c], A, via32), []).append(t)
    return out


def seg_sum(write, read, payload, A: int, mask=None) -> Tuple[List, List]:
    """payload nested [B][T][C][D] of Python floats; exact-order float sums."""
    B, T, C = len(write), len(write[0]), len(write[0][0])
    D = len(payload[0][0][0])
    via32 = key_is_int32(B, T, C, A)
    read = write if read is None else read
    out = [[[[0.0] * D for _ in range(C)] for _ in range(T)] for _ in range(B)]
    has = [[[False] * C for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for c in range(C):
            acc = {}
            for t in range(T):
                ar = wrap(read[b][t][c], A, via32)
                if ar in acc:
                    out[b][t][c] = list(acc[ar])
                    has[b][t][c] = True
                if mask is None or mask[b][t]:
                    aw = wrap(write[b][t][c], A, via32)
                    cur = acc.setdefault(aw, [0.0] * D)
                    for d in range(D):
                        cur[d] += payload[b][t][c][d]
    return out, has


def sorted_keys(write, A: int, mask=None) -> Tuple[List[int], List[int]]:
    """Composite keys of ravel_memory.py:133-135 sorted, and their order."""
    B, T, C = len(write), len(write[0]), len(write[0][0])
    via32 = key_is_int32(B, T, C, A)
    keys = []
    for b in range(B):
        for t in range(T):
            if mask is not None and not mask[b][t]:
                continue
            for c in range(C):
                a = wrap(write[b][t][c], A, via32)
                keys.append(((b * C + c) * A + a) * (T + 1) + t)
    order = sorted(range(len(keys)), key=lambda i: keys[i])
    return [keys[i] for i in order], order


def cache_replay(steps, B: int, C: int, A: int, k: int) -> Tuple[dict, List]:
    """Replay ('read', addr[B][C]) / ('write', addr[B][C], payload[B][C]) steps on a
    k-slot cache; returns the final {(b,c,a): [payloads...]} and every read's
    result [(vals[B][C][k], mask[B][C][k])]."""
    state = {}
    reads = []
    for step in steps:
        if step[0] == "read":
            vals, mask = [], []
            for b in range(B):
                vr, mr = [], []
                for c in range(C):
                    a = min(max(step[1][b][c], 0), A - 1)
                    hist = state.get((b, c, a), [])
                    vr.append([hist[j] if j < len(hist) else None for j in range(k)])
                    mr.append([j < len(hist) for j in range(k)])
                vals.append(vr)
                mask.append(mr)
            reads.append((vals, mask))
        else:
            for b in range(B):
                for c in range(C):
                    a = min(max(step[1][b][c], 0), A - 1)
                    hist = state.setdefault((b, c, a), [])
                    hist.insert(0, step[2][b][c])
                    del hist[k:]
    return state, reads

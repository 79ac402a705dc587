"""ctypes binding of the C ABI in include/ravel_em.h.

The shared library ``libravel_em.so`` sits next to this file (built by
``ravel_em._build``).  There is no fallback: if the library is missing or a
tensor is not on a ROCm device, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_NAME = "libravel_em.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# dtype codes (include/ravel_em.h)
INT32, INT64 = 1, 2
ADDR_GEN = 3  # address code: write/read pointers are AddrGen descriptors
FLOAT32, BFLOAT16, FLOAT16, FLOAT64 = 10, 11, 12, 13

_PAYLOAD_CODES = {
    torch.float32: FLOAT32,
    torch.bfloat16: BFLOAT16,
    torch.float16: FLOAT16,
    torch.float64: FLOAT64,
}
_ADDR_CODES = {torch.int32: INT32, torch.int64: INT64}

_vp, _i, _i64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
_i32 = ctypes.c_int32


class AddrGen(ctypes.Structure):
    """struct ravel_em_addr_gen of include/ravel_em.h (field order and types)."""

    _fields_ = [
        ("tokens", _vp), ("token_dtype", _i32), ("n_literal", _i32),
        ("token_stride_b", _i64), ("token_stride_t", _i64), ("bos_token_id", _i64),
        ("logits", _vp), ("logits_dtype", _i32), ("n_learned", _i32),
        ("n_codebooks", _i32), ("codebook_size", _i32),
        ("logits_stride_b", _i64), ("logits_stride_t", _i64),
        ("history", _vp), ("history_len", _i32), ("reserved", _i32),
        ("history_stride_b", _i64), ("history_stride_t", _i64), ("position_offset", _i64),
    ]

# name -> (restype, argtypes); must list every function of include/ravel_em.h
SIGNATURES = {
    "ravel_em_last_error": (ctypes.c_char_p, []),
    "ravel_em_workspace_status": (_i, [_vp, _sz, _vp, _vp]),
    "ravel_em_abi_version": (_i, []),
    "ravel_em_addresses": (_i, [_vp, _i64, _i64, _i64, _i, _vp, _vp]),
    "ravel_em_key_bits": (_i, [_i64, _i64, _i64, _i64]),
    "ravel_em_set_sort_path": (_i, [_i]),
    "ravel_em_set_split_slots": (_i, [_i64]),
    "ravel_em_profile_start": (_i, []),
    "ravel_em_profile_stop": (_i, [_vp, _vp, _i]),
    "ravel_em_sort_order_workspace": (_sz, [_i64, _i64, _i64, _i64, _i]),
    "ravel_em_sort_order": (_i, [_vp, _i, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "ravel_em_latest_k_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "ravel_em_latest_k_fwd": (
        _i,
        [_vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "ravel_em_latest_k_fwd_static": (
        _i,
        [_vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp],
    ),
    "ravel_em_latest_k_resolve_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i, _i]),
    "ravel_em_latest_k_resolve": (
        _i, [_vp, _vp, _i, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _sz, _vp]
    ),
    "ravel_em_gather_rows": (_i, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "ravel_em_latest1_linear_workspace": (_sz, [_i64, _i64, _i64, _i64, _i, _i]),
    "ravel_em_latest1_linear_fwd": (
        _i, [_vp, _vp, _i, _vp, _i, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]
    ),
    "ravel_em_latest_k_bwd_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i, _i]),
    "ravel_em_latest_k_bwd": (
        _i, [_vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i, _vp, _vp, _sz, _vp]
    ),
    "ravel_em_latest_k_sum_workspace": (
        _sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i]
    ),
    "ravel_em_latest_k_sum_fwd": (
        _i,
        [_vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
         _vp, _sz, _vp],
    ),
    "ravel_em_seg_sum_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "ravel_em_seg_sum_fwd": (
        _i, [_vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]
    ),
    "ravel_em_seg_sum_bwd_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "ravel_em_seg_sum_bwd": (
        _i, [_vp, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _sz, _vp]
    ),
    "ravel_em_cache_read": (_i, [_vp, _vp, _vp, _i, _i, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "ravel_em_cache_write": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _vp]),
    "ravel_em_cache_step": (
        _i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]
    ),
    "ravel_em_cache_prefill_workspace": (_sz, [_i64, _i64, _i64, _i64, _i]),
    "ravel_em_cache_prefill": (
        _i, [_vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]
    ),
}


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or a call into it failed."""


_lib: Optional[ctypes.CDLL] = None


def library() -> ctypes.CDLL:
    """Load libravel_em.so (once) and declare its signatures."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; run `python -m ravel_em._build` "
                "(or __graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = library().ravel_em_last_error().decode(errors="replace")
        raise NativeLibraryError(f"ravel_em error {rc}: {msg}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# torch's raw current-stream accessor (the one its generated kernels' launchers
# call) skips building a Stream object on every call; the public route stays as
# the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on t's device (the launch stream)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def payload_code(dtype: torch.dtype) -> int:
    code = _PAYLOAD_CODES.get(dtype)
    if code is None:
        raise TypeError(f"payload dtype {dtype} is not supported (float32/bfloat16/float16/float64)")
    return code


def addr_code(dtype: torch.dtype) -> int:
    return _ADDR_CODES[dtype]


def addr_gen(tokens: Optional[torch.Tensor], n_literal: int, bos_token_id: int,
             logits: Optional[torch.Tensor], n_learned: int, n_codebooks: int,
             codebook_size: int, history: Optional[torch.Tensor] = None,
             position: int = 0) -> AddrGen:
    """Descriptor of produced addresses.  tokens is [B, T] int32/int64, logits
    [B, T, n_learned * n_codebooks * codebook_size] with a unit last stride,
    history [B, h] the tokens before t = 0 (newest last, tokens' dtype); all
    are read by the kernels through their strides.  position is the time of
    t = 0 for the token/position heads."""
    g = AddrGen()
    if n_literal > 0:
        g.tokens = tokens.data_ptr()
        g.token_dtype = _ADDR_CODES[tokens.dtype]
        g.token_stride_b, g.token_stride_t = tokens.stride(0), tokens.stride(1)
        if history is not None and history.shape[1] > 0:
            g.history = history.data_ptr()
            g.history_len = history.shape[1]
            g.history_stride_b, g.history_stride_t = history.stride(0), history.stride(1)
    g.position_offset = int(position)
    g.n_literal = n_literal
    g.bos_token_id = bos_token_id
    if n_learned > 0:
        g.logits = logits.data_ptr()
        g.logits_dtype = _PAYLOAD_CODES[logits.dtype]
        g.logits_stride_b, g.logits_stride_t = logits.stride(0), logits.stride(1)
    g.n_learned = n_learned
    g.n_codebooks = n_codebooks
    g.codebook_size = codebook_size
    return g


def ref(desc: Optional[AddrGen]) -> Optional[int]:
    """Address of a descriptor for a void* argument (None stays NULL)."""
    return None if desc is None else ctypes.addressof(desc)


def require_device(*tensors: Optional[torch.Tensor]) -> None:
    """The product path runs on ROCm devices only; there is no CPU fallback."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "ravel_em runs on ROCm GPU tensors only (got a tensor on "
                f"{t.device}); there is no CPU fallback"
            )
    library()


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# Status words (include/ravel_em.h): bit values of the word at offset 0 of a
# sorting call's workspace.
STATUS_SORT_WAIT, STATUS_SUM_WAIT = 1, 2
_STATUS_NAMES = {STATUS_SORT_WAIT: "a sort look-back wait gave up",
                 STATUS_SUM_WAIT: "a segmented-sum look-back wait gave up"}


class DeviceWaitError(NativeLibraryError):
    """A call returned OK but one of its bounded device waits gave up, so its
    outputs are not valid (the call's status word is non-zero)."""


# Opt-in: after every sorting call, read the status word back (this
# synchronizes the stream, so it is meant for tests and debugging) and raise
# DeviceWaitError when it is non-zero.  Calls made while a HIP graph is being
# captured are not checked.  RAVEL_EM_CHECK_STATUS=1 turns it on at import.
_status_check = os.environ.get("RAVEL_EM_CHECK_STATUS", "") == "1"
status_checks = 0  # number of status words read so far


def set_status_check(on: bool) -> bool:
    """Turn the status read-back on or off; returns the previous setting."""
    global _status_check
    prev, _status_check = _status_check, bool(on)
    return prev


def status_word(ws: torch.Tensor) -> int:
    """The status word of the last call that used workspace ws (synchronizes
    the current stream of ws's device)."""
    word = ctypes.c_uint32(0)
    check(library().ravel_em_workspace_status(ws.data_ptr(), ws.numel(), ctypes.byref(word),
                                              stream_of(ws)))
    return int(word.value)


def raise_for_status(word: int) -> None:
    if word:
        names = [n for b, n in _STATUS_NAMES.items() if word & b] or ["unknown bits"]
        raise DeviceWaitError(f"ravel_em status word {word:#x}: {'; '.join(names)}; "
                              "the call's outputs are not valid")


def after_call(ws: torch.Tensor) -> None:
    """Check the status word of the call that just used ws, when enabled."""
    global status_checks
    if not _status_check or torch.cuda.is_current_stream_capturing():
        return
    status_checks += 1
    raise_for_status(status_word(ws))

"""C ABI checks that need no GPU: the library loads, exports every function
that include/ravel_em.h declares, and rejects bad arguments before any launch."""
import ctypes
import os
import re

import pytest
import torch

from ravel_em import _native as nat
from ravel_em.ravel_memory import _composite_key_dtype

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ravel_em.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ravel_em_\w+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    names = header_functions()
    assert "ravel_em_latest_k_fwd" in names and "ravel_em_seg_sum_fwd" in names
    assert len(names) >= 18


def test_library_exports_every_declared_symbol():
    lib = nat.library()
    for name in header_functions():
        assert hasattr(lib, name), name


def test_binding_table_matches_header():
    assert sorted(nat.SIGNATURES) == header_functions()


def test_abi_version():
    assert nat.library().ravel_em_abi_version() == 4


def test_static_scratch_rejects_oversized_lookups_without_a_device():
    """The no-allocation entry point checks the size before any HIP call, so a
    lookup beyond its static scratch fails here, on a host without a GPU."""
    lib = nat.library()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the size check comes first
    rc = lib.ravel_em_latest_k_fwd_static(fake, None, nat.INT64, None, fake, nat.BFLOAT16,
                                          16, 65536, 16, 64, 65536, 1, fake, fake, None, None, None)
    assert rc == 1  # RAVEL_EM_EINVAL
    assert "static scratch" in _err()


def test_status_query_rejects_bad_arguments_without_a_device():
    lib = nat.library()
    word = ctypes.c_uint32(7)
    assert lib.ravel_em_workspace_status(None, 256, ctypes.byref(word), None) == 1
    assert "null" in _err()
    assert lib.ravel_em_workspace_status(ctypes.c_void_p(0x1000), 3, ctypes.byref(word), None) == 1
    assert "status word" in _err()
    assert lib.ravel_em_workspace_status(ctypes.c_void_p(0x1000), 256, None, None) == 1


def test_sorting_workspaces_hold_the_status_header():
    lib = nat.library()
    hdr = 256  # RAVEL_EM_STATUS_BYTES
    text = open(HEADER).read()
    assert re.search(r"#define RAVEL_EM_STATUS_BYTES 256\b", text)
    assert "RAVEL_EM_STATUS_SORT_WAIT = 1" in text and "RAVEL_EM_STATUS_SUM_WAIT = 2" in text
    assert (nat.STATUS_SORT_WAIT, nat.STATUS_SUM_WAIT) == (1, 2)
    # the smallest tapes still reserve the header
    assert lib.ravel_em_sort_order_workspace(1, 1, 1, 1, 0) >= hdr
    assert lib.ravel_em_latest_k_workspace(1, 1, 1, 1, 1, 0, 0, 1) >= hdr
    assert lib.ravel_em_latest_k_resolve_workspace(1, 1, 1, 1, 1, 0, 0) >= hdr
    assert lib.ravel_em_seg_sum_workspace(1, 1, 1, 8, 1, 0, 0, nat.FLOAT32) >= hdr
    assert lib.ravel_em_seg_sum_bwd_workspace(1, 1, 1, 8, 1, 0, 0, nat.FLOAT32) >= hdr
    assert lib.ravel_em_cache_prefill_workspace(1, 0, 1, 1, 0) >= hdr
    assert lib.ravel_em_latest1_linear_workspace(1, 1, 1, 1, 0, 1) >= hdr


def test_status_words_raise_on_the_host(monkeypatch):
    """The read-back plumbing: a non-zero word raises DeviceWaitError naming
    the wait; zero passes; nothing is read while checking is off."""
    nat.raise_for_status(0)
    with pytest.raises(nat.DeviceWaitError, match="sort look-back"):
        nat.raise_for_status(nat.STATUS_SORT_WAIT)
    with pytest.raises(nat.DeviceWaitError, match="segmented-sum look-back"):
        nat.raise_for_status(nat.STATUS_SUM_WAIT)
    with pytest.raises(nat.DeviceWaitError, match="0x3"):
        nat.raise_for_status(3)
    words = iter([0, nat.STATUS_SUM_WAIT])
    monkeypatch.setattr(nat, "status_word", lambda ws: next(words))
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    prev = nat.set_status_check(False)
    try:
        nat.after_call(None)  # off: no read
        nat.set_status_check(True)
        before = nat.status_checks
        nat.after_call(None)  # reads 0
        with pytest.raises(nat.DeviceWaitError):
            nat.after_call(None)  # reads the sum bit
        assert nat.status_checks == before + 2
    finally:
        nat.set_status_check(prev)


@pytest.mark.parametrize("shape", [(1, 2048, 3, 1024), (1024, 65536, 64, 65536), (8, 256, 4, 512),
                                   (4, 65536, 16, 65536), (32, 1024, 8, 1024), (1, 1, 1, 1)])
def test_key_bits_matches_python_rule(shape):
    bits = nat.library().ravel_em_key_bits(*shape)
    assert bits == (32 if _composite_key_dtype(*shape) == torch.int32 else 64)


def test_workspace_queries_are_positive_and_monotone():
    lib = nat.library()
    small = lib.ravel_em_latest_k_workspace(2, 64, 3, 11, 1, 0, 0, 0)
    big = lib.ravel_em_latest_k_workspace(4, 65536, 16, 65536, 1, 0, 0, 0)
    assert 0 < small < big
    # cfg4: two u32 key buffers + histograms + src
    N = 4 * 65536 * 16
    assert big >= 2 * 4 * N + 4 * N
    assert lib.ravel_em_seg_sum_workspace(4, 65536, 16, 64, 65536, 0, 0, nat.BFLOAT16) > 0
    assert lib.ravel_em_cache_prefill_workspace(256, 2048, 8, 4096, 0) > 0
    assert lib.ravel_em_sort_order_workspace(2, 64, 3, 11, 1) > lib.ravel_em_sort_order_workspace(2, 64, 3, 11, 0)


def _err():
    return nat.library().ravel_em_last_error().decode()


def test_invalid_arguments_rejected_without_launch():
    lib = nat.library()
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   2, 3, 4, 5, 0, 1, None, None, None, None, 0, None)
    assert rc == 1 and "address_space" in _err()
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   2, 3, 4, 5, 7, 0, None, None, None, None, 0, None)
    assert rc == 1 and "k must be positive" in _err()
    rc = lib.ravel_em_latest_k_fwd(None, None, 7, None, None, nat.FLOAT32,
                                   2, 3, 4, 5, 7, 1, None, None, None, None, 0, None)
    assert rc == 1 and "address dtype" in _err()
    rc = lib.ravel_em_seg_sum_fwd(None, None, nat.INT64, None, None, 99,
                                  2, 3, 4, 5, 7, None, None, None, 0, None)
    assert rc == 1 and "payload dtype" in _err()
    # one batch row must fit the kernels' 32-bit indices ...
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   2, 1 << 27, 1 << 4, 5, 7, 1, None, None, None, None, 0, None)
    assert rc == 1 and "one batch row" in _err()
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   2, 1 << 26, 1 << 4, 5, 7, 2, None, None, None, None, 0, None)
    assert rc == 1 and "one batch row" in _err()
    # ... while a tape of many rows past 2^31 slots is accepted (split by rows)
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   1 << 20, 1 << 12, 1 << 4, 5, 7, 1, None, None, None, None, 0, None)
    assert rc == 1 and "null" in _err()
    # int32 sources of such a tape do not exist
    fake = ctypes.c_void_p(0x1000)
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   1 << 20, 1 << 12, 1 << 4, 5, 7, 1, None, None, fake, None, 0, None)
    assert rc == 1 and "int32 sources" in _err()
    rc = lib.ravel_em_latest_k_resolve(None, None, nat.INT64, None,
                                       1 << 20, 1 << 12, 1 << 4, 7, 1, fake, None, 0, None)
    assert rc == 1 and "2^31" in _err()
    rc = lib.ravel_em_latest_k_bwd(fake, fake, nat.FLOAT32, 1 << 20, 1 << 12, 1 << 4, 5, 1, 0,
                                   fake, None, 0, None)
    assert rc == 1 and "2^31" in _err()
    rc = lib.ravel_em_sort_order(None, nat.INT64, None, 1 << 20, 1 << 12, 1 << 4, 7,
                                 None, None, None, 0, None)
    assert rc == 1 and "null" in _err()  # int64 order: any tape
    # null pointers with a non-empty tape
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   2, 3, 4, 5, 7, 1, None, None, None, None, 0, None)
    assert rc == 1 and "null" in _err()
    rc = lib.ravel_em_cache_read(None, None, None, nat.INT64, nat.BFLOAT16, 2, 3, 0, 1, 4, None, None, None)
    assert rc == 1 and "cache shape" in _err()
    # the joint latest-k + sum entry point checks the union of both operators' arguments
    joint = lambda *a: lib.ravel_em_latest_k_sum_fwd(*a)
    rc = joint(None, None, nat.INT64, None, None, nat.FLOAT32, 2, 3, 4, 5, 7, 0,
               None, None, None, None, None, None, 0, None)
    assert rc == 1 and "k must be positive" in _err()
    rc = joint(None, None, 7, None, None, nat.FLOAT32, 2, 3, 4, 5, 7, 1,
               None, None, None, None, None, None, 0, None)
    assert rc == 1 and "address dtype" in _err()
    rc = joint(None, None, nat.INT64, None, None, 99, 2, 3, 4, 5, 7, 1,
               None, None, None, None, None, None, 0, None)
    assert rc == 1 and "payload dtype" in _err()
    rc = joint(fake, None, nat.INT64, None, fake, nat.FLOAT32, 2, 3, 4, 5, 7, 1,
               fake, fake, None, None, fake, None, 0, None)
    assert rc == 1 and "null" in _err()  # no sum output
    rc = joint(None, None, nat.INT64, None, None, nat.FLOAT32, 2, 1 << 27, 1 << 4, 5, 7, 1,
               None, None, None, None, None, None, 0, None)
    assert rc == 1 and "one batch row" in _err()
    rc = joint(None, None, nat.INT64, None, None, nat.FLOAT32, 1 << 20, 1 << 12, 1 << 4, 5, 7, 1,
               None, None, fake, None, None, None, 0, None)
    assert rc == 1 and "int32 sources" in _err()


def test_workspace_too_small_is_reported_before_launch():
    lib = nat.library()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: the size check comes first
    rc = lib.ravel_em_latest_k_fwd(fake, None, nat.INT64, None, fake, nat.FLOAT32,
                                   2, 64, 3, 4, 11, 1, fake, fake, None, fake, 16, None)
    assert rc == 3 and "workspace" in _err()
    # the joint call in each of its forms (short tape, long tape, the pair for k > 8)
    for (T, k) in [(64, 2), (6000, 1), (64, 12)]:
        need = lib.ravel_em_latest_k_sum_workspace(2, T, 3, 8, 11, k, 0, 0, 0, nat.BFLOAT16)
        assert need > 16
        rc = lib.ravel_em_latest_k_sum_fwd(fake, None, nat.INT64, None, fake, nat.BFLOAT16,
                                           2, T, 3, 8, 11, k, fake, fake, None, fake, fake,
                                           fake, 16, None)
        assert rc == 3 and "workspace" in _err(), (T, k)


def test_empty_tape_is_a_no_op():
    lib = nat.library()
    rc = lib.ravel_em_latest_k_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                   0, 3, 4, 5, 7, 1, None, None, None, None, 0, None)
    assert rc == 0
    rc = lib.ravel_em_latest_k_sum_fwd(None, None, nat.INT64, None, None, nat.FLOAT32,
                                       0, 3, 4, 5, 7, 1, None, None, None, None, None, None, 0,
                                       None)
    assert rc == 0


def test_split_hook_and_split_workspaces():
    lib = nat.library()
    assert lib.ravel_em_set_split_slots(-1) == 1 and "split slots" in _err()
    assert lib.ravel_em_set_split_slots(1 << 31) == 1
    # a tape past 2^26 slots is sized for one range of rows: 2^31 records of
    # 32768 rows x 65536 steps run in ranges of 1024 rows (2^26 records)
    big = lib.ravel_em_latest_k_workspace(1 << 15, 1 << 16, 1, 4096, 1, 0, 0, 0)
    rng = lib.ravel_em_latest_k_workspace(1 << 10, 1 << 16, 1, 4096, 1, 0, 0, 0)
    assert big == rng > 0
    assert lib.ravel_em_latest_k_workspace((1 << 10) + 1, 1 << 16, 1, 4096, 1, 0, 0, 0) == big
    assert lib.ravel_em_seg_sum_workspace(1 << 15, 1 << 16, 1, 1, 4096, 0, 0, nat.FLOAT32) == \
        lib.ravel_em_seg_sum_workspace(1 << 10, 1 << 16, 1, 1, 4096, 0, 0, nat.FLOAT32) > 0
    # k = 4 over 2^29 records: ranges of 256 rows of 2^16 records; the sorted
    # backward adds the range-local sources when it splits
    assert lib.ravel_em_latest_k_bwd_workspace(8192, 1 << 15, 2, 1, 4, nat.FLOAT32, 0) > \
        lib.ravel_em_latest_k_bwd_workspace(256, 1 << 15, 2, 1, 4, nat.FLOAT32, 0) > 0
    # a single row past 2^26 slots runs whole
    assert lib.ravel_em_latest_k_workspace(1, 1 << 28, 2, 4096, 1, 0, 0, 0) > big
    # the hook: ranges of two rows size the workspace of a two-row tape
    try:
        assert lib.ravel_em_set_split_slots(2 * 64 * 3 * 4) == 0
        assert lib.ravel_em_latest_k_workspace(7, 64, 3, 11, 4, 0, 0, 1) == \
            lib.ravel_em_latest_k_workspace(2, 64, 3, 11, 4, 0, 0, 1)
        assert lib.ravel_em_set_split_slots(2 * 64 * 3) == 0  # the sums count records
        assert lib.ravel_em_seg_sum_workspace(7, 64, 3, 8, 11, 1, 0, nat.FLOAT32) == \
            lib.ravel_em_seg_sum_workspace(2, 64, 3, 8, 11, 1, 0, nat.FLOAT32)
    finally:
        assert lib.ravel_em_set_split_slots(0) == 0
    assert lib.ravel_em_latest_k_workspace(7, 64, 3, 11, 4, 0, 0, 1) > \
        lib.ravel_em_latest_k_workspace(2, 64, 3, 11, 4, 0, 0, 1)

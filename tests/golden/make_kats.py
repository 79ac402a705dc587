"""Write tests/golden/reference_kats.json: the known-answer cases of the
reference's own tests, as plain data.

Inputs and the asserted outputs are transcribed from the reference files cited
in each case; "full" expectations (every slot) extend the reference's partial
assertions by replaying each stream's write history by hand, as the
reference's brute-force test does (tests/test_memory.py:43-50).
Run: python tests/golden/make_kats.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

KATS = {
    "key_dtype": {
        "source": "tests/test_memory.py:11-13",
        "cases": [
            {"B": 1, "T": 2048, "C": 3, "A": 1024, "dtype": "int32"},
            {"B": 1024, "T": 65536, "C": 64, "A": 65536, "dtype": "int64"},
        ],
    },
    "latest_exact": {
        "source": "tests/test_memory.py:16-23",
        "write": [[[1], [2], [1], [3], [1]]],
        "payload": [[[[0.0]], [[1.0]], [[2.0]], [[3.0]], [[4.0]]]],
        "address_space": 8,
        "k": 2,
        "asserted": [
            {"index": [0, 0, 0, 0], "mask": False},
            {"index": [0, 2, 0, 0, 0], "value": 0.0},
            {"index": [0, 4, 0, 0, 0], "value": 2.0},
            {"index": [0, 4, 0, 1, 0], "value": 0.0},
        ],
        "full_src": [[[[-1, -1]], [[-1, -1]], [[0, -1]], [[-1, -1]], [[2, 0]]]],
    },
    "latest_separate_reads_masked": {
        "source": "tests/test_memory.py:26-58",
        "write": [[[1], [2], [1], [3], [2], [1]]],
        "read": [[[1], [1], [2], [1], [2], [3]]],
        "write_mask": [[True, True, False, True, True, True]],
        "address_space": 8,
        "k": 2,
        "full_src": [[[[-1, -1]], [[0, -1]], [[1, -1]], [[0, -1]], [[1, -1]], [[3, -1]]]],
    },
    "sum_exact": {
        "source": "tests/test_memory.py:61-67",
        "write": [[[1], [2], [1], [1]]],
        "payload": [[[[1.0]], [[10.0]], [[3.0]], [[7.0]]]],
        "address_space": 8,
        "asserted": [
            {"index": [0, 0, 0, 0], "value": 0.0},
            {"index": [0, 2, 0, 0], "value": 1.0},
            {"index": [0, 3, 0, 0], "value": 4.0},
        ],
        "full_sum": [[[[0.0]], [[0.0]], [[1.0]], [[4.0]]]],
        "full_mask": [[[False], [False], [True], [True]]],
    },
    "decode_cache": {
        "source": "tests/test_memory.py:70-79",
        "batch_size": 1,
        "n_heads": 2,
        "address_space": 16,
        "payload_dim": 3,
        "addresses": [[5, 7]],
        "payload": [[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]],
        "mask_before_write": [[False, False]],
        "mask_after_write": [[True, True]],
    },
    "bench_forced_repeat": {
        "source": "ravel_lm/bench.py:30-48 with the docs/VERIFICATION.md:83-97 shape",
        "torch_manual_seed": 0,
        "B": 2,
        "T": 256,
        "C": 3,
        "D": 16,
        "address_space": 512,
        "forced_times": [10, 100],
        "forced_value": 42.0,
        "note": "addresses torch.randint(0, A-1, (B,T,C)) then [:,10,:] and [:,100,:] set to A-1; "
                "payload torch.randn(B,T,C,D) with [:,10] = 42; the t=100 slot-0 read must be exactly 42",
    },
}


def main():
    path = os.path.join(HERE, "reference_kats.json")
    with open(path, "w") as f:
        json.dump(KATS, f, indent=1)
    print(path)


if __name__ == "__main__":
    main()

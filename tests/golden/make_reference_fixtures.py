"""Writes tests/golden/reference_fixtures.json: the literal input/expected
values that the reference's own end-to-end CPU tests hold for the hot path.

The values are data transcribed from the reference test files named on each
entry (inputs, launch parameters, expected outputs and tolerances); no
reference code is executed or copied.  Run: python tests/golden/make_reference_fixtures.py
"""
import json
import os

FIXTURES = {
    "matmul_4x4": {
        "source": "crates/sile/tests/backend_matmul.rs:21-72 "
                  "(also crates/sile/tests/llvm_ir_cpu_runtime.rs:40-103)",
        "kernel": "matmul", "bm": 2, "bn": 2, "bk": 2, "grid": [4, 1, 1],
        "a": {"shape": [4, 4], "data": [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16]},
        "b": {"shape": [4, 4], "data": [1, 0, 2, 1, 0, 1, 3, 2, 1, 0, 4, 3, 0, 1, 5, 4]},
        "c_init": {"shape": [4, 4], "data": [0] * 16},
        "expected": [4, 6, 40, 30, 12, 14, 96, 70, 20, 22, 152, 110, 28, 30, 208, 150],
        "tolerance_abs": 1e-4,
    },
    "softmax_4x8": {
        "source": "crates/sile/tests/backend_softmax.rs:17-38",
        "kernel": "softmax", "bm": 2, "bn": 8, "grid": [2, 1, 1],
        "x": {"shape": [4, 8], "data": list(range(32))},
        "expected_row_sum": 1.0,
        "tolerance_abs": 1e-4,
    },
    "parallel_reduce_ones": {
        "source": "crates/sile/tests/backend_parallel_reduce.rs:11-29",
        "kernel": "parallel_reduce", "tile": 1000, "grid": [100, 1, 1],
        "a": {"shape": [100000], "fill": 1.0},
        "expected": 100000.0,
        "tolerance_abs": 1e-4,
    },
    "parallel_reduce_arange": {
        "source": "crates/sile/examples/parallel_reduce.rs:11-31",
        "kernel": "parallel_reduce", "tile": 100, "grid": [100, 1, 1],
        "a": {"shape": [10000], "arange_from": 1},
        "expected": 50005000.0,
        "tolerance_rel": 1e-5,
    },
    "relu_8": {
        "source": "crates/sile/tests/llvm_ir_cpu_runtime.rs:105-141",
        "kernel": "relu (max(x, 0) via a >= select; outside the hot path, kept as a map-semantics vector)",
        "x": [-3.0, -1.0, 0.0, 2.5, 4.0, -7.0, 8.0, -0.5],
        "expected": [0.0, 0.0, 0.0, 2.5, 4.0, 0.0, 8.0, 0.0],
    },
    "vec_add": {
        "source": "crates/sile/tests/backend_vec_add.rs:11-25",
        "kernel": "vec_add (outside the hot path)",
        "a_fill": 1.0, "b_fill": 2.0, "expected_fill": 3.0,
    },
}

if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_fixtures.json")
    with open(path, "w") as f:
        json.dump(FIXTURES, f, indent=1)
        f.write("\n")
    print("wrote", path)

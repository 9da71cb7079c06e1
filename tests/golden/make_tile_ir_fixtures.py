"""Writes tests/golden/tile_ir/*.tir: the printed Tile IR of the DSL kernels
with the constants of the reference's own end-to-end tests (matmul 2/2/2,
softmax 2/8, parallel_reduce 1000, vec_add 4, the mlp example's matvec
32/8), derived as tests/tile_ir_text.py
describes.  Run: python tests/golden/make_tile_ir_fixtures.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests import tile_ir_text as T  # noqa: E402

FIXTURES = {
    "matmul_2x2x2.tir": T.matmul(2, 2, 2),            # crates/sile/tests/backend_matmul.rs:21-72
    "softmax_2x8.tir": T.softmax(2, 8),               # crates/sile/tests/backend_softmax.rs:17-38
    "softmax_2x8_unfused.tir": T.softmax(2, 8, passes=False),
    "parallel_reduce_1000.tir": T.parallel_reduce(1000),  # backend_parallel_reduce.rs:11-29
    "vec_add_4.tir": T.vec_add(4),                    # crates/sile/tests/tile_ir_print.rs:7-169
    "vec_add_4_unfused.tir": T.vec_add(4, passes=False),
    "row_sum_4x64.tir": T.row_reduce(4, 64, "sum"),
    "row_max_4x64_rank1.tir": T.row_reduce(4, 64, "max", out_rank=1),
    "attention_32x64x128.tir": T.attention(32, 64, 128, 0.08838834764831845),
    "attention_32x64x128_unfused.tir": T.attention(32, 64, 128, 0.08838834764831845,
                                                   passes=False),
    "matvec_32x8.tir": T.matvec(32, 8),               # crates/sile/examples/mlp.rs:68-89
    "matvec_32x8_unfused.tir": T.matvec(32, 8, passes=False),
}


def main():
    out = os.path.join(HERE, "tile_ir")
    os.makedirs(out, exist_ok=True)
    for name, text in FIXTURES.items():
        with open(os.path.join(out, name), "w") as f:
            f.write(text)
    print(f"wrote {len(FIXTURES)} files to {out}")


if __name__ == "__main__":
    main()

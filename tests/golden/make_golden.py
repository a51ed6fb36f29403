"""Writes tests/golden/*.npz: small known-answer vectors produced by the reference's own CPU code
(qwen_cpu/quants.h Quants::Ref dequant and qwen_cpu/ops.h Ops::matmul), compiled from
/root/reference by `make -C oracle ref` into oracle/_ref/libqkref.so.

Run in the development container (the reference is not present on the GPU box):
    make -C oracle && make -C oracle ref && python tests/golden/make_golden.py

Each file holds data only: the weight bytes (GGUF layout), fp32 activations, the reference's
dequantized rows and its matmul output.  Inputs come from the repository's seeded generator.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib  # noqa: E402

CASES = [  # (name, type, k, n, T)
    ("q4k_k512_n8_t3", oracle_lib.T_Q4_K, 512, 8, 3),
    ("q4k_k1024_n4_t5", oracle_lib.T_Q4_K, 1024, 4, 5),
    ("q6k_k512_n8_t3", oracle_lib.T_Q6_K, 512, 8, 3),
    ("q6k_k1024_n4_t5", oracle_lib.T_Q6_K, 1024, 4, 5),
]


def main():
    gen = oracle_lib.Oracle()
    ref = oracle_lib.RefLib()
    ref.init(1)
    for i, (name, typ, k, n, T) in enumerate(CASES):
        seed = oracle_lib.SEED_BASE | (0x600 + i)
        w = gen.weights(typ, n, k, seed)
        x = gen.normal(seed + 1, T * k).reshape(T, k)
        rb = len(w) // n
        deq = np.stack([ref.dequant(typ, w[r * rb:(r + 1) * rb], k, avx=False) for r in range(n)])
        y = ref.matmul(typ, w, k, n, x)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), type=typ, k=k, n=n, w=w, x=x, deq=deq, y=y)
        print("wrote", name)


if __name__ == "__main__":
    main()

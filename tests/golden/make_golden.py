"""Writes tests/golden/ref_dequant.npz from the reference's own decoders.

Runs oracle/_ref/ref_dequant, built by oracle/Makefile (target `ref`) from the
reference's vendor/strata/include/strata/artifact/dequant.hpp, and stores:
  fp16  f32[65536]    fp16_to_fp32(h) for every pattern h
  q2    f32[256, 64]  dequantize_q2_0 of the 256 blocks of the reference's
                      upstream known-answer recipe (scripts/test-upstream.mjs:20)
Usage: python tests/golden/make_golden.py   (needs /root/reference; run once)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def main():
    oracle.build()
    table = oracle.ref_dequant_table()
    if table is None:
        raise SystemExit("oracle/_ref/ref_dequant is not built (needs the reference tree)")
    fp16, q2 = table
    np.savez_compressed(os.path.join(HERE, "ref_dequant.npz"), fp16=fp16, q2=q2)
    print("wrote", os.path.join(HERE, "ref_dequant.npz"))


if __name__ == "__main__":
    main()

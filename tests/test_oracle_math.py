"""Pins of the oracle's scalar building blocks: fp16 decode, expf, fp16
rounding, the synthetic-data generator. CPU only."""
import ctypes
import os
import re
from fractions import Fraction

import numpy as np
import pytest

from conftest import ROOT


def test_half_bits_exhaustive_vs_numpy(oracle):
    # kernels/strata.cu:13-18 against numpy's IEEE binary16 conversion (an
    # independent implementation), all 65,536 patterns.
    h = np.arange(65536, dtype=np.uint32)
    packed = (h[0::2] | (h[1::2] << 16)).astype(np.uint32)
    ours = oracle.unpack_half(packed, 65536)
    ref = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # includes -0, subnormals, inf


def test_half_bits_vs_reference_decoder(oracle):
    # The reference's own fp16_to_fp32 (vendor/strata/include/strata/artifact/
    # dequant.hpp:33-55) built in oracle/_ref, or its committed output.
    ref = oracle.ref_dequant_table()
    if ref is not None:
        table = ref[0]
    else:
        table = np.load(os.path.join(ROOT, "tests", "golden", "ref_dequant.npz"))["fp16"]
    h = np.arange(65536, dtype=np.uint32)
    ours = oracle.unpack_half((h[0::2] | (h[1::2] << 16)).astype(np.uint32), 65536)
    nan = np.isnan(table)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), table[~nan].view(np.uint32))


def test_half_known_answers(oracle):
    # tests/model.test.mjs:57 of the reference
    assert oracle.half_bits(1) == 2.0 ** -24
    assert oracle.half_bits(0x3C00) == 1.0
    assert np.signbit(oracle.half_bits(0x8000)) and oracle.half_bits(0x8000) == 0.0
    assert oracle.half_bits(0x7C00) == float("inf")


def test_expf_matches_libm_exhaustively(oracle):
    # Every float in [-104, 0] (all exponent arguments a router or sigmoid of
    # a finite input can see after max-subtraction): the restated
    # optimized-routines expf agrees with glibc's expf on all but a handful of
    # inputs (glibc evaluates the same algorithm with FMA on x86-64), and it is
    # not simply a correctly rounded exp (which disagrees ~1e-4 of the time).
    d_libm, d_dbl = oracle.expf_survey(0x80000000, 0xC2D00001, 1)
    assert d_libm <= 4, d_libm
    assert 50000 < d_dbl < 200000, d_dbl


def test_expf_positive_range_and_specials(oracle):
    d_libm, _ = oracle.expf_survey(0x00000000, 0x42B17218, 3)  # [0, 88.72]
    assert d_libm <= 4
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(float("-inf")) == 0.0
    assert oracle.expf(float("inf")) == float("inf")
    assert np.isnan(oracle.expf(float("nan")))
    assert oracle.expf(-104.0) == 0.0
    assert oracle.expf(89.0) == float("inf")
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    for x in (-103.9, -87.5, -1e-30, 1e-30, 0.5, 1.0, 10.0, 88.5):
        assert np.float32(oracle.expf(x)) == np.float32(libm.expf(x)), x


def test_device_exp2_table_is_exact():
    # The device copy of the 2^(i/32) table (strata_device.h) recomputed with
    # exact rational arithmetic: round 2^(i/32) to the nearest double.
    src = open(os.path.join(ROOT, "stratacuda_amd", "csrc", "strata_device.h")).read()
    body = src.split("kExp2Tab[32] = {")[1].split("};")[0]
    table = [int(t, 16) for t in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert len(table) == 32
    import struct
    for i, bits in enumerate(table):
        # 2^(i/32) to 80 bits by bisection on y^32 = 2^i, then round to double.
        lo, hi = Fraction(1), Fraction(2)
        target = Fraction(2) ** i
        for _ in range(90):
            mid = (lo + hi) / 2
            if mid ** 32 < target:
                lo = mid
            else:
                hi = mid
        d = float(lo)  # correctly rounded: the interval is far narrower than an ulp
        assert abs(Fraction(d) - lo) <= Fraction(1, 2 ** 53), i
        u = struct.unpack("<Q", struct.pack("<d", d))[0]
        assert (u - (i << 47)) & ((1 << 64) - 1) == bits, i


def test_f32_to_f16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.normal(0, 0.05, 20000).astype(np.float32),
        (rng.random(5000) * 7e-5).astype(np.float32),  # subnormal fp16 range
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 2.0 ** -24, 3 * 2.0 ** -25, 1.0 + 2.0 ** -11], np.float32),
    ])
    ours = np.array([oracle.f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(ours, xs.astype(np.float16).view(np.uint16))


def test_generator_is_splitmix64(oracle):
    # SplitMix64 from state 0 emits 0xE220A8397B1DCDAF first (published
    # sequence); rand(seed, stream, i) = mix(mix(seed + G*(stream+1)) + i).
    from stratacuda_amd import workload as wl
    assert wl._mix64(0) == 0xE220A8397B1DCDAF
    for seed, stream, i in [(0, 0, 0), (20260101, 16, 12345), (2 ** 63, 7, 2 ** 40)]:
        assert oracle.rand(seed, stream, i) == wl.rand64(seed, stream, i)
    n = np.array([oracle.normal(5, 4, i) for i in range(20000)])
    assert abs(n.mean()) < 0.03 and abs(n.var() - 1.0) < 0.03 and np.abs(n).max() <= 6.0


def test_synth_blob_layout(oracle):
    # Scales are fp16(|0.05 N|): finite, non-negative; codes uniform.
    W, F = 128, 64
    blob = oracle.synth_blob(W, F, 7, 16, 0.05)
    L = oracle.blob_layout(W, F)
    assert blob.size == L["blob_bytes"]
    scales = blob[L["gate_up_scales"]:].view(np.uint16)
    assert np.all((scales & 0x8000) == 0) and np.all((scales & 0x7C00) != 0x7C00)
    codes = np.unpackbits(blob[:L["gate_up_scales"]]).reshape(-1, 2)
    counts = np.bincount(codes[:, 0] * 2 + codes[:, 1], minlength=4)
    assert counts.min() > 0.2 * counts.sum()

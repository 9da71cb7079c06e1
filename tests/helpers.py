"""Seeded inputs and comparison helpers shared by the tests.

Inputs follow the configurations' recipes: numpy default_rng(seed) draws,
rounded to the storage type with round-to-nearest-even.
"""
from __future__ import annotations

import numpy as np

from oracle import cpuref


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def bf16_round(x: np.ndarray):
    """Returns (bits uint16, values float32) of x rounded to bf16."""
    bits = cpuref.bf16_from_f32(x)
    return bits, cpuref.f32_from_bf16(bits)


def f16_round(x: np.ndarray):
    h = np.asarray(x, dtype=np.float32).astype(np.float16)
    return h.view(np.uint16), h.astype(np.float32)


def fp8_quantise(x: np.ndarray):
    """Per-tensor e4m3fn quantisation: s = amax/448, q = rne_sat(x/s).
    Returns (codes uint8, scale float, dequantised float32)."""
    amax = float(np.max(np.abs(x)))
    scale = np.float32(amax / 448.0) if amax > 0 else np.float32(1.0)
    q = cpuref.e4m3_encode(x, float(scale))
    return q, float(scale), cpuref.e4m3_decode(q, float(scale))


def assert_close(got, ref, atol, rtol, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    with np.errstate(invalid="ignore"):  # inf - inf: handled below
        err = np.abs(got - ref)
        bound = atol + rtol * np.abs(ref)
    # NaN compares false: an element is good only if its error is provably within
    # the bound of a finite reference, or it equals the reference (matching
    # infinities, NaN for NaN)
    good = ((err <= bound) & np.isfinite(ref)) | (got == ref) | (np.isnan(got) & np.isnan(ref))
    bad = ~good
    if bad.any():
        with np.errstate(invalid="ignore"):
            excess = np.where(bad, np.nan_to_num(err - bound, nan=np.inf), -np.inf)
        idx = np.unravel_index(np.argmax(excess), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); worst at {idx}: got {got[idx]!r}, ref {ref[idx]!r}")


def say(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a crash log shows it."""
    print(f"[case] {msg}", flush=True)

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


def assert_same_bits(got, ref, what=""):
    """float32 arrays equal bit for bit, except that any NaN matches any NaN
    (the payload of a NaN is not part of the comparison)."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    gn, rn = np.isnan(got), np.isnan(ref)
    bad = (gn != rn) | (~gn & (got.view(np.uint32) != ref.view(np.uint32)))
    if bad.any():
        idx = np.unravel_index(np.argmax(bad), bad.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} differ in bits; first at "
                             f"{idx}: got {got[idx]!r}, ref {ref[idx]!r}")


def max_fold_probe_rows(cols, seed):
    """Rows whose max depends on the reference's fold order (acc = x0;
    acc = x > acc ? x : acc): NaN at column 0 (NaN), NaN later (ignored), all
    NaN, all -inf, -inf then NaNs, +inf beside NaNs, and rows of negative
    values with +0 / -0 ties placed so the first zero in row order lies in
    another lane, wave or 16-byte chunk than the other zeros."""
    r = rng(seed)
    base = lambda: -(np.abs(r.normal(size=cols)) + 0.5).astype(np.float32)
    rows = []
    x = base(); x[0] = np.nan; rows.append(x)
    x = base(); x[cols // 2] = np.nan; x[-1] = np.nan; rows.append(x)
    rows.append(np.full(cols, np.nan, np.float32))
    rows.append(np.full(cols, -np.inf, np.float32))
    x = np.full(cols, np.nan, np.float32); x[0] = -np.inf; rows.append(x)
    x = base(); x[cols - 1] = np.inf; x[1] = np.nan; x[cols // 3] = np.nan; rows.append(x)
    x = base(); x[0] = np.nan; x[cols // 2] = np.inf; rows.append(x)
    for first_neg in (True, False):
        for lo in sorted({1, 5, 9, cols // 5, cols // 2}):
            x = base()
            x[lo] = -0.0 if first_neg else 0.0
            for hi in (cols - 1, (lo + cols) // 2, lo + 1):
                if lo < hi < cols:
                    x[hi] = 0.0 if first_neg else -0.0
            rows.append(x)
    for _ in range(8):   # zeros of random signs at random columns
        x = base()
        pos = r.choice(cols, size=min(cols, 6), replace=False)
        x[pos] = np.where(r.random(pos.size) < 0.5, -0.0, 0.0).astype(np.float32)
        rows.append(x)
    rows.append(r.normal(size=cols).astype(np.float32))
    return np.stack(rows)

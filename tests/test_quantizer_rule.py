"""The device quantizers' division-free rounding (bq_common.h ``Quantizer``), restated in
numpy float32 and held to the exact-quotient rule of the oracle.

The device computes f = fl(v * fl(1/s)), rint(f), and decides only within 4e-5 of a
half-integer b by the sign of the exact remainder v - b*s (its fma keeps the sign; here
float64 holds b*s exactly and keeps the sign of the difference). This pins that the
shortcut never changes a byte: random values at many scales, dense sweeps of ulps around
every half-integer, exact ties, and calibrated scales whose quotients pass the clamp.
"""
import numpy as np

from oracle import quant as O

F32 = np.float32


def device_rule(v, s):
    v = np.asarray(v, F32)
    s = F32(s)
    if s == 0:
        return np.zeros(v.shape, np.int8)
    r = F32(1.0) / s  # correctly rounded
    f = (v * r).astype(F32)
    k = np.rint(f).astype(F32)
    near = ~(np.abs((f - k).astype(F32)) < F32(0.49996))
    out = k.astype(np.float64)
    if near.any():
        fn, kn, vn = f[near], k[near], v[near]
        if not np.isfinite(fn).all():
            raise AssertionError("non-finite quotient: the device takes the division path")
        b = (kn + np.copysign(F32(0.5), (fn - kn).astype(F32))).astype(F32)
        d = vn.astype(np.float64) - b.astype(np.float64) * np.float64(s)  # exact product; sign exact
        lo = b.astype(np.float64) - 0.5
        tie = np.where(np.mod(lo, 2) == 0, lo, lo + 1)
        out[near] = np.where(d > 0, b + 0.5, np.where(d < 0, lo, tie))
    return np.clip(out, -127, 127).astype(np.int8)


def check(v, s):
    got = device_rule(v, s)
    want = O.quantize_with_scale(np.asarray(v, F32), F32(s))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (float(s), np.asarray(v, F32).ravel()[bad[:5]], got.ravel()[bad[:5]], want.ravel()[bad[:5]])


def test_random_values_many_scales():
    rng = np.random.default_rng(0)
    for _ in range(300):
        x = (rng.normal(size=4096) * 10.0 ** rng.uniform(-30, 30)).astype(F32)
        s = O.scale_of(np.abs(x).max())
        check(x, s)


def test_ulp_sweeps_around_every_half_integer():
    rng = np.random.default_rng(1)
    ks = np.arange(-127, 127, dtype=np.float64) + 0.5
    for _ in range(60):
        s = F32(10.0 ** rng.uniform(-20, 20) * rng.uniform(1, 2))
        centre = (ks * np.float64(s)).astype(F32)  # the f32 values nearest each half-integer * s
        vals = [centre]
        lo, hi = centre.copy(), centre.copy()
        for _ in range(24):
            lo = np.nextafter(lo, F32(-np.inf)).astype(F32)
            hi = np.nextafter(hi, F32(np.inf)).astype(F32)
            vals += [lo, hi]
        v = np.concatenate(vals)
        check(v, s)


def test_exact_ties_and_power_of_two_scales():
    for e in (-20, -3, 0, 5, 17):
        s = F32(2.0 ** e)
        v = ((np.arange(-127, 127) + 0.5) * np.float64(s)).astype(F32)  # exact ties
        check(v, s)
        check(-v, s)


def test_calibrated_scales_past_the_clamp():
    rng = np.random.default_rng(2)
    for _ in range(100):
        x = rng.normal(size=2048).astype(F32) * F32(rng.uniform(1, 1e4))
        s = F32(O.scale_of(np.abs(x).max()) * F32(rng.uniform(0.001, 0.9)))
        check(x, s)

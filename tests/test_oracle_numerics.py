"""Pin the restated scalar numerics (numeric.hex) against closed forms and a
high-precision oracle, and check that the library's host build of the same
device numerics is bit-identical to the restatement.

exp follows the reference's contract (tests/portable_exp.rs:41-90,
tests/support/portable_exp.cpp:26-102): <= 1 ULP against a correctly rounded
exp (mpmath at 80 bits adjudicates every input the float64 reference does not
settle), exact at 0, +-inf and the saturation limits, NaN -> 0x7fc00000.
"""
import ctypes
import math
import struct

import mpmath
import numpy as np
import pytest


def word(b):
    return struct.unpack("<f", struct.pack("<I", b & 0xFFFFFFFF))[0]


def bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def exp_inputs():
    xs = []
    for b in [0, 1, 0x007FFFFF, 0x00800000, 0x7F7FFFFF, 0x7F800000, 0x7F800001, 0x7FC12345]:
        xs += [b, b | 0x80000000]
    for center in [0x39000000, 0x3EB17218, 0x42B17218, 0x42CFF1B5, 0x42AEAC50]:
        for i in range(-256, 257):
            xs += [center + i, (center + i) | 0x80000000]
    for k in range(-150, 129):
        b = bits(float(np.float32((k + 0.5) * math.log(2.0))))
        xs += [b + i for i in range(-4, 5)]
    xs += [b << 16 for b in range(65536)]
    rng = np.random.default_rng(123456789)
    xs += rng.integers(0, 2**32, 20000, dtype=np.uint64).tolist()
    xs += [bits(float(v)) for v in rng.uniform(-104.0, 89.0, 20000).astype(np.float32)]
    return np.array([x & 0xFFFFFFFF for x in xs], dtype=np.uint32)


def correctly_rounded_exp_bits(x: float) -> int:
    mpmath.mp.prec = 80
    v = mpmath.exp(mpmath.mpf(x))
    f = np.float32(float(v))  # 80-bit value rounded to double then to float
    # Re-round from the 80-bit value to avoid a double-rounding error.
    lo, hi = np.nextafter(f, np.float32(-np.inf)), np.nextafter(f, np.float32(np.inf))
    best = min([lo, f, hi], key=lambda c: abs(mpmath.mpf(float(c)) - v))
    return bits(float(best))


def test_exp_accuracy_contract(oracle):
    lib = oracle.lib()
    xs = exp_inputs()
    max_ulp = 0
    for b in xs.tolist():
        x = word(b)
        got = bits(lib.ox_exp(x))
        if math.isnan(x):
            assert got == 0x7FC00000
            continue
        with np.errstate(over="ignore", under="ignore"):
            approx = np.float32(np.exp(np.float64(x)))
        expected = bits(float(approx))
        if got != expected:
            expected = correctly_rounded_exp_bits(x)
        ulp = abs(got - expected)
        exact = math.isinf(x) or x == 0.0 or x >= word(0x42B17218) or x <= word(0xC2CFF1B5)
        assert ulp <= 1, (hex(b), hex(got), hex(expected))
        if exact:
            assert got == expected, hex(b)
        max_ulp = max(max_ulp, ulp)
    assert max_ulp <= 1


def test_exp_planted_mistake_is_detected(oracle):
    """A dropped correction term in the rational step (c = r) must break the
    1-ULP contract somewhere in the active range."""
    F = np.float32

    def broken(x):
        n = round(float(F(abs(x)) * F(word(0x3FB8AA3B))))
        k = F(-n if x < 0 else n)
        hi = F(F(x) - F(k * F(word(0x3F317200))))
        lo = F(k * F(word(0x35BFBE8E)))
        r = F(hi - lo)
        c = r  # mistake: correction term dropped
        y = F(F(1) - F(F(lo - F(F(r * c) / F(F(2) - c))) - hi))
        return float(np.ldexp(np.float64(y), int(k)))

    bad = 0
    for x in np.linspace(-20, 20, 101):
        e = float(np.exp(np.float64(np.float32(x))))
        if abs(broken(float(np.float32(x))) - e) > 2 * abs(e) * 2 ** -23:
            bad += 1
    assert bad > 10


def test_sqrt_softplus_sincos_closed_forms(oracle):
    lib = oracle.lib()
    rng = np.random.default_rng(7)
    for x in np.float32(2.0) ** rng.uniform(-100, 100, 3000).astype(np.float32):
        got = lib.ox_sqrt(float(x))
        ref = np.float32(math.sqrt(float(x)))
        assert abs(bits(got) - bits(float(ref))) <= 1, float(x)
    assert lib.ox_sqrt(0.0) == 0.0 and lib.ox_sqrt(-4.0) == 0.0
    for x in np.linspace(-30, 30, 2001).astype(np.float32):
        ref = max(float(x), 0.0) + math.log1p(math.exp(-abs(float(x))))
        assert abs(lib.ox_softplus(float(x)) - ref) <= 2e-7 * max(1.0, abs(ref)), float(x)
    s, c = ctypes.c_float(), ctypes.c_float()
    freqs = [float(np.float32(1e7) ** np.float32(-(2 * i) / 64)) for i in range(32)]
    for pos in list(range(0, 64)) + [511, 1023, 4095, 32767]:
        for f in freqs:
            a = float(np.float32(np.float32(pos) * np.float32(f)))
            lib.ox_sincos(a, ctypes.byref(s), ctypes.byref(c))
            assert abs(s.value - math.sin(a)) < 3e-7 * max(1.0, a / 1000.0), (pos, f)
            assert abs(c.value - math.cos(a)) < 3e-7 * max(1.0, a / 1000.0), (pos, f)


def test_bf16_rounding_closed_form(oracle):
    lib = oracle.lib()
    # nearest-even at an exact tie, NaN quieting, overflow to inf
    assert lib.ox_f2bf(word(0x3F808000)) == 0x3F80
    assert lib.ox_f2bf(word(0x3F818000)) == 0x3F82
    assert lib.ox_f2bf(word(0x7F800001)) == 0x7FC0
    assert lib.ox_f2bf(word(0x7F7FFFFF)) == 0x7F80


@pytest.fixture(scope="module")
def cq35lib():
    import os
    import cq35._build as b
    if not os.path.exists(b.LIBRARY):
        b.build()
    from cq35 import _lib
    return _lib.load()


def test_library_host_numerics_match_restatement(oracle, cq35lib):
    """The library's numerics (the same source as its device code, compiled
    for the host) are bit-identical to the CPU restatement."""
    lib = oracle.lib()
    for b in exp_inputs()[::3].tolist():
        x = word(b)
        assert bits(cq35lib.cq35_numeric_exp(x)) == bits(lib.ox_exp(x)), hex(b)
    rng = np.random.default_rng(3)
    for x in rng.uniform(-40, 40, 4000).astype(np.float32).tolist():
        assert bits(cq35lib.cq35_numeric_softplus(x)) == bits(lib.ox_softplus(x))
        assert bits(cq35lib.cq35_numeric_sqrt(abs(x))) == bits(lib.ox_sqrt(abs(x)))
    s1, c1, s2, c2 = (ctypes.c_float() for _ in range(4))
    for a in rng.uniform(0, 5000, 4000).astype(np.float32).tolist():
        cq35lib.cq35_numeric_sincos(a, ctypes.byref(s1), ctypes.byref(c1))
        lib.ox_sincos(a, ctypes.byref(s2), ctypes.byref(c2))
        assert (bits(s1.value), bits(c1.value)) == (bits(s2.value), bits(c2.value))

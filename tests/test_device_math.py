"""Pins the HIP kernels' segment math on the CPU.

The device functions seg_shares / seg_shares_grad (csrc/ca_common.h) are
re-evaluated here in float32 numpy, with the polynomial constants parsed from
the header itself, and compared with the float64 oracle's segment terms
(oracle/ca_oracle.py: shifted moments, analytic_reference.py:12-75).  A wrong
constant, a sign slip in the signed closed forms or a swapped share fails
these checks without a GPU.
"""
import math
import os
import re

import numpy as np
import pytest

from oracle import ca_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "continuum-attention_amd", "csrc", "ca_common.h")
f32 = np.float32
LN2 = f32(0.69314718055994531)


def coeffs(name):
    src = open(HDR).read()
    m = re.search(r"// %s\n.*?poly\d\(y, ([^)]*)\)" % name, src, flags=re.S)
    assert m, name
    return [f32(float(c.strip().rstrip("f"))) for c in m.group(1).split(",")]


def switch_point():
    m = re.search(r"kSeriesT = ([0-9.]+)f", open(HDR).read())
    return f32(float(m.group(1)))


def poly(y, c):
    """Horner evaluation in float32, highest coefficient first."""
    acc = np.asarray(c[-1], f32) * np.ones_like(np.asarray(y, f32))
    for ci in c[-2::-1]:
        acc = acc * y + ci
    return acc


def device_terms(sl, sr, pl, pr):
    """float32 restatement of seg_shares_grad's value path (csrc/ca_common.h)."""
    sl, sr, pl, pr = (np.asarray(v, f32) for v in (sl, sr, pl, pr))
    with np.errstate(divide="ignore", invalid="ignore"):
        x = (sr - sl) * LN2
        dp = pr - pl
        inv_x = f32(1) / x
        a = dp * inv_x
        rc = (pr - a) * inv_x
        lc = a - rc
        j2c = (pr - f32(2) * rc) * inv_x
    y = x * x
    e1, o1 = poly(y, coeffs("CA_J1_EVEN")), poly(y, coeffs("CA_J1_ODD"))
    e2, o2 = poly(y, coeffs("CA_J2_EVEN")), poly(y, coeffs("CA_J2_ODD"))
    rs = pl * (x * o1 + e1)
    ls = pr * (-x * o1 + e1)
    j2s = pl * (x * o2 + e2)
    small = np.abs(x) < switch_point()
    return (np.where(small, ls, lc), np.where(small, rs, rc), np.where(small, j2s, j2c))


def reference_terms(sl, sr, m):
    """float64 segment terms from the oracle's shifted moments (natural units)."""
    a = np.asarray(sl, np.float64) * math.log(2) + m
    b = np.asarray(sr, np.float64) * math.log(2) + m
    z0, z1, z2 = O.shifted_moments(b - a)
    E = np.exp(np.maximum(a, b) - m)
    return E * (z0 - z1), E * z1, E * z2, E


T_SW = float(switch_point())


@pytest.fixture(scope="module")
def grid():
    rng = np.random.default_rng(7)
    d = np.concatenate([np.linspace(-40, 40, 4001), [0.0, 1e-7, -1e-7],
                        T_SW / math.log(2) + np.linspace(-1e-3, 1e-3, 21),
                        -T_SW / math.log(2) + np.linspace(-1e-3, 1e-3, 21)])
    base = rng.uniform(-9, 7, d.size)            # row-relative scores, log2 units
    sl = base.astype(np.float32)
    sr = (base + d).astype(np.float32)
    keep = (sl <= 8) & (sr <= 8)                # kernels keep s - m <= 8
    return sl[keep], sr[keep]


def test_forward_shares_match_oracle(grid):
    sl, sr = grid
    pl, pr = np.exp2(sl), np.exp2(sr)
    L, R, _ = device_terms(sl, sr, pl, pr)
    Lr, Rr, _, E = reference_terms(sl.astype(np.float64), sr.astype(np.float64), 0.0)
    assert np.all(np.isfinite(L)) and np.all(np.isfinite(R))
    # error relative to the segment's own scale E = e^{max(a,b)-m}
    assert np.max(np.abs(L - Lr) / E) < 2e-6
    assert np.max(np.abs(R - Rr) / E) < 2e-6
    assert np.all(L >= 0) and np.all(R >= 0)


def test_backward_terms_match_oracle(grid):
    sl, sr = grid
    rng = np.random.default_rng(8)
    gl, gr = (rng.standard_normal(sl.size).astype(np.float32) for _ in range(2))
    pl, pr = np.exp2(sl), np.exp2(sr)
    L, R, J2 = device_terms(sl, sr, pl, pr)
    xm = R - J2
    dR = gl * xm + gr * J2
    dL = gl * (L - xm) + gr * xm
    Lr, Rr, J2r, E = reference_terms(sl.astype(np.float64), sr.astype(np.float64), 0.0)
    z0 = (Lr + Rr) / E
    # analytic_reference.py:73-74 in the shifted-moment form
    dR_ref = gl * (Rr - J2r) + gr * J2r
    dL_ref = gl * (E * z0 - 2 * Rr + J2r) + gr * (Rr - J2r)
    scale = E * (np.abs(gl) + np.abs(gr))
    assert np.max(np.abs(dR - dR_ref) / scale) < 5e-6
    assert np.max(np.abs(dL - dL_ref) / scale) < 5e-6


def test_polynomials_against_quadrature():
    """The fitted even/odd constants reproduce J1, J2 on the series interval."""
    from scipy import integrate
    for n, en, on in ((1, "CA_J1_EVEN", "CA_J1_ODD"), (2, "CA_J2_EVEN", "CA_J2_ODD")):
        ce = [float(c) for c in coeffs(en)]
        co = [float(c) for c in coeffs(on)]
        for x in np.linspace(-T_SW, T_SW, 61):
            ref = integrate.quad(lambda u: u ** n * math.exp(x * u), 0, 1, epsabs=1e-14)[0]
            y = x * x
            got = poly(y, ce) + x * poly(y, co)
            assert abs(got - ref) / ref < 3e-7, (n, x)  # quadratic parts: ~2 float32 ulp


def test_planted_sign_error_is_caught(grid):
    """A flipped odd part (R and L swapped below the switch) must fail."""
    sl, sr = grid
    pl, pr = np.exp2(sl), np.exp2(sr)
    L, R, _ = device_terms(sl, sr, pl, pr)
    Lr, Rr, _, E = reference_terms(sl.astype(np.float64), sr.astype(np.float64), 0.0)
    small = np.abs((sr - sl) * LN2) < T_SW
    # swapping the shares is a plausible slip; it must be visible wherever x != 0
    swapped_err = np.max(np.abs(R - Lr)[small & (np.abs(sr - sl) > 0.1)] / E[small & (np.abs(sr - sl) > 0.1)])
    assert swapped_err > 1e-3

"""The bf16x6 product used by the HIP kernels (csrc/ca_common.h: split_pair,
split8, mfma_x6, mfma16_x6), restated in numpy and checked against float64.

An fp32 value is split into three bf16 limbs rounded to nearest even,
x = h + m + l exactly (24 significant bits in three 8-bit limbs), and a*b is
the sum of the six limb products whose orders add to <= 2 (l*h, m*m, h*l,
m*h, h*m, h*h in the kernels' issue order), each exact in fp32, accumulated
in fp32 per 16-term MFMA block.  The checks pin
the exact split, the dot-product error against a sequential fp32 FMA chain,
and that plausible mistakes (a dropped term, a transposed term, two limbs
only) fail the same bound.
"""
import numpy as np

RNG = np.random.default_rng(7)


def bf16_rne(x):
    """fp32 -> bf16 (round to nearest even) -> fp32, as v_cvt_pk_bf16_f32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def bf16_trunc(x):
    u = np.asarray(x, np.float32).view(np.uint32)
    return (u & np.uint32(0xFFFF0000)).view(np.float32)


def split3(x, rnd=bf16_rne):
    x = np.asarray(x, np.float32)
    h = rnd(x)
    r = (x - h).astype(np.float32)
    m = rnd(r)
    r2 = (r - m).astype(np.float32)
    return h, m, rnd(r2)


def dot_limbs(a, b, terms, rnd=bf16_rne, block=16):
    la, lb = split3(a, rnd), split3(b, rnd)
    acc = np.float32(0.0)
    for ia, ib in terms:
        x, y = la[ia], lb[ib]
        for k0 in range(0, len(a), block):
            # one MFMA: exact bf16 products summed, added to the fp32 accumulator
            s = np.dot(x[k0:k0 + block].astype(np.float64), y[k0:k0 + block].astype(np.float64))
            acc = np.float32(acc + np.float32(s))
    return acc


X6 = [(2, 0), (1, 1), (0, 2), (1, 0), (0, 1), (0, 0)]  # l*h, m*m, h*l, m*h, h*m, h*h


def fp32_chain(a, b):
    acc = np.float32(0.0)
    for x, y in zip(a, b):
        acc = np.float32(np.float64(x) * np.float64(y) + np.float64(acc))
    return acc


def test_split_is_exact():
    # three 8-bit limbs hold the 24-bit fp32 significand exactly (rounded limbs
    # carry a sign, truncated ones do not; both are exact) while the limbs stay
    # normal, |x| >= 2^-126 * 2^16; the kernels' values are far above that
    x = (RNG.standard_normal(20000) * 10.0 ** RNG.integers(-30, 30, 20000)).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, 1.0, -1.0, 3.0e38, 1.0 + 2.0 ** -23, -(2.0 - 2.0 ** -23)], np.float32)])
    for rnd in (bf16_rne, bf16_trunc):
        h, m, l = split3(x, rnd)
        resid = x.astype(np.float64) - h.astype(np.float64) - m.astype(np.float64) - l.astype(np.float64)
        assert np.all(resid == 0.0)
        for v in (h, m, l):  # every limb is a bf16 value
            assert np.all((v.view(np.uint32) & 0xFFFF) == 0)


def _errors(n, scale_choices=(1e-3, 1.0, 30.0), D=64, **kw):
    e6, e32 = [], []
    for _ in range(n):
        a = (RNG.standard_normal(D) * RNG.choice(scale_choices)).astype(np.float32)
        b = RNG.standard_normal(D).astype(np.float32)
        ref = np.dot(a.astype(np.float64), b.astype(np.float64))
        scale = np.abs(a.astype(np.float64) * b).sum()
        e6.append(abs(dot_limbs(a, b, kw.get("terms", X6), kw.get("rnd", bf16_rne)) - ref) / scale)
        e32.append(abs(fp32_chain(a, b) - ref) / scale)
    return np.array(e6), np.array(e32)


def test_dot_product_at_fp32_accuracy():
    e6, e32 = _errors(600)
    assert e6.max() <= 1.0e-7        # relative to sum |a_i b_i|
    assert e6.mean() <= e32.mean()   # no worse than a sequential fp32 FMA chain


def test_planted_mistakes_fail_the_bound():
    # two-limb product (h*h, h*m, m*h): bf16x3
    e3, _ = _errors(200, terms=[(1, 0), (0, 1), (0, 0)])
    assert e3.max() > 1.0e-6
    # the m*m term dropped
    ed, _ = _errors(200, terms=[(2, 0), (0, 2), (1, 0), (0, 1), (0, 0)])
    assert ed.max() > 1.0e-7
    # a transposed term: l*l in place of l*h
    et, _ = _errors(200, terms=[(2, 2), (1, 1), (0, 2), (1, 0), (0, 1), (0, 0)])
    assert et.max() > 1.0e-7

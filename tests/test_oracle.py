"""Pins the float64 oracle (oracle/ca_oracle.py) before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle (a dropped cap,
a swapped share, a wrong moment sign, a missing normalisation, a transposed
contraction) fails it.  Sources of the expected values:

* adaptive quadrature (scipy.integrate.quad) of the defining integrals;
* closed forms / limits stated by the reference tests (test_acma.py:71-103,
  test_analytic_backward.py:25-32);
* float64 autograd through an independent torch restatement of the weights
  (oracle/ca_cpu_port.tile_weights), as test_analytic_backward.py:41-62 does;
* central finite differences of the composed operator (brute force).
"""
import math
import warnings

import numpy as np
import pytest
import torch
from scipy import integrate

from oracle import ca_oracle as O
from oracle import ca_cpu_port as P


def quad(f):
    # the tolerance asked for is below what quad can confirm for some
    # integrands (it warns of roundoff); the checks carry their own tolerances
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", integrate.IntegrationWarning)
        val, err = integrate.quad(f, 0.0, 1.0, epsabs=1e-15, epsrel=1e-13, limit=400)
    return val


# ---------------------------------------------------------------- segments --

PAIRS = [(-4.0, 1.5), (2.3, -1.7), (-0.02, 0.01), (3.0, 3.0), (-100.0, 100.0), (100.0, -100.0),
         (0.0, 0.0999), (0.0, -0.1001), (0.0, 0.9999), (0.0, -1.0001), (1e-9, 0.0)]


@pytest.mark.parametrize("a,b", PAIRS)
def test_segment_mass_share_vs_quadrature(a, b):
    """test_acma.py:36-47 with adaptive quadrature instead of trapezoids."""
    L, mu = O.segment_mass_share(np.array([b - a]))
    hi = max(a, b)
    f = lambda u: math.exp(a + (b - a) * u - hi)
    mass = quad(f)
    mom = quad(lambda u: u * f(u))
    assert abs(L[0] - mass) <= 1e-13 * max(1.0, mass)
    assert abs(mu[0] - mom / mass) <= 1e-12


@pytest.mark.parametrize("delta", [-12.0, -1.01, -1.0, -0.999, -0.8, -0.2, -1e-6, 0.0,
                                   1e-6, 0.2, 0.8, 0.999, 1.0, 1.01, 12.0, 60.0, -60.0])
def test_shifted_moments_vs_quadrature(delta):
    """test_analytic_backward.py:33-39 at its deltas plus the branch edges."""
    got = O.shifted_moments(np.array([delta]))
    shift = max(delta, 0.0)
    for n in range(3):
        ref = quad(lambda u: u ** n * math.exp(delta * u - shift))
        assert abs(got[n][0] - ref) <= 1e-13 * max(ref, 1e-3), (n, got[n][0], ref)


def test_moment_limits_ordering():
    """test_analytic_backward.py:25-32: values at 0, z0>=z1>=z2>=0, finiteness."""
    x = np.array([-100., -10., -1., -.1, 0., .1, 1., 10., 100.])
    z0, z1, z2 = O.shifted_moments(x)
    assert np.all(np.isfinite(z0))
    assert np.all((z0 >= z1) & (z1 >= z2) & (z2 >= 0))
    assert z0[4] == pytest.approx(1.0, abs=1e-15)
    assert z1[4] == pytest.approx(0.5, abs=1e-15)
    assert z2[4] == pytest.approx(1 / 3, abs=1e-15)


def test_mass_share_limits_at_zero():
    """test_acma.py:97-103: L(0)=1, mu(0)=1/2, mu'(0)=1/12 (central difference)."""
    L, mu = O.segment_mass_share(np.zeros(3))
    assert np.all(L == 1.0) and np.all(mu == 0.5)
    h = 1e-5
    _, mp = O.segment_mass_share(np.array([h]))
    _, mm = O.segment_mass_share(np.array([-h]))
    assert (mp[0] - mm[0]) / (2 * h) == pytest.approx(1 / 12, abs=1e-9)


def test_mirror_identities_used_by_the_kernels():
    """DERIVED identities the HIP kernels rely on (all pinned here in float64):
    e^{-max(d,0)}(J0-J1)(d) = m1(-d); e^{-max(d,0)}(J0-2J1+J2)(d) = m2(-d);
    m1-m2 is even; and the shares are E*m1 (right) and E*(m0-m1) (left)."""
    d = np.linspace(-7, 7, 2001)
    m0, m1, m2 = O.shifted_moments(d)
    n0, n1, n2 = O.shifted_moments(-d)
    np.testing.assert_allclose(m0 - m1, n1, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(m0 - 2 * m1 + m2, n2, rtol=1e-10, atol=1e-14)
    np.testing.assert_allclose(m1 - m2, n1 - n2, rtol=1e-10, atol=1e-14)
    L, mu = O.segment_mass_share(d)
    np.testing.assert_allclose(L, m0, rtol=1e-13)
    np.testing.assert_allclose(L * mu, m1, rtol=1e-12, atol=1e-15)


# ----------------------------------------------------------------- weights --

def test_known_answer_per_query_integral():
    """test_acma.py:49-69: the exact per-query integral of the piecewise-linear
    K/V path with both half-token caps, by quadrature, on the reference's input."""
    scores = np.array([.35, -1.8, 1.0, 2.5])
    values = np.array([-.7, 1.3, 5., -2.])
    T = 4
    W = O.ca_weights(np.tile(scores, (T, 1)))[0]
    for i in range(T):
        mx = scores[:i + 1].max()
        num = .5 * math.exp(scores[0] - mx) * values[0] + .5 * math.exp(scores[i] - mx) * values[i]
        den = .5 * math.exp(scores[0] - mx) + .5 * math.exp(scores[i] - mx)
        for j in range(1, i + 1):
            f = lambda u, j=j: math.exp(scores[j - 1] * (1 - u) + scores[j] * u - mx)
            num += quad(lambda u, j=j: f(u) * (values[j - 1] * (1 - u) + values[j] * u))
            den += quad(f)
        assert (W[i] * values).sum() == pytest.approx(num / den, abs=1e-13)


def test_constant_scores_give_uniform_causal_attention():
    """test_acma.py:71-76 (also catches a dropped or doubled half-token cap)."""
    W = O.ca_weights(np.full((14, 14), 4.3))[0]
    ref = np.tril(np.ones((14, 14)))
    ref /= ref.sum(-1, keepdims=True)
    np.testing.assert_allclose(W, ref, atol=1e-14, rtol=0)


def test_single_token_is_one():
    """test_acma.py:78-80."""
    W = O.ca_weights(np.array([[123.0]]))[0]
    assert W[0, 0] == 1.0


def test_nonnegative_causal_rows_sum_to_one():
    """test_acma.py:82-89."""
    rng = np.random.default_rng(1)
    s = rng.standard_normal((4, 13, 13)) * 8
    W = O.ca_weights(s)[0]
    assert np.all(np.isfinite(W)) and W.min() >= 0
    np.testing.assert_allclose(W.sum(-1), 1.0, atol=1e-13)
    assert np.abs(W[..., ~np.tril(np.ones((13, 13), bool))]).sum() == 0.0


def test_extreme_logits_and_offset_invariance():
    """test_acma.py:91-95."""
    rng = np.random.default_rng(2)
    s = rng.standard_normal((3, 9, 9)) * 150
    W = O.ca_weights(s)[0]
    assert np.all(np.isfinite(W))
    np.testing.assert_allclose(W, O.ca_weights(s + 1000)[0], atol=1e-9)


def test_not_plain_softmax():
    """test_acma.py:133-138."""
    s = np.array([[0., 0., 0.], [0., 2., 0.], [1., -1., 3.]])
    W = O.ca_weights(s)[0]
    e = np.exp(np.where(np.tril(np.ones((3, 3), bool)), s, -np.inf))
    assert np.abs(W - e / e.sum(-1, keepdims=True)).sum() > 0.01


def test_rows_mode_matches_square_and_tile_offset():
    """Row-wise evaluation (sampled rows / query-tile offset) equals the square
    matrix rows (cuda/continuum_attention.py:622-648 offset semantics)."""
    rng = np.random.default_rng(3)
    s = rng.standard_normal((2, 40, 40)) * 2
    W = O.ca_weights(s)[0]
    rows = np.array([0, 1, 7, 31, 39])
    np.testing.assert_allclose(O.ca_weights(s[:, rows], rows)[0], W[:, rows], atol=1e-15)
    # a tile of queries 12..19 with only keys 0..19 present
    Wt = O.ca_weights(s[:, 12:20, :20], np.arange(12, 20))[0]
    np.testing.assert_allclose(Wt, W[:, 12:20, :20], atol=1e-15)


# --------------------------------------------------------------------- VJP --

def _autograd_ds(s, gw):
    st = torch.tensor(s, dtype=torch.float64, requires_grad=True)
    w = P.tile_weights(st.reshape(1, *s.shape[-2:]), 0)
    return torch.autograd.grad(w, st, torch.tensor(gw).reshape(w.shape))[0].numpy()


@pytest.mark.parametrize("T", [1, 2, 3, 7, 32, 64])
@pytest.mark.parametrize("amp", [0.0, 0.01, 1.0, 4.0, 20.0])
def test_vjp_matches_float64_autograd(T, amp):
    """test_analytic_backward.py:41-51: two independent derivations agree."""
    rng = np.random.default_rng(731 + T)
    s = rng.standard_normal((T, T)) * amp
    gw = rng.standard_normal((T, T))
    ds = O.ca_weights_vjp(s, gw)
    np.testing.assert_allclose(ds, _autograd_ds(s, gw), atol=1e-9, rtol=5e-8)


def test_vjp_long_rows_and_exact_zeros():
    """test_analytic_backward.py:53-61 and test_long.py:45-52 (T=192, 257)."""
    for T, seed in ((192, 23), (257, 257)):
        rng = np.random.default_rng(seed)
        s = rng.standard_normal((T, T))
        gw = rng.standard_normal((T, T))
        ds = O.ca_weights_vjp(s, gw)
        np.testing.assert_allclose(ds, _autograd_ds(s, gw), atol=1e-9, rtol=1e-8)
        assert np.abs(ds[0, 1:]).max() == 0.0
        assert np.abs(ds[np.triu_indices(T, 1)]).max() == 0.0


def test_vjp_invariants():
    """sum_j dS_ij = 0 (shift invariance, verify_backward_mps.py:71-73) and
    T=1 gives dS=0 (verify_backward_mps.py:84-85); equal adjacent scores
    (delta exactly 0, verify_backward_mps.py:49-51) stay finite."""
    rng = np.random.default_rng(5)
    s = rng.standard_normal((50, 50)) * 3
    s[:, 10:20] = s[:, 10:11]          # repeated scores -> delta == 0
    ds = O.ca_weights_vjp(s, rng.standard_normal((50, 50)))
    assert np.all(np.isfinite(ds))
    np.testing.assert_allclose(ds.sum(-1), 0.0, atol=1e-13)
    assert O.ca_weights_vjp(np.array([[2.0]]), np.array([[5.0]]))[0, 0] == 0.0


# ----------------------------------------------------- composed operator ----

def _fd_check(shape, seed, gains, eps=1e-6):
    rng = np.random.default_rng(seed)
    q, k, v, dy = (rng.standard_normal(shape) for _ in range(4))
    rho = np.asarray(gains, float)
    dq, dk, dv, drho = O.ca_backward(q, k, v, rho, dy)

    def loss(q_, k_, v_, r_):
        return float((O.ca_forward(q_, k_, v_, r_)[0] * dy).sum())

    for name, arr, grad in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        idx = [tuple(rng.integers(0, n) for n in shape) for _ in range(6)]
        for ix in idx:
            ap, am = arr.copy(), arr.copy()
            ap[ix] += eps; am[ix] -= eps
            args_p = dict(q=q, k=k, v=v); args_p[name] = ap
            args_m = dict(q=q, k=k, v=v); args_m[name] = am
            fd = (loss(args_p["q"], args_p["k"], args_p["v"], rho)
                  - loss(args_m["q"], args_m["k"], args_m["v"], rho)) / (2 * eps)
            assert grad[ix] == pytest.approx(fd, abs=2e-7, rel=2e-6), (name, ix)
    for h in range(len(rho)):
        rp, rm = rho.copy(), rho.copy()
        rp[h] += eps; rm[h] -= eps
        fd = (loss(q, k, v, rp) - loss(q, k, v, rm)) / (2 * eps)
        assert drho[h] == pytest.approx(fd, abs=2e-7, rel=2e-6)


def test_operator_gradients_vs_finite_differences():
    """Brute force: composed dQ/dK/dV/dRho vs central differences (fp64)."""
    _fd_check((1, 2, 9, 4), 11, [0.0, 0.3])
    _fd_check((2, 1, 6, 3), 12, [-0.4])


def test_backward_rows_decomposition():
    """The row-restricted backward used by the long-T GPU test: its dQ rows
    equal the full backward's, the row sets' dK/dV/dRho parts sum to the full
    gradients, and a suffix of rows alone gives the complete dK/dV of the
    suffix keys.  The full backward is pinned by autograd and finite
    differences above, so a wrong slice or transposition here fails."""
    rng = np.random.default_rng(21)
    shape = (2, 2, 45, 8)
    q, k, v, dy = (rng.standard_normal(shape) * 1.5 for _ in range(4))
    rho = np.array([0.2, -0.5])
    dq, dk, dv, drho = O.ca_backward(q, k, v, rho, dy)
    b, h, T = 1, 1, shape[2]
    parts = [np.arange(0, 7), np.array([7, 8, 20, 33]), np.setdiff1d(np.arange(9, T), [20, 33])]
    acc_k = np.zeros((T, 8)); acc_v = np.zeros((T, 8)); acc_r = 0.0
    for rows in parts:
        dq_r, dk_p, dv_p, dr_p = O.ca_backward_rows(q, k, v, rho, dy, b, h, rows)
        np.testing.assert_allclose(dq_r, dq[b, h, rows], atol=1e-13)
        acc_k += dk_p; acc_v += dv_p; acc_r += dr_p
    np.testing.assert_allclose(acc_k, dk[b, h], atol=1e-13)
    np.testing.assert_allclose(acc_v, dv[b, h], atol=1e-13)
    # drho sums over batches: batch 0 of head 1 adds the rest
    full0 = O.ca_backward_rows(q, k, v, rho, dy, 0, h, np.arange(T))[3]
    assert acc_r + full0 == pytest.approx(drho[h], abs=1e-12)
    suffix = np.arange(30, T)
    _, dk_s, dv_s, _ = O.ca_backward_rows(q, k, v, rho, dy, b, h, suffix)
    np.testing.assert_allclose(dk_s[30:], dk[b, h, 30:], atol=1e-13)
    np.testing.assert_allclose(dv_s[30:], dv[b, h, 30:], atol=1e-13)
    assert np.abs(dk_s[:30] - dk[b, h, :30]).max() > 1e-3  # earlier keys are incomplete


def test_reference_ca_check_case():
    """cuda/continuum_attention.py:1363-1401 (ca_check): [1,2,9,8], tile 4,
    seed 1234: the fp32 CPU port agrees with the fp64 oracle (fwd <= 2e-5,
    grads <= 3e-4), the uniform limit holds, and future values never leak."""
    torch.manual_seed(1234)
    q, k, v = (torch.randn(1, 2, 9, 8) for _ in range(3))
    rho = torch.zeros(2)
    g = torch.randn(1, 2, 9, 8)
    y = P.port_forward(q, k, v, rho, 4)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    assert np.abs(y.numpy() - yo).max() <= 2e-5
    grads = P.port_backward(q, k, v, rho, g, 4)
    ref = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), g.numpy())
    for a, b in zip(grads, ref):
        assert np.abs(a.numpy() - b).max() <= 3e-4
    v2 = v.clone(); v2[:, :, 9 // 2 + 1:] += 1000
    y2 = P.port_forward(q, k, v2, rho, 4)
    torch.testing.assert_close(y[:, :, :5], y2[:, :, :5], atol=1e-5, rtol=1e-5)


def test_config1_cpu_port_vs_oracle():
    """[1,2,64,16] fp32, seed 0, tau=1; the CPU port meets
    the north-star tolerances against the fp64 oracle."""
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 64, 16) for _ in range(3))
    dy = torch.randn(1, 2, 64, 16)
    rho = torch.zeros(2)
    y = P.port_forward(q, k, v, rho, 128)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    rel = lambda a, b: np.abs(a - b).max() / np.abs(b).max()
    assert rel(y.numpy(), yo) <= 1e-4
    for a, b in zip(P.port_backward(q, k, v, rho, dy, 128),
                    O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())):
        assert rel(a.numpy(), b) <= 1e-3


# --------------------------------------------- planted mistakes (CPU only) --

def test_planted_mistakes_are_caught(monkeypatch):
    """Sensitivity of the pins: plant plausible mistakes *in the oracle* and
    check the pins above would fail."""
    s = np.full((6, 6), 1.7)
    # (1) dropping the final half-token cap breaks the uniform limit
    real = O.ca_weights

    def no_end_cap(scores, qidx=None):
        W, m, Z = real(scores, qidx)
        n = W.shape[-1]
        W2 = W.copy()
        W2[np.arange(n), np.arange(n)] -= 0.5 / (np.arange(n) + 1)
        return W2, m, Z
    ref = np.tril(np.ones((6, 6))); ref /= ref.sum(-1, keepdims=True)
    assert np.abs(no_end_cap(s)[0] - ref).max() > 1e-3
    # (2) swapping left/right shares fails the known-answer quadrature
    L, mu = O.segment_mass_share(np.array([2.5 - 1.0]))
    f = lambda u: math.exp(1.0 + 1.5 * u - 2.5)
    assert abs((1 - mu[0]) - quad(lambda u: u * f(u)) / quad(f)) > 1e-2
    # (3) a sign error in the odd moment fails quadrature
    z = O.shifted_moments(np.array([-0.5]))
    wrong = O.shifted_moments(np.array([0.5]))[1][0]
    assert abs(wrong - quad(lambda u: u * math.exp(-0.5 * u))) > 1e-2
    assert abs(z[1][0] - quad(lambda u: u * math.exp(-0.5 * u))) < 1e-13

"""The operator and the weight-level API on CPU tensors (continuum-attention_amd/cpu.py).

The reference runs these on CPU (cuda/continuum_attention.py:658, 688,
737-751; architecture.py:32-105), and its own CPU tests exercise them:
test_acma.py:36-138 (segment coefficients, known-answer quadrature, limits,
causality), ca_check (cuda/continuum_attention.py:1363-1401).  Here the same
checks run against this package's ``architecture`` module and operator, with
the float64 oracle (oracle/ca_oracle.py) as the reference where the
reference compares against its own torch weights.
"""
import math

import numpy as np
import pytest
import torch

from oracle import ca_oracle as O


@pytest.fixture(scope="module")
def A(ca):
    return ca.architecture


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


@pytest.mark.parametrize("a,b", [(-4., 1.5), (2.3, -1.7), (-.02, .01), (3., 3.), (-100., 100.),
                                 (100., -100.), (0.4, -0.55), (-0.999, 0.0)])
def test_segment_coefficients_vs_quadrature(A, a, b):
    """test_acma.py:36-47: L and mu against trapezoid quadrature of the
    segment integral (40001 points), float64, 3e-8."""
    delta = torch.tensor([b - a], dtype=torch.float64)
    L, mu = A.segment_integral_coefficients(delta)
    u = torch.linspace(0, 1, 40001, dtype=torch.float64)
    f = torch.exp(a + u * (b - a) - max(a, b))
    mass = torch.trapezoid(f, u)
    assert abs(L.item() - mass.item()) <= 3e-8
    assert abs(mu.item() - (torch.trapezoid(f * u, u) / mass).item()) <= 3e-8


def test_segment_coefficients_at_zero_and_slope(A):
    """test_acma.py:104-111: L(0) = 1, mu(0) = 1/2, mu'(0) = 1/12 by autograd."""
    d = torch.zeros(3, dtype=torch.float64, requires_grad=True)
    L, mu = A.segment_integral_coefficients(d)
    torch.testing.assert_close(L, torch.ones_like(L))
    torch.testing.assert_close(mu, torch.full_like(mu, 0.5))
    g = torch.autograd.grad(mu.sum(), d)[0]
    torch.testing.assert_close(g, torch.full_like(g, 1 / 12), atol=1e-12, rtol=1e-12)


def test_segment_coefficients_match_oracle_across_branches(A):
    d = torch.tensor(np.concatenate([np.linspace(-3, 3, 601), [-1e-9, 1e-9, 0.9999, 1.0, -1.0001,
                                                                 40.0, -700.0]]))
    L, mu = A.segment_integral_coefficients(d)
    Lo, muo = O.segment_mass_share(d.numpy())
    assert np.abs(L.numpy() - Lo).max() <= 1e-14
    assert np.abs(mu.numpy() - muo).max() <= 1e-14


def test_known_answer_per_query_quadrature(A):
    """test_acma.py:49-69: scores [.35, -1.8, 1.0, 2.5], per-query brute
    quadrature of the piecewise-linear path with both half-token caps."""
    s = torch.tensor([.35, -1.8, 1.0, 2.5], dtype=torch.float64)
    vals = torch.tensor([-.7, 1.3, 5., -2.], dtype=torch.float64)
    T = 4
    W = A.continuous_attention_weights(s.view(1, 1, 1, T).expand(1, 1, T, T).clone())[0, 0]
    u = torch.linspace(0, 1, 20001, dtype=torch.float64)
    for i in range(T):
        m = s[:i + 1].max()
        num = 0.5 * torch.exp(s[0] - m) * vals[0] + 0.5 * torch.exp(s[i] - m) * vals[i]
        den = 0.5 * torch.exp(s[0] - m) + 0.5 * torch.exp(s[i] - m)
        for j in range(1, i + 1):
            f = torch.exp(s[j - 1] * (1 - u) + s[j] * u - m)
            num = num + torch.trapezoid(f * (vals[j - 1] * (1 - u) + vals[j] * u), u)
            den = den + torch.trapezoid(f, u)
        assert abs((W[i] * vals).sum().item() - (num / den).item()) <= 5e-8


def test_weight_limits_and_properties(A):
    """test_acma.py:71-103,133-138: constant scores give uniform causal
    attention, one token gives 1, rows are non-negative, causal and sum to
    one, extreme logits stay finite and offset invariant, and the result is
    not the softmax."""
    z = torch.full((2, 3, 14, 14), 4.3, dtype=torch.float64)
    causal = torch.ones(14, 14, dtype=torch.bool).tril()
    torch.testing.assert_close(A.continuous_attention_weights(z),
                               torch.softmax(z.masked_fill(~causal, -torch.inf), -1),
                               atol=1e-14, rtol=1e-14)
    assert A.continuous_attention_weights(torch.tensor([[[[123.]]]])).item() == 1.0
    torch.manual_seed(1729)
    w = A.continuous_attention_weights(torch.randn(2, 4, 13, 13) * 8)
    assert torch.isfinite(w).all() and w.min().item() >= 0
    torch.testing.assert_close(w.sum(-1), torch.ones(2, 4, 13), atol=1e-6, rtol=1e-6)
    assert w.masked_select(~torch.ones(13, 13, dtype=torch.bool).tril()).abs().sum().item() == 0.0
    lg = torch.randn(1, 3, 9, 9) * 150
    w = A.continuous_attention_weights(lg)
    assert torch.isfinite(w).all()
    torch.testing.assert_close(w, A.continuous_attention_weights(lg + 1000), atol=1e-4, rtol=1e-4)
    lg = torch.tensor([[[[0., 0., 0.], [0., 2., 0.], [1., -1., 3.]]]])
    sm = torch.softmax(lg.masked_fill(~torch.ones(3, 3, dtype=torch.bool).tril(), -torch.inf), -1)
    assert (A.continuous_attention_weights(lg) - sm).abs().sum().item() > 0.01


@pytest.mark.parametrize("T,amp", [(1, 1.0), (2, 1.0), (7, 4.0), (32, 0.01), (64, 20.0), (97, 1.0)])
def test_weights_and_vjp_vs_oracle(A, ca, T, amp):
    """W and its autograd VJP (float64) against the oracle's weights and
    analytic VJP; the package's analytic VJP (cpu.tile_weights_vjp, the
    operator's backward) against the same."""
    g = torch.Generator().manual_seed(T)
    s = torch.randn(3, T, T, generator=g, dtype=torch.float64) * amp
    gw = torch.randn(3, T, T, generator=g, dtype=torch.float64)
    sr = s.clone().requires_grad_(True)
    W = A.continuous_attention_weights(sr)
    ds = torch.autograd.grad((W * gw).sum(), sr)[0]
    Wo = O.ca_weights(s.numpy())[0]
    dso = O.ca_weights_vjp(s.numpy(), gw.numpy())
    assert np.abs(W.detach().numpy() - Wo).max() <= 1e-13
    assert np.abs(ds.numpy() - dso).max() <= 1e-11 * max(1.0, np.abs(dso).max())
    import importlib
    cpu = importlib.import_module("continuum-attention_amd.cpu")
    W2, ds2 = cpu.tile_weights_vjp(s, gw, 0)
    assert np.abs(W2.numpy() - Wo).max() <= 1e-13
    assert np.abs(ds2.numpy() - dso).max() <= 1e-11 * max(1.0, np.abs(dso).max())


def test_weights_twice_differentiable_on_cpu(A):
    """The reference's weights are plain torch, so second derivatives work
    (gradgradcheck in float64)."""
    torch.manual_seed(3)
    s = (torch.randn(1, 1, 5, 5, dtype=torch.float64) * 2).requires_grad_(True)
    assert torch.autograd.gradgradcheck(A.continuous_attention_weights, (s,), atol=1e-6)


def run_cpu(ca, q, k, v, rho, dy, tile=64):
    qd, kd, vd, rd = (x.clone().requires_grad_(True) for x in (q, k, v, rho))
    y = ca.continuum_attention(qd, kd, vd, rd, tile)
    return y.detach(), torch.autograd.grad((y * dy).sum(), (qd, kd, vd, rd))


def test_config1_on_cpu(ca):
    """BASELINE config 1 ([1,2,64,16], torch.manual_seed(0) order q, k, v, dY;
    tau = 1) through continuum_attention on CPU tensors, against the float64
    oracle at the north-star bars (1e-4 outputs, 1e-3 gradients)."""
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 64, 16) for _ in range(3))
    dy = torch.randn(1, 2, 64, 16)
    rho = torch.zeros(2)
    y, g = run_cpu(ca, q, k, v, rho, dy)
    assert y.dtype == torch.float32 and all(t.dtype == torch.float32 for t in g)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    assert rel(y, yo) <= 1e-6
    for a, b in zip(g, go):
        assert rel(a, b) <= 1e-5


def test_reference_ca_check_on_cpu(ca):
    """ca_check (cuda/continuum_attention.py:1363-1401) on CPU: [1,2,9,8],
    seed 1234, query tile 4; forward within 2e-5 and gradients (with the
    trainable gain) within 3e-4 of the exact composition; equal scores give
    uniform causal weights; changing future values leaves earlier outputs."""
    torch.manual_seed(1234)
    q, k, v = (torch.randn(1, 2, 9, 8) for _ in range(3))
    gain = torch.zeros(2)
    g = torch.randn(1, 2, 9, 8)
    y, grads = run_cpu(ca, q, k, v, gain, g, tile=4)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), gain.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), gain.numpy(), g.numpy())
    assert np.abs(y.numpy() - yo).max() <= 2e-5
    for a, b in zip(grads, go):
        assert np.abs(a.numpy() - b).max() <= 3e-4
    v2 = v.clone()
    v2[:, :, 9 // 2 + 1:] += 1000
    z = ca.continuum_attention(q, k, v2, gain, 4)
    torch.testing.assert_close(y[:, :, :5], z[:, :, :5], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("shape,tile,gains,mag", [((2, 3, 150, 24), 64, [0.0, 0.4, -0.7], 1.0),
                                                  ((1, 2, 77, 64), 128, [0.2, 0.0], 3.0),
                                                  ((1, 1, 200, 8), 7, [0.0], 0.01)])
def test_operator_on_cpu_vs_oracle(ca, shape, tile, gains, mag):
    """Any head dim, ragged tiles, gains, small and large score spreads."""
    g = torch.Generator().manual_seed(sum(shape))
    q, k = (torch.randn(shape, generator=g) * mag for _ in range(2))
    v, dy = (torch.randn(shape, generator=g) for _ in range(2))
    rho = torch.tensor(gains)
    y, grads = run_cpu(ca, q, k, v, rho, dy, tile)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    assert rel(y, yo) <= 1e-5
    for a, b in zip(grads, go):
        assert rel(a, b) <= 1e-4


def test_operator_on_cpu_dtypes_and_first_order(ca):
    """Output in v.dtype, gradients in the input dtypes; a second-order
    backward raises as the reference's does (:698-699)."""
    q = torch.randn(1, 2, 20, 16, dtype=torch.float64, requires_grad=True)
    y = ca.continuum_attention(q, q.detach(), q.detach(), torch.zeros(2, dtype=torch.float64))
    assert y.dtype == torch.float64
    gq, = torch.autograd.grad(y.sum(), q)
    assert gq.dtype == torch.float64
    q2 = torch.randn(1, 2, 20, 16, requires_grad=True)
    y2 = ca.continuum_attention(q2, q2, q2, torch.zeros(2))
    with pytest.raises(RuntimeError, match="first-order"):
        torch.autograd.grad(y2.sum(), q2, create_graph=True)

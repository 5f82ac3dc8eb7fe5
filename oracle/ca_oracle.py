"""Float64 CPU oracle for the Continuum Attention (CA) operator.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product path (the HIP kernels behind ``continuum_attention``)
never calls into it.

What it restates (akhadangi/continuum-attention, read as text, never run):

* per-segment mass/share coefficients ``(L, mu)``      -- architecture.py:32-62
* exact causal CA weights with half-token caps        -- architecture.py:65-105,
  with the query-tile offset of cuda/continuum_attention.py:622-648
* shifted exponential moments ``m0, m1, m2``           -- analytic_reference.py:12-49
* analytic first-order VJP dL/dS from dL/dW            -- analytic_reference.py:52-75
* operator composition (scale, W@V, dQ/dK/dV/dRho)    -- cuda/continuum_attention.py:650-766

Every array here is float64.  Rows are addressed by an explicit query index so
that the same code checks a full ``[T, T]`` problem or a few sampled rows of a
T=8192 problem (row ``i`` of W and dS depends only on row ``i`` of S).

Pinning (tests/test_oracle.py; the kernels' scalar forms in
tests/test_device_math.py): trapezoid quadrature of the segment
integrals and of the full per-query integral (the known-answer input of
test_acma.py:49-69), the uniform/softmax limit, single-token W=1, offset
invariance, row sums, exact future zeros, float64 autograd through an
independent torch restatement of the weights, central finite differences of
the composed operator, sum_j dS_ij = 0, and dRho = sum dS*s.
"""
from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------------------
# Segment coefficients.  A segment joins endpoint scores a (left key) and
# b (right key); delta = b - a.  Along u in [0,1] the score is a + delta*u.
# ---------------------------------------------------------------------------

_TAYLOR_DEG = 16


def segment_mass_share(delta):
    """Return ``(L, mu)`` for segment deltas (architecture.py:32-62).

    ``exp(max(a,b)) * L`` is the segment mass, ``L(t) = (1 - e^-t)/t`` with
    ``t = |delta|`` (``L(0)=1``); ``mu = J1/J0`` is the share of the right
    endpoint (``mu(0)=1/2``).  The reference switches to short series below
    ``|delta| < 0.1``; in float64 we use a degree-16 series below ``t < 1``
    (same closed forms above), which is more accurate than either branch.
    """
    d = np.asarray(delta, dtype=np.float64)
    t = np.abs(d)
    small = t < 1.0
    ts = np.where(small, t, 0.0)
    # L(t) = sum_k (-t)^k / (k+1)!
    L_small = np.zeros_like(ts)
    for k in range(_TAYLOR_DEG, -1, -1):
        L_small = L_small * (-ts) + 1.0 / math.factorial(k + 1)
    tl = np.where(small, 1.0, t)
    em1 = np.expm1(-tl)
    L_large = -em1 / tl
    L = np.where(small, L_small, L_large)
    # share of the high endpoint: mu_hi(t) = B(t)/L(t), B(t) = sum (-t)^k/(k+2)!
    B_small = np.zeros_like(ts)
    for k in range(_TAYLOR_DEG, -1, -1):
        B_small = B_small * (-ts) + 1.0 / math.factorial(k + 2)
    mu_hi_large = 1.0 / (-em1) - 1.0 / tl
    mu_hi = np.where(small, B_small / L_small, mu_hi_large)
    mu = np.where(d >= 0, mu_hi, 1.0 - mu_hi)
    return L, mu


def shifted_moments(delta):
    """``m_n(delta) = exp(-max(delta,0)) * int_0^1 u^n exp(delta*u) du``, n=0,1,2.

    Restates analytic_reference.py:12-49: closed forms for ``|delta| >= 1`` and
    degree-16 series below (series of the *shifted* integrals, separately for
    the two signs, so nothing cancels).
    """
    d = np.asarray(delta, dtype=np.float64)
    t = np.abs(d)
    small = t < 1.0
    ts = np.where(small, t, 0.0)

    def series(coef):
        out = np.full_like(ts, coef(_TAYLOR_DEG))
        for k in range(_TAYLOR_DEG - 1, -1, -1):
            out = out * ts + coef(k)
        return out

    f = math.factorial
    # delta <= 0: int u^n e^{-t u} du = sum_k (-t)^k / (k! (k+n+1))
    neg = [series(lambda k, n=n: (-1) ** k / (f(k) * (k + n + 1))) for n in range(3)]
    # delta >= 0: substitute w = 1-u: int (1-w)^n e^{-t w} dw
    p0 = neg[0]
    p1 = series(lambda k: (-1) ** k / f(k + 2))
    p2 = series(lambda k: (-1) ** k * 2.0 / f(k + 3))
    tl = np.where(small, 1.0, t)
    e = np.exp(-tl)
    m0_l = -np.expm1(-tl) / tl
    m1_pos = (tl - 1.0 + e) / tl ** 2
    m2_pos = (tl ** 2 - 2.0 * tl + 2.0 - 2.0 * e) / tl ** 3
    m1_neg = (1.0 - (tl + 1.0) * e) / tl ** 2
    m2_neg = (2.0 - (tl ** 2 + 2.0 * tl + 2.0) * e) / tl ** 3
    pos = d >= 0
    m0 = np.where(small, p0, m0_l)
    m1 = np.where(small, np.where(pos, p1, neg[1]), np.where(pos, m1_pos, m1_neg))
    m2 = np.where(small, np.where(pos, p2, neg[2]), np.where(pos, m2_pos, m2_neg))
    return m0, m1, m2


# ---------------------------------------------------------------------------
# Weights and VJP for score rows.  ``scores[..., r, :]`` is the (unmasked)
# score row of query ``qidx[r]``; keys j > qidx[r] are invisible.
# ---------------------------------------------------------------------------

def _row_setup(scores, qidx):
    s = np.asarray(scores, dtype=np.float64)
    T = s.shape[-1]
    qi = np.asarray(qidx).reshape(-1, 1)
    keys = np.arange(T).reshape(1, T)
    vis = keys <= qi                                  # [R, T]
    seg_vis = keys[:, 1:] <= qi                       # segment (j-1, j) visible iff j <= i
    m = np.max(np.where(vis, s, -np.inf), axis=-1, keepdims=True)
    a = np.where(seg_vis, s[..., :-1], m)            # mask before differencing
    b = np.where(seg_vis, s[..., 1:], m)
    return s, T, qi, keys, vis, seg_vis, m, a, b


def ca_weights(scores, qidx=None):
    """Exact CA weights W for score rows (architecture.py:65-105,
    cuda/continuum_attention.py:622-648).

    ``w_ij = [j=0] 1/2 e^{s_i0-m} + [j=i] 1/2 e^{s_ii-m}
            + [1<=j<=i] mass(j-1,j) mu + [j<i] mass(j,j+1) (1-mu)``,
    normalised per row.  Invisible entries are exactly 0.
    """
    s = np.asarray(scores, dtype=np.float64)
    if qidx is None:
        qidx = np.arange(s.shape[-2])
    s, T, qi, keys, vis, seg_vis, m, a, b = _row_setup(s, qidx)
    L, mu = segment_mass_share(b - a)
    mass = np.exp(np.maximum(a, b) - m) * L * seg_vis
    w = np.zeros_like(s)
    w[..., :-1] += mass * (1.0 - mu)                 # left endpoint share
    w[..., 1:] += mass * mu                          # right endpoint share
    w[..., 0] += 0.5 * np.exp(s[..., 0] - m[..., 0])  # first half-token cap
    diag = np.take_along_axis(s, np.broadcast_to(qi, s.shape[:-1] + (1,)), axis=-1)
    w += (keys == qi) * 0.5 * np.exp(diag - m)       # last half-token cap
    w = np.where(vis, w, 0.0)
    return w / w.sum(axis=-1, keepdims=True), m[..., 0], w.sum(axis=-1)


def ca_weights_vjp(scores, grad_w, weights=None, qidx=None):
    """dL/dS from dL/dW (analytic_reference.py:52-75), float64.

    With ``g = gw - sum_j W gw`` and ``E = e^{max(a,b)-m}``:
      left key  += E (g_l (m0 - 2 m1 + m2) + g_r (m1 - m2))
      right key += E (g_l (m1 - m2) + g_r m2)
      caps      += (1/2) e^{s-m} g
    all divided by Z; invisible entries are exactly 0.
    """
    s = np.asarray(scores, dtype=np.float64)
    gw = np.asarray(grad_w, dtype=np.float64)
    if qidx is None:
        qidx = np.arange(s.shape[-2])
    if weights is None:
        weights = ca_weights(s, qidx)[0]
    s, T, qi, keys, vis, seg_vis, m, a, b = _row_setup(s, qidx)
    z0, z1, z2 = shifted_moments(b - a)
    E = np.exp(np.maximum(a, b) - m) * seg_vis
    cap = np.zeros_like(s)
    cap[..., 0] += 0.5 * np.exp(s[..., 0] - m[..., 0])
    diag = np.take_along_axis(s, np.broadcast_to(qi, s.shape[:-1] + (1,)), axis=-1)
    cap += (keys == qi) * 0.5 * np.exp(diag - m)
    cap = np.where(vis, cap, 0.0)
    Z = (E * z0).sum(axis=-1, keepdims=True) + cap.sum(axis=-1, keepdims=True)
    g = gw - (gw * weights).sum(axis=-1, keepdims=True)
    left = E * (g[..., :-1] * (z0 - 2.0 * z1 + z2) + g[..., 1:] * (z1 - z2))
    right = E * (g[..., :-1] * (z1 - z2) + g[..., 1:] * z2)
    ds = cap * g
    ds[..., :-1] += left
    ds[..., 1:] += right
    return np.where(vis, ds / Z, 0.0)


# ---------------------------------------------------------------------------
# Operator composition (cuda/continuum_attention.py:650-766).
# ---------------------------------------------------------------------------

def head_scale(log_gain, D):
    """Per-head score scale ``exp(rho_h) / sqrt(D)`` (cuda/continuum_attention.py:656-657)."""
    return np.exp(np.asarray(log_gain, dtype=np.float64)) / math.sqrt(D)


def ca_forward(q, k, v, log_gain, row_chunk=1024):
    """y = W(S) V with S = c_h q k^T; returns (y, m, Z) float64.

    ``m`` and ``Z`` are the natural-log row shift and the row normaliser.
    """
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64); v = np.asarray(v, np.float64)
    B, H, T, D = q.shape
    c = head_scale(log_gain, D)
    y = np.zeros_like(v)
    m = np.zeros((B, H, T)); Z = np.zeros((B, H, T))
    for b in range(B):
        for h in range(H):
            for r0 in range(0, T, row_chunk):
                r1 = min(T, r0 + row_chunk)
                s = (q[b, h, r0:r1] @ k[b, h, :r1].T) * c[h]
                W, mm, zz = ca_weights(s, np.arange(r0, r1))
                y[b, h, r0:r1] = W @ v[b, h, :r1]
                m[b, h, r0:r1] = mm; Z[b, h, r0:r1] = zz
    return y, m, Z


def ca_backward(q, k, v, log_gain, dy, row_chunk=1024):
    """Analytic first-order gradients (dq, dk, dv, drho) in float64.

    dV = W^T dY, dQ = c dS K, dK = c dS^T Q, dRho_h = sum_{b,i,j} dS_ij s_ij
    (cuda/continuum_attention.py:754-764).
    """
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64); dy = np.asarray(dy, np.float64)
    B, H, T, D = q.shape
    c = head_scale(log_gain, D)
    dq = np.zeros_like(q); dk = np.zeros_like(k); dv = np.zeros_like(v)
    drho = np.zeros(H)
    for b in range(B):
        for h in range(H):
            for r0 in range(0, T, row_chunk):
                r1 = min(T, r0 + row_chunk)
                qidx = np.arange(r0, r1)
                s = (q[b, h, r0:r1] @ k[b, h, :r1].T) * c[h]
                W = ca_weights(s, qidx)[0]
                gw = dy[b, h, r0:r1] @ v[b, h, :r1].T
                ds = ca_weights_vjp(s, gw, W, qidx)
                dv[b, h, :r1] += W.T @ dy[b, h, r0:r1]
                dq[b, h, r0:r1] += c[h] * (ds @ k[b, h, :r1])
                dk[b, h, :r1] += c[h] * (ds.T @ q[b, h, r0:r1])
                drho[h] += float((ds * s).sum())
    return dq, dk, dv, drho


def ca_forward_rows(q, k, v, log_gain, b, h, rows):
    """Forward output for selected query rows of one (b, h) slice (long-T checks)."""
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64); v = np.asarray(v, np.float64)
    D = q.shape[-1]
    c = head_scale(log_gain, D)[h]
    rows = np.asarray(rows)
    T = int(rows.max()) + 1
    s = (q[b, h, rows] @ k[b, h, :T].T) * c
    W = ca_weights(s, rows)[0]
    return W @ v[b, h, :T]


def ca_backward_rows(q, k, v, log_gain, dy, b, h, rows):
    """Backward restricted to selected query rows of one (b, h) slice.

    Returns ``(dq_rows, dk_part, dv_part, drho_part)``: ``dq_rows`` are the
    complete dQ of those rows (row i of dS depends only on row i of S), and
    ``dk_part``/``dv_part`` (``[T, D]``) and ``drho_part`` are the rows'
    contributions to dK, dV and dRho (cuda/continuum_attention.py:754-764).
    For the suffix ``rows = [T-n, T)`` the parts are the complete dK and dV
    of keys ``j >= T-n`` (only queries ``i >= j`` see key j), which lets a
    long-T test check exact gradients without the ``[T, T]`` problem.
    """
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64); dy = np.asarray(dy, np.float64)
    T, D = q.shape[-2:]
    c = head_scale(log_gain, D)[h]
    rows = np.asarray(rows)
    n = int(rows.max()) + 1
    s = (q[b, h, rows] @ k[b, h, :n].T) * c
    W = ca_weights(s, rows)[0]
    gw = dy[b, h, rows] @ v[b, h, :n].T
    ds = ca_weights_vjp(s, gw, W, rows)
    dk = np.zeros((T, D)); dv = np.zeros((T, D))
    dv[:n] = W.T @ dy[b, h, rows]
    dk[:n] = c * (ds.T @ q[b, h, rows])
    return c * (ds @ k[b, h, :n]), dk, dv, float((ds * s).sum())

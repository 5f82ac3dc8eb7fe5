"""The operator and the weight-level API on CPU tensors.

The reference runs ``_CAExactTiled`` on CPU tensors: with no CUDA extension
(``ext=None``, cuda/continuum_attention.py:658, 704) the forward computes each
query tile's exact weights in torch (``_ca_reference_weights``, :622-648) and
the backward replays them under autograd (:737-751); ``architecture.py:65-105``
(``continuous_attention_weights``) is plain torch too.  ``ca_check``
(cuda/continuum_attention.py:1363-1401) and the reference's CPU model tests run
these paths.  This module is what CPU tensors dispatch to here, so those
callers keep working; GPU tensors never come here (they run the HIP kernels,
and fail loudly when the library is missing).

Own formulation (not the reference's (L, mu) form): a segment between
adjacent keys with endpoint scores a (left) and b (right), x = b - a, and
endpoint weights p_a = e^(a-m), p_b = e^(b-m) relative to the row max m has
moments M_n = p_a J_n(x), J_n(x) = int_0^1 u^n e^(x u) du.  Its right share
is M1, its left share M0 - M1, and its score derivatives are
    d(left)/da = M0 - 2 M1 + M2,  d(left)/db = d(right)/da = M1 - M2,
    d(right)/db = M2.
For |x| >= 1 the moments follow from M0 = (p_b - p_a)/x and the recurrence
M_{n+1} = (p_b - (n+1) M_n)/x; below 1 each combination is a power series in
x with positive coefficients (no cancellation), summed to 20 terms.  The
half-token caps add 0.5 p at key 0 and at the query's own key.

The operator computes in float32 as the reference's does (its scores are
``raw.float()``, :674-676), returns ``v.dtype`` and gradients in the input
dtypes, and keeps the reference's query-tile loop, so ``query_tile`` bounds
the memory of the materialised ``[B*H, tile, K]`` blocks as it does there.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

_SERIES_BELOW = 1.0
_TERMS = 20


def _coefs(fn):
    return [fn(k) for k in range(_TERMS)]


_f = math.factorial
# Series coefficients (in powers of x) of each moment combination divided by p_a.
_C_LEFT = _coefs(lambda k: 1.0 / (_f(k) * (k + 1) * (k + 2)))       # J0 - J1
_C_RIGHT = _coefs(lambda k: 1.0 / (_f(k) * (k + 2)))                # J1
_C_DAA = _coefs(lambda k: 2.0 / (_f(k) * (k + 1) * (k + 2) * (k + 3)))  # J0 - 2 J1 + J2
_C_DAB = _coefs(lambda k: 1.0 / (_f(k) * (k + 2) * (k + 3)))        # J1 - J2
_C_DBB = _coefs(lambda k: 1.0 / (_f(k) * (k + 3)))                  # J2
_C_J0 = _coefs(lambda k: 1.0 / _f(k + 1))                           # J0


def _series(x, coefs):
    out = torch.full_like(x, coefs[-1])
    for c in reversed(coefs[:-1]):
        out = out * x + c
    return out


def segment_shares(pa, pb, x, grads=False):
    """Left/right shares of segments (and, with ``grads``, the three score
    derivatives d(left)/da, d(left)/db = d(right)/da, d(right)/db)."""
    small = x.abs() < _SERIES_BELOW
    xs = torch.where(small, x, torch.zeros_like(x))      # series argument, bounded
    xc = torch.where(small, torch.ones_like(x), x)       # closed-form argument, nonzero
    m0 = (pb - pa) / xc
    m1 = (pb - m0) / xc
    left = torch.where(small, pa * _series(xs, _C_LEFT), m0 - m1)
    right = torch.where(small, pa * _series(xs, _C_RIGHT), m1)
    if not grads:
        return left, right
    m2 = (pb - 2.0 * m1) / xc
    daa = torch.where(small, pa * _series(xs, _C_DAA), m0 - 2.0 * m1 + m2)
    dab = torch.where(small, pa * _series(xs, _C_DAB), m1 - m2)
    dbb = torch.where(small, pa * _series(xs, _C_DBB), m2)
    return left, right, daa, dab, dbb


def _tile_parts(scores, start, grads=False):
    """Unnormalised weights w, their row sums Z and (with ``grads``) the
    segment derivatives of a score tile ``[N, Q, K]`` whose first query is
    ``start`` (query start+r sees keys 0..start+r)."""
    N, Q, K = scores.shape
    dev = scores.device
    qi = torch.arange(start, start + Q, device=dev).view(1, Q, 1)
    kj = torch.arange(K, device=dev).view(1, 1, K)
    vis = kj <= qi
    m = scores.masked_fill(~vis, float("-inf")).amax(-1, keepdim=True)
    sv = torch.where(vis, scores, m)             # invisible scores never reach exp
    p = torch.exp(sv - m) * vis
    seg = vis[..., 1:]                           # segment (j-1, j) needs key j visible
    x = (sv[..., 1:] - sv[..., :-1]) * seg
    parts = segment_shares(p[..., :-1], p[..., 1:], x, grads)
    left, right = parts[0] * seg, parts[1] * seg
    cap = 0.5 * p * ((kj == 0).to(p.dtype) + (kj == qi).to(p.dtype))
    w = F.pad(left, (0, 1)) + F.pad(right, (1, 0)) + cap
    z = w.sum(-1, keepdim=True)
    return w, z, p, cap, seg, parts[2:] if grads else None


def tile_weights(scores, start=0):
    """Exact weights of a query tile (the role of ``_ca_reference_weights``,
    cuda/continuum_attention.py:622-648); differentiable by autograd."""
    w, z, *_ = _tile_parts(scores, start)
    return w / z


def tile_weights_vjp(scores, grad_w, start=0):
    """``(W, dS)``: the weights and the analytic score VJP given dL/dW."""
    w, z, p, cap, seg, (daa, dab, dbb) = _tile_parts(scores, start, grads=True)
    W = w / z
    g = (grad_w - (W * grad_w).sum(-1, keepdim=True)) / z   # dL/dw
    gl, gr = g[..., :-1], g[..., 1:]
    ds = cap * g
    ds = ds + F.pad((gl * daa + gr * dab) * seg, (0, 1))    # left endpoint of each segment
    ds = ds + F.pad((gl * dab + gr * dbb) * seg, (1, 0))    # right endpoint
    return W, ds


def continuous_attention_weights(logits):
    """``architecture.py:65-105`` on CPU tensors: ``[..., T, T]`` logits ->
    causal row-stochastic W, in the logits' dtype, differentiable (any order)
    by autograd like the reference's torch composition."""
    T = logits.size(-1)
    if logits.size(-2) != T:
        raise ValueError("This benchmark requires square full-sequence causal attention")
    lead = logits.shape[:-2]
    W = tile_weights(logits.reshape(-1, T, T), 0)
    return W.reshape(*lead, T, T)


# ---- the operator ----------------------------------------------------------

def _scale(log_gain, H, D):
    return (log_gain.detach().float().exp() * D ** -0.5).view(1, H, 1, 1)


def _tile_scores(qb, kb, scale4, B, H, start, end):
    """float32 scaled scores of queries start..end-1 against keys 0..end-1: [BH, n, end]."""
    raw = torch.bmm(qb[:, start:end].float(), kb[:, :end].float().transpose(1, 2))
    n = end - start
    return (raw.reshape(B, H, n, end) * scale4).reshape(B * H, n, end)


@torch.no_grad()
def forward(q, k, v, log_gain, query_tile):
    """Forward of the operator on CPU tensors (float32 weights, output in v.dtype)."""
    B, H, T, D = q.shape
    scale4 = _scale(log_gain, H, D)
    qb, kb, vb = (x.reshape(B * H, T, D) for x in (q, k, v))
    out = torch.empty((B * H, T, D), dtype=v.dtype)
    for start in range(0, T, query_tile):
        end = min(T, start + query_tile)
        s = _tile_scores(qb, kb, scale4, B, H, start, end)
        out[:, start:end] = torch.bmm(tile_weights(s, start).to(v.dtype), vb[:, :end])
    return out.reshape(B, H, T, D)


@torch.no_grad()
def backward(q, k, v, log_gain, grad_y, query_tile):
    """``(dq, dk, dv, dlog_gain)`` in float32: per query tile, W and the
    analytic score VJP, then the dV / dQ / dK contractions and
    dlog_gain = sum dS * S (S is linear in exp(log_gain))."""
    B, H, T, D = q.shape
    scale4 = _scale(log_gain, H, D)
    qb, kb, vb = (x.reshape(B * H, T, D).float() for x in (q, k, v))
    gb = grad_y.reshape(B * H, T, D).float()
    dq = torch.zeros((B * H, T, D))
    dk = torch.zeros_like(dq)
    dv = torch.zeros_like(dq)
    dg = torch.zeros(H)
    for start in range(0, T, query_tile):
        end = min(T, start + query_tile)
        n = end - start
        s = _tile_scores(qb, kb, scale4, B, H, start, end)
        gys = gb[:, start:end]
        gw = torch.bmm(gys, vb[:, :end].transpose(1, 2))
        W, ds = tile_weights_vjp(s, gw, start)
        dv[:, :end] += torch.bmm(W.transpose(1, 2), gys)
        dsc = (ds.reshape(B, H, n, end) * scale4).reshape(B * H, n, end)
        dq[:, start:end] = torch.bmm(dsc, kb[:, :end])
        dk[:, :end] += torch.bmm(dsc.transpose(1, 2), qb[:, start:end])
        dg += (ds * s).reshape(B, H, n, end).sum(dim=(0, 2, 3))
    shp = (B, H, T, D)
    return dq.reshape(shp), dk.reshape(shp), dv.reshape(shp), dg

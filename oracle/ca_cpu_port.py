"""CPU port of the reference operator's PyTorch CPU path (fp32).

TEST / BASELINE INFRASTRUCTURE ONLY: imported by ``tests/`` and by the
``cpu_baseline`` leg of ``bench.py``.  The product path never calls it.

It restates, in this project's own code, what ``_CAExactTiled`` does when the
CUDA extension is absent (cuda/continuum_attention.py:650-766, ``ext=None``,
``CA_CUDA_MODE=prefix``):

* forward: loop over query tiles; per tile ``S = c_h Q_tile K_prefix^T``,
  exact weights ``tile_weights(S, start)`` (cuda/continuum_attention.py:622-648),
  then ``W @ V_prefix``;
* backward: recompute S and W per tile, ``gw = dY V^T``, dS by autograd
  through ``tile_weights`` (cuda/continuum_attention.py:737-751), then
  ``dV += W^T dY``, ``dQ += c dS K``, ``dK += c dS^T Q``,
  ``dRho += sum dS * S`` (cuda/continuum_attention.py:758-764).

This is the timed CPU baseline (``cpu_baseline.kind = "port"``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def tile_weights(scores: torch.Tensor, start: int) -> torch.Tensor:
    """Exact CA weights for a query tile whose first query is ``start``.

    ``scores`` is ``[N, Q, K]`` (unmasked); query ``start+r`` sees keys
    ``j <= start+r``.  Series branch below ``|delta| < 0.1`` as in the
    reference (cuda/continuum_attention.py:633-640).
    """
    N, Q, K = scores.shape
    dev = scores.device
    qi = torch.arange(start, start + Q, device=dev).view(1, Q, 1)
    kj = torch.arange(K, device=dev).view(1, 1, K)
    vis = kj <= qi
    m = scores.masked_fill(~vis, float("-inf")).amax(-1, keepdim=True)
    seg = kj[..., 1:] <= qi
    a = torch.where(seg, scores[..., :-1], m)
    b = torch.where(seg, scores[..., 1:], m)
    d = b - a
    t = d.abs()
    t2 = t * t
    L_small = 1 - t / 2 + t2 / 6 - t * t2 / 24 + t2 * t2 / 120 - t * t2 * t2 / 720 + t2 * t2 * t2 / 5040
    tc = t.clamp_min(0.1)
    L = torch.where(t < 0.1, L_small, -torch.expm1(-tc) / tc)
    mu_small = 0.5 + d / 12 - d.pow(3) / 720 + d.pow(5) / 30240
    mu_hi = 1 / (-torch.expm1(-tc)) - 1 / tc
    mu = torch.where(t < 0.1, mu_small, torch.where(d >= 0, mu_hi, 1 - mu_hi))
    mass = torch.exp(torch.maximum(a, b) - m) * L * seg
    w = F.pad(mass * (1 - mu), (0, 1)) + F.pad(mass * mu, (1, 0))
    w = w + F.pad(0.5 * torch.exp(scores[..., :1] - m), (0, K - 1))
    diag = scores.gather(-1, qi.expand(N, Q, 1))
    w = w + 0.5 * torch.exp(diag - m) * (kj == qi)
    w = w * vis
    return w / w.sum(-1, keepdim=True)


@torch.no_grad()
def port_forward(q, k, v, log_gain, query_tile=128):
    """Forward of the reference CPU path; q,k,v ``[B,H,T,D]`` fp32."""
    B, H, T, D = q.shape
    scale = (log_gain.detach().exp().float() * D ** -0.5).view(1, H, 1, 1)
    qb, kb, vb = (x.reshape(B * H, T, D) for x in (q, k, v))
    out = []
    for start in range(0, T, query_tile):
        end = min(T, start + query_tile)
        raw = torch.bmm(qb[:, start:end], kb[:, :end].transpose(1, 2))
        s = (raw.reshape(B, H, -1, end) * scale).reshape(B * H, -1, end)
        w = tile_weights(s, start)
        out.append(torch.bmm(w, vb[:, :end]))
    return torch.cat(out, dim=1).reshape(B, H, T, D)


def port_backward(q, k, v, log_gain, dy, query_tile=128):
    """Backward of the reference CPU path (autograd replay per query tile)."""
    B, H, T, D = q.shape
    scale4 = (log_gain.detach().exp().float() * D ** -0.5).view(1, H, 1, 1)
    qb, kb, vb = (x.reshape(B * H, T, D) for x in (q, k, v))
    gb = dy.reshape(B * H, T, D)
    gq = torch.zeros(B * H, T, D)
    gk = torch.zeros(B * H, T, D)
    gv = torch.zeros(B * H, T, D)
    gr = torch.zeros(H)
    for start in range(0, T, query_tile):
        end = min(T, start + query_tile)
        qs, keys, vals, gys = qb[:, start:end], kb[:, :end], vb[:, :end], gb[:, start:end]
        with torch.no_grad():
            raw = torch.bmm(qs, keys.transpose(1, 2))
            s = (raw.reshape(B, H, -1, end) * scale4).reshape(B * H, -1, end)
            gw = torch.bmm(gys, vals.transpose(1, 2))
        with torch.enable_grad():
            sr = s.detach().requires_grad_(True)
            wr = tile_weights(sr, start)
            ds = torch.autograd.grad(wr, sr, gw)[0]
        with torch.no_grad():
            w = wr.detach()
            gv[:, :end] += torch.bmm(w.transpose(1, 2), gys)
            ds4 = ds.reshape(B, H, -1, end)
            sc = (ds4 * scale4).reshape(B * H, -1, end)
            gq[:, start:end] += torch.bmm(sc, keys)
            gk[:, :end] += torch.bmm(sc.transpose(1, 2), qs)
            gr += (ds4 * s.reshape(B, H, -1, end)).sum(dim=(0, 2, 3))
    shp = (B, H, T, D)
    return gq.reshape(shp), gk.reshape(shp), gv.reshape(shp), gr

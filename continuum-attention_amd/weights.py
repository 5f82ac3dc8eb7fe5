"""Materialised CA weights on the GPU: the reference's weight-level API.

* ``ca_weights(scores, start)`` -> ``(W, stats)``: the reference extension's
  ``ext.forward(scores, start)`` (cuda/continuum_attention.py:578-590) and the
  CPU ``_ca_reference_weights(scores, start)`` (:622-648).  ``scores`` is
  ``[BH, Q, K]`` (a query tile starting at absolute query ``start``);
  ``stats`` is ``[BH*Q, 2]`` = (row max, 1/Z).
* ``ca_weights_backward(scores, grad_weights, start)`` -> ``dS`` (and W):
  ``ext.backward_fused`` (:538-554).
* ``continuous_attention_weights(logits)``: ``architecture.py:65-105`` for
  ``[..., T, T]`` logits, differentiable (its backward is the analytic VJP
  kernel).  Same ``ValueError`` for non-square logits.

On GPU tensors all arithmetic runs in the HIP row kernels
(csrc/ca_weights.hip) through the C ABI; inputs of any float dtype are
computed in float32 and results are returned in the input dtype.
``continuous_attention_weights`` on CPU tensors runs ``cpu.py`` in the logits'
own dtype and stays differentiable to any order, as the reference's torch
composition is; ``ca_weights`` / ``ca_weights_backward`` (the CUDA
extension's entry points in the reference) take GPU tensors only.
"""
from __future__ import annotations

import torch

from . import _native
from . import cpu as _cpu


def _f32c(x: torch.Tensor) -> torch.Tensor:
    x = x.detach()
    if x.dtype != torch.float32:
        x = x.float()
    return x.contiguous()


def _cuda(x: torch.Tensor, what: str) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(f"{what} (continuum-attention_amd) runs on ROCm GPU tensors only; "
                           f"got a tensor on {x.device}")


def _rows3(scores: torch.Tensor):
    if scores.dim() < 2:
        raise ValueError(f"scores must be [..., Q, K], got shape {tuple(scores.shape)}")
    Q, K = scores.shape[-2:]
    BH = scores.numel() // max(Q * K, 1)
    return BH, Q, K


def ca_weights(scores: torch.Tensor, start: int = 0):
    """Exact CA weights of a query tile: returns ``(W, stats)`` (float32).

    ``scores[..., r, j]`` is the scaled logit of query ``start + r`` against
    key ``j``; keys beyond ``start + r`` are ignored and get weight 0.
    """
    _cuda(scores, "ca_weights")
    BH, Q, K = _rows3(scores)
    if start < 0 or start + Q > K:
        raise ValueError(f"ca_weights: queries {start}..{start + Q - 1} need K >= {start + Q}, got K={K}")
    lib = _native.load()
    s = _f32c(scores)
    W = torch.empty_like(s)
    stats = torch.empty((BH * Q, 2), device=s.device, dtype=torch.float32)
    with _native.on_device(s.device):
        _native.check(lib.ca_weights_f32(s.data_ptr(), W.data_ptr(), stats.data_ptr(), BH, Q, K,
                                         int(start), _native.stream_handle(s.device)))
    return W, stats


def ca_weights_backward(scores: torch.Tensor, grad_weights: torch.Tensor, start: int = 0,
                        return_weights: bool = False):
    """Score VJP of the CA weights: ``dS = dL/dscores`` from ``dL/dW`` (float32).

    With ``return_weights`` returns ``(W, dS)`` like ``ext.backward_fused``.
    """
    _cuda(scores, "ca_weights_backward")
    if grad_weights.shape != scores.shape:
        raise ValueError(f"grad_weights shape {tuple(grad_weights.shape)} != scores shape "
                         f"{tuple(scores.shape)}")
    BH, Q, K = _rows3(scores)
    if start < 0 or start + Q > K:
        raise ValueError(f"ca_weights_backward: queries {start}..{start + Q - 1} need K >= {start + Q}, "
                         f"got K={K}")
    lib = _native.load()
    s = _f32c(scores)
    gw = _f32c(grad_weights)
    ds = torch.empty_like(s)
    W = torch.empty_like(s) if return_weights else None
    with _native.on_device(s.device):
        _native.check(lib.ca_weights_bwd_f32(s.data_ptr(), gw.data_ptr(),
                                             W.data_ptr() if W is not None else None,
                                             ds.data_ptr(), BH, Q, K, int(start),
                                             _native.stream_handle(s.device)))
    return (W, ds) if return_weights else ds


class _CAWeights(torch.autograd.Function):
    """W(logits) with the analytic first-order VJP (architecture.py:65-105 /
    analytic_reference.py:52-75)."""

    @staticmethod
    def forward(ctx, logits):
        W, _ = ca_weights(logits, 0)
        ctx.save_for_backward(logits)
        return W.to(logits.dtype)

    @staticmethod
    def backward(ctx, grad_w):
        if torch.is_grad_enabled():
            # the analytic VJP kernel is not itself differentiable: a graph
            # built through it (create_graph=True) would be silently cut
            raise RuntimeError("continuous_attention_weights on the GPU supports first-order "
                               "gradients only")
        (logits,) = ctx.saved_tensors
        ds = ca_weights_backward(logits, grad_w, 0)
        return ds.to(logits.dtype)


def continuous_attention_weights(logits: torch.Tensor) -> torch.Tensor:
    """Exact continuous causal piecewise-linear K/V memory weights
    (architecture.py:65-105): ``logits [..., T, T]`` (unmasked, scaled) ->
    row-stochastic causal ``W [..., T, T]`` in ``logits.dtype``."""
    T = logits.size(-1)
    if logits.size(-2) != T:
        raise ValueError("This benchmark requires square full-sequence causal attention")
    if logits.device.type == "cpu":
        return _cpu.continuous_attention_weights(logits)
    return _CAWeights.apply(logits)

"""Continuum Attention operator: the reference's Python API over the HIP kernels.

Drop-in for ``continuum_attention(q, k, v, log_gain, query_tile=64)`` and the
autograd Function ``_CAExactTiled`` (cuda/continuum_attention.py:650-783):

* same signature, argument meaning and return dtype (``v.dtype``);
* same errors: mismatched Q/K/V dtypes -> ValueError
  (cuda/continuum_attention.py:653-654); an unknown ``CA_CUDA_MODE`` ->
  ValueError (:659-661); a backward run with grad enabled (higher order) ->
  RuntimeError (:698-699);
* backward returns ``(dq, dk, dv, dlog_gain, None)`` in the input dtypes
  (:765-766).

Compute is float32 on the device (fp16/bf16 inputs are read as fp32, results
cast back).  ``query_tile`` is accepted and validated; in the reference it only
bounds the memory of the materialised ``[BH, Qt, K]`` weights
(cuda/continuum_attention.py:957), which these kernels never materialise, so it
does not change the arithmetic.  All ``CA_CUDA_MODE`` values select the same
exact fp32 path (the reference modes differ only in fp16 rounding and launch
structure).

There is no CPU path here: the operator runs on ROCm devices only and raises
otherwise.  CPU checking code lives in ``oracle/`` (tests only).
"""
from __future__ import annotations

import os

import torch

from . import _native

_MODES = ("dense", "prefix", "fused", "prefix_v5", "prefix_v6")
SUPPORTED_HEAD_DIMS = (8, 16, 32, 64)


def _mode() -> str:
    mode = os.environ.get("CA_CUDA_MODE", "prefix").lower()
    if mode not in _MODES:
        raise ValueError("CA_CUDA_MODE must be dense, prefix, fused, prefix_v5, or prefix_v6")
    return mode


def _as_f32(x: torch.Tensor) -> torch.Tensor:
    x = x.detach()
    if x.dtype != torch.float32:
        x = x.float()
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "continuum_attention (continuum-attention_amd) runs on ROCm GPU tensors only; "
            f"got a tensor on {dev}")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError("continuum_attention: all tensors must be on the same device")
    return dev


def ca_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, log_gain: torch.Tensor):
    """Runs the HIP forward; returns ``(out_f32, stats)`` (stats: [B*H*T, 2])."""
    lib = _native.load()
    dev = _check_device(q, k, v, log_gain)
    B, H, T, D = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if log_gain.numel() != H:
        raise ValueError(f"log_gain has {log_gain.numel()} entries, expected H={H}")
    qf, kf, vf, gf = _as_f32(q), _as_f32(k), _as_f32(v), _as_f32(log_gain.reshape(H))
    out = torch.empty((B, H, T, D), device=dev, dtype=torch.float32)
    stats = torch.empty((B * H * T, 2), device=dev, dtype=torch.float32)
    nbytes = lib.ca_fwd_workspace_bytes(B, H, T, D)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _native.check(lib.ca_fwd_f32(qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), gf.data_ptr(),
                                     out.data_ptr(), stats.data_ptr(), ws.data_ptr(), nbytes,
                                     B, H, T, D, _stream(dev)))
    return out, stats


def ca_backward(q, k, v, log_gain, out, stats, dout):
    """Runs the HIP backward; returns fp32 ``(dq, dk, dv, dlog_gain)``."""
    lib = _native.load()
    dev = _check_device(q, k, v, log_gain, out, stats, dout)
    B, H, T, D = q.shape
    qf, kf, vf, gf = _as_f32(q), _as_f32(k), _as_f32(v), _as_f32(log_gain.reshape(H))
    of, sf, df = _as_f32(out), _as_f32(stats), _as_f32(dout)
    dq = torch.empty((B, H, T, D), device=dev, dtype=torch.float32)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    dg = torch.empty(H, device=dev, dtype=torch.float32)
    nbytes = lib.ca_bwd_workspace_bytes(B, H, T, D)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _native.check(lib.ca_bwd_f32(qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), gf.data_ptr(),
                                     of.data_ptr(), sf.data_ptr(), df.data_ptr(), dq.data_ptr(),
                                     dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), ws.data_ptr(),
                                     nbytes, B, H, T, D, _stream(dev)))
    return dq, dk, dv, dg


class _CAExactTiled(torch.autograd.Function):
    """Autograd Function with the reference's contract (cuda/continuum_attention.py:650-766)."""

    @staticmethod
    def forward(ctx, q, k, v, log_gain, query_tile):
        if q.dtype != k.dtype or q.dtype != v.dtype:
            raise ValueError("CA Q,K,V must share dtype")
        if q.dim() != 4:
            raise ValueError(f"CA expects [B,H,T,D] tensors, got shape {tuple(q.shape)}")
        if int(query_tile) <= 0:
            raise ValueError("query_tile must be positive")
        _mode()
        with torch.autocast(device_type="cuda", enabled=False):
            out, stats = ca_forward(q, k, v, log_gain)
        ctx.save_for_backward(q, k, v, log_gain, out, stats)
        ctx.query_tile = int(query_tile)
        return out.to(v.dtype)

    @staticmethod
    def backward(ctx, grad_y):
        if torch.is_grad_enabled():
            raise RuntimeError("CA Volta analytic kernel supports first-order gradients only")
        q, k, v, log_gain, out, stats = ctx.saved_tensors
        dq, dk, dv, dg = ca_backward(q, k, v, log_gain, out, stats, grad_y)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(log_gain.dtype), None)


def continuum_attention(q, k, v, log_gain, query_tile=64):
    """Exact causal Continuum Attention (cuda/continuum_attention.py:768-783).

    q, k, v: ``[B, H, T, D]`` (same dtype, D in {8, 16, 32, 64}), log_gain: ``[H]``.
    Scores are ``exp(log_gain[h]) / sqrt(D) * q.k``; keys and values are
    linearly interpolated between adjacent positions with half-token end caps
    and integrated exactly.  Returns ``[B, H, T, D]`` in ``v.dtype``.
    """
    return _CAExactTiled.apply(q.contiguous(), k.contiguous(), v.contiguous(), log_gain,
                               int(query_tile))

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
(cuda/continuum_attention.py:957), which the fused kernels (D in 8, 16, 32,
64, 128) never materialise, so it does not change their arithmetic; other head
dims run the reference's query-tile structure, where it does bound memory.  All ``CA_CUDA_MODE`` values select the same
exact fp32 path (the reference modes differ only in fp16 rounding and launch
structure).

The reference's per-mode limits hold on every device (:662-665):
``CA_CUDA_MODE`` prefix_v5/prefix_v6 need CUDA fp16 tensors and T <= 2048,
and 'fused' needs T <= 2048, D <= 128 and fp16/fp32 values (ValueError).

GPU tensors run the HIP kernels only (a missing library raises; there is no
fallback).  CPU tensors run ``cpu.py``, this package's own float32
formulation of the reference's CPU branch (``ext=None``,
cuda/continuum_attention.py:658, 688, 737-751).
"""
from __future__ import annotations

import functools
import os

import torch

from . import _native
from . import cpu as _cpu

_MODES = ("dense", "prefix", "fused", "prefix_v5", "prefix_v6")
SUPPORTED_HEAD_DIMS = (8, 16, 32, 64, 128)


def _mode() -> str:
    mode = os.environ.get("CA_CUDA_MODE", "prefix").lower()
    if mode not in _MODES:
        raise ValueError("CA_CUDA_MODE must be dense, prefix, fused, prefix_v5, or prefix_v6")
    return mode


def check_mode_limits(mode: str, is_cuda: bool, q_dtype: torch.dtype, v_dtype: torch.dtype,
                      T: int, D: int) -> None:
    """The reference's per-mode limits, raised on every device as there
    (cuda/continuum_attention.py:662-665): prefix_v5/prefix_v6 need CUDA fp16
    Q/K/V and T <= 2048; 'fused' needs T <= 2048, D <= 128 and fp16/fp32
    values.  Within them every mode runs the same exact fp32 kernels."""
    if mode in ("prefix_v5", "prefix_v6") and (not is_cuda or q_dtype != torch.float16 or T > 2048):
        raise ValueError("CA v5/v6 paths require CUDA FP16 Q/K/V and T<=2048")
    if mode == "fused" and (T > 2048 or D > 128 or v_dtype not in (torch.float16, torch.float32)):
        raise ValueError("CA fused forward supports T<=2048, D<=128, FP16/FP32 values")


def _as_f32(x: torch.Tensor) -> torch.Tensor:
    x = x.detach()
    if x.dtype != torch.float32:
        x = x.float()
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


def _stream(dev: torch.device) -> int:
    return _native.stream_handle(dev)


@functools.lru_cache(maxsize=256)
def _fwd_workspace_bytes(B: int, H: int, T: int, D: int) -> int:
    return int(_native.load().ca_fwd_workspace_bytes(B, H, T, D))


@functools.lru_cache(maxsize=256)
def _bwd_workspace_bytes(B: int, H: int, T: int, D: int) -> int:
    return int(_native.load().ca_bwd_workspace_bytes(B, H, T, D))


@functools.lru_cache(maxsize=256)
def _bwd_qkv_workspace_bytes(B: int, H: int, T: int, D: int) -> int:
    return int(_native.load().ca_bwd_qkv_workspace_bytes(B, H, T, D))


@functools.lru_cache(maxsize=256)
def _fwd_qkv_workspace_bytes(B: int, H: int, T: int, D: int) -> int:
    return int(_native.load().ca_fwd_qkv_workspace_bytes(B, H, T, D))


def _clear_workspace_sizes() -> None:
    # the sizes follow the workspace cap and the split override
    for f in (_fwd_workspace_bytes, _bwd_workspace_bytes, _fwd_qkv_workspace_bytes,
              _bwd_qkv_workspace_bytes):
        f.cache_clear()


def set_workspace_cap(nbytes: int) -> None:
    """Bounds the operator's device workspace (bytes; 0 = no bound; default
    1 GiB, or the environment's ``CA_WORKSPACE_CAP_MB``), the role
    ``query_tile`` plays for the reference's materialised weights: beyond it
    the forward uses longer work splits and the backward runs in passes over
    query ranges.  Process-wide."""
    _native.check(_native.load().ca_set_workspace_cap(int(nbytes)))
    _clear_workspace_sizes()


def workspace_cap() -> int:
    return int(_native.load().ca_workspace_cap())


def set_split_override(fwd_split_tiles: int = 0, dq_chunk_stages: int = 0,
                       dkdv_chunk_tiles: int = 0) -> None:
    """Forces the kernels' work-split lengths (0 = automatic; see
    ``ca_debug_set_splits`` in the C header).  For tests: the automatic
    choice depends on the device's CU count, so a forced length runs each one
    at a small shape.  Clears the cached workspace sizes, which follow it."""
    _native.check(_native.load().ca_debug_set_splits(int(fwd_split_tiles), int(dq_chunk_stages),
                                                     int(dkdv_chunk_tiles)))
    _clear_workspace_sizes()


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
    nbytes = _fwd_workspace_bytes(B, H, T, D)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    with _native.on_device(dev):
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
    nbytes = _bwd_workspace_bytes(B, H, T, D)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    with _native.on_device(dev):
        _native.check(lib.ca_bwd_f32(qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), gf.data_ptr(),
                                     of.data_ptr(), sf.data_ptr(), df.data_ptr(), dq.data_ptr(),
                                     dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), ws.data_ptr(),
                                     nbytes, B, H, T, D, _stream(dev)))
    return dq, dk, dv, dg


# ---- any head dimension: the query-tile structure over the HIP weight kernels
#
# Head dims without a fused kernel (D not in SUPPORTED_HEAD_DIMS) run the
# reference operator's own structure (cuda/continuum_attention.py:666-694 and
# :707-764) on the device: per query tile, fp32 GEMMs for the scores, W.V and
# the gradient contractions, and the HIP weight kernels (ca_weights_f32,
# ca_weights_bwd_f32) for the exact weights and their score VJP.  The [BH,
# Qt, K] tile is materialised, so query_tile bounds the memory as in the
# reference.  Matmuls run in IEEE fp32 (no reduced-precision fp32 modes).


class _Fp32Matmul:
    """Turns reduced-precision fp32 GEMM modes off for the enclosed calls."""

    def __enter__(self):
        self.prev = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = False

    def __exit__(self, *exc):
        torch.backends.cuda.matmul.allow_tf32 = self.prev


def _head_scale(log_gain, H, D):
    return (torch.exp(log_gain.reshape(H).float()) * D ** -0.5).reshape(1, H, 1, 1)


def _tile_scores(qf, kt, scale, start, end):
    """c * q[start:end] k[:end]^T for every (b, h): [B, H, end-start, end]."""
    return torch.matmul(qf[:, :, start:end].contiguous(), kt[:, :, :, :end].contiguous()) * scale


def tiled_forward(q, k, v, log_gain, query_tile):
    """fp32 output of the operator for any head dim (query-tile structure)."""
    from .weights import ca_weights
    _check_device(q, k, v, log_gain)
    B, H, T, D = q.shape
    qf, kf, vf = _as_f32(q), _as_f32(k), _as_f32(v)
    scale = _head_scale(log_gain, H, D)
    kt = kf.transpose(2, 3).contiguous()
    out = torch.empty((B, H, T, D), device=q.device, dtype=torch.float32)
    with _Fp32Matmul():
        for start in range(0, T, query_tile):
            end = min(T, start + query_tile)
            s = _tile_scores(qf, kt, scale, start, end)
            w, _ = ca_weights(s.reshape(B * H, end - start, end), start)
            out[:, :, start:end] = torch.matmul(w.reshape(B, H, end - start, end), vf[:, :, :end])
    return out


def tiled_backward(q, k, v, log_gain, dout, query_tile):
    """fp32 (dq, dk, dv, dlog_gain) for any head dim, recomputing each tile."""
    from .weights import ca_weights_backward
    _check_device(q, k, v, log_gain, dout)
    B, H, T, D = q.shape
    qf, kf, vf, gf = _as_f32(q), _as_f32(k), _as_f32(v), _as_f32(dout)
    scale = _head_scale(log_gain, H, D)
    kt = kf.transpose(2, 3).contiguous()
    vt = vf.transpose(2, 3).contiguous()
    dq = torch.zeros_like(qf)
    dk = torch.zeros_like(kf)
    dv = torch.zeros_like(vf)
    dg = torch.zeros((B, H), device=q.device, dtype=torch.float32)
    with _Fp32Matmul():
        for start in range(0, T, query_tile):
            end = min(T, start + query_tile)
            n = end - start
            s = _tile_scores(qf, kt, scale, start, end)
            gy = gf[:, :, start:end].contiguous()
            gw = torch.matmul(gy, vt[:, :, :, :end].contiguous())            # dL/dW
            w, ds = ca_weights_backward(s.reshape(B * H, n, end), gw.reshape(B * H, n, end), start,
                                        return_weights=True)
            w = w.reshape(B, H, n, end)
            ds = ds.reshape(B, H, n, end)
            dv[:, :, :end] += torch.matmul(w.transpose(2, 3).contiguous(), gy)
            dsc = ds * scale                                                    # dL/d(q.k)
            dq[:, :, start:end] = torch.matmul(dsc, kf[:, :, :end])
            dk[:, :, :end] += torch.matmul(dsc.transpose(2, 3).contiguous(), qf[:, :, start:end].contiguous())
            dg += (ds * s).sum(dim=(2, 3))                                      # d/dlog_gain: s is linear in e^g
    return dq, dk, dv, dg.sum(0)


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
        mode = _mode()
        ctx.query_tile = int(query_tile)
        ctx.fused = q.shape[-1] in SUPPORTED_HEAD_DIMS
        ctx.empty = False
        ctx.on_cpu = q.device.type == "cpu"
        check_mode_limits(mode, q.device.type == "cuda", q.dtype, v.dtype, q.shape[2], q.shape[3])
        if ctx.on_cpu:
            for t in (k, v, log_gain):
                if t.device != q.device:
                    raise RuntimeError("continuum_attention: all tensors must be on the same device")
        if q.shape[2] == 0:
            # the reference's query-tile loop has no tile to concatenate (:670-694)
            raise RuntimeError("continuum_attention: empty sequence (T = 0)")
        if q.shape[0] * q.shape[1] == 0:
            # an empty batch: the reference's tile loop yields empty tiles
            if not ctx.on_cpu:
                _check_device(q, k, v, log_gain)
            ctx.empty = True
            ctx.save_for_backward(q, k, v, log_gain)
            return torch.empty(q.shape, device=q.device, dtype=v.dtype)
        if ctx.on_cpu:
            ctx.save_for_backward(q, k, v, log_gain)
            return _cpu.forward(q, k, v, log_gain, ctx.query_tile)
        with torch.autocast(device_type="cuda", enabled=False):
            if ctx.fused:
                out, stats = ca_forward(q, k, v, log_gain)
                ctx.save_for_backward(q, k, v, log_gain, out, stats)
            else:
                out = tiled_forward(q, k, v, log_gain, ctx.query_tile)
                ctx.save_for_backward(q, k, v, log_gain)
        return out.to(v.dtype)

    @staticmethod
    def backward(ctx, grad_y):
        if torch.is_grad_enabled():
            raise RuntimeError("CA Volta analytic kernel supports first-order gradients only")
        if ctx.empty:
            q, k, v, log_gain = ctx.saved_tensors
            return (torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v),
                    torch.zeros_like(log_gain), None)
        if ctx.on_cpu:
            q, k, v, log_gain = ctx.saved_tensors
            dq, dk, dv, dg = _cpu.backward(q, k, v, log_gain, grad_y, ctx.query_tile)
        elif ctx.fused:
            q, k, v, log_gain, out, stats = ctx.saved_tensors
            dq, dk, dv, dg = ca_backward(q, k, v, log_gain, out, stats, grad_y)
        else:
            q, k, v, log_gain = ctx.saved_tensors
            with torch.autocast(device_type="cuda", enabled=False):
                dq, dk, dv, dg = tiled_backward(q, k, v, log_gain, grad_y, ctx.query_tile)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(log_gain.dtype), None)


def continuum_attention(q, k, v, log_gain, query_tile=64):
    """Exact causal Continuum Attention (cuda/continuum_attention.py:768-783).

    q, k, v: ``[B, H, T, D]`` (same dtype), log_gain: ``[H]``.  On the GPU,
    D in {8, 16, 32, 64, 128} runs the fused kernels and any other D the
    query-tile structure over the HIP weight kernels (``query_tile`` rows at a
    time); CPU tensors run the float32 CPU path (``cpu.py``).
    Scores are ``exp(log_gain[h]) / sqrt(D) * q.k``; keys and values are
    linearly interpolated between adjacent positions with half-token end caps
    and integrated exactly.  Returns ``[B, H, T, D]`` in ``v.dtype``.
    """
    return _CAExactTiled.apply(q.contiguous(), k.contiguous(), v.contiguous(), log_gain,
                               int(query_tile))

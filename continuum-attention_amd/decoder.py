"""CA-S byte decoder: the reference's main caller of the CA operator.

Counterpart of ``ContinuumDecoderConfig`` / ``ContinuumDecoderLM``
(cuda/continuum_attention.py:784-923): a pre-norm decoder with RMSNorm
(eps 1e-6), interleaved RoPE (theta 1e4), exact Continuum Attention with a
learned per-head score gain ``log_qk_gain`` (init 0, tau = 1), tanh-GELU MLP
and an untied byte head.  Module names, parameter shapes, initialisation
(std .02, residual projections .02/sqrt(2L)) and state-dict keys are the
reference's, so its checkpoints load unchanged; the default configuration has
101,205,120 parameters (cuda/test_cpu.py:25-27).

Only the attention operator is this package's: ``continuum_attention`` runs
the HIP kernels with float32 scores whatever the autocast dtype, and returns
``v.dtype``.  ``train_step`` is one optimisation step as the reference's
training loop takes it (cuda/continuum_attention.py:1195-1230): autocast
forward + cross-entropy, backward, gradient clipping, AdamW.
"""
from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from . import _native
from .ops import (SUPPORTED_HEAD_DIMS, _bwd_qkv_workspace_bytes, _fwd_qkv_workspace_bytes, _mode,
                  check_mode_limits, continuum_attention)

_DTYPE_CODE = {torch.float32: _native.CA_DTYPE_F32, torch.bfloat16: _native.CA_DTYPE_BF16,
               torch.float16: _native.CA_DTYPE_F16}


@dataclass
class ContinuumDecoderConfig:
    """Decoder hyper-parameters (cuda/continuum_attention.py:784-814)."""
    vocab_size: int = 256
    block_size: int = 2048
    d_model: int = 1024
    n_heads: int = 16
    n_layers: int = 8
    mlp_ratio: float = 4.0
    dropout: float = 0.0
    eps: float = 1e-6
    rope_theta: float = 10000.0
    grad_checkpointing: bool = False
    ca_query_tile: int = 64

    def __post_init__(self):
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if (self.d_model // self.n_heads) % 2:
            raise ValueError("RoPE needs even head dimension")
        if self.n_layers <= 0 or self.block_size < 2 or self.ca_query_tile <= 0:
            raise ValueError("Invalid layer, context or CA query tile count")
        if self.dropout != 0:
            raise ValueError("The CA operator has no attention dropout; use --dropout 0.0")


class _RMSNormFn(torch.autograd.Function):
    """RMSNorm forward and backward as single HIP passes (ca_rmsnorm_fwd /
    ca_rmsnorm_bwd).  The output is written in ``out_dtype``: under autocast
    every RMSNorm output feeds a linear layer, whose autocast would round it to
    that dtype, so the rounded value is the reference's."""

    @staticmethod
    def forward(ctx, x, weight, eps, out_dtype):
        lib = _native.load()
        C = x.shape[-1]
        N = x.numel() // C
        xc = _aligned(x.detach(), 16)
        w = weight.detach().contiguous()
        y = torch.empty(x.shape, device=x.device, dtype=out_dtype)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        stream = _native.stream_handle(x.device)
        with _native.on_device(x.device):
            _native.check(lib.ca_rmsnorm_fwd(xc.data_ptr(), w.data_ptr(), y.data_ptr(),
                                             _DTYPE_CODE[out_dtype], rstd.data_ptr(), N, C,
                                             float(eps), stream))
        ctx.save_for_backward(xc, w, rstd)
        return y

    @staticmethod
    def backward(ctx, gy):
        if torch.is_grad_enabled():
            raise RuntimeError("the fused RMSNorm supports first-order gradients only")
        xc, w, rstd = ctx.saved_tensors
        lib = _native.load()
        C = xc.shape[-1]
        N = xc.numel() // C
        g = gy.contiguous()
        if g.dtype not in _DTYPE_CODE:
            g = g.float()
        dx = torch.empty_like(xc)
        dw = torch.empty_like(w)
        nbytes = int(lib.ca_rmsnorm_bwd_workspace_bytes(N, C))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=xc.device)
        stream = _native.stream_handle(xc.device)
        with _native.on_device(xc.device):
            _native.check(lib.ca_rmsnorm_bwd(g.data_ptr(), _DTYPE_CODE[g.dtype], xc.data_ptr(),
                                             w.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                                             dw.data_ptr(), ws.data_ptr(), ws.numel(), N, C,
                                             stream))
        return dx, dw, None, None


class _AddRMSNormFn(torch.autograd.Function):
    """The decoder's residual add and the RMSNorm that reads it, s = x + res
    and y = RMSNorm(s), as one HIP pass each way (ca_add_rmsnorm_fwd /
    ca_add_rmsnorm_bwd).  Returns (s, y): s continues the fp32 residual stream,
    y is written in ``out_dtype`` as in _RMSNormFn.  The backward adds the
    gradient s receives downstream to the norm's and returns it for x (fp32)
    and, in res's dtype, for res."""

    @staticmethod
    def forward(ctx, x, res, weight, eps, out_dtype):
        lib = _native.load()
        C = x.shape[-1]
        N = x.numel() // C
        xc = _aligned(x.detach(), 16)
        rc = _aligned(res.detach(), 16)
        w = weight.detach().contiguous()
        s = torch.empty(x.shape, device=x.device, dtype=torch.float32)
        y = torch.empty(x.shape, device=x.device, dtype=out_dtype)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        stream = _native.stream_handle(x.device)
        with _native.on_device(x.device):
            _native.check(lib.ca_add_rmsnorm_fwd(xc.data_ptr(), rc.data_ptr(), _DTYPE_CODE[res.dtype],
                                                 s.data_ptr(), w.data_ptr(), y.data_ptr(),
                                                 _DTYPE_CODE[out_dtype], rstd.data_ptr(), N, C,
                                                 float(eps), stream))
        ctx.save_for_backward(s, w, rstd)
        ctx.res_dtype = res.dtype
        ctx.set_materialize_grads(False)  # an unused s (after the last block) reads no zeros
        return s, y

    @staticmethod
    def backward(ctx, gs, gy):
        if torch.is_grad_enabled():
            raise RuntimeError("the fused add + RMSNorm supports first-order gradients only")
        s, w, rstd = ctx.saved_tensors
        lib = _native.load()
        C = s.shape[-1]
        N = s.numel() // C
        g = torch.zeros_like(s) if gy is None else gy.contiguous()
        if g.dtype not in _DTYPE_CODE:
            g = g.float()
        gsum = None if gs is None else gs.float().contiguous()
        dx = torch.empty_like(s)
        dres = torch.empty(s.shape, device=s.device, dtype=ctx.res_dtype)
        dw = torch.empty_like(w)
        nbytes = int(lib.ca_rmsnorm_bwd_workspace_bytes(N, C))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=s.device)
        stream = _native.stream_handle(s.device)
        with _native.on_device(s.device):
            _native.check(lib.ca_add_rmsnorm_bwd(g.data_ptr(), _DTYPE_CODE[g.dtype],
                                                 None if gsum is None else gsum.data_ptr(),
                                                 s.data_ptr(), w.data_ptr(), rstd.data_ptr(),
                                                 dx.data_ptr(), dres.data_ptr(),
                                                 _DTYPE_CODE[ctx.res_dtype], dw.data_ptr(),
                                                 ws.data_ptr(), ws.numel(), N, C, stream))
        return dx, dres, dw, None, None


class RMSNorm(nn.Module):
    """weight * x / rms(x) (cuda/continuum_attention.py:817-823)."""

    # fp32 GPU inputs run as one HIP pass each way (_RMSNormFn); False, or any
    # other input, runs the reference's op-by-op composition
    fused = True

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def _fusable(self, x):
        return (self.fused and x.is_cuda and x.dtype == torch.float32
                and self.weight.dtype == torch.float32 and x.shape[-1] <= 4096)

    @staticmethod
    def _out_dtype():
        if torch.is_autocast_enabled("cuda"):
            ad = torch.get_autocast_dtype("cuda")
            if ad in (torch.bfloat16, torch.float16):
                return ad
        return torch.float32

    def _composition(self, x):
        return self.weight * x * torch.rsqrt(x.square().mean(-1, keepdim=True) + self.eps)

    def forward(self, x):
        if self._fusable(x):
            return _RMSNormFn.apply(x, self.weight, self.eps, self._out_dtype())
        return self._composition(x)

    def add_and_norm(self, x, res):
        """(x + res, self(x + res)): the residual add of a decoder block and
        the norm that reads its result, fused when the input qualifies."""
        if (self._fusable(x) and res.shape == x.shape and res.device == x.device
                and res.dtype in _DTYPE_CODE):
            return _AddRMSNormFn.apply(x, res, self.weight, self.eps, self._out_dtype())
        s = x + res
        return s, self(s)


_ROPE_CACHE: dict = {}


def _rope_tables(T, D, theta, device, dtype):
    """cos/sin of position x frequency, each frequency repeated for its pair,
    in ``dtype`` (cuda/continuum_attention.py:826-831); cached per shape."""
    key = (T, D, float(theta), device, dtype)
    tab = _ROPE_CACHE.get(key)
    if tab is None:
        freq = 1.0 / (theta ** (torch.arange(0, D, 2, device=device, dtype=torch.float32) / D))
        phase = torch.outer(torch.arange(T, device=device, dtype=torch.float32), freq)
        cos = phase.cos().repeat_interleave(2, -1).to(dtype)[None, None]
        sin = phase.sin().repeat_interleave(2, -1).to(dtype)[None, None]
        tab = (cos, sin)
        if len(_ROPE_CACHE) > 64:
            _ROPE_CACHE.clear()
        _ROPE_CACHE[key] = tab
    return tab


def _rotate_pairs(t):
    """(x0, x1) -> (-x1, x0) for each interleaved pair of the last axis."""
    pairs = t.unflatten(-1, (-1, 2))
    return torch.stack((-pairs[..., 1], pairs[..., 0]), -1).flatten(-2)


def apply_rope(q, k, theta):
    """Interleaved rotary embedding at each position, computed in q's dtype
    (cuda/continuum_attention.py:826-835)."""
    cos, sin = _rope_tables(q.shape[-2], q.shape[-1], theta, q.device, q.dtype)
    return q * cos + _rotate_pairs(q) * sin, k * cos + _rotate_pairs(k) * sin


_CS_CACHE: dict = {}


def rope_cos_sin(T, D, theta, device, dtype=torch.float32):
    """fp32 table ``[T, D/2, 2]`` of (cos, sin) of ``t * theta^(-2i/D)``, the
    reference's angles, rounded to ``dtype`` as the reference casts them to
    the operands' dtype (cuda/continuum_attention.py:828-830) and stored as
    fp32; ``theta=None`` gives the identity rotation (cos 1, sin 0, exact in
    every dtype); cached per shape and dtype."""
    key = (T, D, None if theta is None else float(theta), device, dtype)
    cs = _CS_CACHE.get(key)
    if cs is None:
        if theta is None:
            cs = torch.stack((torch.ones(T, D // 2, device=device), torch.zeros(T, D // 2, device=device)),
                             -1).contiguous()
        else:
            freq = 1.0 / (theta ** (torch.arange(0, D, 2, device=device, dtype=torch.float32) / D))
            phase = torch.outer(torch.arange(T, device=device, dtype=torch.float32), freq)
            cs = torch.stack((phase.cos(), phase.sin()), -1)
            cs = cs.to(dtype).float().contiguous()
        if len(_CS_CACHE) > 64:
            _CS_CACHE.clear()
        _CS_CACHE[key] = cs
    return cs


def _aligned(x, nbytes):
    x = x.contiguous()
    return x if x.data_ptr() % nbytes == 0 else x.clone()


class _RopeContinuumAttention(torch.autograd.Function):
    """qkv projection output -> RoPE -> CA operator -> token-major output, with
    the operator's kernels reading the projection output [B, T, 3, H, D]
    directly (q and k rotated as they are read, with the reference's
    rounding to the projection's dtype) and writing the output token-major in
    that dtype (ca_fwd_qkv); the backward (ca_bwd_qkv) reads the output
    gradient token-major and writes the qkv gradient, the q and k parts
    rotated back (in fp32, rounded once).  The forward is ``apply_rope`` +
    ``continuum_attention`` + transpose; the gradients differ from that
    composition's only in rounding (it rounds each step of the rotation's
    backward to the dtype)."""

    @staticmethod
    def forward(ctx, qkv, log_gain, theta, heads, query_tile):
        if int(query_tile) <= 0:
            raise ValueError("query_tile must be positive")
        mode = _mode()
        if qkv.dtype not in _DTYPE_CODE:
            raise ValueError(f"unsupported qkv dtype {qkv.dtype}")
        if qkv.device.type != "cuda":
            raise RuntimeError("continuum attention (continuum-attention_amd) runs on ROCm GPU "
                               f"tensors only; got a tensor on {qkv.device}")
        Bsz, T, C3 = qkv.shape
        C = C3 // 3
        D = C // heads
        # the operator's mode limits, on the rotated q and v in the projection's
        # dtype as the reference passes them (cuda/continuum_attention.py:853)
        check_mode_limits(mode, True, qkv.dtype, qkv.dtype, T, D)
        lib = _native.load()
        dev, dt = qkv.device, _DTYPE_CODE[qkv.dtype]
        x = _aligned(qkv.detach(), 16)
        cs = rope_cos_sin(T, D, theta, dev, qkv.dtype) if theta is not None else None
        gain = log_gain.detach().float().contiguous()
        y = torch.empty(Bsz, heads, T, D, device=dev, dtype=torch.float32)
        out = torch.empty(Bsz, T, C, device=dev, dtype=qkv.dtype)
        stats = torch.empty(Bsz * heads * T, 2, device=dev, dtype=torch.float32)
        nbytes = _fwd_qkv_workspace_bytes(Bsz, heads, T, D)
        ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
        with _native.on_device(dev):
            _native.check(lib.ca_fwd_qkv(x.data_ptr(), dt, cs.data_ptr() if cs is not None else None,
                                         gain.data_ptr(), y.data_ptr(), out.data_ptr(),
                                         stats.data_ptr(), ws.data_ptr(), nbytes, Bsz, T, heads, D,
                                         _native.stream_handle(dev)))
        ctx.save_for_backward(x, gain, y, stats)
        ctx.cs = cs
        ctx.shape = (Bsz, T, heads, D)
        ctx.gain_dtype = log_gain.dtype
        return out

    @staticmethod
    def backward(ctx, gout):
        if torch.is_grad_enabled():
            raise RuntimeError("CA Volta analytic kernel supports first-order gradients only")
        x, gain, y, stats = ctx.saved_tensors
        cs = ctx.cs
        Bsz, T, heads, D = ctx.shape
        lib = _native.load()
        dev = x.device
        g = _aligned(gout.to(x.dtype), 16)
        dqkv = torch.empty(Bsz, T, 3 * heads * D, device=dev, dtype=x.dtype)
        dg = torch.empty(heads, device=dev, dtype=torch.float32)
        nbytes = _bwd_qkv_workspace_bytes(Bsz, heads, T, D)
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        with _native.on_device(dev):
            _native.check(lib.ca_bwd_qkv(x.data_ptr(), _DTYPE_CODE[x.dtype],
                                         cs.data_ptr() if cs is not None else None, gain.data_ptr(),
                                         y.data_ptr(), stats.data_ptr(), g.data_ptr(),
                                         dqkv.data_ptr(), dg.data_ptr(), ws.data_ptr(), nbytes, Bsz,
                                         T, heads, D, _native.stream_handle(dev)))
        return dqkv, dg.to(ctx.gain_dtype), None, None, None


def rope_continuum_attention(qkv, log_gain, theta, heads, query_tile=64):
    """``[B, T, 3C]`` qkv projection output -> ``[B, T, C]`` attention output
    (before the output projection), in qkv's dtype; see _RopeContinuumAttention.
    ``theta=None``: no rotary embedding (the prologue only splits the heads)."""
    return _RopeContinuumAttention.apply(qkv, log_gain, None if theta is None else float(theta),
                                         int(heads), int(query_tile))


# Largest vocabulary whose embedding gradient is formed as a one-hot GEMM
# (its [tokens, vocab] one-hot matrix costs O(tokens * vocab)); the byte
# vocabulary (256) is far below it.
ONE_HOT_MAX_VOCAB = 4096


class _TokenEmbedding(torch.autograd.Function):
    """The token lookup ``weight[tokens]`` with its weight gradient formed as
    ``one_hot(tokens)^T @ grad`` (a scatter of ones into a zeroed matrix, then
    one GEMM): deterministic, and free of the sorting path torch's embedding
    backward takes above 3072 lookups, which records memset nodes that HIP
    graph replays do not reliably redo.  Same values as nn.Embedding's
    gradient up to the summation order of the rows of equal tokens, for
    finite gradients; a non-finite gradient row reaches every vocabulary row
    (0 * inf is NaN in the GEMM) where nn.Embedding's touches only the looked-up
    row.  Used for vocabularies of at most ONE_HOT_MAX_VOCAB rows."""

    @staticmethod
    def forward(ctx, tokens, weight):
        ctx.save_for_backward(tokens)
        ctx.num = weight.shape[0]
        return F.embedding(tokens, weight)

    @staticmethod
    def backward(ctx, grad):
        (tokens,) = ctx.saved_tensors
        flat = tokens.reshape(-1, 1)
        onehot = torch.zeros(flat.shape[0], ctx.num, device=grad.device, dtype=grad.dtype)
        onehot.scatter_(1, flat, 1.0)
        return None, onehot.t().mm(grad.reshape(-1, grad.shape[-1]))


def token_embedding(tokens, emb: nn.Embedding):
    """``emb(tokens)``, on GPU tensors with the one-hot GEMM weight gradient of
    _TokenEmbedding when the vocabulary is at most ONE_HOT_MAX_VOCAB rows
    (torch's embedding backward for the CA-S decoder's 2048 byte lookups took
    109 us per step, a [2048, 256] x [2048, 1024] GEMM a few)."""
    if tokens.is_cuda and emb.num_embeddings <= ONE_HOT_MAX_VOCAB and emb.padding_idx is None \
            and emb.max_norm is None and not emb.scale_grad_by_freq and not emb.sparse:
        return _TokenEmbedding.apply(tokens, emb.weight)
    return emb(tokens)


class ContinuumSelfAttention(nn.Module):
    """qkv projection -> RoPE -> CA operator -> output projection
    (cuda/continuum_attention.py:838-854)."""

    def __init__(self, dim, heads, rope_theta, ca_query_tile):
        super().__init__()
        self.heads = heads
        self.head_dim = dim // heads
        self.rope_theta = rope_theta
        self.ca_query_tile = ca_query_tile
        self.qkv = nn.Linear(dim, 3 * dim, bias=False)
        self.out = nn.Linear(dim, dim, bias=False)
        self.out._residual_proj = True
        # positive per-head score gain exp(log_qk_gain), starting at 1
        self.log_qk_gain = nn.Parameter(torch.zeros(heads))

    # fused HIP prologue/epilogue around the operator on GPU tensors (head
    # dims with fused operator kernels); False runs the reference's op-by-op
    # composition (same operator kernels)
    fused_prologue = True

    def forward(self, x):
        Bsz, T, C = x.shape
        if self.fused_prologue and x.is_cuda and self.head_dim in SUPPORTED_HEAD_DIMS:
            y = rope_continuum_attention(self.qkv(x), self.log_qk_gain, self.rope_theta, self.heads,
                                         self.ca_query_tile)
            return self.out(y)
        q, k, v = self.qkv(x).view(Bsz, T, 3, self.heads, self.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
        q, k = apply_rope(q, k, self.rope_theta)
        y = continuum_attention(q, k, v, self.log_qk_gain, self.ca_query_tile)
        return self.out(y.transpose(1, 2).reshape(Bsz, T, C))


class GELUMLP(nn.Module):
    """fc1 -> tanh-GELU -> fc2 (cuda/continuum_attention.py:857-866)."""

    def __init__(self, dim, ratio, dropout):
        super().__init__()
        hidden = int(dim * ratio)
        self.fc1 = nn.Linear(dim, hidden, bias=False)
        self.fc2 = nn.Linear(hidden, dim, bias=False)
        self.fc2._residual_proj = True
        self.dropout = nn.Dropout(dropout)

    def forward(self, x):
        return self.fc2(self.dropout(F.gelu(self.fc1(x), approximate="tanh")))


class CADecoderBlock(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.norm1 = RMSNorm(cfg.d_model, cfg.eps)
        self.attn = ContinuumSelfAttention(cfg.d_model, cfg.n_heads, cfg.rope_theta, cfg.ca_query_tile)
        self.norm2 = RMSNorm(cfg.d_model, cfg.eps)
        self.mlp = GELUMLP(cfg.d_model, cfg.mlp_ratio, cfg.dropout)

    def forward(self, x):
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))


class ContinuumDecoderLM(nn.Module):
    """Byte decoder with exact Continuum Attention
    (cuda/continuum_attention.py:882-923)."""

    def __init__(self, cfg: ContinuumDecoderConfig):
        super().__init__()
        self.cfg = cfg
        self.byte_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.drop = nn.Dropout(cfg.dropout)
        self.blocks = nn.ModuleList([CADecoderBlock(cfg) for _ in range(cfg.n_layers)])
        self.norm_f = RMSNorm(cfg.d_model, cfg.eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)  # untied
        self.residual_layers = cfg.n_layers
        self.residual_init_scale = 1.0 / math.sqrt(2.0 * cfg.n_layers)
        self.apply(self._init_weights)

    def _init_weights(self, m):
        if isinstance(m, nn.Linear):
            std = 0.02 * self.residual_init_scale if getattr(m, "_residual_proj", False) else 0.02
            nn.init.normal_(m.weight, mean=0, std=std)
        elif isinstance(m, nn.Embedding):
            nn.init.normal_(m.weight, mean=0, std=0.02)

    def forward(self, input_ids, targets=None):
        if input_ids.dim() != 2 or input_ids.shape[1] > self.cfg.block_size:
            raise ValueError("Input must be [B,T] with T<=block_size")
        x = self.drop(token_embedding(input_ids, self.byte_emb))
        if self.blocks and not (self.cfg.grad_checkpointing and self.training) and self.norm_f._fusable(x):
            # the blocks' chain x = x + attn(norm1(x)); x = x + mlp(norm2(x)),
            # with every residual add fused into the norm that reads its sum
            # (the next block's norm1, or norm_f after the last block)
            h = self.blocks[0].norm1(x)
            for n, block in enumerate(self.blocks):
                x, h = block.norm2.add_and_norm(x, block.attn(h))
                nxt = self.blocks[n + 1].norm1 if n + 1 < len(self.blocks) else self.norm_f
                x, h = nxt.add_and_norm(x, block.mlp(h))
            logits = self.lm_head(h)
        else:
            for block in self.blocks:
                if self.cfg.grad_checkpointing and self.training:
                    x = torch.utils.checkpoint.checkpoint(block, x, use_reentrant=False)
                else:
                    x = block(x)
            logits = self.lm_head(self.norm_f(x))
        out = {"logits": logits}
        if targets is not None:
            V = self.cfg.vocab_size
            out["loss"] = F.cross_entropy(logits[:, :-1, :].reshape(-1, V), targets[:, 1:].reshape(-1),
                                          reduction="mean")
        return out

    def parameter_breakdown(self):
        return {"byte_embedding": _numel(self.byte_emb), "decoder_blocks": _numel(self.blocks),
                "continuum_head_gains": self.cfg.n_layers * self.cfg.n_heads,
                "final_norm": _numel(self.norm_f), "lm_head": _numel(self.lm_head)}


def _numel(module):
    return sum(p.numel() for p in module.parameters())


def count_parameters(model):
    """``{'total', 'trainable'}`` parameter counts (cuda/runtime.py:63-66)."""
    ps = list(model.parameters())
    return {"total": sum(p.numel() for p in ps),
            "trainable": sum(p.numel() for p in ps if p.requires_grad)}


def build_adamw(model, lr=3e-4, weight_decay=0.1, betas=(0.9, 0.95)):
    """AdamW over all parameters (cuda/runtime.py:87-88, defaults
    cuda/continuum_attention.py:960-966); the fused multi-tensor kernel when
    the device supports it."""
    params = list(model.parameters())
    on_gpu = all(p.is_cuda for p in params)
    try:
        return torch.optim.AdamW(params, lr=lr, weight_decay=weight_decay, betas=betas, fused=on_gpu)
    except (RuntimeError, TypeError):
        return torch.optim.AdamW(params, lr=lr, weight_decay=weight_decay, betas=betas)


def build_fused_adamw(model, lr=3e-4, weight_decay=0.1, betas=(0.9, 0.95)):
    """build_adamw's optimizer as the library's HIP AdamW (optim.FusedAdamW):
    the same update over the same parameters, with bf16 shadows of every
    nn.Linear weight so bf16 autocast runs no weight casts."""
    from .optim import FusedAdamW
    linears = [m for m in model.modules() if isinstance(m, nn.Linear)]
    return FusedAdamW(model.parameters(), lr=lr, betas=betas, weight_decay=weight_decay,
                      shadow_modules=linears)


def train_step(model, optimizer, batch, amp_dtype=torch.bfloat16, grad_clip=1.0):
    """One optimisation step on a ``[B, T]`` byte batch (next-byte targets from
    the batch itself, as cuda/continuum_attention.py:1205-1228): autocast
    forward + loss, backward, clip to ``grad_clip``, AdamW.  Returns the loss
    tensor (no host synchronisation)."""
    from .optim import FusedAdamW
    optimizer.zero_grad(set_to_none=True)
    amp = (torch.autocast(device_type="cuda", dtype=amp_dtype) if amp_dtype is not None
           else contextlib.nullcontext())
    with amp:
        loss = model(batch, targets=batch)["loss"]
    loss.backward()
    if isinstance(optimizer, FusedAdamW):
        optimizer.step(max_norm=grad_clip or 0.0)
        return loss.detach()
    if grad_clip and grad_clip > 0:
        if _fused_on_gpu(optimizer):
            # clip_grad_norm_'s scaling g * max_norm / (norm + 1e-6) (applied
            # when that factor is < 1) is handed to the fused AdamW kernel as
            # its gradient divisor (norm + 1e-6) / max_norm, instead of a
            # separate multiply pass over every gradient
            grads = [p.grad for g in optimizer.param_groups for p in g["params"] if p.grad is not None]
            norm = torch.linalg.vector_norm(torch.stack(torch._foreach_norm(grads, 2.0)), 2.0)
            optimizer.grad_scale = torch.clamp((norm + 1e-6) / grad_clip, min=1.0)
            try:
                optimizer.step()
            finally:
                del optimizer.grad_scale
            return loss.detach()
        torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
    optimizer.step()
    return loss.detach()


# HIP graph node type of a memset (hipGraphNodeTypeMemset) and of a child
# graph (hipGraphNodeTypeGraph), hip_runtime_api.h.
_HIP_NODE_MEMSET, _HIP_NODE_GRAPH = 2, 4


def _loaded_hip_runtime():
    """The HIP runtime library this process already has loaded (torch's), as
    a ctypes handle: its path is read from /proc/self/maps, so dlopen returns
    that same library rather than loading a second runtime by a fixed name."""
    import ctypes

    paths = []
    with open("/proc/self/maps") as maps:
        for line in maps:
            path = line.split(None, 5)[-1].strip() if line.count(" ") >= 5 else ""
            if "/libamdhip64.so" in path and path not in paths:
                paths.append(path)
    if not paths:
        raise RuntimeError("GraphedTrainStep: no HIP runtime (libamdhip64.so) is loaded in this "
                           "process; the captured graph cannot be inspected")
    if len(paths) > 1:
        raise RuntimeError(f"GraphedTrainStep: several HIP runtimes are loaded ({paths}); the "
                           "captured graph cannot be inspected reliably")
    return ctypes.CDLL(paths[0])


def _hip_graph_memset_nodes(graph: "torch.cuda.CUDAGraph") -> int:
    """Memset nodes of a captured HIP graph kept by torch (keep_graph=True),
    child graphs included.  Queried through the HIP runtime torch loaded."""
    import ctypes

    hip = _loaded_hip_runtime()
    get_nodes, get_type = hip.hipGraphGetNodes, hip.hipGraphNodeGetType
    get_child = hip.hipGraphChildGraphNodeGetGraph
    get_nodes.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                          ctypes.POINTER(ctypes.c_size_t)]
    get_type.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    get_child.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    for f in (get_nodes, get_type, get_child):
        f.restype = ctypes.c_int

    def check(err, what):
        if err != 0:
            raise RuntimeError(f"GraphedTrainStep: {what} failed (hipError {err})")

    def walk(g):
        n = ctypes.c_size_t(0)
        check(get_nodes(g, None, ctypes.byref(n)), "hipGraphGetNodes")
        nodes = (ctypes.c_void_p * max(n.value, 1))()
        check(get_nodes(g, nodes, ctypes.byref(n)), "hipGraphGetNodes")
        count = 0
        for k in range(n.value):
            t = ctypes.c_int(-1)
            check(get_type(nodes[k], ctypes.byref(t)), "hipGraphNodeGetType")
            if t.value == _HIP_NODE_MEMSET:
                count += 1
            elif t.value == _HIP_NODE_GRAPH:
                child = ctypes.c_void_p()
                check(get_child(nodes[k], ctypes.byref(child)), "hipGraphChildGraphNodeGetGraph")
                count += walk(child)
        return count

    return walk(ctypes.c_void_p(graph.raw_cuda_graph()))


class GraphedTrainStep:
    """A training step with the forward and backward captured once as a HIP
    graph and replayed each step (the optimizer step runs eagerly after the
    replay: optim.FusedAdamW's clip + update, or clip_grad_norm_ + a torch
    optimizer).

    ``batch`` is a tensor or a tuple of tensors fixing the input shapes; each
    call copies its inputs into the captured ones.  ``loss_fn(model, *inputs)``
    returns the scalar loss; by default the decoder's next-byte loss
    ``model(ids, targets=ids)["loss"]``.  Forward and backward are warmed up
    (twice, on a side stream, without an optimizer step: parameters are
    unchanged) before capture, as graph capture requires.  While the object
    is used the gradients are the captured graph's buffers: they are
    overwritten by each replay and must not be set to None (do not call
    ``zero_grad``).  A replay uses the parameters and the bf16 shadows as they
    are in memory, so in-place changes to them between steps are seen;
    hyper-parameters of the eager optimizer step can change freely.

    A capture that recorded any memset node is refused with ValueError before
    it is instantiated (nothing of it runs): graph replays on this platform do
    not reliably redo memset nodes.  Library code records them by itself
    (torch's sorting embedding backward, used above 3072 indices per lookup,
    through rocprim's partition; reductions over many blocks), so the check
    walks the captured graph rather than guessing which ops do."""

    def __init__(self, model, optimizer, batch, amp_dtype=torch.bfloat16, grad_clip=1.0, warmup=2,
                 loss_fn=None):
        from .optim import FusedAdamW
        self.model, self.optimizer = model, optimizer
        self.amp_dtype, self.grad_clip = amp_dtype, grad_clip
        self.fused = isinstance(optimizer, FusedAdamW)
        self.loss_fn = loss_fn or (lambda m, ids: m(ids, targets=ids)["loss"])
        inputs = batch if isinstance(batch, (tuple, list)) else (batch,)
        self.static_inputs = tuple(t.detach().clone() for t in inputs)
        dev = self.static_inputs[0].device
        _native.timing_enable(False)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(max(warmup, 1)):
                optimizer.zero_grad(set_to_none=True)
                self._forward_backward()
        torch.cuda.current_stream(dev).wait_stream(side)
        optimizer.zero_grad(set_to_none=True)
        self.graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.graph):
            self.static_loss = self._forward_backward()
        memsets = _hip_graph_memset_nodes(self.graph)
        if memsets:
            self.graph.reset()
            raise ValueError(
                f"GraphedTrainStep: the captured forward/backward holds {memsets} memset "
                "node(s), which graph replays do not reliably redo (e.g. torch's embedding "
                "backward above 3072 indices per lookup); train this model with the eager step")
        self.graph.instantiate()

    def _forward_backward(self):
        amp = (torch.autocast(device_type="cuda", dtype=self.amp_dtype, cache_enabled=False)
               if self.amp_dtype is not None else contextlib.nullcontext())
        with amp:
            loss = self.loss_fn(self.model, *self.static_inputs)
        loss.backward()
        return loss.detach()

    def __call__(self, *batch):
        """One training step on ``batch`` (the same tensors, in the same order,
        as at construction); returns the loss (a device tensor that the next
        call overwrites)."""
        for dst, src in zip(self.static_inputs, batch):
            dst.copy_(src)
        self.graph.replay()
        if self.fused:
            self.optimizer.step(max_norm=self.grad_clip or 0.0)
        else:
            if self.grad_clip and self.grad_clip > 0:
                torch.nn.utils.clip_grad_norm_(self.model.parameters(), self.grad_clip)
            self.optimizer.step()
        return self.static_loss


def _fused_on_gpu(optimizer):
    """A fused torch AdamW/Adam whose parameters are all on the GPU (its
    kernel divides every gradient by ``optimizer.grad_scale`` when set)."""
    if not isinstance(optimizer, (torch.optim.AdamW, torch.optim.Adam)):
        return False
    return all(g.get("fused") for g in optimizer.param_groups) and all(
        p.is_cuda for g in optimizer.param_groups for p in g["params"])

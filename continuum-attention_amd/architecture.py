"""Small-variant caller of the CA operator: ``CausalAttention`` and ``TinyLM``.

Counterpart of the reference's architecture.py:108-245 (the TinyStories
backbone: variants A/B/F/G are ordinary causal softmax, P/R/S/H exact
continuous memory).  Module names, parameter shapes, initialisation and
state-dict keys are the reference's, so its checkpoints load unchanged and the
parameter budgets agree (5,008,640 / 5,008,664 at seq_len 192, test_acma.py:
21-26; 5,090,560 / 5,090,584 at 512, test_hp_only.py:13-23).

The weight-level functions of the reference module are here too:
``segment_integral_coefficients(delta) -> (L, mu)`` (architecture.py:32-62)
and ``continuous_attention_weights(logits)`` (architecture.py:65-105), so the
reference's tests import them from this module unchanged.

Backends for the continuous variants on GPU tensors (CPU tensors run the
operator's and the weights' CPU path, as the reference's modules do):

* ``'hip'``: the fused operator ``continuum_attention`` (no ``[T, T]`` tensor);
  the variant's q scaling (``1/tau`` or ``exp(log_qk_gain)``) is applied to q
  before the call and the operator gets ``log_gain = 0``, so its own scale is
  the reference's ``1/sqrt(D)`` (architecture.py:134-146).
* ``'hip_weights'``: materialised logits -> ``continuous_attention_weights``
  (HIP row kernels) -> ``W @ v``, the reference backend's structure
  (architecture.py:146-177).
* The reference's own backend names are accepted for drop-in use:
  ``'reference'`` and ``'mixed'``, and the Metal ones ``'metal_weights'``,
  ``'metal_analytic'`` and ``'metal_long'``, map to ``'hip_weights'``
  (identical weights); ``'metal_direct'`` maps to ``'hip'``.

The softmax variants use torch's softmax / SDPA exactly as the reference does
(architecture.py:157-161); they are not part of the CA operator.
"""
from __future__ import annotations

import math

import torch
from torch import nn
from torch.nn import functional as F

from . import _native
from .decoder import RMSNorm as _DecoderRMSNorm
from .decoder import token_embedding as _token_embedding
from .decoder import rope_continuum_attention
from .ops import SUPPORTED_HEAD_DIMS, continuum_attention
from .cpu import _C_J0, _C_RIGHT, _SERIES_BELOW, _series
from .weights import continuous_attention_weights

__all__ = ["segment_integral_coefficients", "continuous_attention_weights", "RMSNorm",
           "CausalAttention", "SwiGLU", "Block", "TinyLM", "parameters", "build_adamw",
           "build_fused_adamw", "train_step", "VARIANTS"]


def segment_integral_coefficients(delta):
    """``(L, mu)`` for segments with endpoint logits a, b and ``delta = b - a``
    (architecture.py:32-62): ``exp(max(a, b)) * L`` is the segment's mass,
    ``L = (1 - e^-|delta|) / |delta|`` = J0(-|delta|) (1 at 0), and
    ``mu = J1(delta) / J0(delta)`` is the share of the right endpoint (1/2 at
    0), with ``J_n(x) = int_0^1 u^n e^(x u) du``.  Below |delta| = 1 both are
    20-term power series (J0, J1 coefficients 1/(k+1)!, 1/(k!(k+2))), above it
    the closed forms; torch ops on any device, differentiable."""
    t = delta.abs()
    small = t < _SERIES_BELOW
    ts = torch.where(small, t, torch.zeros_like(t))
    tc = torch.where(small, torch.ones_like(t), t)
    L = torch.where(small, _series(-ts, _C_J0), -torch.expm1(-tc) / tc)
    ds = torch.where(small, delta, torch.zeros_like(delta))
    mu_series = _series(ds, _C_RIGHT) / _series(ds, _C_J0)
    mu_hi = 1.0 / (-torch.expm1(-tc)) - 1.0 / tc             # mu at +|delta|
    mu = torch.where(small, mu_series, torch.where(delta >= 0, mu_hi, 1.0 - mu_hi))
    return L, mu

VARIANTS = ("A", "B", "F", "G", "P", "R", "S", "H")
_BACKEND_MAP = {"hip": "hip", "hip_weights": "hip_weights", "reference": "hip_weights",
                "mixed": "hip_weights", "metal_weights": "hip_weights",
                "metal_analytic": "hip_weights", "metal_long": "hip_weights",
                "metal_direct": "hip"}


class RMSNorm(_DecoderRMSNorm):
    """x / rms(x) * weight, eps 1e-5 (architecture.py:21-29).  On fp32 GPU
    inputs one HIP pass each way (the decoder's fused RMSNorm kernels, also
    for the residual add that feeds it); otherwise, or with
    ``RMSNorm.fused = False``, the reference's composition."""

    def __init__(self, width, eps=1e-5):
        super().__init__(width, eps)

    def _composition(self, x):
        return x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + self.eps) * self.weight


class CausalAttention(nn.Module):
    """Multi-head causal attention with the reference's eight variants
    (architecture.py:108-177)."""

    def __init__(self, width, heads, seq_len, variant="B", backend="hip", fixed_tau=0.30):
        super().__init__()
        if variant not in VARIANTS:
            raise ValueError("variant must be A, B, F, G, P, R, S or H")
        if backend not in _BACKEND_MAP:
            raise ValueError("backend must be one of " + ", ".join(_BACKEND_MAP))
        if width % heads:
            raise ValueError("width must be divisible by heads")
        if fixed_tau <= 0:
            raise ValueError("fixed_tau must be > 0")
        self.variant = variant
        self.backend = backend
        self.path = _BACKEND_MAP[backend]
        self.heads = heads
        self.width = width
        self.head_dim = width // heads
        self.fixed_tau = float(fixed_tau)
        self.continuous = variant in ("P", "R", "S", "H")
        if variant in ("F", "G", "S", "H"):
            g0 = -math.log(0.30) if variant in ("G", "H") else 0.0
            self.log_qk_gain = nn.Parameter(torch.full((heads,), g0))
        self.qkv = nn.Linear(width, 3 * width, bias=False)
        self.out = nn.Linear(width, width, bias=False)
        self.register_buffer("causal_mask", torch.ones(seq_len, seq_len, dtype=torch.bool).tril(),
                             persistent=False)

    def _qkv(self, x):
        Bsz, T, _ = x.shape
        q, k, v = (t.view(Bsz, T, self.heads, self.head_dim).transpose(1, 2)
                   for t in self.qkv(x).chunk(3, dim=-1))
        if self.variant in ("B", "P"):
            q = q * (1.0 / self.fixed_tau)
        elif self.variant in ("F", "G", "S", "H"):
            q = q * self.log_qk_gain.exp().view(1, -1, 1, 1)
        return q, k, v

    def _logits(self, q, k):
        return (q @ k.transpose(-2, -1).contiguous()) * (self.head_dim ** -0.5)

    def _weights(self, q, k, v=None):
        logits = self._logits(q, k)
        if self.continuous:
            return continuous_attention_weights(logits)
        T = q.size(-2)
        return F.softmax(logits.masked_fill(~self.causal_mask[:T, :T], -torch.inf), dim=-1)

    def attention_weights(self, x):
        q, k, v = self._qkv(x)
        return self._weights(q, k, v)

    # fused HIP prologue/epilogue (qkv -> fp32 heads -> operator -> tokens) on
    # GPU tensors for the continuous variants on the 'hip' backend, with the
    # variant's q scale passed as the operator's log-gain; False runs the
    # reference's composition (same operator kernels)
    fused_prologue = True

    def _log_gain(self, device):
        if self.variant in ("F", "G", "S", "H"):
            return self.log_qk_gain
        g = math.log(1.0 / self.fixed_tau) if self.variant in ("B", "P") else 0.0
        # a constant: kept per (device, value), not rebuilt every step
        cache = self.__dict__.setdefault("_gain_cache", {})
        key = (device, self.heads, g)
        t = cache.get(key)
        if t is None:
            t = cache[key] = torch.full((self.heads,), g, device=device, dtype=torch.float32)
        return t

    def forward(self, x):
        Bsz, T, _ = x.shape
        if (self.fused_prologue and self.continuous and self.path == "hip" and x.is_cuda
                and self.head_dim in SUPPORTED_HEAD_DIMS and self.head_dim % 4 == 0):
            y = rope_continuum_attention(self.qkv(x), self._log_gain(x.device), None, self.heads)
            return self.out(y)
        q, k, v = self._qkv(x)
        if self.continuous and self.path == "hip":
            zero = torch.zeros(self.heads, device=q.device, dtype=torch.float32)
            y = continuum_attention(q, k, v, zero)
        elif not self.continuous and self.backend != "reference":
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True, dropout_p=0.0)
        else:
            y = self._weights(q, k, v) @ v
        return self.out(y.transpose(1, 2).reshape(Bsz, T, self.width))


class _SwiGLUFn(torch.autograd.Function):
    """silu(gate) * value over the halves of u = [gate | value] as one HIP
    pass each way (ca_swiglu_fwd_f32 / ca_swiglu_bwd_f32); the backward writes
    the gradient of u whole, so no concatenation of the halves' gradients."""

    @staticmethod
    def forward(ctx, u):
        lib = _native.load()
        H = u.shape[-1] // 2
        N = u.numel() // (2 * H)
        uc = u.detach()
        h = torch.empty(u.shape[:-1] + (H,), device=u.device, dtype=torch.float32)
        with _native.on_device(u.device):
            _native.check(lib.ca_swiglu_fwd_f32(uc.data_ptr(), h.data_ptr(), N, H,
                                                _native.stream_handle(u.device)))
        ctx.save_for_backward(uc)
        return h

    @staticmethod
    def backward(ctx, dh):
        if torch.is_grad_enabled():
            raise RuntimeError("the fused SwiGLU supports first-order gradients only")
        (uc,) = ctx.saved_tensors
        lib = _native.load()
        H = uc.shape[-1] // 2
        N = uc.numel() // (2 * H)
        g = dh.float().contiguous()
        if g.data_ptr() % 16:
            g = g.clone()
        du = torch.empty_like(uc)
        with _native.on_device(uc.device):
            _native.check(lib.ca_swiglu_bwd_f32(uc.data_ptr(), g.data_ptr(), du.data_ptr(), N, H,
                                                _native.stream_handle(uc.device)))
        return du


class SwiGLU(nn.Module):
    """SwiGLU MLP (architecture.py:180-188).  On fp32 GPU activations the
    gate runs as _SwiGLUFn; ``SwiGLU.fused = False`` restores the composition."""
    fused = True

    def __init__(self, width, hidden):
        super().__init__()
        self.gate_up = nn.Linear(width, 2 * hidden, bias=False)
        self.down = nn.Linear(hidden, width, bias=False)

    def forward(self, x):
        u = self.gate_up(x)
        if (self.fused and u.is_cuda and u.dtype == torch.float32 and u.is_contiguous()
                and u.shape[-1] % 8 == 0 and u.data_ptr() % 16 == 0 and u.numel() > 0):
            return self.down(_SwiGLUFn.apply(u))
        gate, value = u.chunk(2, dim=-1)
        return self.down(F.silu(gate) * value)


class Block(nn.Module):
    def __init__(self, width, hidden, heads, seq_len, variant, backend, fixed_tau):
        super().__init__()
        self.norm_attn = RMSNorm(width)
        self.attn = CausalAttention(width, heads, seq_len, variant, backend, fixed_tau)
        self.norm_mlp = RMSNorm(width)
        self.mlp = SwiGLU(width, hidden)

    def forward(self, x):
        x = x + self.attn(self.norm_attn(x))
        return x + self.mlp(self.norm_mlp(x))


class TinyLM(nn.Module):
    """Pre-norm byte LM with learned positions and a tied head
    (architecture.py:180-241).  ``layers`` defaults to the reference's six
    blocks ``b0 .. b5``; BASELINE's CA-P configuration uses four."""

    def __init__(self, variant="B", backend="hip", seq_len=192, width=256, hidden=720, heads=4,
                 fixed_tau=0.30, layers=6):
        super().__init__()
        if layers < 1:
            raise ValueError("layers must be >= 1")
        self.seq_len = seq_len
        self.variant = variant
        self.layers = layers
        self.tok_embed = nn.Embedding(256, width)
        self.pos_embed = nn.Embedding(seq_len, width)
        for i in range(layers):
            self.add_module(f"b{i}", Block(width, hidden, heads, seq_len, variant, backend, fixed_tau))
        self.final_norm = RMSNorm(width)
        self.lm_head = nn.Linear(width, 256, bias=False)
        self.lm_head.weight = self.tok_embed.weight
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, tokens):
        _, length = tokens.shape
        if length > self.seq_len:
            raise ValueError("Sequence exceeds model seq_len")
        pos = torch.arange(length, device=tokens.device)
        tok = _token_embedding(tokens, self.tok_embed)
        x = tok + self.pos_embed(pos)[None, :, :]
        blocks = [getattr(self, f"b{i}") for i in range(self.layers)]
        if self.final_norm._fusable(x):
            # the blocks' chain x = x + attn(norm_attn(x)); x = x + mlp(norm_mlp(x)),
            # with every residual add fused into the norm that reads its sum
            h = blocks[0].norm_attn(x)
            for n, block in enumerate(blocks):
                x, h = block.norm_mlp.add_and_norm(x, block.attn(h))
                nxt = blocks[n + 1].norm_attn if n + 1 < len(blocks) else self.final_norm
                x, h = nxt.add_and_norm(x, block.mlp(h))
            return self.lm_head(h)
        for block in blocks:
            x = block(x)
        return self.lm_head(self.final_norm(x))


def parameters(model):
    """Trainable parameter count (architecture.py:244-245)."""
    return sum(p.numel() for p in model.parameters() if p.requires_grad)


def build_adamw(model, lr=4e-4, weight_decay=0.1, geometry_lr_mult=8.0):
    """AdamW as the reference trains TinyLM (benchmark.py:189-201): learned
    gains get ``lr * geometry_lr_mult`` and no weight decay; betas (.9, .95).
    Uses the fused multi-tensor kernel on the GPU."""
    gains = [p for n, p in model.named_parameters() if n.endswith("log_qk_gain")]
    dense = [p for n, p in model.named_parameters() if not n.endswith("log_qk_gain")]
    groups = [{"params": dense, "lr": lr, "weight_decay": weight_decay}]
    if gains:
        groups.append({"params": gains, "lr": lr * geometry_lr_mult, "weight_decay": 0.0})
    fused = all(p.is_cuda for p in model.parameters())
    try:
        return torch.optim.AdamW(groups, betas=(0.9, 0.95), fused=fused)
    except (RuntimeError, TypeError):
        return torch.optim.AdamW(groups, betas=(0.9, 0.95))


def build_fused_adamw(model, lr=4e-4, weight_decay=0.1, geometry_lr_mult=8.0):
    """build_adamw's groups and hyper-parameters as the library's HIP AdamW
    (optim.FusedAdamW; TinyLM trains in fp32, so no bf16 weight shadows)."""
    from .optim import FusedAdamW
    gains = [p for n, p in model.named_parameters() if n.endswith("log_qk_gain")]
    dense = [p for n, p in model.named_parameters() if not n.endswith("log_qk_gain")]
    groups = [{"params": dense, "lr": lr, "weight_decay": weight_decay}]
    if gains:
        groups.append({"params": gains, "lr": lr * geometry_lr_mult, "weight_decay": 0.0})
    return FusedAdamW(groups, lr=lr, betas=(0.9, 0.95), weight_decay=weight_decay)


def train_step(model, optimizer, x, target, grad_clip=1.0):
    """One TinyLM step (benchmark.py:207-214): cross-entropy of the byte
    logits, backward, clip to ``grad_clip``, AdamW.  Returns the loss tensor."""
    from .optim import FusedAdamW
    logits = model(x)
    loss = F.cross_entropy(logits.reshape(-1, 256), target.reshape(-1))
    optimizer.zero_grad(set_to_none=True)
    loss.backward()
    if isinstance(optimizer, FusedAdamW):
        optimizer.step(max_norm=grad_clip or 0.0)
        return loss.detach()
    torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
    optimizer.step()
    return loss.detach()

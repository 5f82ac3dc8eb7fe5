"""AdamW with gradient clipping for the decoders' training steps, in HIP.

The reference trains with ``torch.optim.AdamW`` (cuda/runtime.py:87-88) after
``torch.nn.utils.clip_grad_norm_`` (cuda/continuum_attention.py:1205-1228),
under bf16/fp16 autocast.  ``FusedAdamW`` computes the same step with the
library's kernels (``ca_grad_clip_coef``, ``ca_adamw_step``):

* one pass for the global gradient norm and the clip coefficient (kept on the
  device, no host synchronisation) and one pass for the AdamW update of every
  tensor, in place of torch's per-tensor norms, the clip multiply and the
  optimizer kernels;
* ``nn.Linear`` weights get a bf16 *shadow*: a copy rounded to nearest even,
  exactly what bf16 autocast casts the weight to before each matmul.  Under
  bf16 autocast the layer multiplies by the shadow, so the forward runs no
  cast, the weight gradient stays in bf16 (the value autocast's cast backward
  would have upcast), and the update rewrites the shadow from the new fp32
  weight.  Outside bf16 autocast the layer uses its fp32 weight and the step
  reads the fp32 gradient.

The fp32 weights stay the parameters (state dicts are unchanged); a shadow is
recopied whenever its weight's version counter shows a change made outside
the optimizer (``load_state_dict``, in-place edits).  Gradients of shadowed
weights are collected by the optimizer, not left on the weight's ``.grad``:
a hook takes each backward's bf16 gradient off the shadow as soon as autograd
has stored it.  One backward per step keeps that bf16 tensor (the value
autocast's cast backward would upcast); gradient accumulation over several
backwards (the reference's ``grad_accum`` micro-steps,
cuda/continuum_attention.py:1194-1207) sums them in an fp32 buffer, as torch
sums upcast gradients into an fp32 ``.grad``, never rounding the running sum
to bf16.  ``FusedAdamW.grads()`` lists the gradient each tensor's step uses.
The update is torch's AdamW formula in fp32 (one global step count: every
parameter is expected to receive a gradient each step, as in the decoders).
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native


class _OptTensor(ctypes.Structure):
    """``ca_opt_tensor`` of the C ABI."""
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("exp_avg", ctypes.c_void_p),
                ("exp_avg_sq", ctypes.c_void_p), ("shadow", ctypes.c_void_p), ("numel", ctypes.c_longlong),
                ("grad_dtype", ctypes.c_int), ("reserved", ctypes.c_int)]


class ShadowLinear(nn.Linear):
    """nn.Linear whose bf16-autocast forward multiplies by a bf16 copy of the
    weight kept by FusedAdamW (same parameters and state-dict keys)."""

    def forward(self, x):
        sh = getattr(self, "_ca_shadow", None)
        if (sh is not None and x.is_cuda and torch.is_autocast_enabled("cuda")
                and torch.get_autocast_dtype("cuda") == torch.bfloat16):
            if self._ca_shadow_version != self.weight._version:
                # the fp32 weight was changed outside the optimizer
                with torch.no_grad():
                    sh.copy_(self.weight)
                self._ca_shadow_version = self.weight._version
            return F.linear(x, sh, self.bias)
        return F.linear(x, self.weight, self.bias)


def _aligned16(t):
    return t.data_ptr() % 16 == 0


class FusedAdamW(torch.optim.Optimizer):
    """torch.optim.AdamW + clip_grad_norm_ in HIP kernels (see the module
    docstring).  ``params`` are parameters or torch-style parameter groups
    (dicts with ``params`` and optional ``lr`` / ``weight_decay``);
    ``shadow_modules`` are the nn.Linear modules whose weights get bf16
    shadows (they become ShadowLinear).  A torch Optimizer, so torch's LR
    schedulers drive ``param_groups[i]["lr"]`` as usual."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2,
                 shadow_modules=()):
        super().__init__(params, {"lr": lr, "betas": tuple(betas), "eps": eps,
                                  "weight_decay": weight_decay})
        self.lib = _native.load()
        self.step_count = 0
        self.chunk = int(self.lib.ca_opt_chunk_elems())
        self.shadow = {}
        for mod in shadow_modules:
            if type(mod) is not nn.Linear and not isinstance(mod, ShadowLinear):
                raise TypeError("shadow_modules must be nn.Linear modules")
            w = mod.weight
            sh = torch.empty(w.shape, device=w.device, dtype=torch.bfloat16)
            with torch.no_grad():
                sh.copy_(w)
            sh.requires_grad_(True)
            mod.__class__ = ShadowLinear
            mod._ca_shadow = sh
            mod._ca_shadow_version = w._version
            self.shadow[id(w)] = sh
            sh.register_post_accumulate_grad_hook(self._collect_shadow_grad)
        self._shadow_grads = {}  # id(shadow) -> bf16 gradient (one backward) or fp32 sum
        self._groups = []
        devices = {p.device for group in self.param_groups for p in group["params"]}
        if len(devices) != 1:
            raise ValueError("FusedAdamW: all parameters must be on one GPU")
        for group in self.param_groups:
            tensors = list(group["params"])
            for p in tensors:
                if not (p.is_cuda and p.dtype == torch.float32 and p.is_contiguous() and _aligned16(p)):
                    raise ValueError("FusedAdamW: parameters must be contiguous fp32 GPU tensors")
                self.state[p] = {"exp_avg": torch.zeros_like(p), "exp_avg_sq": torch.zeros_like(p)}
            chunks = []
            for ti, p in enumerate(tensors):
                for c in range((p.numel() + self.chunk - 1) // self.chunk):
                    chunks.extend((ti, c))
            dev = tensors[0].device if tensors else None
            self._groups.append({
                "tensors": tensors,
                "chunks": torch.tensor(chunks, dtype=torch.int32, device=dev) if tensors else None,
                "nchunks": len(chunks) // 2,
                "table": torch.empty(len(tensors) * ctypes.sizeof(_OptTensor), dtype=torch.uint8,
                                     device=dev) if tensors else None,
            })
        nchunks = max(g["nchunks"] for g in self._groups)
        dev = next(g["tensors"][0].device for g in self._groups if g["tensors"])
        self._partial = torch.empty(max(nchunks, 1), device=dev, dtype=torch.float32)
        self._norm = torch.empty(1, device=dev, dtype=torch.float32)
        self._coef = torch.empty(1, device=dev, dtype=torch.float32)

    # ---- gradients -----------------------------------------------------
    def _collect_shadow_grad(self, sh):
        """Post-accumulate hook of a shadow: moves the gradient autograd just
        stored on it into the optimizer.  The shadow's .grad is then empty
        again, so the next backward stores its gradient afresh instead of
        adding it to a bf16 sum; from the second backward on the gradients
        are summed in fp32."""
        g = sh.grad
        if g is None:
            return
        sh.grad = None
        key = id(sh)
        prev = self._shadow_grads.get(key)
        if prev is None:
            self._shadow_grads[key] = g
        elif prev.dtype == torch.float32:
            prev.add_(g)
        else:
            self._shadow_grads[key] = prev.float().add_(g)

    def _grad_of(self, p):
        sh = self.shadow.get(id(p))
        gs = None
        if sh is not None:
            gs = self._shadow_grads.get(id(sh))
            if sh.grad is not None:  # stored without the hook (e.g. assigned by hand)
                gs = sh.grad if gs is None else gs.float().add_(sh.grad)
        if gs is not None and p.grad is not None:
            raise RuntimeError("FusedAdamW: a weight has both a bf16-shadow and an fp32 gradient")
        return gs if gs is not None else p.grad

    def grads(self):
        """The gradient each parameter's step uses (None when it has none)."""
        return [self._grad_of(p) for g in self._groups for p in g["tensors"]]

    def zero_grad(self, set_to_none: bool = True):
        # collected shadow gradients are dropped either way: the next backward
        # starts a new sum, which equals adding to zeros
        self._shadow_grads.clear()
        for g in self._groups:
            for p in g["tensors"]:
                for t in (p, self.shadow.get(id(p))):
                    if t is not None and t.grad is not None:
                        if set_to_none:
                            t.grad = None
                        else:
                            t.grad.zero_()

    # ---- tables ----------------------------------------------------------
    def _fill_table(self, g):
        n = len(g["tensors"])
        arr = (_OptTensor * n)()
        for i, p in enumerate(g["tensors"]):
            grad = self._grad_of(p)
            st = self.state[p]
            sh = self.shadow.get(id(p))
            if grad is not None:
                if grad.shape != p.shape or not grad.is_contiguous() or not _aligned16(grad):
                    raise ValueError("FusedAdamW: gradients must be contiguous, 16-byte aligned, "
                                     "and shaped like their parameters")
                if grad.dtype not in (torch.float32, torch.bfloat16):
                    raise ValueError(f"FusedAdamW: unsupported gradient dtype {grad.dtype}")
            arr[i].param = p.data_ptr()
            arr[i].grad = grad.data_ptr() if grad is not None else None
            arr[i].exp_avg = st["exp_avg"].data_ptr()
            arr[i].exp_avg_sq = st["exp_avg_sq"].data_ptr()
            arr[i].shadow = sh.data_ptr() if sh is not None else None
            # a tensor without a gradient is skipped (no chunk of it does work)
            arr[i].numel = p.numel() if grad is not None else 0
            arr[i].grad_dtype = _native.CA_DTYPE_F32 if (grad is None or grad.dtype == torch.float32) \
                else _native.CA_DTYPE_BF16
        host = torch.empty(ctypes.sizeof(arr), dtype=torch.uint8, pin_memory=True)
        ctypes.memmove(host.data_ptr(), ctypes.addressof(arr), ctypes.sizeof(arr))
        g["table"].copy_(host, non_blocking=True)

    # ---- step ------------------------------------------------------------
    @torch.no_grad()
    def step(self, closure=None, max_norm=0.0):
        """One AdamW step; with max_norm > 0 the gradients are first scaled by
        clip_grad_norm_'s factor min(1, max_norm / (norm + 1e-6)).  Returns the
        total gradient norm (a device tensor) when clipping."""
        if closure is not None:
            with torch.enable_grad():
                closure()
        self.step_count += 1
        groups = [g for g in self._groups if g["tensors"]]
        stream = _native.stream_handle(groups[0]["tensors"][0].device)
        for g in groups:
            self._fill_table(g)
        coef = None
        if max_norm and max_norm > 0:
            if len(groups) == 1:
                g = groups[0]
                _native.check(self.lib.ca_grad_clip_coef(g["table"].data_ptr(), len(g["tensors"]),
                                                         g["chunks"].data_ptr(), g["nchunks"],
                                                         self._partial.data_ptr(), float(max_norm),
                                                         self._norm.data_ptr(), self._coef.data_ptr(),
                                                         stream))
            else:
                # several groups: one norm over all of them
                sq = []
                for g in groups:
                    part = torch.empty(1, device=self._norm.device, dtype=torch.float32)
                    _native.check(self.lib.ca_grad_clip_coef(g["table"].data_ptr(), len(g["tensors"]),
                                                             g["chunks"].data_ptr(), g["nchunks"],
                                                             self._partial.data_ptr(), 0.0,
                                                             part.data_ptr(), self._coef.data_ptr(),
                                                             stream))
                    sq.append(part.square())
                total = torch.stack(sq).sum().sqrt()
                self._norm.copy_(total.reshape(1))
                self._coef.copy_(torch.clamp(max_norm / (total + 1e-6), max=1.0).reshape(1))
            coef = self._coef
        for group, g in zip(self.param_groups, self._groups):
            if not g["tensors"]:
                continue
            b1, b2 = group["betas"]
            _native.check(self.lib.ca_adamw_step(g["table"].data_ptr(), len(g["tensors"]),
                                                 g["chunks"].data_ptr(), g["nchunks"],
                                                 coef.data_ptr() if coef is not None else None,
                                                 float(group["lr"]), float(b1), float(b2),
                                                 float(group["eps"]), float(group["weight_decay"]),
                                                 self.step_count, stream))
        return self._norm if coef is not None else None

    # ---- checkpoints (own format: the step count is global) ----------------
    def state_dict(self):
        return {"step": self.step_count,
                "state": [{"exp_avg": self.state[p]["exp_avg"].clone(),
                           "exp_avg_sq": self.state[p]["exp_avg_sq"].clone()}
                          for g in self._groups for p in g["tensors"]],
                "param_groups": [{k: v for k, v in g.items() if k != "params"} for g in self.param_groups]}

    def load_state_dict(self, sd):
        flat = [p for g in self._groups for p in g["tensors"]]
        if len(sd["state"]) != len(flat):
            raise ValueError("FusedAdamW.load_state_dict: parameter count differs")
        self.step_count = int(sd["step"])
        for p, st in zip(flat, sd["state"]):
            self.state[p]["exp_avg"].copy_(st["exp_avg"])
            self.state[p]["exp_avg_sq"].copy_(st["exp_avg_sq"])
        for g, gs in zip(self.param_groups, sd["param_groups"]):
            g.update({k: v for k, v in gs.items() if k in ("lr", "betas", "eps", "weight_decay")})

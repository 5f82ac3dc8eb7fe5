"""ctypes binding of libca_hip.so (the C ABI declared in include/continuum_attention_amd.h).

This replaces the reference's JIT-built pybind extension
(``_ca_cuda_extension``, cuda/continuum_attention.py:608-620).  The library is
built in-tree by ``build.py`` (``__graft_entry__.build()``); loading fails
loudly when it is missing -- there is no fallback path.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import torch  # must be imported first: the library binds torch's HIP runtime

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libca_hip.so")

CA_OK = 0
CA_ERR_INVALID = 1
CA_ERR_UNSUPPORTED = 2
CA_ERR_WORKSPACE = 3
CA_ERR_HIP = 4
CA_DTYPE_F32, CA_DTYPE_BF16, CA_DTYPE_F16 = 0, 1, 2
ABI_VERSION = 1

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); one entry per declaration in the public header
SIGNATURES = {
    "ca_abi_version": (_i, []),
    "ca_last_error": (ctypes.c_char_p, []),
    "ca_set_workspace_cap": (_i, [_sz]),
    "ca_workspace_cap": (_sz, []),
    "ca_fwd_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ca_bwd_qkv_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ca_fwd_qkv_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ca_fwd_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "ca_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ca_bwd_f32": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                        _i, _i, _i, _i, _vp]),
    "ca_bwd_f32_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _i, _i, _i, _i, _vp]),
    "ca_weights_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ca_weights_bwd_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ca_fwd_qkv": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "ca_bwd_qkv": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "ca_rmsnorm_fwd": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp]),
    "ca_rmsnorm_bwd_workspace_bytes": (_sz, [_i, _i]),
    "ca_rmsnorm_bwd": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _vp]),
    "ca_add_rmsnorm_fwd": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp]),
    "ca_add_rmsnorm_bwd": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _sz, _i, _i,
                                _vp]),
    "ca_opt_chunk_elems": (_i, []),
    "ca_grad_clip_coef": (_i, [_vp, _i, _vp, _i, _vp, ctypes.c_float, _vp, _vp, _vp]),
    "ca_adamw_step": (_i, [_vp, _i, _vp, _i, _vp, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                           ctypes.c_float, ctypes.c_float, _i, _vp]),
    "ca_bf16_shadow": (_i, [_vp, _i, _vp, _i, _vp]),
    "ca_swiglu_fwd_f32": (_i, [_vp, _vp, _i, _i, _vp]),
    "ca_swiglu_bwd_f32": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "ca_timing_enable": (_i, [_i]),
    "ca_timing_read": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i), _i]),
    "ca_debug_set_splits": (_i, [_i, _i, _i]),
}

KERNEL_NAMES = ("ca_fwd", "ca_fwd_combine", "ca_bwd_prep", "ca_bwd_dkdv", "ca_bwd_dq",
                "ca_bwd_merge", "ca_weights", "ca_weights_bwd", "ca_rmsnorm_fwd",
                "ca_rmsnorm_bwd", "ca_swiglu_fwd", "ca_swiglu_bwd")

_lib = None


class CAError(RuntimeError):
    """Error status returned by the native library."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(dev: torch.device) -> int:
    """The current HIP stream of ``dev`` as the handle the C ABI takes: the
    value of ``torch.cuda.current_stream(dev).cuda_stream``, read without
    building a Stream object (that costs microseconds per launch)."""
    if _raw_stream is not None and dev.index is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def on_device(dev: torch.device):
    """``torch.cuda.device(dev)``, or a no-op context when ``dev`` is already
    the current device (the library launches on the current device)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def load() -> ctypes.CDLL:
    """Loads and type-annotates libca_hip.so (once)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"continuum-attention_amd: native library {LIB_PATH} is not built; run "
            "`python continuum-attention_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.ca_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libca_hip.so ABI version {ver}, expected {ABI_VERSION}")
    cap_mb = os.environ.get("CA_WORKSPACE_CAP_MB")
    if cap_mb is not None:
        # the workspace bound (MiB, 0 = none) in place of the library's 1 GiB
        lib.ca_set_workspace_cap(int(float(cap_mb) * (1 << 20)))
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Raises on a non-zero status: ValueError for argument errors, else RuntimeError."""
    if rc == CA_OK:
        return
    msg = load().ca_last_error().decode(errors="replace")
    if rc in (CA_ERR_INVALID, CA_ERR_UNSUPPORTED):
        raise ValueError(f"continuum-attention_amd: {msg}")
    raise CAError(rc, f"continuum-attention_amd: {msg}")


def timing_enable(on: bool = True) -> None:
    check(load().ca_timing_enable(1 if on else 0))


def timing_read() -> dict:
    """Per-kernel ``{name: (total_ms, launches)}`` since the last read/enable."""
    n = len(KERNEL_NAMES)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int * n)()
    check(load().ca_timing_read(ms, cnt, n))
    return {KERNEL_NAMES[i]: (ms[i], cnt[i]) for i in range(n)}

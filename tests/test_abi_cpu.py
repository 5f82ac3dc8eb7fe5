"""CPU-only checks of the drop-in boundary: the C-ABI library loads, exports
every symbol its header declares, validates arguments before touching the GPU,
and the Python operator keeps the reference's error contract.

No test here launches a kernel (this container has no GPU).
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "continuum_attention_amd.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ca_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = header_functions()
    for n in ("ca_fwd_f32", "ca_bwd_f32", "ca_fwd_workspace_bytes", "ca_bwd_workspace_bytes",
              "ca_last_error", "ca_abi_version"):
        assert n in names


def test_library_exports_every_header_symbol(ca):
    lib = ca.native.load()
    for name in header_functions():
        assert hasattr(lib, name), name
        assert name in ca.native.SIGNATURES, name
    assert lib.ca_abi_version() == ca.native.ABI_VERSION


def test_workspace_sizes(ca):
    lib = ca.native.load()
    # every 128-query group fits one forward split (<= 12 key tiles) and the
    # grid fills the device: no partials
    assert lib.ca_fwd_workspace_bytes(16, 32, 384, 64) == 0
    assert lib.ca_fwd_workspace_bytes(2, 16, 512, 64) > 0
    # a small grid takes shorter splits (4 tiles: 3 splits of the 12-tile group)
    assert lib.ca_fwd_workspace_bytes(2, 16, 384, 64) == 2 * 16 * 3 * 384 * 66 * 4
    assert lib.ca_fwd_workspace_bytes(2, 16, 2048, 64) > 0
    nqt = 2048 // 32
    ds_bytes = 2 * 16 * (nqt * (nqt + 1) // 2) * 1024 * 4
    assert lib.ca_bwd_workspace_bytes(2, 16, 2048, 64) >= ds_bytes + 2 * 16 * 2048 * 4
    assert lib.ca_bwd_workspace_bytes(0, 1, 1, 64) == 0


@pytest.mark.parametrize("T,tiles", [(2048, 12), (3000, 16), (4096, 16), (8192, 24), (16384, 32)])
def test_forward_split_length_follows_the_row_length(ca, T, tiles):
    """The forward's split length (seen through its partials' size: one
    [T][D + 2] fp32 block per slice and split of the longest row) is 12 tiles
    up to T = 2048 and 12 sqrt(T / 2048), to a multiple of 4, beyond."""
    lib = ca.native.load()
    prev = lib.ca_workspace_cap()
    ca.ops.set_workspace_cap(0)
    try:
        splits = -(-min(4 * ((T + 127) // 128), (T + 31) // 32) // tiles)
        assert lib.ca_fwd_workspace_bytes(1, 16, T, 64) == 16 * splits * T * 66 * 4
    finally:
        ca.ops.set_workspace_cap(prev)


@pytest.mark.parametrize("shape,code", [((0, 1, 8, 64), 1), ((1, 1, 0, 64), 1),
                                        ((1, 1, 8, 256), 2), ((1, 1, 8, 24), 2)])
def test_argument_errors_before_any_launch(ca, shape, code):
    lib = ca.native.load()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    rc = lib.ca_fwd_f32(p, p, p, p, p, p, None, 0, *shape, None)
    assert rc == code
    assert lib.ca_last_error().decode()
    rc = lib.ca_bwd_f32(p, p, p, p, p, p, p, p, p, p, p, None, 0, *shape, None)
    assert rc == code


def test_null_misaligned_and_workspace_errors(ca):
    lib = ca.native.load()
    p = ctypes.c_void_p(4096)
    assert lib.ca_fwd_f32(None, p, p, p, p, p, None, 0, 1, 1, 8, 64, None) == 1
    assert b"null" in lib.ca_last_error()
    odd = ctypes.c_void_p(4100)
    assert lib.ca_fwd_f32(odd, p, p, p, p, p, None, 0, 1, 1, 8, 64, None) == 1
    assert b"aligned" in lib.ca_last_error()
    # a smaller workspace lengthens the forward's splits instead of failing;
    # with a forced split the partials cannot shrink, so too little is refused
    # before any launch
    assert lib.ca_debug_set_splits(1, 0, 0) == 0
    try:
        need = lib.ca_fwd_workspace_bytes(1, 1, 4096, 64)
        assert need > 0
        assert lib.ca_fwd_f32(p, p, p, p, p, p, p, need - 1, 1, 1, 4096, 64, None) == 3
        assert b"workspace" in lib.ca_last_error()
    finally:
        assert lib.ca_debug_set_splits(0, 0, 0) == 0
    assert lib.ca_bwd_f32(p, p, p, p, p, p, p, p, p, p, p, p, 16, 1, 1, 64, 64, None) == 3


def test_python_errors_follow_reference_contract(ca, monkeypatch):
    q = torch.zeros(1, 1, 4, 16)
    with pytest.raises(ValueError, match="must share dtype"):
        ca.continuum_attention(q, q.double(), q, torch.zeros(1))
    monkeypatch.setenv("CA_CUDA_MODE", "bogus")
    with pytest.raises(ValueError, match="CA_CUDA_MODE"):
        ca.continuum_attention(q, q, q, torch.zeros(1))
    # CPU tensors: the reference's CPU-side errors (cuda/continuum_attention.py:662-665)
    for mode in ("prefix_v5", "prefix_v6"):
        monkeypatch.setenv("CA_CUDA_MODE", mode)
        with pytest.raises(ValueError, match="v5/v6 paths require CUDA FP16"):
            ca.continuum_attention(q, q, q, torch.zeros(1))
    monkeypatch.setenv("CA_CUDA_MODE", "fused")
    with pytest.raises(ValueError, match="fused forward supports T<=2048"):
        z = torch.zeros(1, 1, 2049, 16)
        ca.continuum_attention(z, z, z, torch.zeros(1))
    with pytest.raises(ValueError, match="fused forward supports"):
        ca.continuum_attention(q.double(), q.double(), q.double(), torch.zeros(1))
    monkeypatch.setenv("CA_CUDA_MODE", "prefix")
    with pytest.raises(ValueError, match="query_tile"):
        ca.continuum_attention(q, q, q, torch.zeros(1), 0)
    # other devices are neither the HIP nor the CPU path
    m = torch.zeros(1, 1, 4, 16, device="meta")
    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        ca.continuum_attention(m, m, m, torch.zeros(1, device="meta"))


def test_package_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "continuum-attention_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                src = open(os.path.join(dirpath, f)).read()
                src = re.sub(r'""".*?"""', "", src, flags=re.S)
                src = re.sub(r"#.*|//.*", "", src)
                assert "oracle" not in src, f


@pytest.mark.parametrize("BH,Q,K,start", [(0, 4, 8, 0), (1, 0, 8, 0), (1, 4, 0, 0), (1, 4, 8, -1),
                                          (1, 4, 8, 5), (2, 9, 8, 0)])
def test_weights_argument_errors_before_any_launch(ca, BH, Q, K, start):
    """start + Q > K (a query without its keys), empty or negative shapes."""
    lib = ca.native.load()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert lib.ca_weights_f32(p, p, p, BH, Q, K, start, None) == 1
    assert lib.ca_last_error().decode().startswith("ca_weights_f32")
    assert lib.ca_weights_bwd_f32(p, p, p, p, BH, Q, K, start, None) == 1
    assert lib.ca_weights_f32(None, p, p, 1, 4, 8, 0, None) == 1
    assert lib.ca_weights_bwd_f32(p, None, p, p, 1, 4, 8, 0, None) == 1


def test_opt_tensor_layout_matches_header(tmp_path):
    """The ctypes mirror of ca_opt_tensor (optim._OptTensor) has the C
    header's size and field offsets (compiled with gcc from the header)."""
    import ctypes
    import importlib
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = tmp_path / "layout.c"
    fields = ["param", "grad", "exp_avg", "exp_avg_sq", "shadow", "numel", "grad_dtype", "reserved"]
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "continuum_attention_amd.h"\n'
                   'int main(void) { printf("%zu", sizeof(ca_opt_tensor));'
                   + "".join(f' printf(" %zu", offsetof(ca_opt_tensor, {f}));' for f in fields)
                   + ' return 0; }\n')
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", os.path.join(root, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    opt = importlib.import_module("continuum-attention_amd.optim")
    want = [ctypes.sizeof(opt._OptTensor)] + [getattr(opt._OptTensor, f).offset for f in fields]
    assert got == want


@pytest.mark.parametrize("N,H", [(0, 8), (4, 0), (4, 6), (-1, 8)])
def test_swiglu_argument_errors_before_any_launch(ca, N, H):
    """ca_swiglu_fwd_f32 / ca_swiglu_bwd_f32 reject empty or negative shapes
    and H not a multiple of 4, before touching the pointers."""
    lib = ca.native.load()
    p = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert lib.ca_swiglu_fwd_f32(p, p, N, H, None) == 1
    assert lib.ca_last_error().decode().startswith("ca_swiglu_fwd_f32")
    assert lib.ca_swiglu_bwd_f32(p, p, p, N, H, None) == 1


def test_swiglu_null_and_misaligned_pointers(ca):
    lib = ca.native.load()
    p, odd = ctypes.c_void_p(4096), ctypes.c_void_p(4100)
    assert lib.ca_swiglu_fwd_f32(None, p, 4, 8, None) == 1
    assert b"null" in lib.ca_last_error()
    assert lib.ca_swiglu_bwd_f32(p, odd, p, 4, 8, None) == 1
    assert b"aligned" in lib.ca_last_error()


def test_noalloc_backward_checks_before_any_launch(ca):
    """ca_bwd_f32_noalloc validates the shape (B, H, T and D) before anything
    else, with no HIP call: non-positive sizes are CA_ERR_INVALID, head dims
    and sizes outside the kernels' range CA_ERR_UNSUPPORTED."""
    lib = ca.native.load()
    p = ctypes.c_void_p(16)
    assert lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 0, 16, 64, 64, None) == 1
    assert lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 1, 16, 64, -64, None) == 1
    assert b"positive" in lib.ca_last_error()
    assert lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 1, 16, 64, 0, None) == 1
    assert lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 1, 16, 64, 24, None) == 2
    assert lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 64, 16, 65536, 64, None) == 2
    assert b"2^31" in lib.ca_last_error()


def test_no_valid_shape_exceeds_the_noalloc_array(ca):
    """Head sets bound the backward's workspace by one head's 128-query group:
    at the largest T the kernels take (65536) that is about 32 MiB, so every
    shape check_shape accepts fits the static 512 MiB array."""
    lib = ca.native.load()
    prev = lib.ca_workspace_cap()
    try:
        ca.ops.set_workspace_cap(1)  # below any plan: the least workspace is reported
        least = lib.ca_bwd_workspace_bytes(1, 1, 65536, 128)
        assert least < 64 << 20
        scratch_mb = int(re.search(r"#define CA_NOALLOC_SCRATCH_MB (\d+)", open(HEADER).read()).group(1))
        assert least <= scratch_mb << 20
    finally:
        ca.ops.set_workspace_cap(prev)


def test_workspace_cap_bounds_the_sizes(ca):
    """The workspace bound: under the default 1 GiB cap the backward of a
    long sequence asks for at most the cap (it runs in passes), the forward
    for at most the cap (longer splits), and so do the token-major entry
    points (the backward then sums dK and dV over its passes in fp32 in the
    workspace); without a cap, the full sizes."""
    lib = ca.native.load()
    prev = lib.ca_workspace_cap()
    try:
        assert prev == 1 << 30
        assert lib.ca_bwd_workspace_bytes(1, 16, 32768, 64) <= 1 << 30
        assert lib.ca_fwd_workspace_bytes(1, 16, 32768, 64) <= 1 << 30
        assert lib.ca_bwd_qkv_workspace_bytes(1, 16, 32768, 64) <= 1 << 30
        assert lib.ca_fwd_qkv_workspace_bytes(1, 16, 32768, 64) <= 1 << 30
        small = lib.ca_bwd_workspace_bytes(2, 16, 2048, 64)
        # the token-major entry points add room for the keys rotated once
        # ([B*H][T][D], 4-byte elements, rounded up to 256 bytes)
        rot = 2 * 16 * 2048 * 64 * 4
        assert lib.ca_bwd_qkv_workspace_bytes(2, 16, 2048, 64) == small + rot  # fits: one pass
        # one CA-S layer (268 MiB) is one pass under the default cap
        assert lib.ca_bwd_qkv_workspace_bytes(1, 16, 2048, 64) == \
            lib.ca_bwd_workspace_bytes(1, 16, 2048, 64) + 16 * 2048 * 64 * 4
        assert lib.ca_fwd_qkv_workspace_bytes(2, 16, 2048, 64) == \
            rot + lib.ca_fwd_workspace_bytes(2, 16, 2048, 64)
        ca.ops.set_workspace_cap(0)
        full = lib.ca_bwd_qkv_workspace_bytes(1, 16, 32768, 64)
        assert full > 30 << 30
        assert lib.ca_bwd_workspace_bytes(1, 16, 32768, 64) == full - 16 * 32768 * 64 * 4
        assert lib.ca_fwd_workspace_bytes(1, 16, 32768, 64) > 1 << 30
        # the token-major backward of one CA-S layer at T = 16384 under 256 MiB:
        # its fp32 dK/dV sums (128 MiB for 16 heads) leave too little for one
        # group of every head, so it runs in sets of heads
        ca.ops.set_workspace_cap(256 << 20)
        assert lib.ca_bwd_qkv_workspace_bytes(1, 16, 16384, 64) <= 256 << 20
        assert lib.ca_bwd_workspace_bytes(1, 16, 16384, 64) <= 256 << 20
        ca.ops.set_workspace_cap(32 << 20)
        assert lib.ca_bwd_workspace_bytes(1, 2, 8192, 64) <= 32 << 20
        assert lib.ca_fwd_workspace_bytes(1, 2, 8192, 64) <= 32 << 20
        # below what one 128-query group needs, the minimum is reported
        ca.ops.set_workspace_cap(1 << 20)
        least = lib.ca_bwd_workspace_bytes(1, 2, 8192, 64)
        assert 1 << 20 < least < 32 << 20
        assert lib.ca_fwd_workspace_bytes(1, 2, 8192, 64) == 0  # unsplit forward
    finally:
        ca.ops.set_workspace_cap(prev)


def test_workspace_size_caches_follow_the_cap_and_splits(ca):
    # the Python side caches every workspace size; changing the cap or the
    # split override must drop all four caches
    ops = ca.ops
    shape = (1, 2, 8192, 64)
    sizes = (ops._fwd_workspace_bytes, ops._bwd_workspace_bytes, ops._fwd_qkv_workspace_bytes,
             ops._bwd_qkv_workspace_bytes)
    prev = ops.workspace_cap()
    try:
        ops.set_workspace_cap(0)
        before = [f(*shape) for f in sizes]
        ops.set_workspace_cap(32 << 20)
        after = [f(*shape) for f in sizes]
        assert after[1] < before[1]  # passes over query ranges
        assert after[3] < before[3]  # the token-major backward too
        lib = ca.native.load()
        assert after == [lib.ca_fwd_workspace_bytes(*shape), lib.ca_bwd_workspace_bytes(*shape),
                         lib.ca_fwd_qkv_workspace_bytes(*shape), lib.ca_bwd_qkv_workspace_bytes(*shape)]
        ops.set_split_override(4, 0, 0)
        forced = [f(*shape) for f in sizes]
        assert forced[0] == lib.ca_fwd_workspace_bytes(*shape) != after[0]
        assert forced == [lib.ca_fwd_workspace_bytes(*shape), lib.ca_bwd_workspace_bytes(*shape),
                          lib.ca_fwd_qkv_workspace_bytes(*shape), lib.ca_bwd_qkv_workspace_bytes(*shape)]
    finally:
        ops.set_split_override(0, 0, 0)
        ops.set_workspace_cap(prev)

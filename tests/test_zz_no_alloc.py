"""The allocation-free backward ``ca_bwd_f32_noalloc`` (workspace in a static
device array) against ``ca_bwd_f32`` (caller-allocated workspace), both
through the C ABI: bit-for-bit equal gradients on two calls in a row, the
second on a smaller input (the array keeps the first call's contents), and a
clear CA_ERR_WORKSPACE for a shape beyond the array."""
import ctypes
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def noalloc_backward(ca, q, k, v, rho, out, stats, dy):
    lib = ca.native.load()
    B, H, T, D = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    dg = torch.empty(H, device=q.device)
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.ca_bwd_f32_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), rho.data_ptr(),
                                out.data_ptr(), stats.data_ptr(), dy.data_ptr(), dq.data_ptr(),
                                dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), B, H, T, D,
                                ca.native.stream_handle(q.device))
    ca.native.check(rc)
    torch.cuda.synchronize()
    return (dq, dk, dv, dg), free0 - torch.cuda.mem_get_info()[0]


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_backward_matches_workspace_backward(gpu_ca, order):
    ops = gpu_ca.ops
    for n, (shape, seed) in enumerate([((1, 16, 2048, 64), 1), ((2, 4, 300, 64), 2)]):
        say(f"[case] noalloc call {n + 1}: shape {shape}")
        g = torch.Generator().manual_seed(seed)
        q, k, v, dy = (torch.randn(shape, generator=g).cuda() for _ in range(4))
        rho = torch.linspace(-0.3, 0.3, shape[1]).cuda()
        out, stats = ops.ca_forward(q, k, v, rho)
        ref = ops.ca_backward(q, k, v, rho, out, stats, dy)
        got, grew = noalloc_backward(gpu_ca, q, k, v, rho, out, stats, dy)
        say(f"   free device memory dropped by {grew / 2**20:.1f} MiB during the call")
        for name, a, b in zip(("dq", "dk", "dv", "dlog_gain"), got, ref):
            assert torch.equal(a, b), name


def test_noalloc_backward_in_passes(gpu_ca):
    """A shape whose full backward workspace (3.1 GB) exceeds the 512 MiB
    array runs in passes over query ranges: bitwise equal to ca_bwd_f32
    given a workspace of the same size (the same pass plan)."""
    ops = gpu_ca.ops
    lib = gpu_ca.native.load()
    shape = (1, 16, 8192, 64)
    say(f"[case] noalloc in passes: shape {shape}")
    assert lib.ca_bwd_qkv_workspace_bytes(*shape) > 512 << 20
    g = torch.Generator().manual_seed(3)
    q, k, v, dy = (torch.randn(shape, generator=g).cuda() for _ in range(4))
    rho = torch.linspace(-0.2, 0.2, 16).cuda()
    out, stats = ops.ca_forward(q, k, v, rho)
    ws = torch.empty(512 << 20, device="cuda", dtype=torch.uint8)
    ref = [torch.empty_like(q) for _ in range(3)] + [torch.empty(16, device="cuda")]
    gpu_ca.native.check(lib.ca_bwd_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), rho.data_ptr(),
                                       out.data_ptr(), stats.data_ptr(), dy.data_ptr(),
                                       *[t.data_ptr() for t in ref], ws.data_ptr(), 512 << 20,
                                       *shape, gpu_ca.native.stream_handle(q.device)))
    got, _ = noalloc_backward(gpu_ca, q, k, v, rho, out, stats, dy)
    for name, a, b in zip(("dq", "dk", "dv", "dlog_gain"), got, ref):
        assert torch.equal(a, b), name


def test_noalloc_rejects_shapes_beyond_the_array(gpu_ca):
    lib = gpu_ca.native.load()
    p = ctypes.c_void_p(16)
    rc = lib.ca_bwd_f32_noalloc(p, p, p, p, p, p, p, p, p, p, p, 8, 16, 65536, 64, None)
    assert rc == gpu_ca.native.CA_ERR_WORKSPACE
    assert b"scratch" in lib.ca_last_error()

"""The allocation-free backward ``ca_bwd_f32_noalloc`` (workspace in a static
device array) against ``ca_bwd_f32`` (caller-allocated workspace), both
through the C ABI: bit-for-bit equal gradients on two calls in a row, the
second on a smaller input (the array keeps the first call's contents), with
no drop in free device memory during a call once the array is loaded, and
a shape that runs in passes sized to the array.  (The refusal of invalid
shapes before any launch is a CPU test: test_abi_cpu.py.)"""
import sys

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
    torch.cuda.synchronize()
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
    # a first call loads the library's static array on the device (its code
    # object is loaded on first use); after it, calls allocate nothing
    w = make(gpu_ca, (1, 1, 64, 64), 0)
    noalloc_backward(gpu_ca, *w)
    for n, (shape, seed) in enumerate([((1, 16, 2048, 64), 1), ((2, 4, 300, 64), 2)]):
        say(f"[case] noalloc call {n + 1}: shape {shape}")
        q, k, v, rho, out, stats, dy = make(gpu_ca, shape, seed)
        ref = ops.ca_backward(q, k, v, rho, out, stats, dy)
        torch.cuda.synchronize()
        got, grew = noalloc_backward(gpu_ca, q, k, v, rho, out, stats, dy)
        say(f"   free device memory dropped by {grew} bytes during the call")
        assert grew == 0
        for name, a, b in zip(("dq", "dk", "dv", "dlog_gain"), got, ref):
            assert torch.equal(a, b), name


def make(ca, shape, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v, dy = (torch.randn(shape, generator=g).cuda() for _ in range(4))
    rho = torch.linspace(-0.3, 0.3, shape[1]).cuda()
    out, stats = ca.ops.ca_forward(q, k, v, rho)
    return q, k, v, rho, out, stats, dy


def test_noalloc_backward_in_passes(gpu_ca):
    """A shape whose full backward workspace (3.1 GB) exceeds the 512 MiB
    array runs in passes over query ranges: bitwise equal to ca_bwd_f32
    given a workspace of the same size (the same pass plan)."""
    ops = gpu_ca.ops
    lib = gpu_ca.native.load()
    shape = (1, 16, 8192, 64)
    say(f"[case] noalloc in passes: shape {shape}")
    prev = gpu_ca.ops.workspace_cap()
    try:
        gpu_ca.ops.set_workspace_cap(0)
        assert lib.ca_bwd_workspace_bytes(*shape) > 512 << 20
    finally:
        gpu_ca.ops.set_workspace_cap(prev)
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

"""GPU parity of the HIP operator against the float64 oracle (oracle/ca_oracle.py).

Bar: max relative error max|x-ref|/max|ref| <= 1e-4
on outputs and <= 1e-3 on gradients (dq, dk, dv, dlog_gain); exact causality
(outputs bitwise unchanged, future gradients exactly 0).  Every call goes
through the C ABI (libca_hip.so via ctypes) behind continuum_attention().
"""
import json
import math
import sys

import numpy as np
import pytest
import torch

from oracle import ca_oracle as O

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-4
GRAD_TOL = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def make_inputs(shape, seed, mag=1.0, gains=None, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(shape, generator=g) * mag
    k = torch.randn(shape, generator=g) * mag
    v = torch.randn(shape, generator=g)
    dy = torch.randn(shape, generator=g)
    H = shape[1]
    rho = torch.zeros(H) if gains is None else torch.tensor(gains, dtype=torch.float32)
    return q, k, v, rho, dy


def run_hip(ca, q, k, v, rho, dy, tile=64):
    qd, kd, vd, rd = (x.cuda().requires_grad_(True) for x in (q, k, v, rho))
    y = ca.continuum_attention(qd, kd, vd, rd, tile)
    grads = torch.autograd.grad((y * dy.cuda()).sum(), (qd, kd, vd, rd))
    torch.cuda.synchronize()
    return y.detach().cpu().numpy(), [g.cpu().numpy() for g in grads]


def check_case(ca, shape, seed, mag=1.0, gains=None, label=""):
    say(f"[case] {label} shape={shape} seed={seed} mag={mag} gains={gains}")
    q, k, v, rho, dy = make_inputs(shape, seed, mag, gains)
    y, grads = run_hip(ca, q, k, v, rho, dy)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    ey = rel(y, yo)
    eg = [rel(a, b) for a, b in zip(grads, go)]
    say(f"   out {ey:.2e}  dq {eg[0]:.2e} dk {eg[1]:.2e} dv {eg[2]:.2e} drho {eg[3]:.2e}")
    assert np.all(np.isfinite(y)) and all(np.all(np.isfinite(g)) for g in grads)
    assert ey <= OUT_TOL
    for name, e in zip(("dq", "dk", "dv", "drho"), eg):
        assert e <= GRAD_TOL, name
    return ey, eg


def test_config1_cpu_operator_shape(gpu_ca):
    """[1,2,64,16] fp32, seed 0 (torch.manual_seed order q,k,v,dy), tau=1."""
    say("[case] config1 [1,2,64,16] seed 0")
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 64, 16) for _ in range(3))
    dy = torch.randn(1, 2, 64, 16)
    rho = torch.zeros(2)
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    assert rel(y, yo) <= OUT_TOL
    for a, b in zip(grads, go):
        assert rel(a, b) <= GRAD_TOL


def error_metrics(a, b):
    """Errors of a against the float64 reference b: the bar's max relative
    error (max|a-b| / max|b|), the reference benchmark's relative L2 and
    max-abs (cuda/benchmark.py:22-31: |a-b|_2 / |a|_2), and the element-wise
    relative error with an absolute floor of 1e-3 * rms(b)."""
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    d = np.abs(a - b)
    floor = 1e-3 * float(np.sqrt(np.mean(b * b))) + 1e-300
    return {"max_rel": rel(a, b), "relative_l2": float(np.linalg.norm(d) / max(np.linalg.norm(a), 1e-9)),
            "max_abs": float(d.max()), "elem_rel_floor": float((d / np.maximum(np.abs(b), floor)).max())}


@pytest.mark.parametrize("shape", [(1, 2, 64, 16), (1, 4, 1024, 64)])
def test_error_metrics_reference_style(gpu_ca, shape):
    """Every error metric the measurement spec names, printed per tensor as
    the reference's COMPARE lines, at config 1 and a 1024-token shape of
    config 2's head size (seed 0, tau = 1): max relative error within the
    bars (outputs 1e-4, gradients 1e-3) and relative L2 within the
    reference's own 1e-3 (cuda/benchmark.py:22-31)."""
    say(f"[case] error metrics {shape}")
    q, k, v, rho, dy = make_inputs(shape, 0)
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    for name, a, b, bar in zip(("y", "dq", "dk", "dv", "drho"), [y] + grads, [yo] + list(go),
                               [OUT_TOL] + [GRAD_TOL] * 4):
        m = error_metrics(a, b)
        say("COMPARE " + json.dumps({"name": name, **{k2: float(f"{v2:.3e}") for k2, v2 in m.items()}}))
        assert m["max_rel"] <= bar and m["relative_l2"] <= min(bar, 1e-3), name


def test_reference_ca_check_shape(gpu_ca):
    """cuda/continuum_attention.py:1363-1401: [1,2,9,8], seed 1234, fwd <= 2e-5 abs, grads <= 3e-4 abs."""
    say("[case] ca_check [1,2,9,8]")
    torch.manual_seed(1234)
    q, k, v = (torch.randn(1, 2, 9, 8) for _ in range(3))
    rho = torch.zeros(2)
    g = torch.randn(1, 2, 9, 8)
    y, grads = run_hip(gpu_ca, q, k, v, rho, g, tile=4)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), g.numpy())
    assert np.abs(y - yo).max() <= 2e-5
    for a, b in zip(grads, go):
        assert np.abs(a - b).max() <= 3e-4


@pytest.mark.parametrize("T", [1, 2, 3, 31, 32, 33, 62, 63, 64, 65, 124, 125, 127, 128, 129, 192, 257])
def test_ragged_lengths(gpu_ca, T):
    check_case(gpu_ca, (1, 2, T, 64), 100 + T, 1.0, [0.0, 0.3], f"ragged T={T}")


@pytest.mark.parametrize("D", [8, 16, 32, 64, 128])
def test_head_dims(gpu_ca, D):
    check_case(gpu_ca, (2, 2, 129, D), 7 + D, 1.0, [0.0, math.log(1 / 0.3)], f"D={D}")


@pytest.mark.parametrize("D,T,tile,dtype", [(80, 200, 64, torch.float32), (96, 129, 32, torch.float32),
                                             (48, 65, 16, torch.float32), (24, 100, 128, torch.float32),
                                             (4, 33, 7, torch.float32), (128, 1, 64, torch.float32),
                                             (128, 130, 37, torch.bfloat16)])
def test_any_head_dim_query_tiles(gpu_ca, D, T, tile, dtype):
    """Head dims without fused kernels (80, 96, 48, 24, 4) run the
    reference's query-tile structure on the device (fp32 GEMMs + the HIP
    weight kernels); D = 128 runs the fused kernels.  Outputs and all four
    gradients against the oracle, across tile boundaries and a tile that does
    not divide T, nonzero gains, and bf16 inputs."""
    say(f"[case] any head dim D={D} T={T} query_tile={tile} {dtype}")
    q, k, v, rho, dy = make_inputs((2, 2, T, D), 300 + D + T, 1.0, [0.2, -0.4])
    q, k, v, dy = (x.to(dtype).float() for x in (q, k, v, dy))
    qd, kd, vd = (x.to(dtype).cuda().requires_grad_(True) for x in (q, k, v))
    rd = rho.cuda().requires_grad_(True)
    y = gpu_ca.continuum_attention(qd, kd, vd, rd, tile)
    assert y.dtype == dtype
    grads = torch.autograd.grad((y.float() * dy.cuda()).sum(), (qd, kd, vd, rd))
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    out_bar, grad_bar = (OUT_TOL, GRAD_TOL) if dtype == torch.float32 else (1e-2, 1e-2)
    ey = rel(y.detach().float().cpu().numpy(), yo)
    eg = [rel(g.float().cpu().numpy(), b) for g, b in zip(grads, go)]
    say(f"   out {ey:.2e}  dq {eg[0]:.2e} dk {eg[1]:.2e} dv {eg[2]:.2e} drho {eg[3]:.2e}")
    assert ey <= out_bar
    for name, e in zip(("dq", "dk", "dv", "drho"), eg):
        assert e <= grad_bar, name


@pytest.mark.parametrize("mag", [0.0, 0.01, 2.5, 4.0])
def test_score_magnitudes(gpu_ca, mag):
    """Equal scores (mag 0: delta exactly 0, uniform limit), tiny and large deltas."""
    check_case(gpu_ca, (1, 2, 200, 64), 31, mag, [0.0, 0.2], f"mag={mag}")


def test_forward_splits_and_combine(gpu_ca):
    """T=1000 and 1537 span several forward splits (combine kernel) and many
    backward key blocks."""
    check_case(gpu_ca, (1, 2, 1000, 64), 5, 1.0, [0.1, -0.2], "splits T=1000")
    check_case(gpu_ca, (1, 1, 1537, 32), 6, 1.5, [0.0], "splits T=1537")


def test_dq_split_k(gpu_ca):
    """Grids far below one resident round split the dQ pass into chunks of
    7 key stages (224 keys, the shortest automatic length), merged in chunk
    order.  T=2049, one slice: the last query group's 65 stages make 10
    chunks, checked in full against the oracle.  T=4000, two D=32 slices with
    different gains: up to 18 chunks, checked on the last 200 queries (every
    chunk of the last groups) and on sampled rows.  Two calls agree bit for
    bit (fixed merge order)."""
    check_case(gpu_ca, (1, 1, 2049, 64), 12, 1.0, [0.25], "dq split T=2049")
    say("[case] dq split T=4000 D=32")
    T = 4000
    q, k, v, rho, dy = make_inputs((1, 2, T, 32), 13, 1.0, [0.0, -0.3])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    y2, grads2 = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.array_equal(y, y2) and all(np.array_equal(a, b) for a, b in zip(grads, grads2))
    qn, kn, vn, dyn, rn = q.numpy(), k.numpy(), v.numpy(), dy.numpy(), rho.numpy()
    rows = np.unique(np.concatenate([np.arange(T - 200, T), [0, 1, 959, 960, 1983, 1984, 3007]]))
    for h in (0, 1):
        dq_r = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, rows)[0]
        e = rel(grads[0][0, h, rows], dq_r)
        say(f"   head {h}: dq rows {e:.2e}")
        assert e <= GRAD_TOL


def test_repeated_keys_taylor_branch(gpu_ca):
    """Adjacent equal keys make delta exactly 0 (verify_backward_mps.py:49-51)
    and near-duplicate keys keep |delta| ~ 1e-4 (config 5 heads 0-7)."""
    say("[case] repeated / near-duplicate keys")
    torch.manual_seed(77)
    T = 300
    q = torch.randn(1, 2, T, 64)
    k = torch.randn(1, 2, T, 64)
    k[:, 0, 1::2] = k[:, 0, 0::2][:, :T // 2]               # exact repeats
    k[:, 1] = torch.cumsum(torch.randn(T, 64) * 1e-4, 0) + torch.randn(1, 64)
    v = torch.randn(1, 2, T, 64)
    dy = torch.randn(1, 2, T, 64)
    rho = torch.tensor([0.0, 0.5])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    assert rel(y, yo) <= OUT_TOL
    for a, b in zip(grads, go):
        assert rel(a, b) <= GRAD_TOL


def test_uniform_limit_exact(gpu_ca):
    """q = 0 gives equal scores: CA reduces to uniform causal averaging
    (test_acma.py:71-76)."""
    say("[case] uniform limit")
    T = 333
    v = torch.randn(1, 3, T, 32)
    q = torch.zeros(1, 3, T, 32)
    k = torch.randn(1, 3, T, 32)
    y = gpu_ca.continuum_attention(q.cuda(), k.cuda(), v.cuda(), torch.zeros(3).cuda()).cpu()
    ref = torch.cumsum(v.double(), 2) / torch.arange(1, T + 1, dtype=torch.float64).view(1, 1, T, 1)
    assert (y.double() - ref).abs().max().item() <= 2e-5


def test_causality_exact_T2048(gpu_ca):
    """cuda/benchmark.py:54-81: future edits leave earlier outputs bitwise
    unchanged; a prefix loss gives exactly zero gradient to future q, k, v."""
    say("[case] causality T=2048")
    torch.manual_seed(1649)
    T = 2048
    q, k, v = (torch.randn(1, 2, T, 64, device="cuda") for _ in range(3))
    rho = torch.tensor([0.0, 0.2], device="cuda")
    with torch.no_grad():
        y0 = gpu_ca.continuum_attention(q, k, v, rho, 128)
        for cut in (0, 127, 128, 1023, 1024, 2046):
            qp, kp, vp = q.clone(), k.clone(), v.clone()
            qp[:, :, cut + 1:] = torch.randn_like(qp[:, :, cut + 1:]) * 2.5
            kp[:, :, cut + 1:] = torch.randn_like(kp[:, :, cut + 1:]) * 2.5
            vp[:, :, cut + 1:] = torch.randn_like(vp[:, :, cut + 1:]) * 2.5
            y1 = gpu_ca.continuum_attention(qp, kp, vp, rho, 128)
            assert torch.equal(y0[:, :, :cut + 1], y1[:, :, :cut + 1]), cut
    for cut in (0, 127, 128, 1023, 1024, 2046):
        qt, kt, vt = (x.clone().requires_grad_(True) for x in (q, k, v))
        y = gpu_ca.continuum_attention(qt, kt, vt, rho, 128)
        gq, gk, gv = torch.autograd.grad(y[:, :, :cut + 1].sum(), (qt, kt, vt))
        for g in (gq, gk, gv):
            fut = g[:, :, cut + 1:]
            assert fut.numel() == 0 or fut.abs().max().item() == 0.0, cut


def test_config2_full_size(gpu_ca):
    """[2,16,2048,64] fp32, seed 0, rho=0.  Full outputs and
    gradients vs the oracle for two heads (both batches); size-independent
    invariants for every head: sum_j dV_j = sum_i dY_i, sum_j dK_j = 0,
    sum_i q_i.dQ_i = sum_j k_j.dK_j = dRho_h."""
    say("[case] config2 [2,16,2048,64]")
    torch.manual_seed(0)
    shape = (2, 16, 2048, 64)
    q, k, v = (torch.randn(shape) for _ in range(3))
    dy = torch.randn(shape)
    rho = torch.zeros(16)
    y, (dq, dk, dv, dr) = run_hip(gpu_ca, q, k, v, rho, dy)
    for h in (0, 9):
        sl = (slice(None), slice(h, h + 1))
        yo, _, _ = O.ca_forward(q[sl].numpy(), k[sl].numpy(), v[sl].numpy(), rho[h:h + 1].numpy())
        go = O.ca_backward(q[sl].numpy(), k[sl].numpy(), v[sl].numpy(), rho[h:h + 1].numpy(),
                           dy[sl].numpy())
        say(f"   head {h}: out {rel(y[sl], yo):.2e} dq {rel(dq[sl], go[0]):.2e} "
            f"dk {rel(dk[sl], go[1]):.2e} dv {rel(dv[sl], go[2]):.2e} drho {rel(dr[h:h+1], go[3]):.2e}")
        assert rel(y[sl], yo) <= OUT_TOL
        assert rel(dq[sl], go[0]) <= GRAD_TOL
        assert rel(dk[sl], go[1]) <= GRAD_TOL
        assert rel(dv[sl], go[2]) <= GRAD_TOL
        assert rel(dr[h:h + 1], go[3]) <= GRAD_TOL
    dvs = dv.astype(np.float64).sum(2)
    np.testing.assert_allclose(dvs, dy.double().sum(2).numpy(), rtol=0, atol=2e-3)
    assert np.abs(dk.astype(np.float64).sum(2)).max() <= 2e-3
    qdq = (q.double().numpy() * dq).sum(axis=(0, 2, 3))
    kdk = (k.double().numpy() * dk).sum(axis=(0, 2, 3))
    np.testing.assert_allclose(qdq, dr, rtol=1e-3, atol=1e-2)
    np.testing.assert_allclose(kdk, dr, rtol=1e-3, atol=1e-2)


def config5_inputs(seed=0, T=8192):
    """[1,16,T,64]; heads 0-7 k_j = k_{j-1} + N(0, 1e-4^2)
    (delta ~ 1e-4, the Taylor branch), heads 8-15 k = 4 N(0,1) (large |delta|);
    q, v, dY ~ N(0,1); log_gain = 0."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 16, T, 64, generator=g)
    k0 = torch.randn(8, 1, 64, generator=g)
    walk = torch.cumsum(torch.randn(8, T - 1, 64, generator=g) * 1e-4, 1)
    k = torch.cat([torch.cat([k0, k0 + walk], 1), 4.0 * torch.randn(8, T, 64, generator=g)], 0)[None]
    v = torch.randn(1, 16, T, 64, generator=g)
    dy = torch.randn(1, 16, T, 64, generator=g)
    return q, k.contiguous(), v, torch.zeros(16), dy


def test_config5_long_context_T8192(gpu_ca):
    """BASELINE config 5 at full size through the C ABI.  Oracle checks that
    need no [T, T] problem: forward and dQ on sampled rows of every head
    (row i depends only on row i of S), exact dK/dV of the last 256 keys of
    four heads (only queries i >= j see key j), and for every head
    sum_j dV_j = sum_i dY_i, sum_j dK_j = 0, sum q.dQ = sum k.dK = dRho.
    Errors are measured per head group (Taylor heads 0-7, large-delta heads
    8-15) so the larger group cannot mask the other."""
    say("[case] config5 [1,16,8192,64]")
    T = 8192
    q, k, v, rho, dy = config5_inputs(0, T)
    y, (dq, dk, dv, dr) = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.all(np.isfinite(y)) and all(np.all(np.isfinite(x)) for x in (dq, dk, dv, dr))
    qn, kn, vn, dyn, rn = q.numpy(), k.numpy(), v.numpy(), dy.numpy(), rho.numpy()
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([[0, 1, 2, 31, 32, 33, 61, 62, 63, 64, 127, 128, 129, 2047, 2048,
                                      4095, 4096, 6000, T - 2, T - 1], rng.integers(0, T, 8)]))
    for grp, heads in (("taylor", range(0, 8)), ("large", range(8, 16))):
        yr = np.stack([O.ca_forward_rows(qn, kn, vn, rn, 0, h, rows) for h in heads])
        dqr = np.stack([O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, rows)[0] for h in heads])
        hs = list(heads)
        ey = rel(y[0, hs][:, rows], yr)
        eq = rel(dq[0, hs][:, rows], dqr)
        say(f"   {grp}: sampled rows out {ey:.2e} dq {eq:.2e}")
        assert ey <= OUT_TOL
        assert eq <= GRAD_TOL
    suffix = np.arange(T - 256, T)
    for h in (0, 5, 8, 13):
        dq_s, dk_s, dv_s, _ = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, suffix)
        ek = rel(dk[0, h, suffix], dk_s[suffix])
        ev = rel(dv[0, h, suffix], dv_s[suffix])
        eq = rel(dq[0, h, suffix], dq_s)
        say(f"   head {h} last 256 keys: dk {ek:.2e} dv {ev:.2e} dq {eq:.2e}")
        assert ek <= GRAD_TOL and ev <= GRAD_TOL and eq <= GRAD_TOL
    d64 = lambda a: np.asarray(a, np.float64)
    dvs = d64(dv).sum(2)
    dys = d64(dyn).sum(2)
    scale_v = d64(np.abs(dyn)).sum(2).max()
    say(f"   sum dV - sum dY: {np.abs(dvs - dys).max():.2e} (scale {scale_v:.1f})")
    assert np.abs(dvs - dys).max() <= 1e-5 * scale_v
    dks = np.abs(d64(dk).sum(2)).max(-1)[0]
    scale_k = np.abs(d64(dk)).sum(2).max(-1)[0]
    say(f"   |sum dK| / sum |dK| per head: {np.max(dks / scale_k):.2e}")
    assert np.all(dks <= 1e-4 * scale_k)
    qdq = (d64(qn) * dq).sum(axis=(0, 2, 3))
    kdk = (d64(kn) * dk).sum(axis=(0, 2, 3))
    mag = (np.abs(d64(qn) * dq)).sum(axis=(0, 2, 3))
    say(f"   max |q.dQ - dRho| / sum|q.dQ|: {np.max(np.abs(qdq - dr) / mag):.2e}, "
        f"|k.dK - dRho|: {np.max(np.abs(kdk - dr) / mag):.2e}")
    assert np.all(np.abs(qdq - dr) <= 1e-4 * mag)
    assert np.all(np.abs(kdk - dr) <= 1e-4 * mag)


def test_long_context_T16384(gpu_ca):
    """Twice config 5's length, beyond the reference's fused-kernel limit
    (T <= 2048, cuda/continuum_attention.py:664-665): [1,2,16384,64] with one
    near-duplicate-key head (config 5 head 0) and one large-delta head (head
    8).  Forward and dQ on sampled rows, exact dK/dV/dQ of the last 256 keys,
    and sum dV = sum dY, sum dK = 0, sum q.dQ = sum k.dK = dRho per head."""
    say("[case] long context [1,2,16384,64]")
    T = 16384
    q, k, v, rho, dy = config5_inputs(3, T)
    sel = [0, 8]
    q, k, v, dy = (x[:, sel].contiguous() for x in (q, k, v, dy))
    rho = rho[sel].contiguous()
    y, (dq, dk, dv, dr) = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.all(np.isfinite(y)) and all(np.all(np.isfinite(x)) for x in (dq, dk, dv, dr))
    qn, kn, vn, dyn, rn = q.numpy(), k.numpy(), v.numpy(), dy.numpy(), rho.numpy()
    rng = np.random.default_rng(9)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 2047, 2048, 8191, 8192, 12000, T - 2, T - 1],
                                     rng.integers(0, T, 6)]))
    for h in (0, 1):
        yr = O.ca_forward_rows(qn, kn, vn, rn, 0, h, rows)
        dqr = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, rows)[0]
        ey, eq = rel(y[0, h][rows], yr), rel(dq[0, h][rows], dqr)
        suffix = np.arange(T - 256, T)
        dq_s, dk_s, dv_s, _ = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, suffix)
        ek, ev = rel(dk[0, h, suffix], dk_s[suffix]), rel(dv[0, h, suffix], dv_s[suffix])
        say(f"   head {h}: rows out {ey:.2e} dq {eq:.2e}; last 256 keys dk {ek:.2e} dv {ev:.2e}")
        assert ey <= OUT_TOL and eq <= GRAD_TOL and ek <= GRAD_TOL and ev <= GRAD_TOL
    d64 = lambda a: np.asarray(a, np.float64)
    scale_v = d64(np.abs(dyn)).sum(2).max()
    assert np.abs(d64(dv).sum(2) - d64(dyn).sum(2)).max() <= 1e-5 * scale_v
    dks = np.abs(d64(dk).sum(2)).max(-1)[0]
    assert np.all(dks <= 1e-4 * np.abs(d64(dk)).sum(2).max(-1)[0])
    qdq = (d64(qn) * dq).sum(axis=(0, 2, 3))
    kdk = (d64(kn) * dk).sum(axis=(0, 2, 3))
    mag = (np.abs(d64(qn) * dq)).sum(axis=(0, 2, 3))
    assert np.all(np.abs(qdq - dr) <= 1e-4 * mag) and np.all(np.abs(kdk - dr) <= 1e-4 * mag)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_precision_inputs(gpu_ca, dtype):
    """bf16/fp16 q, k, v (the reference's autocast inputs): the operator reads
    them as fp32, returns v.dtype and gradients in the input dtypes.  Against
    the oracle on the same rounded inputs, the only extra error is the final
    rounding of the outputs to dtype."""
    say(f"[case] {dtype} inputs")
    q, k, v, rho, dy = make_inputs((1, 2, 150, 64), 41, 1.0, [0.0, 0.4])
    qh, kh, vh = (x.to(dtype) for x in (q, k, v))
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (qh, kh, vh))
    rd = rho.cuda().requires_grad_(True)
    y = gpu_ca.continuum_attention(qd, kd, vd, rd)
    assert y.dtype == dtype
    grads = torch.autograd.grad(y, (qd, kd, vd, rd), dy.cuda().to(dtype))
    assert [g.dtype for g in grads] == [dtype, dtype, dtype, torch.float32]
    q64, k64, v64 = (x.double().numpy() for x in (qh, kh, vh))
    dy64 = dy.to(dtype).double().numpy()
    yo = O.ca_forward(q64, k64, v64, rho.numpy())[0]
    go = O.ca_backward(q64, k64, v64, rho.numpy(), dy64)
    tol = 2 ** -8 if dtype == torch.bfloat16 else 2 ** -11
    ey = rel(y.float().detach().cpu().numpy(), yo)
    eg = [rel(g.float().cpu().numpy(), r) for g, r in zip(grads, go)]
    say(f"   out {ey:.2e} grads {[f'{e:.1e}' for e in eg]} (dtype rounding {tol:.1e})")
    assert ey <= tol
    assert all(e <= tol for e in eg[:3]) and eg[3] <= GRAD_TOL


def test_hip_graph_capture_and_replay(gpu_ca):
    """The operator's forward and backward launch only kernels on the current
    stream (no host sync, no memset), so they can be captured in a HIP graph.
    The graph is replayed several times with eager work and synchronisation in
    between; every replay must equal the eager result bitwise."""
    say("[case] graph capture")
    q, k, v, rho, dy = make_inputs((2, 4, 300, 64), 43, 1.0, [0.0, 0.2, -0.1, 0.3])
    qd, kd, vd, rd, dyd = (x.cuda() for x in (q, k, v, rho, dy))
    ref_y, ref_stats = gpu_ca.ca_forward(qd, kd, vd, rd)
    ref_g = gpu_ca.ca_backward(qd, kd, vd, rd, ref_y, ref_stats, dyd)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on the capture stream
        gpu_ca.ca_backward(qd, kd, vd, rd, *gpu_ca.ca_forward(qd, kd, vd, rd), dyd)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y, stats = gpu_ca.ca_forward(qd, kd, vd, rd)
        grads = gpu_ca.ca_backward(qd, kd, vd, rd, y, stats, dyd)
    for rep in range(4):
        junk = torch.randn(1 << 20, device="cuda") * rep  # eager work between replays
        junk.sum().item()
        for t in (y, *grads):
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref_y), rep
        for a, b in zip(grads, ref_g):
            assert torch.equal(a, b), rep


def test_stream_handle_follows_current_stream(gpu_ca):
    """The launch stream handle equals torch's current stream on the default
    stream and under a side stream (forward and the autograd backward launched
    there give the default stream's results)."""
    say("[case] stream handle")
    N = gpu_ca.native
    dev = torch.device("cuda", torch.cuda.current_device())
    assert N.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    q, k, v, rho, dy = (x.cuda() for x in make_inputs((1, 2, 200, 32), 44, 1.0, [0.1, -0.2]))
    ref = run_hip(gpu_ca, q, k, v, rho, dy)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        assert N.stream_handle(dev) == s.cuda_stream != torch.cuda.default_stream(dev).cuda_stream
        got = run_hip(gpu_ca, q, k, v, rho, dy)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert np.array_equal(got[0], ref[0])
    for a, b in zip(got[1], ref[1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("shape", [(0, 2, 16, 64), (2, 0, 16, 64), (0, 1, 5, 24)])
def test_empty_batch(gpu_ca, shape):
    """An empty batch (B or H = 0) gives empty outputs and gradients, as the
    reference's tile loop does; T = 0 raises (its concatenation of no tiles)."""
    say(f"[case] empty batch {shape}")
    q, k, v = (torch.randn(shape, device="cuda", requires_grad=True) for _ in range(3))
    rho = torch.zeros(shape[1], device="cuda", requires_grad=True)
    y = gpu_ca.continuum_attention(q, k, v, rho)
    assert y.shape == q.shape and y.dtype == v.dtype
    grads = torch.autograd.grad(y.sum(), (q, k, v, rho), allow_unused=True)
    for g, t in zip(grads, (q, k, v, rho)):
        assert g is None or g.shape == t.shape
    z = torch.randn(1, 1, 0, 64, device="cuda")
    with pytest.raises(RuntimeError, match="T = 0"):
        gpu_ca.continuum_attention(z, z, z, torch.zeros(1, device="cuda"))


def test_mode_limits_on_gpu(gpu_ca, monkeypatch):
    """The CA_CUDA_MODE limits raise on GPU tensors as in the reference
    (cuda/continuum_attention.py:662-665), in the operator and in the
    decoder's fused attention; within them every mode returns the default
    mode's result bit for bit."""
    say("[case] CA_CUDA_MODE limits on GPU tensors")
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 2, 64, 64, generator=g).cuda() for _ in range(3))
    rho = torch.zeros(2, device="cuda")
    one = torch.zeros(1, device="cuda")
    monkeypatch.delenv("CA_CUDA_MODE", raising=False)
    ref32 = gpu_ca.continuum_attention(q, k, v, rho)
    ref16 = gpu_ca.continuum_attention(q.half(), k.half(), v.half(), rho)
    long16 = torch.zeros(1, 1, 2049, 16, device="cuda", dtype=torch.float16)
    for mode in ("prefix_v5", "prefix_v6"):
        monkeypatch.setenv("CA_CUDA_MODE", mode)
        with pytest.raises(ValueError, match="v5/v6 paths require CUDA FP16"):
            gpu_ca.continuum_attention(q, k, v, rho)
        with pytest.raises(ValueError, match="v5/v6 paths require CUDA FP16"):
            gpu_ca.continuum_attention(long16, long16, long16, one)
        assert torch.equal(gpu_ca.continuum_attention(q.half(), k.half(), v.half(), rho), ref16)
    monkeypatch.setenv("CA_CUDA_MODE", "fused")
    long32 = long16.float()
    wide = torch.zeros(1, 1, 8, 160, device="cuda")
    for t in (long32, wide, q.bfloat16()):
        with pytest.raises(ValueError, match="fused forward supports"):
            gpu_ca.continuum_attention(t, t, t, one if t.shape[1] == 1 else rho)
    assert torch.equal(gpu_ca.continuum_attention(q, k, v, rho), ref32)
    # the decoder's fused attention: bf16 values are outside 'fused'
    qkv = torch.randn(1, 64, 3 * 128, generator=g).cuda().bfloat16()
    with pytest.raises(ValueError, match="fused forward supports"):
        gpu_ca.decoder.rope_continuum_attention(qkv, rho, 10000.0, 2)
    monkeypatch.setenv("CA_CUDA_MODE", "prefix_v5")
    with pytest.raises(ValueError, match="v5/v6 paths require CUDA FP16"):
        gpu_ca.decoder.rope_continuum_attention(qkv, rho, 10000.0, 2)
    gpu_ca.decoder.rope_continuum_attention(qkv.half(), rho, 10000.0, 2)

"""GPU parity at the BASELINE config-3 and config-4 operator shapes, at every
work-split length, and for non-finite inputs.

* Config 3's layer shape [16,4,512,64] with log_gain = ln(1/0.3) on every
  head (the CA-P decoder's fixed tau = 0.30 reaches the operator as its
  log-gain) and config 4's [1,16,2048,64] with non-zero per-head gains: the
  small-grid split paths (short forward ranges, dQ and dK/dV chunks) that
  the automatic choice takes at these shapes on a 256-CU MI355X.
* Every split length the automatic choice can pick (forward ranges of 12, 8,
  6, 4 tiles; dQ chunks of 64, 48, 32, 24, 16 key blocks; dK/dV chunks of
  24, 16, 12, 8, 6 query tiles), and odd and single lengths, forced through
  ``ca_debug_set_splits`` at small shapes and compared in full.
* NaN inputs propagate to the outputs a NaN reaches in the reference and
  leave every other row bit for bit unchanged.

Bars as elsewhere: max|x-ref|/max|ref| <= 1e-4 on outputs, <= 1e-3 on
gradients, against the float64 oracle (oracle/ca_oracle.py).
"""
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


def inputs(shape, seed, gains, mag=1.0):
    g = torch.Generator().manual_seed(seed)
    q, k = (torch.randn(shape, generator=g) * mag for _ in range(2))
    v, dy = (torch.randn(shape, generator=g) for _ in range(2))
    return q, k, v, torch.tensor(gains, dtype=torch.float32), dy


def run_hip(ca, q, k, v, rho, dy, tile=64):
    qd, kd, vd, rd = (x.cuda().requires_grad_(True) for x in (q, k, v, rho))
    y = ca.continuum_attention(qd, kd, vd, rd, tile)
    grads = torch.autograd.grad((y * dy.cuda()).sum(), (qd, kd, vd, rd))
    torch.cuda.synchronize()
    return y.detach().cpu().numpy(), [g.cpu().numpy() for g in grads]


def check_full(q, k, v, rho, dy, y, grads, label):
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    ey = rel(y, yo)
    eg = [rel(a, b) for a, b in zip(grads, go)]
    say(f"   {label}: out {ey:.2e} dq {eg[0]:.2e} dk {eg[1]:.2e} dv {eg[2]:.2e} drho {eg[3]:.2e}")
    assert ey <= OUT_TOL
    for name, e in zip(("dq", "dk", "dv", "drho"), eg):
        assert e <= GRAD_TOL, name


def check_invariants(q, k, dy, dq, dk, dv, dr):
    """sum_j dV_j = sum_i dY_i and sum_j dK_j = 0 per slice; sum_i q.dQ =
    sum_j k.dK = dRho_h per head (dRho_h sums over the batch)."""
    d64 = lambda a: np.asarray(a, np.float64)
    dyn = dy.numpy()
    scale_v = d64(np.abs(dyn)).sum(2).max()
    assert np.abs(d64(dv).sum(2) - d64(dyn).sum(2)).max() <= 1e-5 * scale_v
    dks = np.abs(d64(dk).sum(2)).max(-1)
    assert np.all(dks <= 1e-4 * np.abs(d64(dk)).sum(2).max(-1))
    qdq = (d64(q.numpy()) * dq).sum(axis=(0, 2, 3))
    kdk = (d64(k.numpy()) * dk).sum(axis=(0, 2, 3))
    mag = (np.abs(d64(q.numpy()) * dq)).sum(axis=(0, 2, 3))
    assert np.all(np.abs(qdq - dr) <= 1e-4 * mag) and np.all(np.abs(kdk - dr) <= 1e-4 * mag)


def check_sampled_rows(q, k, v, rho, dy, y, dq, rows):
    """Output and dQ rows of every (b, h) slice against the row oracle."""
    qn, kn, vn, rn, dyn = q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy()
    worst_y = worst_q = 0.0
    B, H = q.shape[:2]
    for b in range(B):
        for h in range(H):
            yr = O.ca_forward_rows(qn, kn, vn, rn, b, h, rows)
            dqr = O.ca_backward_rows(qn, kn, vn, rn, dyn, b, h, rows)[0]
            worst_y = max(worst_y, rel(y[b, h][rows], yr))
            worst_q = max(worst_q, rel(dq[b, h][rows], dqr))
    say(f"   sampled rows of all {B * H} slices: out {worst_y:.2e} dq {worst_q:.2e}")
    assert worst_y <= OUT_TOL and worst_q <= GRAD_TOL


def test_config3_layer_shape(gpu_ca):
    """BASELINE config 3's operator call: [16,4,512,64], log_gain = ln(1/0.3)
    on all four heads, N(0,1) q, k, v, dY.  Every slice in full against the
    oracle (outputs, dQ, dK, dV, dRho), and the invariants."""
    say("[case] config3 layer [16,4,512,64] log_gain ln(1/0.3)")
    shape = (16, 4, 512, 64)
    q, k, v, rho, dy = inputs(shape, 3, [math.log(1 / 0.3)] * 4)
    y, (dq, dk, dv, dr) = run_hip(gpu_ca, q, k, v, rho, dy)
    check_full(q, k, v, rho, dy, y, (dq, dk, dv, dr), "all 64 slices")
    check_invariants(q, k, dy, dq, dk, dv, dr)


def test_config4_layer_shape(gpu_ca):
    """BASELINE config 4's operator call: [1,16,2048,64] with non-zero gains
    (-0.5 .. 0.5).  Two slices in full (outputs and all four gradients,
    dRho of those heads), sampled rows of all 16 slices, and the invariants
    for every head."""
    say("[case] config4 layer [1,16,2048,64] gains -0.5..0.5")
    shape = (1, 16, 2048, 64)
    gains = np.linspace(-0.5, 0.5, 16).tolist()
    q, k, v, rho, dy = inputs(shape, 4, gains)
    y, (dq, dk, dv, dr) = run_hip(gpu_ca, q, k, v, rho, dy)
    for h in (0, 11):
        sl = (slice(None), slice(h, h + 1))
        check_full(q[sl], k[sl], v[sl], rho[h:h + 1], dy[sl], y[sl],
                   (dq[sl], dk[sl], dv[sl], dr[h:h + 1]), f"head {h}")
    rows = np.array([0, 1, 2, 31, 32, 127, 128, 511, 512, 1023, 1024, 1500, 2046, 2047])
    check_sampled_rows(q, k, v, rho, dy, y, dq, rows)
    check_invariants(q, k, dy, dq, dk, dv, dr)


# (forward split tiles, dQ chunk stages of 32 keys, dK/dV chunk tiles); 0 =
# automatic.  The automatic choices are forward 12/8/6/4, dQ 28/21/14/10/7 and
# dK/dV 24/16/12/8/6; each appears below, at a shape where it cuts some group.
SPLITS = [(4, 7, 6), (6, 10, 8), (8, 14, 12), (12, 21, 16), (12, 28, 24), (5, 5, 5), (1, 1, 1),
          (3, 2, 2)]


@pytest.fixture
def split_override(gpu_ca):
    yield gpu_ca.ops.set_split_override
    gpu_ca.ops.set_split_override(0, 0, 0)


@pytest.mark.parametrize("splits", SPLITS, ids=lambda s: "fwd%d-dq%d-kv%d" % s)
def test_every_split_length(gpu_ca, split_override, splits):
    """Each forced split length at [1,2,1100,64] (35 query tiles and key
    stages, 79 key blocks: every length cuts some ranges unevenly) in full
    against the oracle, and two calls bitwise equal (fixed merge order)."""
    say(f"[case] forced splits {splits} [1,2,1100,64]")
    split_override(*splits)
    q, k, v, rho, dy = inputs((1, 2, 1100, 64), 21, [0.3, -0.4])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    y2, grads2 = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.array_equal(y, y2) and all(np.array_equal(a, b) for a, b in zip(grads, grads2))
    check_full(q, k, v, rho, dy, y, grads, f"splits {splits}")


def test_default_splits_past_t2048(gpu_ca):
    """[1,2,3000,64] with the automatic splits, which past T = 2048 grow with
    the row length (16-tile forward splits here, a ragged last query group
    and key stage) in full against the oracle."""
    say("[case] default splits [1,2,3000,64]")
    q, k, v, rho, dy = inputs((1, 2, 3000, 64), 23, [0.1, -0.2])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    check_full(q, k, v, rho, dy, y, grads, "T=3000 default splits")


def test_default_splits_dkdv_fallback_shape(gpu_ca):
    """[1,16,3000,64] with the automatic splits: there the fp32 dK/dV rule's
    16-tile chunks would need more partials than the workspace is sized for,
    so the launch takes the longer chunks it was sized for.  Heads 0 and 15
    (independent slices, each with its own dlog_gain) against the oracle."""
    say("[case] default splits [1,16,3000,64], heads 0 and 15")
    q, k, v, rho, dy = inputs((1, 16, 3000, 64), 24, [0.1 * (h % 5) - 0.2 for h in range(16)])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    for h in (0, 15):
        sl = slice(h, h + 1)
        check_full(q[:, sl], k[:, sl], v[:, sl], rho[sl], dy[:, sl], y[:, sl],
                   [grads[0][:, sl], grads[1][:, sl], grads[2][:, sl], grads[3][sl]],
                   f"T=3000 H=16 head {h}")


@pytest.mark.parametrize("D,splits", [(128, (4, 16, 6)), (32, (6, 10, 8)), (16, (1, 3, 1))])
def test_forced_splits_other_head_dims(gpu_ca, split_override, D, splits):
    say(f"[case] forced splits {splits} [1,2,700,{D}]")
    split_override(*splits)
    q, k, v, rho, dy = inputs((1, 2, 700, D), 22 + D, [0.0, 0.25])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    check_full(q, k, v, rho, dy, y, grads, f"D={D} splits {splits}")


def test_nan_inputs_propagate_like_the_reference(gpu_ca):
    """A NaN in q row r makes output row r NaN (every score of the row is
    NaN, as in the reference) and leaves every other row bitwise unchanged;
    a NaN in key j makes every row i >= j NaN and leaves rows i < j bitwise
    unchanged (the reference masks future scores before they meet
    arithmetic).  In the backward, dQ row r is NaN, dRho of that head is
    NaN, and every other slice's gradients are unchanged."""
    say("[case] NaN inputs [2,2,300,64]")
    shape = (2, 2, 300, 64)
    q, k, v, rho, dy = inputs(shape, 8, [0.1, -0.2])
    y0, g0 = run_hip(gpu_ca, q, k, v, rho, dy)
    r, j = 137, 201
    qn = q.clone()
    qn[1, 0, r, 5] = float("nan")
    y1, g1 = run_hip(gpu_ca, qn, k, v, rho, dy)
    bad = np.zeros(shape[:3], bool)
    bad[1, 0, r] = True
    assert np.isnan(y1[bad]).all()
    assert np.array_equal(y1[~bad], y0[~bad])
    dq1, dk1, dv1, dr1 = g1
    assert np.isnan(dq1[1, 0, r]).all() and np.isnan(dr1[0])
    rows = np.ones(shape[2], bool)
    rows[r] = False
    assert np.isfinite(dq1[1, 0][rows]).all()
    for b, h in ((0, 0), (0, 1), (1, 1)):
        for a0, a1 in zip(g0[:3], g1[:3]):
            assert np.array_equal(a0[b, h], a1[b, h])
    assert dr1[1] == g0[3][1]
    kn = k.clone()
    kn[0, 1, j, 9] = float("nan")
    y2, _ = run_hip(gpu_ca, q, kn, v, rho, dy)
    bad = np.zeros(shape[:3], bool)
    bad[0, 1, j:] = True
    assert np.isnan(y2[bad]).all()
    assert np.array_equal(y2[~bad], y0[~bad])


@pytest.fixture
def workspace_cap(gpu_ca):
    prev = gpu_ca.ops.workspace_cap()
    yield gpu_ca.ops.set_workspace_cap
    gpu_ca.ops.set_workspace_cap(prev)


def _row_and_suffix_checks(q, k, v, rho, dy, y, grads, rows, label):
    """Forward and dQ on sampled rows; dK, dV, dQ of the last 256 keys exactly
    (only queries i >= j see key j); the invariants."""
    dq, dk, dv, dr = grads
    qn, kn, vn, rn, dyn = q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy()
    T = q.shape[2]
    suffix = np.arange(T - 256, T)
    for h in range(q.shape[1]):
        yr = O.ca_forward_rows(qn, kn, vn, rn, 0, h, rows)
        dqr = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, rows)[0]
        dq_s, dk_s, dv_s, _ = O.ca_backward_rows(qn, kn, vn, rn, dyn, 0, h, suffix)
        e = (rel(y[0, h][rows], yr), rel(dq[0, h][rows], dqr), rel(dk[0, h, suffix], dk_s[suffix]),
             rel(dv[0, h, suffix], dv_s[suffix]), rel(dq[0, h, suffix], dq_s))
        say(f"   {label} head {h}: rows out {e[0]:.2e} dq {e[1]:.2e}; last 256 keys dk {e[2]:.2e} "
            f"dv {e[3]:.2e} dq {e[4]:.2e}")
        assert e[0] <= OUT_TOL and all(x <= GRAD_TOL for x in e[1:])
    check_invariants(q, k, dy, dq, dk, dv, dr)


@pytest.mark.parametrize("T,H,cap_mb", [(16384, 2, 256), (32768, 1, 512), (16384, 1, 96)])
def test_bounded_workspace_long_context(gpu_ca, workspace_cap, T, H, cap_mb):
    """The workspace bound that stands in for the reference's query_tile
    (cuda/continuum_attention.py:957): with a cap far below the full
    backward workspace (4.2 GB for [1,2,16384,64], 8.3 GB for [1,1,32768,64])
    the size functions report at most the cap, the backward runs in passes
    over query ranges and the forward with longer splits, and the results
    match the oracle: sampled rows, the last 256 keys exactly, invariants."""
    say(f"[case] workspace cap {cap_mb} MiB, [1,{H},{T},64]")
    lib = gpu_ca.native.load()
    workspace_cap(0)
    full = lib.ca_bwd_workspace_bytes(1, H, T, 64)  # one pass, uncapped
    workspace_cap(cap_mb << 20)
    wb, wf = lib.ca_bwd_workspace_bytes(1, H, T, 64), lib.ca_fwd_workspace_bytes(1, H, T, 64)
    say(f"   backward workspace {wb / 2**20:.0f} MiB (full {full / 2**20:.0f} MiB), "
        f"forward {wf / 2**20:.0f} MiB")
    assert wb <= cap_mb << 20 and wf <= cap_mb << 20 and full > 4 * (cap_mb << 20)
    q, k, v, rho, dy = config5_like(T, H)
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.all(np.isfinite(y)) and all(np.all(np.isfinite(x)) for x in grads)
    rows = np.array([0, 1, 31, 32, 127, 128, 2047, 2048, 8191, 8192, T // 2 + 5, T - 129, T - 2, T - 1])
    _row_and_suffix_checks(q, k, v, rho, dy, y, grads, rows, f"cap {cap_mb} MiB")


def config5_like(T, H):
    """Config 5's two head kinds: near-duplicate keys (delta ~ 1e-4, the Taylor
    branch) in head 0 and keys x4 (large delta) in head 1."""
    g = torch.Generator().manual_seed(T + H)
    q = torch.randn(1, H, T, 64, generator=g)
    k0 = torch.randn(1, 64, generator=g)
    heads = [torch.cat([k0, k0 + torch.cumsum(torch.randn(T - 1, 64, generator=g) * 1e-4, 0)])]
    if H > 1:
        heads.append(4.0 * torch.randn(T, 64, generator=g))
    k = torch.stack(heads)[None].contiguous()
    v = torch.randn(1, H, T, 64, generator=g)
    dy = torch.randn(1, H, T, 64, generator=g)
    return q, k, v, torch.zeros(H), dy


@pytest.mark.parametrize("cap_mb,shape", [(3, (2, 3, 3000, 64)), (1, (1, 2, 1500, 32))])
def test_backward_passes_in_full(gpu_ca, workspace_cap, cap_mb, shape):
    """A cap that forces many passes at a size the oracle checks in full:
    outputs and all four gradients, and two calls bitwise equal."""
    say(f"[case] backward passes, cap {cap_mb} MiB, {shape}")
    lib = gpu_ca.native.load()
    B, H, T, D = shape
    workspace_cap(0)
    full = lib.ca_bwd_workspace_bytes(B, H, T, D)  # one pass, uncapped
    workspace_cap(cap_mb << 20)
    assert lib.ca_bwd_workspace_bytes(B, H, T, D) < full // 4
    q, k, v, rho, dy = inputs(shape, 30, [0.2, -0.3, 0.1][:H])
    y, grads = run_hip(gpu_ca, q, k, v, rho, dy)
    y2, grads2 = run_hip(gpu_ca, q, k, v, rho, dy)
    assert np.array_equal(y, y2) and all(np.array_equal(a, b) for a, b in zip(grads, grads2))
    check_full(q, k, v, rho, dy, y, grads, f"cap {cap_mb} MiB")

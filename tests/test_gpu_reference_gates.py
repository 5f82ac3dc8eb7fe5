"""The reference's own GPU gates, replayed on the HIP paths against the float64
oracle (oracle/ca_oracle.py).

* The CUDA preflight's two weight-kernel case lists
  (cuda/continuum_attention.py:1407-1447): tiles of Q queries starting at
  `start` over T (or start + Q) keys, magnitudes up to 2.5, late tiles
  (T 2048, start 2024) and 2048-key zero-magnitude rows, with the
  preflight's own tolerances (W: atol = rtol = 3e-5; dS: atol 3e-4, rtol
  3e-3).  The scores come from a CPU generator seeded 20260814 (the
  preflight seeds torch.manual_seed(20260814) and draws on the CUDA device,
  whose stream this box does not reproduce).
* The Metal verifiers' stress patterns on the weight VJP: magnitude 7 and
  equal adjacent scores at T in {7, 32, 192} (verify_backward_mps.py:49-51,
  159-161), and equal-score segments s[..., 1:3] = s[..., :1] at
  magnitude 3 (verify_mps.py:37-40).
* The v6 benchmark's fp16 numerical cases (cuda/benchmark.py:36-52): six
  [1,2,T,64] fp16 problems, magnitudes up to 2.5, log-gains
  (0, ln(1/0.3)), through the operator, against the oracle on the
  fp16-rounded inputs.
* The full CA-S decoder causality gate (cuda/benchmark.py:85-105): the
  101,205,120-parameter model at T 2048 under fp16 (the reference's) and
  bf16 autocast; logits before each cut bitwise unchanged when every later
  token is replaced.
* Config 2 ([2,16,2048,64]): sampled rows of all 32 slices against the row
  oracle (forward and dQ).
* The decoder's fused attention gradients (dqkv with RoPE transposed back)
  against the oracle directly, in one pass and in passes under a small
  workspace cap (T 16384 at 256 MiB for one CA-S layer's 16 heads).
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import ca_oracle as O

pytestmark = pytest.mark.gpu

PREFLIGHT_SEED = 20260814


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def close(got, ref, atol, rtol):
    """torch.testing.assert_close's criterion |got - ref| <= atol + rtol |ref|."""
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    excess = np.abs(got - ref) - (atol + rtol * np.abs(ref))
    return float(excess.max())


# cuda/continuum_attention.py:1414-1420 (ext.forward + ext.backward over T keys)
PREFLIGHT_FULL = [(9, 0, 9, 1.0), (192, 144, 32, 1.0), (512, 480, 32, 2.5),
                  (2048, 2024, 24, 2.5), (2048, 0, 24, 0.0)]
# cuda/continuum_attention.py:1441-1447 (ext.backward_fused over K = start + Q keys)
PREFLIGHT_FUSED = [(9, 0, 9, 1.0), (192, 160, 32, 2.5), (512, 480, 32, 2.5),
                   (2048, 2024, 24, 2.5), (2048, 0, 24, 0.0)]


def _preflight_case(gpu_ca, K, start, Q, mag, gen):
    s = torch.randn(1, Q, K, generator=gen) * mag
    gw = torch.randn(1, Q, K, generator=gen)
    W, stats = gpu_ca.ca_weights(s.cuda(), start)
    W2, ds = gpu_ca.ca_weights_backward(s.cuda(), gw.cuda(), start, return_weights=True)
    qidx = np.arange(start, start + Q)
    Wo = O.ca_weights(s.double().numpy(), qidx)[0]
    dso = O.ca_weights_vjp(s.double().numpy(), gw.double().numpy(), qidx=qidx)
    W, W2, ds = (x.cpu().numpy() for x in (W, W2, ds))
    ew, ew2, eds = close(W, Wo, 3e-5, 3e-5), close(W2, Wo, 3e-5, 3e-5), close(ds, dso, 3e-4, 3e-3)
    say(f"   K={K} q={start}:{start + Q} magnitude={mag}: forward_abs {np.abs(W - Wo).max():.3g} "
        f"grad_abs {np.abs(ds - dso).max():.3g} (rel {rel(W, Wo):.2e} / {rel(ds, dso):.2e})")
    assert ew <= 0 and ew2 <= 0, "weights beyond the preflight tolerance"
    assert eds <= 0, "score gradient beyond the preflight tolerance"
    # the north-star bars as well
    assert rel(W, Wo) <= 1e-4 and rel(ds, dso) <= 1e-3
    # exact zeros past each row's visible prefix
    for r in range(Q):
        assert np.all(W[:, r, start + r + 1:] == 0.0) and np.all(ds[:, r, start + r + 1:] == 0.0)


def test_cuda_preflight_weight_cases(gpu_ca):
    say("[case] CUDA preflight weight cases (full key range)")
    gen = torch.Generator().manual_seed(PREFLIGHT_SEED)
    for T, start, Q, mag in PREFLIGHT_FULL:
        _preflight_case(gpu_ca, T, start, Q, mag, gen)


def test_cuda_preflight_fused_cases(gpu_ca):
    say("[case] CUDA preflight fused cases (K = start + Q)")
    gen = torch.Generator().manual_seed(PREFLIGHT_SEED + 1)
    for T, start, Q, mag in PREFLIGHT_FUSED:
        _preflight_case(gpu_ca, start + Q, start, Q, mag, gen)


def _weights_vs_oracle(gpu_ca, s, gw):
    sd = s.cuda().requires_grad_(True)
    W = gpu_ca.continuous_attention_weights(sd)
    (ds,) = torch.autograd.grad(W, sd, gw.cuda())
    Wo = O.ca_weights(s.double().numpy())[0]
    dso = O.ca_weights_vjp(s.double().numpy(), gw.double().numpy())
    W, ds = W.detach().cpu().numpy(), ds.cpu().numpy()
    return W, ds, Wo, dso


@pytest.mark.parametrize("T", [7, 32, 192])
@pytest.mark.parametrize("pattern", ["magnitude7", "repeat"])
def test_metal_backward_stress_patterns(gpu_ca, T, pattern):
    """verify_backward_mps.py:49-51, 159-161: scores x7, and every odd key's
    score equal to its even neighbour's (zero-width segments, the Taylor
    branch at delta = 0), B = H = 2; forward at the verifier's 5e-4 and both
    at the north-star bars."""
    say(f"[case] Metal VJP pattern {pattern} T={T}")
    g = torch.Generator().manual_seed(1729 + T)
    mag = 7.0 if pattern == "magnitude7" else 1.0
    s = torch.randn(2, 2, T, T, generator=g) * mag
    if pattern == "repeat" and T > 1:
        s[..., 1::2] = s[..., ::2][..., :s[..., 1::2].shape[-1]]
    gw = torch.randn(2, 2, T, T, generator=g)
    W, ds, Wo, dso = _weights_vs_oracle(gpu_ca, s, gw)
    say(f"   W {rel(W, Wo):.2e} dS {rel(ds, dso):.2e}")
    assert close(W, Wo, 5e-4, 5e-4) <= 0
    assert rel(W, Wo) <= 1e-4 and rel(ds, dso) <= 1e-3
    np.testing.assert_allclose(W.sum(-1), 1.0, atol=2e-6)


@pytest.mark.parametrize("T", [1, 2, 7, 32, 192, 256])
def test_metal_equal_score_segments(gpu_ca, T):
    """verify_mps.py:37-40: scores x3 with keys 1 and 2 given key 0's score
    (two equal-score segments at the start of every row); W, W.V and the
    row mass against the oracle, and the VJP at the north-star bar."""
    say(f"[case] equal-score segments T={T}")
    g = torch.Generator().manual_seed(1729 + 7 * T)
    s = torch.randn(2, 3, T, T, generator=g) * 3.0
    v = torch.randn(2, 3, T, 16, generator=g)
    if T >= 2:
        s[:, :, :, 1:3] = s[:, :, :, :1]
    gw = torch.randn(2, 3, T, T, generator=g)
    W, ds, Wo, dso = _weights_vs_oracle(gpu_ca, s, gw)
    y, yo = W @ v.numpy(), Wo @ v.double().numpy()
    say(f"   W {rel(W, Wo):.2e} W.V {rel(y, yo):.2e} dS {rel(ds, dso):.2e}")
    assert rel(W, Wo) <= 1e-4 and rel(y, yo) <= 1e-4 and rel(ds, dso) <= 1e-3
    np.testing.assert_allclose(W.sum(-1), 1.0, atol=2e-6)


# cuda/benchmark.py:36-38
FP16_CASES = [(9, 1.0), (32, 2.2), (129, 1.0), (192, 2.5), (512, 1.0), (2048, 1.0)]


@pytest.mark.parametrize("T,mag", FP16_CASES)
def test_v6_benchmark_fp16_cases(gpu_ca, T, mag):
    """cuda/benchmark.py:36-52 on the HIP operator: fp16 q, k, v, dY (q and k
    scaled by the magnitude), log-gains (0, ln(1/0.3)), query tile 128.
    Against the oracle on the same fp16 values: the outputs and q/k/v
    gradients are rounded to fp16 (half an ulp, 2^-11 relative, per
    element), so each element must lie within that rounding plus the
    north-star bar (1e-4 of the largest output, 1e-3 of the largest
    gradient); dlog_gain (fp32) at 1e-3; and the reference's own metric,
    relative L2 <= 1e-3 (cuda/benchmark.py:22-31)."""
    say(f"[case] v6 fp16 case T={T} magnitude={mag}")
    g = torch.Generator().manual_seed(1633 + T)
    q = (torch.randn(1, 2, T, 64, generator=g) * mag).half()
    k = (torch.randn(1, 2, T, 64, generator=g) * mag).half()
    v = torch.randn(1, 2, T, 64, generator=g).half()
    dy = torch.randn(1, 2, T, 64, generator=g).half()
    rho = torch.tensor([0.0, math.log(1 / .3)])
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (q, k, v))
    rd = rho.cuda().requires_grad_(True)
    y = gpu_ca.continuum_attention(qd, kd, vd, rd, 128)
    assert y.dtype == torch.float16
    grads = torch.autograd.grad((y.float() * dy.cuda().float()).sum(), (qd, kd, vd, rd))
    q64, k64, v64, dy64 = (x.double().numpy() for x in (q, k, v, dy))
    yo = O.ca_forward(q64, k64, v64, rho.double().numpy())[0]
    go = O.ca_backward(q64, k64, v64, rho.double().numpy(), dy64)
    half_ulp = 2.0 ** -11
    res = [("Y", y, yo, 1e-4)] + [(n, gr, r, 1e-3) for n, gr, r in zip(("dQ", "dK", "dV"), grads, go)]
    for name, got, ref, bar in res:
        got = got.detach().float().cpu().numpy().astype(np.float64)
        err = np.abs(got - ref) - (bar * np.abs(ref).max() + half_ulp * np.abs(ref))
        l2 = np.linalg.norm(got - ref) / max(np.linalg.norm(got), 1e-9)
        say(f"   {name}: max rel {rel(got, ref):.2e}, relative L2 {l2:.2e}")
        assert np.all(np.isfinite(got))
        assert err.max() <= 0, name
        assert l2 <= 1e-3, name
    er = rel(grads[3].cpu().numpy(), go[3])
    say(f"   dRho: max rel {er:.2e}")
    assert er <= 1e-3


@pytest.mark.parametrize("amp", [torch.float16, torch.bfloat16])
def test_full_decoder_causality(gpu_ca, amp):
    """cuda/benchmark.py:85-105: the 101,205,120-parameter CA-S decoder
    (seed 4242, eval, T 2048) under autocast; replacing every token after
    each cut leaves the logits up to the cut bitwise unchanged."""
    say(f"[case] full-decoder causality under {amp} autocast")
    Dm = gpu_ca.decoder
    torch.manual_seed(4242)
    cfg = Dm.ContinuumDecoderConfig(block_size=2048, d_model=1024, n_heads=16, n_layers=8,
                                    mlp_ratio=4., dropout=0., ca_query_tile=128)
    model = Dm.ContinuumDecoderLM(cfg).cuda().eval()
    assert sum(p.numel() for p in model.parameters()) == 101_205_120
    gen = torch.Generator().manual_seed(4243)
    ids = torch.randint(0, 256, (1, 2048), generator=gen).cuda()
    with torch.no_grad(), torch.autocast("cuda", dtype=amp):
        base = model(ids)["logits"]
        assert torch.isfinite(base).all()
        for cut in (127, 1023, 1024, 2046):
            edited = ids.clone()
            edited[:, cut + 1:] = torch.randint(0, 256, (1, 2047 - cut), generator=gen).cuda()
            changed = model(edited)["logits"]
            err = (base[:, :cut + 1] - changed[:, :cut + 1]).abs().max().item()
            moved = (base[:, cut + 1:] - changed[:, cut + 1:]).abs().max().item()
            say(f"   cut {cut}: earlier logits max_abs {err}, later logits moved {moved:.3g}")
            assert err == 0.0, cut
            assert moved > 0.0  # the edit did reach the model


def test_config2_sampled_rows_every_slice(gpu_ca):
    """Config 2 ([2,16,2048,64], seed 0, log_gain 0): rows 0, 1, 127, 128,
    1023, 1024, 2046, 2047 of all 32 slices against the row oracle (output
    and dQ: row i of both depends on row i of S alone)."""
    say("[case] config2 sampled rows of all 32 slices")
    torch.manual_seed(0)
    shape = (2, 16, 2048, 64)
    q, k, v = (torch.randn(shape) for _ in range(3))
    dy = torch.randn(shape)
    rho = torch.zeros(16)
    qd, kd, vd, rd = (x.cuda().requires_grad_(True) for x in (q, k, v, rho))
    y = gpu_ca.continuum_attention(qd, kd, vd, rd)
    dq = torch.autograd.grad((y * dy.cuda()).sum(), qd)[0]
    y, dq = y.detach().cpu().numpy(), dq.cpu().numpy()
    rows = np.array([0, 1, 127, 128, 1023, 1024, 2046, 2047])
    qn, kn, vn, dyn, rn = q.numpy(), k.numpy(), v.numpy(), dy.numpy(), rho.numpy()
    wy = wq = 0.0
    for b in range(2):
        for h in range(16):
            yr = O.ca_forward_rows(qn, kn, vn, rn, b, h, rows)
            dqr = O.ca_backward_rows(qn, kn, vn, rn, dyn, b, h, rows)[0]
            wy = max(wy, rel(y[b, h, rows], yr))
            wq = max(wq, rel(dq[b, h, rows], dqr))
    say(f"   worst slice: out {wy:.2e} dq {wq:.2e}")
    assert wy <= 1e-4 and wq <= 1e-3


def _rope_np(x, cs):
    """Interleaved rotation of x [..., T, D] by the table cs [T, D/2, 2] in float64."""
    c, s = cs[..., 0], cs[..., 1]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x1 * c + x0 * s
    return out


def _rope_back_np(g, cs):
    """The transposed rotation (the gradient of the un-rotated operand)."""
    c, s = cs[..., 0], cs[..., 1]
    g0, g1 = g[..., 0::2], g[..., 1::2]
    out = np.empty_like(g)
    out[..., 0::2] = g0 * c + g1 * s
    out[..., 1::2] = g1 * c - g0 * s
    return out


def _fused_layer(gpu_ca, T, H, D, dtype, seed, theta=1e4, bwd_caps=(None,)):
    """rope_continuum_attention on a random [1, T, 3HD] qkv in `dtype`:
    returns the inputs, the upstream gradient, the output and, per entry of
    bwd_caps (a workspace cap for the backward, None: the current one), the
    gradients (dqkv, dlog_gain) of the same forward."""
    Dm = gpu_ca.decoder
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(1, T, 3 * H * D, generator=g).to(dtype).cuda().requires_grad_(True)
    gain = (0.2 * torch.randn(H, generator=g)).cuda().requires_grad_(True)
    gout = torch.randn(1, T, H * D, generator=g).to(dtype).cuda()
    out = Dm.rope_continuum_attention(qkv, gain, theta, H)
    grads = []
    for i, cap in enumerate(bwd_caps):
        with (_capped(gpu_ca, cap) if cap is not None else _nothing()):
            grads.append(torch.autograd.grad(out, (qkv, gain), gout,
                                             retain_graph=i + 1 < len(bwd_caps)))
    torch.cuda.synchronize()
    return qkv.detach(), gain.detach(), gout, out.detach(), grads


class _nothing:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def _oracle_operands(gpu_ca, qkv, H, D, theta, dtype):
    """q, k (rotated as the kernels rotate them: the reference's apply_rope in
    the operand dtype) and v as float64 [1, H, T, D], plus the float64 table."""
    Dm = gpu_ca.decoder
    B, T, _ = qkv.shape
    q, k, v = qkv.view(B, T, 3, H, D).permute(2, 0, 3, 1, 4).unbind(0)
    qr, kr = Dm.apply_rope(q.contiguous(), k.contiguous(), theta)
    cs = Dm.rope_cos_sin(T, D, theta, qkv.device, dtype).double().cpu().numpy()
    return (qr.double().cpu().numpy(), kr.double().cpu().numpy(), v.double().cpu().numpy(), cs)


def test_fused_decoder_gradients_vs_oracle_fp32(gpu_ca):
    """The decoder's fused attention in fp32 ([1,300,3*2*64], RoPE, gains
    0.2 N(0,1)): output, dq and dk with RoPE transposed back, dv and
    dlog_gain against the oracle composed with the float64 rotation."""
    say("[case] fused decoder attention gradients vs oracle, fp32")
    T, H, D, theta = 300, 2, 64, 1e4
    qkv, gain, gout, out, [(dqkv, dgain)] = _fused_layer(gpu_ca, T, H, D, torch.float32, 17, theta)
    qn, kn, vn, cs = _oracle_operands(gpu_ca, qkv, H, D, theta, torch.float32)
    gn = gain.double().cpu().numpy()
    dy = gout.double().cpu().numpy().reshape(1, T, H, D).transpose(0, 2, 1, 3)
    yo = O.ca_forward(qn, kn, vn, gn)[0]
    dq, dk, dv, dr = O.ca_backward(qn, kn, vn, gn, dy)
    got = dqkv.double().cpu().numpy().reshape(1, T, 3, H, D).transpose(2, 0, 3, 1, 4)
    ey = rel(out.double().cpu().numpy().reshape(1, T, H, D).transpose(0, 2, 1, 3), yo)
    eq = rel(got[0], _rope_back_np(dq, cs))
    ek = rel(got[1], _rope_back_np(dk, cs))
    ev = rel(got[2], dv)
    er = rel(dgain.cpu().numpy(), dr)
    say(f"   out {ey:.2e} dq {eq:.2e} dk {ek:.2e} dv {ev:.2e} dgain {er:.2e}")
    assert ey <= 1e-4 and max(eq, ek, ev, er) <= 1e-3


def _capped(gpu_ca, nbytes):
    class _Cap:
        def __enter__(self):
            self.prev = gpu_ca.ops.workspace_cap()
            gpu_ca.ops.set_workspace_cap(nbytes)

        def __exit__(self, *exc):
            gpu_ca.ops.set_workspace_cap(self.prev)
    return _Cap()


def test_fused_decoder_backward_in_passes_matches_one_pass(gpu_ca):
    """One CA-S layer ([1,2048,3*16*64], bf16, RoPE) under a 24 MiB cap: the
    token-major backward runs in sets of heads, each in passes over query
    ranges, with dK and dV summed over the passes in fp32 and rounded once.
    Against the one-pass backward: every gradient differs only in the fp32
    summation order (dq: the dQ pass's chunking depends on the grid; dk, dv:
    the pass sums), then bf16 rounding: at most one bf16 ulp of the element,
    plus fp32 rounding (1e-6 of the tensor's largest value) where a sum
    cancels to near zero."""
    say("[case] token-major backward in passes vs one pass, bf16")
    lib = gpu_ca.native.load()
    T, H, D = 2048, 16, 64
    with _capped(gpu_ca, 24 << 20):
        need = lib.ca_bwd_qkv_workspace_bytes(1, H, T, D)
    say(f"   capped token-major backward workspace {need / 2**20:.1f} MiB")
    assert need <= 24 << 20
    # one forward, its backward in one pass and under the cap
    *_, (one, many) = _fused_layer(gpu_ca, T, H, D, torch.bfloat16, 23, bwd_caps=(None, 24 << 20))
    a = one[0].float().view(1, T, 3, H, D)
    b = many[0].float().view(1, T, 3, H, D)
    for i, name in enumerate(("dq", "dk", "dv")):
        d = (a[:, :, i] - b[:, :, i]).abs()
        scale = a[:, :, i].abs().max().item()
        bound = 2.0 ** -7 * torch.maximum(a[:, :, i].abs(), b[:, :, i].abs()) + 1e-6 * scale
        frac = (d > 0).float().mean().item()
        say(f"   {name}: max |diff| {d.max().item():.3g} (of max {scale:.3g}), "
            f"{100 * frac:.2f}% of elements differ, worst excess {(d - bound).max().item():.3g}")
        assert bool((d <= bound).all()), name
    eg = (one[1] - many[1]).abs().max().item() / one[1].abs().max().item()
    say(f"   dlog_gain rel diff {eg:.2e}")
    assert eg <= 1e-5


def test_fused_decoder_long_context_under_cap(gpu_ca):
    """One CA-S layer's attention at T 16384 (bf16, RoPE, 16 heads) under a
    256 MiB workspace cap, which the one-pass backward (about 8.6 GB) and
    even one query group of all 16 heads with the fp32 dK/dV sums exceed:
    sampled rows of the output and dq of every head, and dk, dv of the last
    256 keys of four heads, against the oracle (bf16 outputs: 4e-3 of the
    largest value, as for config 4)."""
    say("[case] token-major attention T=16384 under a 256 MiB cap, bf16")
    lib = gpu_ca.native.load()
    T, H, D, theta = 16384, 16, 64, 1e4
    with _capped(gpu_ca, 256 << 20):
        assert lib.ca_bwd_qkv_workspace_bytes(1, H, T, D) <= 256 << 20
        assert lib.ca_fwd_qkv_workspace_bytes(1, H, T, D) <= 256 << 20
        qkv, gain, gout, out, [(dqkv, dgain)] = _fused_layer(gpu_ca, T, H, D, torch.bfloat16, 29,
                                                             theta)
    qn, kn, vn, cs = _oracle_operands(gpu_ca, qkv, H, D, theta, torch.bfloat16)
    gn = gain.double().cpu().numpy()
    dy = gout.double().cpu().numpy().reshape(1, T, H, D).transpose(0, 2, 1, 3)
    y = out.double().cpu().numpy().reshape(1, T, H, D).transpose(0, 2, 1, 3)
    got = dqkv.double().cpu().numpy().reshape(1, T, 3, H, D).transpose(2, 0, 3, 1, 4)
    assert np.all(np.isfinite(got)) and np.all(np.isfinite(y))
    rng = np.random.default_rng(31)
    rows = np.unique(np.concatenate([[0, 1, 127, 128, 2047, 2048, 8191, 8192, T - 2, T - 1],
                                     rng.integers(0, T, 6)]))
    wy = wq = 0.0
    for h in range(H):
        yr = O.ca_forward_rows(qn, kn, vn, gn, 0, h, rows)
        dqr = O.ca_backward_rows(qn, kn, vn, gn, dy, 0, h, rows)[0]
        wy = max(wy, rel(y[0, h, rows], yr))
        wq = max(wq, rel(got[0][0, h, rows], _rope_back_np(dqr, cs[rows])))
    say(f"   sampled rows of 16 heads: out {wy:.2e} dq {wq:.2e}")
    assert wy <= 4e-3 and wq <= 4e-3
    suffix = np.arange(T - 256, T)
    for h in (0, 5, 10, 15):
        _, dk_s, dv_s, _ = O.ca_backward_rows(qn, kn, vn, gn, dy, 0, h, suffix)
        ek = rel(got[1][0, h, suffix], _rope_back_np(dk_s[suffix], cs[suffix]))
        ev = rel(got[2][0, h, suffix], dv_s[suffix])
        say(f"   head {h} last 256 keys: dk {ek:.2e} dv {ev:.2e}")
        assert ek <= 4e-3 and ev <= 4e-3
    # dlog_gain = sum_j k_j . dK_j over all keys (every dS row sums to zero),
    # with k and dK of the rotated keys: the kernels rotate the gradient back
    # with the table R = [[c, s], [-s, c]] of rounded (c, s), so R^T applied
    # to it gives (c^2 + s^2) times the rotated keys' gradient
    cs2 = (cs[..., 0] ** 2 + cs[..., 1] ** 2).repeat(2, -1)
    dk_rot = _rope_np(got[1], cs) / cs2
    kdk = (kn * dk_rot).sum(axis=(0, 2, 3))
    mag = np.abs(kn * dk_rot).sum(axis=(0, 2, 3))
    dg = dgain.double().cpu().numpy()
    say(f"   max |k.dK - dlog_gain| / sum|k.dK|: {np.max(np.abs(kdk - dg) / mag):.2e}")
    assert np.all(np.abs(kdk - dg) <= 4e-3 * mag)


def test_operator_backward_in_head_sets(gpu_ca):
    """The fp32 operator ([2,4,1000,64], gains, seed 37) under a 2 MiB cap,
    below one query group of all eight slices: the backward runs in sets of
    heads per batch (dlog_gain summed over the batches' sets in order),
    against the oracle."""
    say("[case] fp32 operator backward in head sets")
    lib = gpu_ca.native.load()
    shape = (2, 4, 1000, 64)
    g = torch.Generator().manual_seed(37)
    q, k, v, dy = (torch.randn(shape, generator=g) for _ in range(4))
    rho = torch.tensor([0.0, 0.3, -0.2, 0.5])
    with _capped(gpu_ca, 2 << 20):
        need = lib.ca_bwd_workspace_bytes(*shape)
        say(f"   backward workspace {need / 2**20:.2f} MiB")
        assert need <= 2 << 20
        qd, kd, vd, rd = (x.cuda().requires_grad_(True) for x in (q, k, v, rho))
        y = gpu_ca.continuum_attention(qd, kd, vd, rd)
        grads = torch.autograd.grad((y * dy.cuda()).sum(), (qd, kd, vd, rd))
    yo = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), rho.numpy())[0]
    go = O.ca_backward(q.numpy(), k.numpy(), v.numpy(), rho.numpy(), dy.numpy())
    ey = rel(y.detach().cpu().numpy(), yo)
    eg = [rel(a.cpu().numpy(), b) for a, b in zip(grads, go)]
    say(f"   out {ey:.2e} dq {eg[0]:.2e} dk {eg[1]:.2e} dv {eg[2]:.2e} drho {eg[3]:.2e}")
    assert ey <= 1e-4 and max(eg) <= 1e-3

"""GPU parity of the weight-materialising kernels and of the operator's callers.

* ``ca_weights`` / ``continuous_attention_weights`` / ``ca_weights_backward``
  (csrc/ca_weights.hip through the C ABI) against the float64 oracle
  (oracle/ca_oracle.py: ``ca_weights``, ``ca_weights_vjp``); bars 1e-4 on
  weights, 1e-3 on score gradients (max|x-ref|/max|ref|), exact zeros beyond
  each row's prefix; the reference tests' weight properties
  (test_fusion.py:27-35, test_acma.py:104-110,127-138).
* ``CausalAttention`` with the fused operator ('hip') against the
  materialised path ('hip_weights') and against a float64 composition with
  the oracle; ``TinyLM`` causality (test_acma.py:118-126) and controls
  (test_acma.py:140-146); one CA-S decoder training step and decoder logits
  against a float64 CPU model whose attention is the oracle.
"""
import contextlib
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ca_oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


@pytest.mark.parametrize("T,mag", [(1, 1.0), (2, 1.0), (7, 1.0), (15, 1.0), (63, 2.0), (64, 0.0),
                                   (65, 4.0), (257, 1.0), (1000, 3.0)])
def test_weights_and_vjp_vs_oracle(gpu_ca, T, mag):
    say(f"[case] weights T={T} mag={mag}")
    g = torch.Generator().manual_seed(T)
    s = torch.randn(2, 3, T, T, generator=g) * mag
    gw = torch.randn(2, 3, T, T, generator=g)
    sd = s.cuda().requires_grad_(True)
    W = gpu_ca.continuous_attention_weights(sd)
    (ds,) = torch.autograd.grad(W, sd, gw.cuda())
    Wo = O.ca_weights(s.double().numpy())[0]
    dso = O.ca_weights_vjp(s.double().numpy(), gw.double().numpy())
    W, ds = W.detach().cpu().numpy(), ds.cpu().numpy()
    ew, eds = rel(W, Wo), rel(ds, dso)
    say(f"   W {ew:.2e} dS {eds:.2e}")
    assert ew <= 1e-4 and eds <= 1e-3
    fut = np.triu(np.ones((T, T), bool), 1)
    assert np.all(W[..., fut] == 0.0) and np.all(ds[..., fut] == 0.0)
    assert np.all(W >= 0.0)
    np.testing.assert_allclose(W.sum(-1), 1.0, atol=2e-6)


def test_weights_query_tile_offset_and_stats(gpu_ca):
    """ext.forward(scores, start) semantics: a tile of queries start..start+Q-1
    over K >= start+Q keys (cuda/continuum_attention.py:622-648); stats are the
    row max and 1/Z; ext.backward_fused returns (W, dS)."""
    say("[case] weights tile offset")
    g = torch.Generator().manual_seed(9)
    K, start, Q = 300, 128, 64
    s = torch.randn(4, Q, K, generator=g) * 2.0
    gw = torch.randn(4, Q, K, generator=g)
    W, stats = gpu_ca.ca_weights(s.cuda(), start)
    W2, ds = gpu_ca.ca_weights_backward(s.cuda(), gw.cuda(), start, return_weights=True)
    qidx = np.arange(start, start + Q)
    Wo, mo, zo = O.ca_weights(s.double().numpy(), qidx)
    dso = O.ca_weights_vjp(s.double().numpy(), gw.double().numpy(), qidx=qidx)
    W, W2, ds, stats = (x.cpu().numpy() for x in (W, W2, ds, stats))
    assert rel(W, Wo) <= 1e-4 and rel(W2, Wo) <= 1e-4
    assert rel(ds, dso) <= 1e-3
    np.testing.assert_allclose(stats[:, 0], mo.reshape(-1), rtol=0, atol=1e-6)
    np.testing.assert_allclose(stats[:, 1], 1.0 / zo.reshape(-1), rtol=1e-5)
    for r in range(Q):
        assert np.all(W[:, r, start + r + 1:] == 0.0)
    with pytest.raises(ValueError):
        gpu_ca.ca_weights(s[:, :, :start + Q - 1].contiguous().cuda(), start)


def test_weight_properties_from_reference_tests(gpu_ca):
    """test_fusion.py:27-35 (non-negative, rows sum to 1, W00 = 1),
    test_acma.py:104-110 (scores receive finite non-zero gradients),
    test_acma.py:127-138 (not plain softmax)."""
    say("[case] weight properties")
    torch.manual_seed(22)
    s = torch.randn(2, 3, 15, 15, device="cuda")
    W = gpu_ca.continuous_attention_weights(s)
    assert (W >= 0).all().item()
    torch.testing.assert_close(W.sum(-1), torch.ones_like(W.sum(-1)), atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(W[..., 0, 0], torch.ones_like(W[..., 0, 0]))
    logits = torch.randn(2, 2, 7, 7, device="cuda", requires_grad=True)
    w = gpu_ca.continuous_attention_weights(logits)
    (w * torch.randn_like(w)).sum().backward()
    assert torch.isfinite(logits.grad).all().item() and logits.grad.abs().sum().item() > 0
    lg = torch.tensor([[[[0., 0., 0.], [0., 2., 0.], [1., -1., 3.]]]], device="cuda")
    w = gpu_ca.continuous_attention_weights(lg)
    causal = torch.ones(3, 3, dtype=torch.bool, device="cuda").tril()
    std = torch.softmax(lg.masked_fill(~causal, -torch.inf), -1)
    assert (w - std).abs().sum().item() > .01


def _oracle_attention_np(x, attn):
    """float64 composition of CausalAttention.forward with the oracle weights."""
    Wqkv = attn.qkv.weight.detach().double().cpu().numpy()
    Wout = attn.out.weight.detach().double().cpu().numpy()
    B, T, C = x.shape
    H, Dh = attn.heads, attn.head_dim
    qkv = x @ Wqkv.T
    q, k, v = (qkv[..., i * C:(i + 1) * C].reshape(B, T, H, Dh).transpose(0, 2, 1, 3) for i in range(3))
    if attn.variant in ("B", "P"):
        q = q / attn.fixed_tau
    elif attn.variant in ("F", "G", "S", "H"):
        q = q * np.exp(attn.log_qk_gain.detach().double().cpu().numpy())[None, :, None, None]
    y = O.ca_forward(q, k, v, np.zeros(H))[0]
    return y.transpose(0, 2, 1, 3).reshape(B, T, C) @ Wout.T


@pytest.mark.parametrize("variant", ["P", "R", "S", "H"])
def test_causal_attention_fused_vs_weights_vs_oracle(gpu_ca, variant):
    say(f"[case] CausalAttention variant {variant}")
    A = gpu_ca.architecture
    torch.manual_seed(11)
    x = torch.randn(2, 70, 128)
    outs, grads = {}, {}
    for backend in ("hip", "hip_weights"):
        torch.manual_seed(1)
        attn = A.CausalAttention(128, 2, 128, variant=variant, backend=backend).cuda()
        xd = x.cuda().requires_grad_(True)
        y = attn(xd)
        params = [xd, attn.qkv.weight] + ([attn.log_qk_gain] if hasattr(attn, "log_qk_gain") else [])
        grads[backend] = [gg.cpu().numpy() for gg in torch.autograd.grad((y * y).sum(), params)]
        outs[backend] = y.detach().cpu().numpy()
    ref = _oracle_attention_np(x.double().numpy(), attn)
    e_f, e_w = rel(outs["hip"], ref), rel(outs["hip_weights"], ref)
    say(f"   out fused {e_f:.2e} weights {e_w:.2e}")
    assert e_f <= 1e-4 and e_w <= 1e-4
    for a, b in zip(grads["hip"], grads["hip_weights"]):
        assert rel(a, b) <= 1e-3


def test_tinylm_no_future_leak_and_controls(gpu_ca):
    """test_acma.py:118-126 (a prefix's logits do not see later tokens) and
    test_acma.py:140-146 (R == S at initialisation, exactly)."""
    say("[case] TinyLM causality")
    A = gpu_ca.architecture
    ids = torch.randint(0, 256, (2, 13), device="cuda")
    mod = ids.clone()
    mod[:, 7:] = torch.randint(0, 256, (2, 6), device="cuda")
    for backend in ("hip", "hip_weights"):
        for variant in ("P", "R", "S"):
            torch.manual_seed(97)
            m = A.TinyLM(variant=variant, backend=backend, seq_len=16, width=32, hidden=64,
                         heads=4).cuda().eval()
            with torch.no_grad():
                torch.testing.assert_close(m(ids)[:, :7], m(mod)[:, :7], atol=2e-5, rtol=2e-5)
    with torch.no_grad():
        torch.manual_seed(97)
        r = A.TinyLM(variant="R", seq_len=16, width=32, hidden=64, heads=4).cuda()
        torch.manual_seed(97)
        s = A.TinyLM(variant="S", seq_len=16, width=32, hidden=64, heads=4).cuda()
        torch.testing.assert_close(r(ids), s(ids), atol=0, rtol=0)


def test_tinylm_512_finite(gpu_ca):
    """test_long.py:54-61."""
    A = gpu_ca.architecture
    torch.manual_seed(1729)
    m = A.TinyLM(variant="S", seq_len=512, width=32, hidden=64, heads=4).cuda()
    with torch.no_grad():
        out = m(torch.randint(0, 256, (1, 512), device="cuda"))
    assert tuple(out.shape) == (1, 512, 256) and torch.isfinite(out).all().item()


class _OracleCA(torch.autograd.Function):
    """Float64 CPU attention through the oracle (forward only)."""

    @staticmethod
    def forward(ctx, q, k, v, log_gain, query_tile=64):
        y = O.ca_forward(q.numpy(), k.numpy(), v.numpy(), log_gain.detach().numpy())[0]
        return torch.from_numpy(y)


@pytest.mark.parametrize("d_model", [128, 256])
def test_decoder_logits_vs_float64_oracle_model(gpu_ca, monkeypatch, d_model):
    """Small CA-S decoder: fp32 GPU logits against a float64 CPU copy of the
    same model whose attention is the oracle (head dims 64 and 128)."""
    say(f"[case] decoder logits vs float64 oracle model, d_model {d_model}")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=d_model, n_heads=2, n_layers=2, block_size=96)
    torch.manual_seed(4)
    m = Dm.ContinuumDecoderLM(cfg)
    with torch.no_grad():
        for blk in m.blocks:
            blk.attn.log_qk_gain.copy_(torch.tensor([0.3, -0.2]))
    ids = torch.randint(0, 256, (2, 96))
    with torch.no_grad():
        got = m.cuda()(ids.cuda())["logits"].cpu().numpy()
        m64 = Dm.ContinuumDecoderLM(cfg).double()
        m64.load_state_dict({k: v.double().cpu() for k, v in m.state_dict().items()})
        monkeypatch.setattr(Dm, "continuum_attention",
                            lambda q, k, v, g, t=64: _OracleCA.apply(q, k, v, g, t))
        ref = m64(ids)["logits"].numpy()
    e = rel(got, ref)
    say(f"   logits rel {e:.2e}")
    assert e <= 1e-4


def test_decoder_train_step_bf16(gpu_ca):
    """One CA-S training step (bf16 autocast, fp32 CA scores): finite loss near
    ln 256 at initialisation, finite gradients reaching every gain."""
    say("[case] decoder train step")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=256, n_heads=4, n_layers=2, block_size=256)
    torch.manual_seed(0)
    m = Dm.ContinuumDecoderLM(cfg).cuda()
    opt = Dm.build_adamw(m)
    batch = torch.randint(0, 256, (2, 256), device="cuda")
    g0 = [b.attn.log_qk_gain.detach().clone() for b in m.blocks]
    loss = Dm.train_step(m, opt, batch)
    torch.cuda.synchronize()
    assert abs(loss.item() - np.log(256)) < 0.1
    for b, g in zip(m.blocks, g0):
        assert b.attn.log_qk_gain.grad is not None
        assert torch.isfinite(b.attn.log_qk_gain.grad).all().item()
        assert not torch.equal(b.attn.log_qk_gain.detach(), g)  # the step moved the gains


def _unfused_attention(Dm, qkv, log_gain, theta, heads):
    """Reference op-by-op composition: view/permute, RoPE, operator, transpose."""
    Bsz, T, C3 = qkv.shape
    q, k, v = qkv.view(Bsz, T, 3, heads, C3 // 3 // heads).permute(2, 0, 3, 1, 4).unbind(0)
    q, k = Dm.apply_rope(q, k, theta)
    y = Dm.continuum_attention(q, k, v, log_gain, 64)
    return y.transpose(1, 2).reshape(Bsz, T, C3 // 3)


def _qkv_call(ca, qkv, gain, cs, H, dout, rotate_keys_first=(False, True)):
    """ca_fwd_qkv + ca_bwd_qkv through the C ABI: (y fp32 heads, out, dqkv, dgain).
    rotate_keys_first: (forward, backward) workspaces with room for the keys
    rotated once (ca_fwd_qkv_workspace_bytes / ca_bwd_qkv_workspace_bytes), or
    without it (the kernels then rotate the keys they read)."""
    lib = ca.native.load()
    Bsz, T, C3 = qkv.shape
    D = C3 // 3 // H
    code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[qkv.dtype]
    y = torch.empty(Bsz, H, T, D, device="cuda")
    out = torch.empty(Bsz, T, H * D, device="cuda", dtype=qkv.dtype)
    st = torch.empty(Bsz * H * T, 2, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    nf = (lib.ca_fwd_qkv_workspace_bytes if rotate_keys_first[0] else lib.ca_fwd_workspace_bytes)(
        Bsz, H, T, D)
    wf = torch.empty(max(nf, 1), device="cuda", dtype=torch.uint8)
    csp = cs.data_ptr() if cs is not None else None
    ca.native.check(lib.ca_fwd_qkv(qkv.data_ptr(), code, csp, gain.data_ptr(), y.data_ptr(),
                                   out.data_ptr(), st.data_ptr(), wf.data_ptr(), nf, Bsz, T, H, D, s))
    nb = lib.ca_bwd_qkv_workspace_bytes(Bsz, H, T, D)
    if not rotate_keys_first[1]:
        nb -= (Bsz * H * T * D * 4 + 255) // 256 * 256
    wb = torch.empty(nb, device="cuda", dtype=torch.uint8)
    dqkv = torch.empty_like(qkv)
    dg = torch.empty(H, device="cuda")
    ca.native.check(lib.ca_bwd_qkv(qkv.data_ptr(), code, csp, gain.data_ptr(), y.data_ptr(),
                                   st.data_ptr(), dout.data_ptr(), dqkv.data_ptr(), dg.data_ptr(),
                                   wb.data_ptr(), nb, Bsz, T, H, D, s))
    torch.cuda.synchronize()
    return y, out, dqkv, dg


@pytest.mark.parametrize("D,T,splits", [(64, 130, (0, 0, 0)), (16, 77, (0, 0, 0)),
                                        (128, 300, (0, 0, 0)), (64, 700, (1, 1, 1)),
                                        (32, 520, (4, 16, 6))])
def test_qkv_entry_points_match_the_operator(gpu_ca, D, T, splits):
    """ca_fwd_qkv / ca_bwd_qkv read the token-major qkv [B,T,3,H,D] and write
    the output and dqkv token-major.  Without rotation they are the
    operator's kernels on the same values, so for fp32, bf16 and fp16 qkv:
    y is bitwise the operator's output on the upcast q, k, v; the token-major
    output is y rounded to the dtype; dqkv is the operator's gradients
    rounded to the dtype.  bf16 is the exception for the gradients: its dK/dV
    kernel forms q.k of the bf16 values and scales it after the product,
    where the fp32 kernel scales k first, so its scores differ in fp32
    rounding and a few gradient elements round to the neighbouring bf16
    value.  With RoPE, against the operator on q, k rotated in fp32
    beforehand (rounding-level differences only).  Forced splits run the
    combine and merge kernels' token-major writes."""
    say(f"[case] qkv entry points D={D} T={T} splits {splits}")
    Dm = gpu_ca.decoder
    gpu_ca.ops.set_split_override(*splits)
    try:
        Bsz, H = 2, 3
        g = torch.Generator().manual_seed(D + T)
        gain = torch.tensor([0.0, 0.3, -0.25], device="cuda")
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            qkv = (torch.randn(Bsz, T, 3 * H * D, generator=g) * 1.3).to(dt).cuda()
            dout = torch.randn(Bsz, T, H * D, generator=g).to(dt).cuda()
            y, out, dqkv, dg = _qkv_call(gpu_ca, qkv, gain, None, H, dout)
            q, k, v = (t.contiguous() for t in qkv.float().view(Bsz, T, 3, H, D).permute(2, 0, 3, 1, 4))
            dyh = dout.float().view(Bsz, T, H, D).transpose(1, 2).contiguous()
            yr, st = gpu_ca.ca_forward(q, k, v, gain)
            dq, dk, dv, dgr = gpu_ca.ca_backward(q, k, v, gain, yr, st, dyh)
            assert torch.equal(y, yr), dt
            assert torch.equal(out, yr.transpose(1, 2).reshape(Bsz, T, H * D).to(dt)), dt
            ref = torch.stack((dq, dk, dv), 2).transpose(1, 3).reshape(Bsz, T, 3 * H * D).to(dt)
            if dt == torch.bfloat16:
                unequal = (dqkv != ref).float().mean().item()
                e_q = rel(dqkv.float().cpu().numpy(), ref.float().cpu().numpy())
                e_g = rel(dg.cpu().numpy(), dgr.cpu().numpy())
                say(f"   bf16: {unequal:.2e} of dqkv differ, rel {e_q:.1e}; dgain rel {e_g:.1e}")
                assert unequal <= 0.02 and e_q <= 2.0 ** -7 and e_g <= 1e-5
            else:
                assert torch.equal(dqkv, ref), dt
                assert torch.equal(dg, dgr), dt
        # RoPE in the kernels vs rotating first
        qkv = (torch.randn(Bsz, T, 3 * H * D, generator=g) * 1.3).cuda()
        dout = torch.randn(Bsz, T, H * D, generator=g).cuda()
        cs = Dm.rope_cos_sin(T, D, 10000.0, qkv.device)
        y, out, dqkv, dg = _qkv_call(gpu_ca, qkv, gain, cs, H, dout)
        q, k, v = qkv.view(Bsz, T, 3, H, D).permute(2, 0, 3, 1, 4)

        def rot(x, inverse=False):
            x0, x1 = x[..., 0::2], x[..., 1::2]
            c, s_ = cs[..., 0], (-cs[..., 1] if inverse else cs[..., 1])
            return torch.stack((x0 * c - x1 * s_, x1 * c + x0 * s_), -1).flatten(-2).contiguous()
        qr, kr = rot(q), rot(k)
        dyh = dout.view(Bsz, T, H, D).transpose(1, 2).contiguous()
        yr, st = gpu_ca.ca_forward(qr, kr, v.contiguous(), gain)
        dq, dk, dv, dgr = gpu_ca.ca_backward(qr, kr, v.contiguous(), gain, yr, st, dyh)
        ref = torch.stack((rot(dq, True), rot(dk, True), dv), 2).transpose(1, 3).reshape(Bsz, T, 3 * H * D)
        e = [rel(a.cpu().numpy(), b.cpu().numpy()) for a, b in
             ((y, yr), (out, yr.transpose(1, 2).reshape(Bsz, T, H * D)), (dqkv, ref), (dg, dgr))]
        say("   rope: y %.1e out %.1e dqkv %.1e dgain %.1e" % tuple(e))
        assert e[0] <= 1e-6 and e[1] <= 1e-6 and e[2] <= 1e-5 and e[3] <= 1e-5
    finally:
        gpu_ca.ops.set_split_override(0, 0, 0)


def test_qkv_bf16_at_the_ca_s_layer_shape(gpu_ca):
    """One CA-S layer's shape, [1,16,2048,64], through the token-major entry
    points in bf16 with the automatic work splits (bf16 dK/dV takes 16-tile
    chunks there, the fp32 kernels 24) against the fp32 operator on the same
    values (pinned against the oracle by the parity tests): the output equal
    bit for bit, the gradients within bf16 rounding of the fp32 operator's
    and the gain gradient within fp32 rounding."""
    say("[case] bf16 qkv entry points at [1,16,2048,64]")
    Bsz, T, H, D = 1, 2048, 16, 64
    g = torch.Generator().manual_seed(64)
    gain = (torch.randn(H, generator=g) * 0.3).cuda()
    qkv = (torch.randn(Bsz, T, 3 * H * D, generator=g) * 1.3).to(torch.bfloat16).cuda()
    dout = torch.randn(Bsz, T, H * D, generator=g).to(torch.bfloat16).cuda()
    y, out, dqkv, dg = _qkv_call(gpu_ca, qkv, gain, None, H, dout)
    q, k, v = (t.contiguous() for t in qkv.float().view(Bsz, T, 3, H, D).permute(2, 0, 3, 1, 4))
    dyh = dout.float().view(Bsz, T, H, D).transpose(1, 2).contiguous()
    yr, st = gpu_ca.ca_forward(q, k, v, gain)
    dq, dk, dv, dgr = gpu_ca.ca_backward(q, k, v, gain, yr, st, dyh)
    assert torch.equal(y, yr)
    ref = torch.stack((dq, dk, dv), 2).transpose(1, 3).reshape(Bsz, T, 3 * H * D)
    ref16 = ref.to(torch.bfloat16)
    unequal = (dqkv != ref16).float().mean().item()
    e_q = rel(dqkv.float().cpu().numpy(), ref.cpu().numpy())
    e_g = rel(dg.cpu().numpy(), dgr.cpu().numpy())
    say(f"   {unequal:.2e} of dqkv differ from the rounded fp32 gradients, rel {e_q:.1e}; "
        f"dgain rel {e_g:.1e}")
    assert unequal <= 0.02 and e_q <= 2.0 ** -7 and e_g <= 1e-5


@pytest.mark.parametrize("D,T", [(64, 300), (16, 77), (128, 130)])
def test_qkv_keys_rotated_once_match_in_kernel_rotation(gpu_ca, D, T):
    """With RoPE the token-major entry points rotate the keys once into their
    workspace when it has the room, else the kernels rotate the keys they
    read: the same arithmetic (the reference's rounding to the operand type),
    so outputs and gradients agree bit for bit, for each operand type."""
    say(f"[case] keys rotated once vs in-kernel, D={D} T={T}")
    Bsz, H = 2, 3
    g = torch.Generator().manual_seed(3 * D + T)
    gain = torch.tensor([0.0, 0.3, -0.25], device="cuda")
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        qkv = (torch.randn(Bsz, T, 3 * H * D, generator=g) * 1.3).to(dt).cuda()
        dout = torch.randn(Bsz, T, H * D, generator=g).to(dt).cuda()
        cs = gpu_ca.decoder.rope_cos_sin(T, D, 10000.0, qkv.device, dt)
        a = _qkv_call(gpu_ca, qkv, gain, cs, H, dout, (True, True))
        b = _qkv_call(gpu_ca, qkv, gain, cs, H, dout, (False, False))
        for x, y in zip(a, b):
            assert torch.equal(x, y), dt


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_rope_attention_vs_unfused(gpu_ca, dtype):
    """The decoder's fused prologue/epilogue against the reference composition
    (apply_rope + operator + transpose): outputs and gradients of qkv and the
    gains.  fp32: RoPE rounding only.  bf16: both rotate as the reference does
    in bf16 (cuda/continuum_attention.py:826-835) and the fused kernels skip
    the zero limb products of the bf16-valued operands, so the output is the
    composition's bit for bit; the gain gradient differs in fp32 rounding
    (the fused dK/dV kernel scales q.k after the product, as bf16 operands
    allow, the composition's fp32 kernel scales k first), and the qkv gradient
    by the rotation backward's rounding (the composition rounds each of its
    steps to bf16, the fused epilogue rotates in fp32 and rounds once)."""
    say(f"[case] fused rope attention {dtype}")
    Dm = gpu_ca.decoder
    torch.manual_seed(8)
    Bsz, T, H, D, theta = 2, 130, 4, 64, 10000.0
    qkv = (torch.randn(Bsz, T, 3 * H * D) * 1.5).cuda().to(dtype)
    gain = torch.tensor([0.0, 0.3, -0.2, 0.1], device="cuda")
    dout = torch.randn(Bsz, T, H * D).cuda().to(dtype)
    res = {}
    for name, fn in (("fused", lambda a, b: Dm.rope_continuum_attention(a, b, theta, H)),
                     ("unfused", lambda a, b: _unfused_attention(Dm, a, b, theta, H))):
        a = qkv.clone().requires_grad_(True)
        b = gain.clone().requires_grad_(True)
        y = fn(a, b)
        assert y.dtype == dtype and y.shape == (Bsz, T, H * D)
        ga, gb = torch.autograd.grad(y, (a, b), dout)
        res[name] = [t.float().cpu().numpy() for t in (y.detach(), ga, gb)]
    errs = [rel(x, r) for x, r in zip(res["fused"], res["unfused"])]
    say(f"   out {errs[0]:.2e} dqkv {errs[1]:.2e} dgain {errs[2]:.2e}")
    if dtype == torch.float32:
        assert errs[0] <= 2e-5 and errs[1] <= 2e-4 and errs[2] <= 2e-4
    else:
        assert errs[0] == 0.0 and errs[2] <= 1e-5 and errs[1] <= 2e-2


def _rmsnorm_composition(x, w, eps):
    return w * x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps)


@pytest.mark.parametrize("rows,C", [(1, 256), (37, 1024), (130, 1000), (2048, 1024), (5, 4096),
                                     (3, 257), (300, 771), (3000, 64)])
def test_rmsnorm_fused_vs_composition(gpu_ca, rows, C):
    """The decoder's fused RMSNorm (ca_rmsnorm_fwd/bwd through the C ABI)
    against the reference's torch composition (cuda/continuum_attention.py:
    817-823) and its autograd: fp32 output and dx, dweight; bf16/fp16 outputs
    equal the composition's rounded to that dtype (within one ulp, the
    composition's mean is summed in another order), and dy in that dtype."""
    Dm = gpu_ca.decoder
    g = torch.Generator().manual_seed(rows + C)
    x = (torch.randn(rows, C, generator=g) * 3 + 0.5).cuda()
    w = (torch.rand(C, generator=g) + 0.5).cuda()
    for out_dtype in (torch.float32, torch.bfloat16, torch.float16):
        say(f"[case] rmsnorm rows={rows} C={C} {out_dtype}")
        dy = torch.randn(rows, C, generator=g).cuda().to(out_dtype)
        xa, wa = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        y = Dm._RMSNormFn.apply(xa, wa, 1e-6, out_dtype)
        assert y.dtype == out_dtype
        dx, dw = torch.autograd.grad(y, (xa, wa), dy)
        xb, wb = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        yr = _rmsnorm_composition(xb, wb, 1e-6)
        dxr, dwr = torch.autograd.grad(yr, (xb, wb), dy.float())
        if out_dtype == torch.float32:
            ey = rel(y.detach().cpu().numpy(), yr.detach().cpu().numpy())
            assert ey <= 1e-6
        else:
            yc = yr.detach().to(out_dtype).float()
            ulp = 2.0 ** (-7 if out_dtype == torch.bfloat16 else -10)
            diff = (y.detach().float() - yc).abs() / yc.abs().clamp_min(1e-30)
            ey = diff.max().item()
            assert ey <= ulp
        ex = rel(dx.cpu().numpy(), dxr.cpu().numpy())
        ew = rel(dw.cpu().numpy(), dwr.cpu().numpy())
        say(f"   y {ey:.2e} dx {ex:.2e} dweight {ew:.2e}")
        assert ex <= 1e-5 and ew <= 1e-5


@pytest.mark.parametrize("rows,C,rdt", [(37, 1024, torch.float32), (2048, 1024, torch.bfloat16),
                                         (300, 771, torch.bfloat16), (5, 4096, torch.float16)])
@pytest.mark.parametrize("use_s", [True, False])
def test_add_rmsnorm_fused_vs_composition(gpu_ca, rows, C, rdt, use_s):
    """ca_add_rmsnorm_fwd/bwd (the decoder's residual add fused into the norm
    that reads it) against torch's s = x + res, RMSNorm(s) and autograd:
    s bit-exact, y as the fused RMSNorm, gradients of x (plus the gradient s
    receives downstream, or none), res (in its dtype) and weight."""
    say(f"[case] add+rmsnorm rows={rows} C={C} res {rdt} s used {use_s}")
    Dm = gpu_ca.decoder
    g = torch.Generator().manual_seed(rows + C)
    x = (torch.randn(rows, C, generator=g) * 2).cuda()
    res = torch.randn(rows, C, generator=g).cuda().to(rdt)
    w = (torch.rand(C, generator=g) + 0.5).cuda()
    gy = torch.randn(rows, C, generator=g).cuda().to(rdt)
    gsum = torch.randn(rows, C, generator=g).cuda()
    xa, ra, wa = (t.clone().requires_grad_(True) for t in (x, res, w))
    s, y = Dm._AddRMSNormFn.apply(xa, ra, wa, 1e-6, rdt)
    outs, grads = ((s, y), (gsum, gy)) if use_s else ((y,), (gy,))
    dx, dr, dw = torch.autograd.grad(outs, (xa, ra, wa), grads)
    xb, rb, wb = (t.clone().requires_grad_(True) for t in (x, res, w))
    sr = xb + rb
    yr = _rmsnorm_composition(sr, wb, 1e-6)
    outs_r, grads_r = ((sr, yr), (gsum, gy.float())) if use_s else ((yr,), (gy.float(),))
    dxr, drr, dwr = torch.autograd.grad(outs_r, (xb, rb, wb), grads_r)
    assert torch.equal(s.detach(), sr.detach())
    assert dr.dtype == rdt
    if rdt == torch.float32:
        assert rel(y.detach().cpu().numpy(), yr.detach().cpu().numpy()) <= 1e-6
    else:
        yc = yr.detach().to(rdt).float()
        ulp = 2.0 ** (-7 if rdt == torch.bfloat16 else -10)
        assert ((y.detach().float() - yc).abs() / yc.abs().clamp_min(1e-30)).max().item() <= ulp
    ex = rel(dx.cpu().numpy(), dxr.cpu().numpy())
    er = rel(dr.float().cpu().numpy(), drr.float().cpu().numpy())
    ew = rel(dw.cpu().numpy(), dwr.cpu().numpy())
    say(f"   dx {ex:.2e} dres {er:.2e} dweight {ew:.2e}")
    assert ex <= 1e-5 and ew <= 1e-5
    assert er <= (1e-5 if rdt == torch.float32 else 4e-3)


@pytest.mark.parametrize("clip", [0.05, 1e9])
def test_train_step_clip_in_adamw(gpu_ca, clip):
    """train_step hands clip_grad_norm_'s factor to the fused AdamW kernel as
    its gradient divisor: the clipped gradients left in .grad, AdamW's first
    moments and the parameters match torch's clip_grad_norm_ + step
    (cuda/continuum_attention.py:1205-1228), with the clip active (0.05) and
    inactive."""
    say(f"[case] clip in AdamW, max_norm {clip}")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(3)
    ma = Dm.ContinuumDecoderLM(cfg).cuda()
    mb = Dm.ContinuumDecoderLM(cfg).cuda()
    mb.load_state_dict(ma.state_dict())
    oa, ob = Dm.build_adamw(ma), Dm.build_adamw(mb)
    assert Dm._fused_on_gpu(oa)
    ids = torch.randint(0, 256, (2, 64), device="cuda")
    # one step from equal parameters: equal gradients before the clip, so any
    # difference is the clip's (a second step would compare bf16 forwards of
    # parameters that differ in their last bits)
    Dm.train_step(ma, oa, ids, grad_clip=clip)
    ob.zero_grad(set_to_none=True)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss = mb(ids, targets=ids)["loss"]
    loss.backward()
    torch.nn.utils.clip_grad_norm_(mb.parameters(), clip)
    ob.step()
    worst = {}
    for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
        sa, sb = oa.state[pa]["exp_avg"], ob.state[pb]["exp_avg"]
        for key, a, b in (("grad", pa.grad, pb.grad), ("exp_avg", sa, sb), ("param", pa, pb)):
            e = ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()
            worst[key] = max(worst.get(key, 0.0), e)
    say("   " + " ".join(f"{k} {v:.1e}" for k, v in worst.items()))
    assert worst["grad"] <= 1e-5 and worst["exp_avg"] <= 1e-5 and worst["param"] <= 1e-6


def test_decoder_fused_prologue_matches_composition(gpu_ca):
    """Whole decoder (fp32): fused-prologue attention and fused RMSNorm vs the
    op-by-op path, logits and every parameter gradient."""
    say("[case] decoder fused vs composition")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(6)
    m = Dm.ContinuumDecoderLM(cfg).cuda()
    ids = torch.randint(0, 256, (2, 64), device="cuda")
    outs = {}
    for fused in (True, False):
        Dm.ContinuumSelfAttention.fused_prologue = fused
        Dm.RMSNorm.fused = fused
        try:
            m.zero_grad(set_to_none=True)
            loss = m(ids, targets=ids)["loss"]
            loss.backward()
            outs[fused] = (loss.item(), {n: p.grad.detach().clone() for n, p in m.named_parameters()})
        finally:
            Dm.ContinuumSelfAttention.fused_prologue = True
            Dm.RMSNorm.fused = True
    assert abs(outs[True][0] - outs[False][0]) <= 1e-5 * abs(outs[False][0])
    for n, gref in outs[False][1].items():
        assert rel(outs[True][1][n].cpu().numpy(), gref.cpu().numpy()) <= 1e-3, n


def _torch_reference_step(m, opt, ids, clip, amp):
    opt.zero_grad(set_to_none=True)
    ctx = torch.autocast(device_type="cuda", dtype=torch.bfloat16) if amp else contextlib.nullcontext()
    with ctx:
        loss = m(ids, targets=ids)["loss"]
    loss.backward()
    grads = [p.grad.detach().clone() for p in m.parameters()]
    torch.nn.utils.clip_grad_norm_(m.parameters(), clip)
    opt.step()
    return loss.item(), grads


@pytest.mark.parametrize("amp,clip", [(True, 0.05), (True, 1e9), (False, 0.05)])
def test_fused_adamw_matches_torch(gpu_ca, amp, clip):
    """optim.FusedAdamW (HIP clip + AdamW, bf16 shadows of the Linear
    weights) against torch's clip_grad_norm_ + AdamW (cuda/runtime.py:87-88,
    cuda/continuum_attention.py:1205-1228) on one decoder step from equal
    parameters: the same loss, the gradients the step uses equal to torch's
    (the bf16 shadow gradients are the values autocast upcasts), first and
    second moments and parameters within fp32 rounding, and every shadow
    equal to its new weight rounded to bf16."""
    say(f"[case] FusedAdamW vs torch, autocast {amp}, clip {clip}")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(5)
    ma = Dm.ContinuumDecoderLM(cfg).cuda()
    mb = Dm.ContinuumDecoderLM(cfg).cuda()
    mb.load_state_dict(ma.state_dict())
    oa = Dm.build_fused_adamw(ma)
    ob = torch.optim.AdamW(mb.parameters(), lr=3e-4, weight_decay=0.1, betas=(0.9, 0.95))
    ids = torch.randint(0, 256, (2, 64), device="cuda")
    loss_a = Dm.train_step(ma, oa, ids, amp_dtype=torch.bfloat16 if amp else None, grad_clip=clip).item()
    loss_b, grads_b = _torch_reference_step(mb, ob, ids, clip, amp)
    assert loss_a == loss_b
    for ga, gb in zip(oa.grads(), grads_b):
        assert torch.equal(ga.float(), gb)
    worst = {}
    for pa, pb in zip(ma.parameters(), mb.parameters()):
        sa, sb = oa.state[pa], ob.state[pb]
        for key, a, b in (("exp_avg", sa["exp_avg"], sb["exp_avg"]),
                          ("exp_avg_sq", sa["exp_avg_sq"], sb["exp_avg_sq"]), ("param", pa, pb)):
            e = ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()
            worst[key] = max(worst.get(key, 0.0), e)
    say("   " + " ".join(f"{k} {v:.1e}" for k, v in worst.items()))
    assert worst["exp_avg"] <= 1e-5 and worst["exp_avg_sq"] <= 1e-5 and worst["param"] <= 1e-6
    for mod in ma.modules():
        sh = getattr(mod, "_ca_shadow", None)
        if sh is not None:
            assert torch.equal(sh, mod.weight.detach().to(torch.bfloat16))


def test_fused_adamw_shadow_refresh_and_groups(gpu_ca):
    """A weight changed outside the optimizer (load_state_dict) is recopied
    to its shadow before the next bf16 forward; two parameter groups (gains
    at 8x lr without decay, as TinyLM's build_adamw) share one clip norm and
    match torch; an LR scheduler drives the fused optimizer."""
    say("[case] FusedAdamW shadow refresh, groups, scheduler")
    Dm = gpu_ca.decoder
    from importlib import import_module
    Opt = import_module("continuum-attention_amd.optim")
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(8)
    ma = Dm.ContinuumDecoderLM(cfg).cuda()
    mb = Dm.ContinuumDecoderLM(cfg).cuda()
    mb.load_state_dict(ma.state_dict())

    def groups(m):
        gains = [p for n, p in m.named_parameters() if "log_qk_gain" in n]
        rest = [p for n, p in m.named_parameters() if "log_qk_gain" not in n]
        return [{"params": rest}, {"params": gains, "lr": 2.4e-3, "weight_decay": 0.0}]

    oa = Opt.FusedAdamW(groups(ma), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1,
                        shadow_modules=[m for m in ma.modules() if isinstance(m, torch.nn.Linear)])
    ob = torch.optim.AdamW(groups(mb), lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1)
    sched = torch.optim.lr_scheduler.StepLR(oa, step_size=1, gamma=0.5)
    ids = torch.randint(0, 256, (2, 64), device="cuda")
    Dm.train_step(ma, oa, ids, grad_clip=0.05)
    _torch_reference_step(mb, ob, ids, 0.05, True)
    sched.step()
    assert abs(oa.param_groups[0]["lr"] - 1.5e-4) < 1e-12
    for pa, pb in zip(ma.parameters(), mb.parameters()):
        e = ((oa.state[pa]["exp_avg"] - ob.state[pb]["exp_avg"]).abs().max()
             / ob.state[pb]["exp_avg"].abs().max().clamp_min(1e-30)).item()
        assert e <= 1e-5
        assert ((pa - pb).abs().max() / pb.abs().max()).item() <= 1e-6
    # weights replaced from outside: the next bf16 forward recopies the shadows
    fresh = Dm.ContinuumDecoderLM(cfg).cuda()
    ma.load_state_dict(fresh.state_dict())
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        la = ma(ids, targets=ids)["loss"].item()
        lb = fresh(ids, targets=ids)["loss"].item()
    assert la == lb
    for mod in ma.modules():
        sh = getattr(mod, "_ca_shadow", None)
        if sh is not None:
            assert torch.equal(sh, mod.weight.detach().to(torch.bfloat16))


def test_tinylm_fused_norms_and_adamw(gpu_ca):
    """TinyLM (CA-P family) with its RMSNorms and residual adds fused (one
    HIP pass each) against the reference's composition: logits and every
    parameter gradient; then one step of the HIP AdamW (TinyLM's groups:
    gains at 8x lr without decay) against torch's clip_grad_norm_ + AdamW
    (benchmark.py:189-214)."""
    say("[case] TinyLM fused norms + HIP AdamW")
    A = gpu_ca.architecture
    Dm = gpu_ca.decoder
    torch.manual_seed(12)
    m = A.TinyLM(variant="H", backend="hip", seq_len=128, layers=2).cuda()
    x = torch.randint(0, 256, (2, 128), device="cuda")
    outs = {}
    for fused in (True, False):
        Dm.RMSNorm.fused = fused
        try:
            m.zero_grad(set_to_none=True)
            logits = m(x)
            torch.nn.functional.cross_entropy(logits.reshape(-1, 256), x.reshape(-1)).backward()
            outs[fused] = (logits.detach().clone(), [p.grad.detach().clone() for p in m.parameters()])
        finally:
            Dm.RMSNorm.fused = True
    el = rel(outs[True][0].cpu().numpy(), outs[False][0].cpu().numpy())
    eg = max(rel(a.cpu().numpy(), b.cpu().numpy()) for a, b in zip(outs[True][1], outs[False][1]))
    say(f"   logits {el:.2e} grads {eg:.2e}")
    assert el <= 1e-5 and eg <= 1e-4
    ma = A.TinyLM(variant="H", backend="hip", seq_len=128, layers=2).cuda()
    mb = A.TinyLM(variant="H", backend="hip", seq_len=128, layers=2).cuda()
    mb.load_state_dict(ma.state_dict())
    oa, ob = A.build_fused_adamw(ma), A.build_adamw(mb)
    la = A.train_step(ma, oa, x, x, grad_clip=0.05).item()
    Dm.RMSNorm.fused = True
    lb = A.train_step(mb, ob, x, x, grad_clip=0.05).item()
    assert la == lb
    for pa, pb in zip(ma.parameters(), mb.parameters()):
        e = ((oa.state[pa]["exp_avg"] - ob.state[pb]["exp_avg"]).abs().max()
             / ob.state[pb]["exp_avg"].abs().max().clamp_min(1e-30)).item()
        assert e <= 1e-5
        assert ((pa - pb).abs().max() / pb.abs().max()).item() <= 1e-6


def test_graphed_train_step_matches_eager(gpu_ca):
    """decoder.GraphedTrainStep (forward + backward captured as one HIP graph,
    replayed each step, HIP AdamW after each replay) against the eager
    train_step on a twin model over three steps with different batches, with
    eager work and synchronisation between the replays: every replay's loss,
    and the parameters after every step, equal the eager ones."""
    say("[case] graphed train step vs eager")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(21)
    ma = Dm.ContinuumDecoderLM(cfg).cuda()
    mb = Dm.ContinuumDecoderLM(cfg).cuda()
    mb.load_state_dict(ma.state_dict())
    oa, ob = Dm.build_fused_adamw(ma), Dm.build_fused_adamw(mb)
    g = torch.Generator().manual_seed(22)
    batches = [torch.randint(0, 256, (2, 64), generator=g).cuda() for _ in range(3)]
    step = Dm.GraphedTrainStep(ma, oa, batches[0], grad_clip=0.05)
    for n, b in enumerate(batches):
        la = step(b).item()
        torch.cuda.synchronize()
        lb = Dm.train_step(mb, ob, b, grad_clip=0.05).item()
        torch.cuda.synchronize()
        say(f"   step {n}: graphed {la:.6f} eager {lb:.6f}")
        assert abs(la - lb) <= 1e-6 * abs(lb)
        worst = max(((pa - pb).abs().max() / pb.abs().max()).item()
                    for pa, pb in zip(ma.parameters(), mb.parameters()))
        assert worst <= 1e-6, worst


@pytest.mark.parametrize("batch", [6, 16])
def test_graphed_tinylm_step_matches_eager(gpu_ca, batch):
    """GraphedTrainStep with a caller's loss (TinyLM's next-byte cross-entropy
    on (inputs, targets)), fp32 without autocast, a tied head and FusedAdamW's
    two parameter groups under a global clip, against the eager step over
    three replays; at batch 16 (8192 token lookups, the CA-P configuration)
    TinyLM's one-hot token-embedding gradient keeps the capture free of the
    memset nodes torch's sorting embedding backward records, which a direct
    nn.Embedding lookup of that size still does (that capture is refused
    before it is instantiated)."""
    say(f"[case] graphed TinyLM step vs eager (B {batch}, T 512)")
    A, Dm = gpu_ca.architecture, gpu_ca.decoder
    torch.manual_seed(31)
    kw = dict(variant="P", backend="hip", seq_len=512, width=64, hidden=128, heads=4,
              fixed_tau=0.30, layers=2)
    ma, mb = A.TinyLM(**kw).cuda(), A.TinyLM(**kw).cuda()
    mb.load_state_dict(ma.state_dict())
    oa, ob = A.build_fused_adamw(ma), A.build_fused_adamw(mb)
    g = torch.Generator().manual_seed(32)
    data = [torch.randint(0, 256, (batch, 513), generator=g).cuda() for _ in range(3)]
    loss_fn = lambda m, x, t: F.cross_entropy(m(x).reshape(-1, 256), t.reshape(-1))
    step = Dm.GraphedTrainStep(ma, oa, (data[0][:, :-1], data[0][:, 1:]), amp_dtype=None,
                               grad_clip=0.5, loss_fn=loss_fn)
    for n, d in enumerate(data):
        la = step(d[:, :-1], d[:, 1:]).item()
        torch.cuda.synchronize()
        lb = A.train_step(mb, ob, d[:, :-1], d[:, 1:], grad_clip=0.5).item()
        torch.cuda.synchronize()
        say(f"   step {n}: graphed {la:.6f} eager {lb:.6f}")
        assert abs(la - lb) <= 1e-6 * abs(lb)
        worst = max(((pa - pb).abs().max() / pb.abs().max()).item()
                    for pa, pb in zip(ma.parameters(), mb.parameters()))
        assert worst <= 1e-6, worst
    if batch == 16:
        say("[case] graphed step with a direct nn.Embedding lookup of 8192 tokens refused")
        lookup = lambda m, x, t: m.tok_embed(x).square().mean()
        with pytest.raises(ValueError, match="memset node"):
            Dm.GraphedTrainStep(mb, ob, (data[0][:, :-1], data[0][:, 1:]), amp_dtype=None,
                                loss_fn=lookup)


@pytest.mark.parametrize("variant", ["P", "R", "S", "H"])
def test_tinylm_fused_prologue_matches_composition(gpu_ca, variant):
    """TinyLM's continuous variants with the fused qkv -> heads prologue (the
    variant's q scale passed as the operator's log-gain, no rotation) against
    the reference's composition (q scaled, heads split and copied): logits and
    every parameter gradient, the learned gains' included."""
    say(f"[case] TinyLM {variant} fused prologue vs composition")
    A = gpu_ca.architecture
    torch.manual_seed(31)
    m = A.TinyLM(variant=variant, backend="hip", seq_len=96, layers=2).cuda()
    if variant in ("S", "H"):
        with torch.no_grad():
            for n, p in m.named_parameters():
                if n.endswith("log_qk_gain"):
                    p.add_(torch.linspace(-0.3, 0.3, p.numel(), device="cuda"))
    x = torch.randint(0, 256, (2, 96), device="cuda")
    outs = {}
    for fused in (True, False):
        A.CausalAttention.fused_prologue = fused
        try:
            m.zero_grad(set_to_none=True)
            logits = m(x)
            torch.nn.functional.cross_entropy(logits.reshape(-1, 256), x.reshape(-1)).backward()
            outs[fused] = (logits.detach().clone(), {n: p.grad.detach().clone() for n, p in m.named_parameters()})
        finally:
            A.CausalAttention.fused_prologue = True
    el = rel(outs[True][0].cpu().numpy(), outs[False][0].cpu().numpy())
    eg = {n: rel(outs[True][1][n].cpu().numpy(), outs[False][1][n].cpu().numpy()) for n in outs[True][1]}
    worst = max(eg.values())
    say(f"   logits {el:.2e} worst grad {worst:.2e} ({max(eg, key=eg.get)})")
    assert el <= 1e-5 and worst <= 1e-4


@pytest.mark.parametrize("N,H,scale", [(37, 4, 1.0), (8192, 720, 1.0), (300, 256, 30.0),
                                       (5, 16, 120.0)])
def test_fused_swiglu_matches_composition(gpu_ca, N, H, scale):
    """The fused SwiGLU gate (ca_swiglu_fwd_f32 / ca_swiglu_bwd_f32) against
    torch's silu(gate) * value and its autograd: same formulas in the same
    order, so equal to a few ulp; |g| > 88 (scale 120) checks the capped
    exponent, where torch's silu gives -0 and the kernel a denormal.  Bar:
    1e-6 as max|x - ref| / max|ref| on h and du."""
    say(f"[case] fused SwiGLU N={N} H={H} scale={scale}")
    A = gpu_ca.architecture
    torch.manual_seed(N + H)
    u = (torch.randn(N, 2 * H, device="cuda") * scale).requires_grad_(True)
    dh = torch.randn(N, H, device="cuda")
    h = A._SwiGLUFn.apply(u)
    (du,) = torch.autograd.grad(h, u, dh)
    u2 = u.detach().clone().requires_grad_(True)
    g, v = u2.chunk(2, dim=-1)
    h2 = F.silu(g) * v
    (du2,) = torch.autograd.grad(h2, u2, dh)
    # per tensor, max|x - ref| / max|ref|: element-wise the two differ
    # relatively where values are tiny (silu of g << 0, whose exp argument
    # reduction errs by about |g| ulp) or where 1 + g (1 - s) cancels (g near
    # -1.28, a one-ulp difference in s amplified)
    eh = rel(h.detach().cpu().numpy(), h2.detach().cpu().numpy())
    e = rel(du.cpu().numpy(), du2.cpu().numpy())
    say(f"   h max rel {eh:.2e}, du max rel {e:.2e}")
    assert eh <= 1e-6 and e <= 1e-6


def test_tinylm_fused_swiglu_step(gpu_ca):
    """A TinyLM (variant P, fp32) loss and every parameter gradient with the
    fused SwiGLU gate against SwiGLU.fused = False (torch's composition)."""
    say("[case] TinyLM fused SwiGLU vs composition")
    A = gpu_ca.architecture
    torch.manual_seed(41)
    m = A.TinyLM(variant="P", backend="hip", seq_len=128, width=64, hidden=96, heads=4,
                 fixed_tau=0.30, layers=2).cuda()
    ids = torch.randint(0, 256, (3, 129), device="cuda")
    out = {}
    try:
        for fused in (True, False):
            A.SwiGLU.fused = fused
            m.zero_grad(set_to_none=True)
            loss = F.cross_entropy(m(ids[:, :-1]).reshape(-1, 256), ids[:, 1:].reshape(-1))
            loss.backward()
            out[fused] = (loss.item(), [p.grad.clone() for p in m.parameters()])
    finally:
        A.SwiGLU.fused = True
    assert abs(out[True][0] - out[False][0]) <= 1e-6 * abs(out[False][0])
    for a, b in zip(out[True][1], out[False][1]):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("micro", [2, 8])
def test_fused_adamw_gradient_accumulation(gpu_ca, micro):
    """The reference's grad_accum loop (cuda/continuum_attention.py:1194-1207:
    loss / grad_accum, one backward per micro-batch, then clip and step)
    under bf16 autocast: the gradients FusedAdamW steps with are the fp32
    sums of the micro-batches' bf16 weight gradients, bit for bit what torch
    accumulates in each fp32 .grad, and the updated parameters agree with
    torch's clip_grad_norm_ + AdamW to fp32 rounding."""
    say(f"[case] FusedAdamW gradient accumulation over {micro} backwards")
    Dm = gpu_ca.decoder
    cfg = Dm.ContinuumDecoderConfig(d_model=128, n_heads=2, n_layers=2, block_size=64)
    torch.manual_seed(11)
    ma = Dm.ContinuumDecoderLM(cfg).cuda()
    mb = Dm.ContinuumDecoderLM(cfg).cuda()
    mb.load_state_dict(ma.state_dict())
    oa = Dm.build_fused_adamw(ma)
    ob = torch.optim.AdamW(mb.parameters(), lr=3e-4, weight_decay=0.1, betas=(0.9, 0.95))
    batches = [torch.randint(0, 256, (2, 64), device="cuda") for _ in range(micro)]
    for m, o in ((ma, oa), (mb, ob)):
        o.zero_grad(set_to_none=True)
        for ids in batches:
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
                loss = m(ids, targets=ids)["loss"] / micro
            loss.backward()
    grads_b = [p.grad.detach().clone() for p in mb.parameters()]
    for ga, gb in zip(oa.grads(), grads_b):
        assert ga.dtype == torch.float32 and torch.equal(ga, gb)
    oa.step(max_norm=1.0)
    torch.nn.utils.clip_grad_norm_(mb.parameters(), 1.0)
    ob.step()
    worst = max(((pa - pb).abs().max() / pb.abs().max()).item()
                for pa, pb in zip(ma.parameters(), mb.parameters()))
    say(f"   parameters after the step: {worst:.1e}")
    assert worst <= 1e-6


@pytest.mark.parametrize("bad", [float("inf"), float("nan")])
def test_clip_and_adamw_with_non_finite_gradient(gpu_ca, bad):
    """A diverging step: one gradient element is inf or NaN.  The HIP clip
    and AdamW give torch's total norm (inf / NaN), clip factor (0 / NaN) and
    updated parameters (NaN where torch's are NaN, equal elsewhere)."""
    say(f"[case] clip + AdamW with a {bad} gradient")
    torch.manual_seed(12)
    shapes = [(64, 33), (1000,), (7,)]
    pa = [torch.randn(s, device="cuda") for s in shapes]
    pb = [p.clone() for p in pa]
    grads = [torch.randn(s, device="cuda") for s in shapes]
    grads[1][123] = bad
    for p, q, gr in zip(pa, pb, grads):
        p.grad = gr.clone()
        q.grad = gr.clone()
    oa = gpu_ca.optim.FusedAdamW(pa, lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1)
    ob = torch.optim.AdamW(pb, lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1)
    norm_a = oa.step(max_norm=1.0)
    norm_b = torch.nn.utils.clip_grad_norm_(pb, 1.0)
    ob.step()
    torch.testing.assert_close(norm_a.reshape(()), norm_b, equal_nan=True)
    for a, b in zip(pa, pb):
        assert torch.equal(torch.isnan(a), torch.isnan(b))
        torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6, equal_nan=True)

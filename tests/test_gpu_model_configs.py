"""The BASELINE config-3 and config-4 workloads as GPU tests: one full training
step of each model at its benchmark size, the fused paths against the
op-by-op composition, and layer 0's attention output against the float64
oracle on sampled rows.

* Config 3: the CA-P TinyLM (4 blocks, d 256, 4 heads, fixed tau 0.30,
  T 512, batch 16, fp32) with the library's AdamW (bench.py ``ca_p``).
* Config 4: the 101,205,120-parameter CA-S decoder at T 2048, batch 1, bf16
  autocast with fp32 CA scores, with the library's AdamW and bf16 weight
  shadows (bench.py ``ca_s``); the fused-vs-composition comparison runs the
  same model in fp32, where both paths should agree to fp32 rounding.

The reference checks its full decoder the same way (cuda/benchmark.py:85-105)
and pins the parameter budgets (test_hp_only.py:13-23, cuda/test_cpu.py:25-27).
"""
import math
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ca_oracle as O

pytestmark = pytest.mark.gpu

LN256 = math.log(256.0)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def capture(attn):
    """Forward hooks recording the qkv projection's output and the attention
    output that enters the output projection."""
    store = {}
    hs = [attn.qkv.register_forward_hook(lambda m, i, o: store.__setitem__("qkv", o.detach().clone())),
          attn.out.register_forward_pre_hook(lambda m, i: store.__setitem__("y", i[0].detach().clone()))]
    return store, hs


def heads(qkv, H):
    B, T, C3 = qkv.shape
    return qkv.float().view(B, T, 3, H, C3 // (3 * H)).permute(2, 0, 3, 1, 4).unbind(0)


def attention_vs_oracle(q, k, v, log_gain, y_tokens, rows, bar):
    """Sampled rows of every (b, h) slice of the [B, T, H*D] attention output
    against the float64 row oracle."""
    qn, kn, vn = (x.double().cpu().numpy() for x in (q, k, v))
    rn = log_gain.double().cpu().numpy()
    B, H, T, D = q.shape
    y = y_tokens.float().view(B, T, H, D).cpu().numpy()
    worst = 0.0
    for b in range(B):
        for h in range(H):
            yr = O.ca_forward_rows(qn, kn, vn, rn, b, h, rows)
            worst = max(worst, rel(y[b, rows, h], yr))
    say(f"   layer 0 attention, sampled rows of {B * H} slices: {worst:.2e}")
    assert worst <= bar


def init_loss_bar(logits):
    """Expected cross-entropy of a randomly initialised byte model: with
    logits ~ N(0, sigma^2) independent of the target, E[CE] = E[logsumexp]
    - E[z_target] ~= ln 256 + sigma^2 / 2 (second order in sigma; sigma is
    about 0.3 for TinyLM's tied head and 0.64 for CA-S's untied
    d_model-1024 head at std 0.02)."""
    return LN256 + 0.5 * logits.float().var().item()


def grads_of(model):
    return {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}


def test_config3_ca_p_step(gpu_ca):
    """Config 3: loss at init within 0.05 of ln 256 + sigma^2/2 (sigma^2 the
    logits' variance), every gradient finite,
    parameters finite after the HIP AdamW step; fused prologue / RMSNorm /
    SwiGLU logits and gradients equal to the composition within fp32
    rounding; layer 0's attention against the oracle (log_gain = ln(1/0.3))."""
    say("[case] config3 CA-P TinyLM step (4 blocks, d256, T512, b16)")
    A = gpu_ca.architecture
    torch.manual_seed(0)
    model = A.TinyLM(variant="P", backend="hip", seq_len=512, width=256, hidden=720, heads=4,
                     fixed_tau=0.30, layers=4).cuda()
    assert A.parameters(model) == 3_459_328
    g = torch.Generator().manual_seed(2)
    data = torch.randint(0, 256, (16, 513), generator=g).cuda()
    x, tgt = data[:, :-1], data[:, 1:]
    store, hooks = capture(model.b0.attn)
    outs = {}
    try:
        for fused in (True, False):
            A.CausalAttention.fused_prologue = fused
            A.RMSNorm.fused = fused
            A.SwiGLU.fused = fused
            model.zero_grad(set_to_none=True)
            logits = model(x)
            loss = F.cross_entropy(logits.reshape(-1, 256), tgt.reshape(-1))
            loss.backward()
            outs[fused] = (logits.detach().clone(), loss.item(), grads_of(model))
            if fused:
                qkv, y0 = store["qkv"], store["y"]
    finally:
        A.CausalAttention.fused_prologue = True
        A.RMSNorm.fused = True
        A.SwiGLU.fused = True
        for h in hooks:
            h.remove()
    loss0 = outs[True][1]
    bar = init_loss_bar(outs[True][0])
    say(f"   loss at init {loss0:.4f} (ln 256 + sigma^2/2 = {bar:.4f})")
    assert abs(loss0 - bar) <= 0.05
    el = rel(outs[True][0].cpu().numpy(), outs[False][0].cpu().numpy())
    eg = max(rel(outs[True][2][n].cpu().numpy(), gr.cpu().numpy()) for n, gr in outs[False][2].items())
    say(f"   fused vs composition: logits {el:.2e}, worst gradient {eg:.2e}")
    assert el <= 1e-5 and eg <= 1e-4
    assert set(outs[True][2]) == {n for n, _ in model.named_parameters()}
    assert all(torch.isfinite(gr).all() for gr in outs[True][2].values())
    q, k, v = heads(qkv, 4)
    rows = np.array([0, 1, 31, 32, 100, 255, 256, 384, 510, 511])
    attention_vs_oracle(q, k, v, torch.full((4,), math.log(1 / 0.3)), y0, rows, 1e-4)
    opt = A.build_fused_adamw(model)
    loss = A.train_step(model, opt, x, tgt).item()
    assert abs(loss - loss0) <= 1e-4 * loss0
    assert all(torch.isfinite(p).all() for p in model.parameters())


def test_config4_ca_s_step(gpu_ca):
    """Config 4: the 101,205,120-parameter CA-S decoder, T 2048, batch 1,
    bf16 autocast with the HIP AdamW and bf16 weight shadows: loss at init
    within 0.05 of ln 256 + sigma^2/2, every gradient the step uses finite, parameters
    finite after the step, layer 0's attention (bf16 output of the fused
    prologue, RoPE in fp32) against the oracle within bf16 rounding."""
    say("[case] config4 CA-S step (101,205,120 params, T2048, b1, bf16 autocast)")
    Dm = gpu_ca.decoder
    torch.manual_seed(0)
    cfg = Dm.ContinuumDecoderConfig()
    model = Dm.ContinuumDecoderLM(cfg).cuda()
    assert Dm.count_parameters(model)["total"] == 101_205_120
    opt = Dm.build_fused_adamw(model)
    ids = torch.randint(0, 256, (1, cfg.block_size), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        bar = init_loss_bar(model(ids)["logits"])
    attn = model.blocks[0].attn
    store, hooks = capture(attn)
    try:
        loss = Dm.train_step(model, opt, ids).item()
    finally:
        for h in hooks:
            h.remove()
    say(f"   loss at init {loss:.4f} (ln 256 + sigma^2/2 = {bar:.4f})")
    assert abs(loss - bar) <= 0.05
    grads = opt.grads()
    assert len(grads) == len(list(model.parameters())) and all(gr is not None for gr in grads)
    assert all(torch.isfinite(gr).all() for gr in grads)
    assert all(torch.isfinite(p).all() for p in model.parameters())
    assert store["y"].dtype == torch.bfloat16
    q, k, v = heads(store["qkv"], cfg.n_heads)
    # RoPE as the reference computes it under bf16 autocast (the kernels' own
    # rotation): in bf16, cuda/continuum_attention.py:826-835
    qb, kb = Dm.apply_rope(q.to(torch.bfloat16), k.to(torch.bfloat16), cfg.rope_theta)
    q, k = qb.float(), kb.float()
    rows = np.array([0, 1, 2, 63, 64, 511, 1024, 1535, 2046, 2047])
    # the output is rounded to bf16: half an ulp (2^-8 relative) per element
    attention_vs_oracle(q, k, v, torch.zeros(cfg.n_heads), store["y"], rows, 4e-3)


def test_config4_ca_s_fused_vs_composition_fp32(gpu_ca):
    """The config-4 model in fp32: the fused prologue and fused RMSNorm /
    residual-add chain against the op-by-op composition, logits and every
    parameter gradient (fp32 on both sides, so only rounding differs)."""
    say("[case] config4 CA-S fused vs composition, fp32")
    Dm = gpu_ca.decoder
    torch.manual_seed(0)
    cfg = Dm.ContinuumDecoderConfig()
    model = Dm.ContinuumDecoderLM(cfg).cuda()
    ids = torch.randint(0, 256, (1, cfg.block_size), generator=torch.Generator().manual_seed(1)).cuda()
    outs = {}
    try:
        for fused in (True, False):
            Dm.ContinuumSelfAttention.fused_prologue = fused
            Dm.RMSNorm.fused = fused
            model.zero_grad(set_to_none=True)
            out = model(ids, targets=ids)
            out["loss"].backward()
            outs[fused] = (out["logits"].detach().clone(), out["loss"].item(), grads_of(model))
    finally:
        Dm.ContinuumSelfAttention.fused_prologue = True
        Dm.RMSNorm.fused = True
    el = rel(outs[True][0].cpu().numpy(), outs[False][0].cpu().numpy())
    worst = max((rel(outs[True][2][n].cpu().numpy(), gr.cpu().numpy()), n)
                for n, gr in outs[False][2].items())
    say(f"   loss {outs[True][1]:.5f} vs {outs[False][1]:.5f}; logits {el:.2e}; "
        f"worst gradient {worst[0]:.2e} ({worst[1]})")
    assert abs(outs[True][1] - outs[False][1]) <= 1e-5 * outs[False][1]
    assert el <= 1e-4 and worst[0] <= 1e-3

"""CPU checks of the operator's callers (continuum-attention_amd/architecture.py
and decoder.py): parameter budgets, initialisation, configuration errors,
state-dict layout, RoPE, and the CA variants on CPU tensors.

Expected values come from the reference's own tests: test_acma.py:21-34,
140-154; test_hp_only.py:13-23; test_fusion.py:17-25; cuda/test_cpu.py:25-27.
"""
import math

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def A(ca):
    return ca.architecture


@pytest.fixture(scope="module")
def Dm(ca):
    return ca.decoder


def tiny(A, variant, backend="hip", seed=97):
    torch.manual_seed(seed)
    return A.TinyLM(variant=variant, backend=backend, seq_len=16, width=32, hidden=64, heads=4,
                    fixed_tau=.30)


@pytest.mark.parametrize("variant,T,count", [("B", 192, 5_008_640), ("P", 192, 5_008_640),
                                             ("R", 192, 5_008_640), ("F", 192, 5_008_664),
                                             ("S", 192, 5_008_664), ("H", 192, 5_008_664),
                                             ("H", 512, 5_090_584), ("P", 512, 5_090_560)])
def test_tinylm_parameter_budget(A, variant, T, count):
    """test_acma.py:21-26, test_hp_only.py:13-23."""
    m = A.TinyLM(variant=variant, backend="hip", seq_len=T)
    assert A.parameters(m) == count


def test_ca_p_four_layer_budget(A):
    """BASELINE's CA-P configuration: 4 blocks of the TinyLM backbone at T=512."""
    m = A.TinyLM(variant="P", seq_len=512, layers=4)
    assert A.parameters(m) == 3_459_328
    assert not hasattr(m, "b4")


def test_h_variant_gain_init(A):
    """test_hp_only.py:19-20: H starts at tau = 0.30."""
    m = A.TinyLM(variant="H", seq_len=192)
    assert m.b0.attn.continuous
    assert torch.exp(-m.b0.attn.log_qk_gain).mean().item() == pytest.approx(0.3, abs=1e-6)


def test_shared_initial_weights_equal(A):
    """test_acma.py:28-34: every variant starts from the same weights."""
    states = {v: tiny(A, v).state_dict() for v in ("A", "B", "F", "P", "R", "S")}
    common = set.intersection(*(set(s) for s in states.values()))
    assert len(common) >= 40
    for key in common:
        for v in states:
            assert torch.equal(states["B"][key], states[v][key]), key


def test_state_dict_keys_follow_reference_names(A, Dm):
    m = tiny(A, "S")
    keys = set(m.state_dict())
    for k in ("tok_embed.weight", "pos_embed.weight", "b0.attn.qkv.weight", "b0.attn.out.weight",
              "b0.attn.log_qk_gain", "b5.mlp.gate_up.weight", "b5.mlp.down.weight",
              "b3.norm_attn.weight", "b3.norm_mlp.weight", "final_norm.weight", "lm_head.weight"):
        assert k in keys, k
    cfg = Dm.ContinuumDecoderConfig(d_model=64, n_heads=4, n_layers=2, block_size=32)
    d = Dm.ContinuumDecoderLM(cfg)
    keys = set(d.state_dict())
    for k in ("byte_emb.weight", "blocks.0.norm1.weight", "blocks.0.attn.qkv.weight",
              "blocks.0.attn.out.weight", "blocks.0.attn.log_qk_gain", "blocks.1.norm2.weight",
              "blocks.1.mlp.fc1.weight", "blocks.1.mlp.fc2.weight", "norm_f.weight", "lm_head.weight"):
        assert k in keys, k


def test_softmax_controls_on_cpu(A):
    """Softmax variants use torch only (test_acma.py:140-154, test_fusion.py:17-25):
    A == F initially (gain exp(0) = 1), reference weights == SDPA path."""
    torch.manual_seed(5)
    ids = torch.randint(0, 256, (1, 13))
    with torch.no_grad():
        torch.testing.assert_close(tiny(A, "A")(ids), tiny(A, "F")(ids), atol=0, rtol=0)
        for v in ("B", "F"):
            torch.testing.assert_close(tiny(A, v, "reference")(ids), tiny(A, v, "mixed")(ids),
                                       atol=3e-5, rtol=3e-5)


def test_ca_variants_run_on_cpu(A, ca):
    """CPU tensors run the CA variants as the reference's modules do: the
    fused-operator backend and the weights backend agree, and the weight-level
    entry points keep the GPU-only ones GPU-only."""
    ids = torch.randint(0, 256, (2, 9))
    for v in ("P", "R", "S", "H"):
        a = tiny(A, v, "hip")(ids)
        b = tiny(A, v, "hip_weights")(ids)
        assert torch.isfinite(a).all()
        torch.testing.assert_close(a, b, atol=2e-5, rtol=2e-5)
    with pytest.raises(ValueError, match="square"):
        ca.continuous_attention_weights(torch.randn(1, 1, 3, 4))
    with pytest.raises(RuntimeError, match="GPU tensors only"):
        ca.ca_weights(torch.randn(1, 4, 4))


def test_bad_variant_backend_and_config(A, Dm):
    with pytest.raises(ValueError):
        A.CausalAttention(32, 4, 16, variant="Q")
    with pytest.raises(ValueError):
        A.CausalAttention(32, 4, 16, variant="P", backend="cuda")
    with pytest.raises(ValueError):
        A.CausalAttention(30, 4, 16)
    with pytest.raises(ValueError):
        A.CausalAttention(32, 4, 16, fixed_tau=0.0)
    with pytest.raises(ValueError, match="divisible"):
        Dm.ContinuumDecoderConfig(d_model=100, n_heads=3)
    with pytest.raises(ValueError, match="RoPE"):
        Dm.ContinuumDecoderConfig(d_model=12, n_heads=4)
    with pytest.raises(ValueError, match="dropout"):
        Dm.ContinuumDecoderConfig(dropout=0.1)
    with pytest.raises(ValueError):
        Dm.ContinuumDecoderConfig(n_layers=0)
    cfg = Dm.ContinuumDecoderConfig(d_model=32, n_heads=2, n_layers=1, block_size=8)
    with pytest.raises(ValueError, match="block_size"):
        Dm.ContinuumDecoderLM(cfg)(torch.zeros(1, 9, dtype=torch.long))


def test_ca_s_parameter_budget(Dm):
    """cuda/test_cpu.py:25-27: the default CA-S decoder has 101,205,120 parameters."""
    m = Dm.ContinuumDecoderLM(Dm.ContinuumDecoderConfig())
    assert Dm.count_parameters(m) == {"total": 101_205_120, "trainable": 101_205_120}
    br = m.parameter_breakdown()
    assert sum(br.values()) - br["continuum_head_gains"] == 101_205_120
    assert br["continuum_head_gains"] == 8 * 16


def test_ca_s_initialisation(Dm):
    """std .02, residual projections .02/sqrt(2L), untied head, gains 0."""
    torch.manual_seed(0)
    cfg = Dm.ContinuumDecoderConfig(d_model=256, n_heads=4, n_layers=8, block_size=64)
    m = Dm.ContinuumDecoderLM(cfg)
    b = m.blocks[3]
    assert b.attn.qkv.weight.std().item() == pytest.approx(0.02, rel=0.02)
    assert b.mlp.fc1.weight.std().item() == pytest.approx(0.02, rel=0.02)
    assert b.attn.out.weight.std().item() == pytest.approx(0.02 / 4.0, rel=0.03)
    assert b.mlp.fc2.weight.std().item() == pytest.approx(0.02 / 4.0, rel=0.03)
    assert m.lm_head.weight.data_ptr() != m.byte_emb.weight.data_ptr()
    assert torch.equal(b.attn.log_qk_gain, torch.zeros(4))


def test_rope_matches_complex_rotation(Dm):
    """Interleaved RoPE equals multiplying each pair (x0 + i x1) by
    exp(i * pos * theta^(-2k/D)) -- an independent formulation."""
    torch.manual_seed(3)
    B, H, T, D, theta = 2, 3, 17, 8, 10000.0
    q, k = torch.randn(B, H, T, D, dtype=torch.float64), torch.randn(B, H, T, D, dtype=torch.float64)
    qr, kr = Dm.apply_rope(q.float(), k.float(), theta)
    pos = np.arange(T)[:, None]
    freq = theta ** (-np.arange(0, D, 2) / D)
    rot = np.exp(1j * pos * freq)
    for x, xr in ((q, qr), (k, kr)):
        z = x.numpy()[..., 0::2] + 1j * x.numpy()[..., 1::2]
        z = z * rot
        ref = np.stack([z.real, z.imag], -1).reshape(B, H, T, D)
        np.testing.assert_allclose(xr.numpy(), ref, atol=2e-6, rtol=0)


def test_graph_memset_node_count(Dm, monkeypatch):
    """GraphedTrainStep's capture check counts the memset nodes of the
    captured HIP graph, child graphs included, through the HIP graph API
    (replaced here by a fake runtime holding a known node structure:
    graph 1 = kernel, memset, child graph 2, memcpy; graph 2 = memset,
    kernel, child graph 3; graph 3 = memset)."""
    import ctypes

    graphs = {1: [("k", None), ("m", None), ("g", 2), ("c", None)],
              2: [("m", None), ("k", None), ("g", 3)], 3: [("m", None)]}
    types = {"k": 0, "c": 1, "m": 2, "g": 4}
    nodes = {}  # node handle -> (type, child graph)
    for g, ns in graphs.items():
        for k, (t, child) in enumerate(ns):
            nodes[100 * g + k + 1] = (types[t], child)

    def get_nodes(g, out, n):
        ids = [100 * g.value + k + 1 for k in range(len(graphs[g.value]))]
        if out is not None:
            for k, h in enumerate(ids):
                out[k] = h
        n._obj.value = len(ids)
        return 0

    def get_type(node, t):
        t._obj.value = nodes[node][0]
        return 0

    def get_child(node, out):
        out._obj.value = nodes[node][1]
        return 0

    class FakeHip:
        hipGraphGetNodes = staticmethod(get_nodes)
        hipGraphNodeGetType = staticmethod(get_type)
        hipGraphChildGraphNodeGetGraph = staticmethod(get_child)

    class FakeGraph:
        def __init__(self, h):
            self.h = h

        def raw_cuda_graph(self):
            return self.h

    monkeypatch.setattr(Dm, "_loaded_hip_runtime", lambda: FakeHip())
    assert Dm._hip_graph_memset_nodes(FakeGraph(1)) == 3
    assert Dm._hip_graph_memset_nodes(FakeGraph(3)) == 1
    graphs[4] = [("k", None), ("c", None)]
    nodes[401], nodes[402] = (0, None), (1, None)
    assert Dm._hip_graph_memset_nodes(FakeGraph(4)) == 0


def test_graph_check_uses_the_loaded_hip_runtime(Dm):
    """The memset-node check queries the HIP runtime torch already loaded
    (found in /proc/self/maps), not a library opened by a fixed soname."""
    import torch  # noqa: F401  (loads the HIP runtime of this ROCm build)

    maps = open("/proc/self/maps").read()
    lib = Dm._loaded_hip_runtime()
    assert "/libamdhip64.so" in lib._name and lib._name in maps
    assert hasattr(lib, "hipGraphGetNodes")


def test_token_embedding_gradient_matches_nn_embedding():
    """The GPU token lookup of TinyLM and the CA-S decoder
    (decoder._TokenEmbedding: the weight gradient as one_hot(tokens)^T @ grad)
    gives nn.Embedding's output and weight gradient, repeated tokens included
    (run here on CPU tensors); token_embedding takes it only for small
    vocabularies and plain embeddings."""
    import importlib
    A = importlib.import_module("continuum-attention_amd.decoder")
    small, big = torch.nn.Embedding(256, 8), torch.nn.Embedding(A.ONE_HOT_MAX_VOCAB + 1, 8)
    t = torch.randint(0, 256, (2, 5))
    assert torch.equal(A.token_embedding(t, small), small(t))  # CPU tensors: nn.Embedding
    assert torch.equal(A.token_embedding(t, big), big(t))
    g = torch.Generator().manual_seed(5)
    w = torch.randn(256, 24, generator=g, dtype=torch.float64)
    tokens = torch.randint(0, 256, (7, 300), generator=g)
    tokens[0, :50] = 3  # many repeats of one token
    up = torch.randn(7, 300, 24, generator=g, dtype=torch.float64)
    wa = w.clone().requires_grad_(True)
    ya = A._TokenEmbedding.apply(tokens, wa)
    (ga,) = torch.autograd.grad(ya, (wa,), up)
    wb = w.clone().requires_grad_(True)
    yb = torch.nn.functional.embedding(tokens, wb)
    (gb,) = torch.autograd.grad(yb, (wb,), up)
    assert torch.equal(ya, yb)
    assert torch.allclose(ga, gb, rtol=1e-12, atol=1e-12)

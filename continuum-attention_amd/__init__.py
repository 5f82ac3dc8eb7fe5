"""MI355X-native Continuum Attention (CA) operator.

Public API (mirrors akhadangi/continuum-attention, cuda/continuum_attention.py:650-783):
    continuum_attention(q, k, v, log_gain, query_tile=64)
    _CAExactTiled  (torch.autograd.Function)
    continuous_attention_weights(logits), ca_weights(scores, start)
        (materialised weights, architecture.py:65-105, ext.forward)
    architecture.CausalAttention / TinyLM   (small variants, architecture.py)
    decoder.ContinuumDecoderLM              (CA-S decoder, cuda/continuum_attention.py:784-923)

The arithmetic runs in hand-written HIP kernels (csrc/, built into
libca_hip.so by build.py) behind the C ABI in include/continuum_attention_amd.h.
The package directory name contains a hyphen; import it with
``importlib.import_module("continuum-attention_amd")``.
"""
from . import _native as native
from .ops import (SUPPORTED_HEAD_DIMS, _CAExactTiled, ca_backward, ca_forward,
                  continuum_attention)
from .weights import ca_weights, ca_weights_backward, continuous_attention_weights
from . import architecture, decoder, ops, optim

__all__ = ["continuum_attention", "_CAExactTiled", "ca_forward", "ca_backward", "native",
           "SUPPORTED_HEAD_DIMS", "ca_weights", "ca_weights_backward",
           "continuous_attention_weights", "architecture", "decoder", "ops", "optim"]

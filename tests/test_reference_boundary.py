"""The drop-in against the reference's own classes, on the CPU: a config with exactly the
reference TransformerConfig's fields (src/core/transformer.py:25-78, listed in
tests/reference_surface.py) goes through the patched get_attention
(src/core/attention.py:190-194) and builds the paged module with the reference's
parameter shapes; the whole model builds from it; "triton" gives the torch module as the
reference's AttentionTriton does; a contiguous KVCache is taken over (the paged kernels
then refuse CPU tensors); kv_ops is an autograd.Function like KVOpsTriton."""
from __future__ import annotations

import pytest
import torch

from reference_surface import (REFERENCE_FIELDS, RefTransformerConfig, field_list,
                               patched_get_attention)


@pytest.fixture(scope="module")
def M(iva):
    from importlib import import_module
    return import_module("iva_amd.model")


def test_config_has_exactly_the_reference_fields():
    assert field_list() == REFERENCE_FIELDS
    assert len(REFERENCE_FIELDS) == 29
    for name in ("n_kv_heads", "sink_tokens", "rope_in_attention", "kv_block_size",
                 "kv_cache_dtype"):
        assert not hasattr(RefTransformerConfig(), name)
    RefTransformerConfig(attn_impl="hip_paged")
    with pytest.raises(ValueError, match="attn_impl"):
        RefTransformerConfig(attn_impl="flash")


def test_patched_get_attention_builds_the_paged_module(M):
    cfg = RefTransformerConfig(attn_impl="hip_paged", d_model=128, n_heads=4, n_layers=2,
                               dropout=0.0)
    att = patched_get_attention(cfg)
    assert isinstance(att, M.PagedAttention)
    assert att.n_kv_heads == att.n_heads == 4       # the reference has no GQA
    assert att.sink_tokens == 0 and att.rope is False
    # same parameters as the reference's AttentionTorch (attention.py:28-31): a reference
    # state dict loads unchanged
    ref = patched_get_attention(RefTransformerConfig(d_model=128, n_heads=4, dropout=0.0))
    assert isinstance(ref, M.AttentionTorch)
    shapes = {k: tuple(v.shape) for k, v in ref.state_dict().items()}
    assert shapes == {f"{p}_proj.weight": (128, 128) for p in "qkvo"}
    att.load_state_dict(ref.state_dict())


def test_triton_gives_the_torch_module(M):
    cfg = RefTransformerConfig(attn_impl="triton", d_model=64, n_heads=4, dropout=0.0)
    assert type(M.get_attention(cfg)) is M.AttentionTorch


def test_model_builds_from_the_reference_config(M):
    cfg = RefTransformerConfig(attn_impl="hip_paged", d_model=64, n_heads=4, n_layers=3,
                               vocab_size=50, seq_len=64, dropout=0.0)
    model = M.Transformer(cfg).eval()
    assert all(isinstance(b.attention, M.PagedAttention) for b in model.blocks)
    cache = model.new_kv_cache(2, 16, device="cpu", dtype=torch.float32)
    assert cache.num_layers == 3 and cache.n_heads == 4


def test_contiguous_cache_is_taken_over(M):
    """A reference KVCache is adopted as a PagedKVCache; on the CPU the kernels refuse."""
    cfg = RefTransformerConfig(attn_impl="hip_paged", d_model=64, n_heads=4, n_layers=2,
                               dropout=0.0)
    att = M.PagedAttention(cfg).eval()
    kv = M.KVCache(1, 4, 16, 0, torch.device("cpu"))
    with pytest.raises(RuntimeError, match="GPU"):
        att(torch.randn(1, 3, 64), kv_cache=kv)
    with pytest.raises(ValueError, match="sequences"):
        att(torch.randn(2, 3, 64), kv_cache=kv)
    with pytest.raises(TypeError, match="no 'k'"):
        att(torch.randn(1, 3, 64), kv_cache=object())


def test_kv_ops_is_an_autograd_function(iva):
    """kv_ops runs as KVOps.apply (KVOpsTriton.apply, kv_ops_triton.py:95-156), with the
    reference's errors raised from inside it."""
    assert issubclass(iva.KVOps, torch.autograd.Function)
    assert iva.KVOps.backward(None, torch.ones(1)) == (None, None, None, None)
    kv = torch.zeros(1, 1, 4, 8, requires_grad=True)
    with pytest.raises(ValueError, match="Values tensor required"):
        iva.kv_ops(kv, torch.tensor([0]), None, "scatter")
    with pytest.raises(ValueError, match="Unknown operation"):
        iva.kv_ops(kv, torch.tensor([0]), None, "compact")

"""The drop-in boundary on the GPU: attn_impl="hip_paged" against the torch backend
with identical weights.

  * PagedAttention vs AttentionTorch, prefill then single-token decode, fp32 model:
    outputs agree to 2e-5 (the decode kernel's fp32 bound is 1e-5 on attention
    output; the projections add fp32 rounding);
  * window + sink masks through the model (decode kernel page walk vs dense masks);
  * the no-cache forward (one-layer paged cache of the input's own tokens) vs the torch
    backend without a cache, module and model;
  * padding masks (no cache, and a masked prefill followed by masked single-token steps)
    vs the torch backend;
  * Transformer bf16 (config C3's shape family, scaled down): teacher-forced logits of
    prefill + 16 decode steps agree within bf16 tolerance, and greedy tokens agree
    wherever the torch backend's top-2 margin exceeds twice that tolerance, over a
    stated minimum of compared steps (greedy_parity.py);
  * the reference's own surface: a config with exactly the reference's fields through
    the patched get_attention, and the reference's generate loop (a KVCache of length 0,
    the whole sequence fed again each step) on the paged backend;
  * kv_ops under autograd: outputs join the graph, backward gives no gradient;
  * PagedKVCache as a KVCache: update / k / v / get_slice / seq_len / select_layer.
"""
from __future__ import annotations

import pytest
import torch

from greedy_parity import check_greedy_parity
from reference_surface import RefTransformerConfig, reference_generate

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M(iva):
    from importlib import import_module
    return import_module("iva_amd.model")


def twin_models(M, dtype, dev, **kw):
    base = dict(d_model=256, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, seq_len=512,
                dropout=0.0)
    base.update(kw)
    torch.manual_seed(0)
    ref = M.Transformer(M.TransformerConfig(attn_impl="torch", **base)).to(dev, dtype).eval()
    paged = M.Transformer(M.TransformerConfig(attn_impl="hip_paged", **base)).to(dev, dtype).eval()
    paged.load_state_dict(ref.state_dict())
    return ref, paged


def run_steps(model, ids, prefill, dev):
    cache = model.new_kv_cache(ids.shape[0], ids.shape[1], device=dev)
    outs = [model(ids[:, :prefill], kv_cache=cache)["logits"]]
    for t in range(prefill, ids.shape[1]):
        outs.append(model(ids[:, t:t + 1], kv_cache=cache)["logits"])
    assert cache.seq_len == ids.shape[1]
    return torch.cat(outs, dim=1).float(), cache


def test_attention_module_fp32(M, dev):
    cfg = M.TransformerConfig(d_model=512, n_layers=1, n_heads=8, n_kv_heads=2, vocab_size=64,
                              dropout=0.0, attn_impl="hip_paged")
    torch.manual_seed(3)
    pa = M.PagedAttention(cfg).to(dev).eval()
    ta = M.AttentionTorch(M.TransformerConfig(**{**cfg.__dict__, "attn_impl": "torch"})).to(dev).eval()
    ta.load_state_dict(pa.state_dict())
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    pcache = pc.PagedKVCache(3, 2, 64, 0, dev, torch.float32, num_layers=1, max_seq_len=200)
    tcache = M.LayeredKVCache(3, 2, 64, 1, dev, torch.float32)
    x = torch.randn(3, 150, 512, device=dev) * 0.5
    with torch.no_grad():
        a, _ = pa(x[:, :100], kv_cache=pcache)
        b, _ = ta(x[:, :100], kv_cache=tcache)
        assert (a - b).abs().max().item() <= 2e-5
        for t in range(100, 150):
            a, _ = pa(x[:, t:t + 1], kv_cache=pcache)
            b, _ = ta(x[:, t:t + 1], kv_cache=tcache)
            assert (a - b).abs().max().item() <= 2e-5, f"decode step {t}"
    assert pcache.seq_len == tcache.seq_len == 150


def test_no_cache_forward_matches_torch_backend(M, dev):
    """Without a cache (the path of a plain ``model(input_ids)`` and of the reference's
    generate_stream, src/api/generate.py:183-188) PagedAttention runs the paged append and
    prefill kernels on a one-layer cache of its own tokens and returns None, as
    AttentionTorch does (src/core/attention.py:74-75)."""
    cfg = M.TransformerConfig(d_model=512, n_layers=1, n_heads=8, n_kv_heads=2, vocab_size=64,
                              dropout=0.0, attn_impl="hip_paged")
    torch.manual_seed(5)
    pa = M.PagedAttention(cfg).to(dev).eval()
    ta = M.AttentionTorch(M.TransformerConfig(**{**cfg.__dict__, "attn_impl": "torch"})).to(dev).eval()
    ta.load_state_dict(pa.state_dict())
    x = torch.randn(3, 333, 512, device=dev) * 0.5
    with torch.no_grad():
        for window, sinks in ((None, None), (40, {"sink_tokens": 4})):
            a, ca = pa(x, sliding_window=window, sink_cfg=sinks)
            b, cb = ta(x, sliding_window=window, sink_cfg=sinks)
            assert ca is None and cb is None
            assert (a - b).abs().max().item() <= 2e-5, f"window {window}"
    ref, paged = twin_models(M, torch.float32, dev, sliding_window=64, sink_tokens=4)
    ids = torch.randint(0, 512, (2, 200), device=dev)
    with torch.no_grad():
        lr, lp = ref(ids)["logits"], paged(ids)["logits"]
    assert (lr - lp).abs().max().item() <= 1e-4


def test_padding_masks_match_the_torch_backend(M, dev):
    """Padding masks (the reference's broadcast, src/core/attention.py:95-97) on the paged
    backend: the step's rows go through the append and gather kernels, the masked
    attention is evaluated on the gathered keys; against the torch backend with the same
    weights, without a cache (left padding, right padding, holes; fully masked rows are
    zero in both) and with one (a masked prefill, then single-token steps whose width-1
    masks keep or drop whole rows)."""
    ref, paged = twin_models(M, torch.float32, dev, sliding_window=None)
    ids = torch.randint(0, 512, (3, 40), device=dev)
    mask = torch.ones(3, 40, dtype=torch.long, device=dev)
    mask[0, :7] = 0
    mask[1, 31:] = 0
    mask[2, 5:9] = 0
    with torch.no_grad():
        lr = ref(ids, attention_mask=mask)["logits"]
        lp = paged(ids, attention_mask=mask)["logits"]
        assert (lr - lp).abs().max().item() <= 1e-4
        cr = ref.new_kv_cache(3, 48, device=dev)
        cp = paged.new_kv_cache(3, 48, device=dev)
        outs = []
        for m in (ref, paged):
            c = cr if m is ref else cp
            o = [m(ids[:, :32], attention_mask=mask[:, :32], kv_cache=c)["logits"]]
            for t, keep in zip(range(32, 40), ([1, 1, 1], [1, 0, 1], [0, 1, 1], [1, 1, 1])* 2):
                step_mask = torch.tensor(keep, device=dev).view(3, 1)
                o.append(m(ids[:, t:t + 1], attention_mask=step_mask, kv_cache=c)["logits"])
            outs.append(torch.cat(o, dim=1))
        assert (outs[0] - outs[1]).abs().max().item() <= 1e-4
        assert cp.seq_len == 40


def test_window_and_sinks_through_the_model(M, dev):
    ref, paged = twin_models(M, torch.float32, dev, sliding_window=24, sink_tokens=4)
    ids = torch.randint(0, 512, (2, 90), device=dev)
    with torch.no_grad():
        lr, _ = run_steps(ref, ids, 40, dev)
        lp, _ = run_steps(paged, ids, 40, dev)
    assert (lr - lp).abs().max().item() <= 1e-4


def test_transformer_bf16_logits_and_greedy_tokens(M, dev):
    ref, paged = twin_models(M, torch.bfloat16, dev)
    ids = torch.randint(0, 512, (4, 64 + 16), device=dev)
    with torch.no_grad():
        lr, _ = run_steps(ref, ids, 64, dev)
        lp, _ = run_steps(paged, ids, 64, dev)
    tol = 0.05  # bf16 logits of a 2-layer model: both paths round activations to bf16
    assert (lr - lp).abs().max().item() <= tol
    # top-2 logit gaps of this model (vocab 512, logit std ~0.32) are ~0.09: 8 x 48 steps
    # give about a hundred steps above the 2 * tol margin
    prompts = torch.randint(0, 512, (8, 64), generator=torch.Generator().manual_seed(1)).to(dev)
    r = check_greedy_parity(ref, paged, prompts, steps=48, tol=tol, min_compared=32)
    print(f"compared {r['compared']} of 384 steps; first divergences {r['first_divergence']}")


def test_paged_cache_duck_type(M, iva, dev):
    from importlib import import_module
    pc = import_module("iva_amd.paged_cache")
    cache = pc.PagedKVCache(2, 4, 64, 0, dev, torch.float16, num_layers=2, max_seq_len=100)
    k1 = torch.randn(2, 4, 37, 64, device=dev).half()
    v1 = torch.randn(2, 4, 37, 64, device=dev).half()
    cache.select_layer(1)
    cache.update(k1, v1, 0)
    assert cache.seq_len == 37
    assert torch.equal(cache.k.view(torch.int16), k1.view(torch.int16))
    assert torch.equal(cache.v.view(torch.int16), v1.view(torch.int16))
    k2 = torch.randn(2, 4, 5, 64, device=dev).half()
    cache.update(k2, k2, 37)
    ks, vs = cache.get_slice(30, 42)
    assert torch.equal(ks[:, :, 7:].view(torch.int16), k2.view(torch.int16))
    assert torch.equal(ks[:, :, :7].view(torch.int16), k1[:, :, 30:].view(torch.int16))
    cache.select_layer(0)
    assert not cache.k.view(torch.int16).any()  # layer 0 untouched
    n_free = cache.pool.num_free_pages
    cache.free()
    assert cache.pool.num_free_pages > n_free


def test_graph_decode_matches_eager(M, dev):
    """generate(use_graph=True) replays one captured decode step with device-side cache
    bookkeeping; it must emit exactly the tokens of the eager loop."""
    _, paged = twin_models(M, torch.bfloat16, dev)
    ids = torch.randint(0, 512, (4, 40), device=dev)
    with torch.no_grad():
        a = paged.generate(ids, max_length=12, do_sample=False, eos_token_id=None, use_graph=True)
        b = paged.generate(ids, max_length=12, do_sample=False, eos_token_id=None, use_graph=False)
    assert a.shape == (4, 52) and torch.equal(a, b)
    # a cache passed in keeps its length bookkeeping in step with the device
    cache = paged.new_kv_cache(4, 60)
    with torch.no_grad():
        paged.generate(ids, max_length=10, do_sample=False, eos_token_id=None, use_graph=True,
                       kv_cache=cache)
    assert cache.seq_len == 40 + 9   # the last sampled token is not fed back
    assert all(cache.pool.length(s) == 49 for s in cache.seq_ids)
    cache.free()


def test_fp8_kv_cache_through_the_model(M, dev):
    """kv_cache_dtype="fp8": prefill over e4m3fn pages (gathered, dequantized) and FP8
    decode steps.  Logits stay close to the same model with a bf16 cache (the pages are
    quantized, so this is a closeness check, not parity); graph decode == eager."""
    _, paged = twin_models(M, torch.bfloat16, dev)
    _, paged8 = twin_models(M, torch.bfloat16, dev, kv_cache_dtype="fp8")
    paged8.load_state_dict(paged.state_dict())
    ids = torch.randint(0, 512, (4, 48 + 12), device=dev)
    with torch.no_grad():
        l16, _ = run_steps(paged, ids, 48, dev)
        l8, cache = run_steps(paged8, ids, 48, dev)
        assert cache.pool.fp8
        assert (l16 - l8).abs().max().item() <= 0.25
        a = paged8.generate(ids[:, :40], max_length=8, do_sample=False, eos_token_id=None, use_graph=True)
        b = paged8.generate(ids[:, :40], max_length=8, do_sample=False, eos_token_id=None, use_graph=False)
    assert torch.equal(a, b)


def test_rope_in_attention_paged_vs_torch(M, dev):
    """rope_in_attention=True: the paged backend rotates q in place and K inside the
    append (fused) or before the fused decode op; logits match the torch backend's
    vectorized reference RoPE; graph decode (device-side positions) == eager."""
    ref, paged = twin_models(M, torch.float32, dev, rope_in_attention=True)
    ids = torch.randint(0, 512, (3, 40 + 10), device=dev)
    with torch.no_grad():
        lr, _ = run_steps(ref, ids, 40, dev)
        lp, _ = run_steps(paged, ids, 40, dev)
    assert (lr - lp).abs().max().item() <= 1e-4
    _, p16 = twin_models(M, torch.bfloat16, dev, rope_in_attention=True)
    with torch.no_grad():
        a = p16.generate(ids[:, :24], max_length=8, do_sample=False, eos_token_id=None, use_graph=True)
        b = p16.generate(ids[:, :24], max_length=8, do_sample=False, eos_token_id=None, use_graph=False)
    assert torch.equal(a, b)


def test_fp8_cache_with_rope_in_attention(M, dev):
    """kv_cache_dtype="fp8" with rope_in_attention=True: prefill chunks take the fused FP8
    RoPE append (ivakv_append_rope_fp8), decode steps rotate K before the fused FP8 step.
    Logits stay close to the bf16-cache model with the same RoPE (quantized pages: a
    closeness check); graph decode == eager."""
    _, p16 = twin_models(M, torch.bfloat16, dev, rope_in_attention=True)
    _, p8 = twin_models(M, torch.bfloat16, dev, rope_in_attention=True, kv_cache_dtype="fp8")
    p8.load_state_dict(p16.state_dict())
    ids = torch.randint(0, 512, (3, 40 + 10), device=dev)
    with torch.no_grad():
        l16, _ = run_steps(p16, ids, 40, dev)
        l8, cache = run_steps(p8, ids, 40, dev)
        assert cache.pool.fp8
        assert (l16 - l8).abs().max().item() <= 0.25
        a = p8.generate(ids[:, :24], max_length=8, do_sample=False, eos_token_id=None, use_graph=True)
        b = p8.generate(ids[:, :24], max_length=8, do_sample=False, eos_token_id=None, use_graph=False)
    assert torch.equal(a, b)


def test_reference_config_and_generate_loop(M, dev):
    """The reference's own TransformerConfig fields (no n_kv_heads, sinks or RoPE flag)
    build the paged model; the reference's generate loop (transformer.py:257-320: a
    contiguous KVCache of length 0, the whole sequence fed again every step) runs on it:
    each forward takes the KVCache over as a paged cache with one layer per block, so
    every step is a paged prefill of the whole sequence.  fp32: logits equal the torch
    backend's no-cache forward to 1e-4, and the greedy tokens equal the torch backend's
    incremental generate wherever its top-2 margin exceeds 2e-4."""
    kw = dict(d_model=256, n_layers=2, n_heads=4, vocab_size=512, seq_len=512, dropout=0.0)
    torch.manual_seed(0)
    ref = M.Transformer(RefTransformerConfig(attn_impl="torch", **kw)).to(dev).eval()
    paged = M.Transformer(RefTransformerConfig(attn_impl="hip_paged", **kw)).to(dev).eval()
    paged.load_state_dict(ref.state_dict())
    assert all(isinstance(b.attention, M.PagedAttention) for b in paged.blocks)
    ids = torch.randint(0, 512, (3, 40), generator=torch.Generator().manual_seed(2)).to(dev)
    with torch.no_grad():
        cache = M.KVCache(3, 4, 64, 0, dev)
        lp = paged(ids, kv_cache=cache)["logits"]
        lr = ref(ids)["logits"]
    assert cache.seq_len == 0 and cache.k.numel() == 0   # the caller's cache is untouched
    assert (lp - lr).abs().max().item() <= 1e-4
    steps = 12
    got = reference_generate(paged, ids, max_length=steps, do_sample=False, eos_token_id=-1)
    want = ref.generate(ids, max_length=steps, do_sample=False, eos_token_id=None)
    assert got.shape == want.shape == (3, 40 + steps)
    with torch.no_grad():
        lw, _ = run_steps(ref, want, 40, dev)
    top2 = lw[:, 39:-1].topk(2, dim=-1).values
    margin = top2[..., 0] - top2[..., 1]
    assert int((margin > 2e-4).sum()) >= 30
    for b in range(3):   # a stream may leave the torch one only at a near-tie
        differ = (got[b, 40:] != want[b, 40:]).nonzero()
        if differ.numel():
            assert margin[b, int(differ[0])] <= 2e-4, f"sequence {b} at step {int(differ[0])}"


def test_kv_ops_autograd(iva, dev):
    """kv_ops is KVOps.apply (KVOpsTriton, kv_ops_triton.py:95-147): an output of a cache
    that requires grad joins the graph, and backward through it gives no gradient."""
    kv = torch.randn(2, 3, 16, 8, device=dev, requires_grad=True)
    idx = torch.tensor([3, 0, 7], device=dev)
    out = iva.kv_ops(kv, idx)
    assert out.requires_grad and out.grad_fn is not None
    assert torch.equal(out.detach(), kv.detach()[:, :, idx])
    (out.sum() * 2).backward()
    assert kv.grad is None
    vals = torch.randn(2, 3, 3, 8, device=dev)
    sc = iva.kv_ops(kv, idx, vals, operation="scatter")
    assert sc.requires_grad and torch.equal(sc.detach()[:, :, idx], vals)

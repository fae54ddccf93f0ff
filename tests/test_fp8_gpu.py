"""FP8 (OCP e4m3fn) KV pages on the GPU vs the CPU oracle.

  * append: codes and per-(slot, kv head) scaling factors bit-exact (untouched bytes
    and factors unchanged), for fp32 / fp16 / bf16 source rows over six decades of
    row magnitude, all-zero rows and skipped slots;
  * gather: dequantized rows exact (float32 division, then the output cast), and all
    256 codes decode as torch.float8_e4m3fn does;
  * decode attention over FP8 pages (unit-scale data, as the other attention tests):
    within 2e-3 (+ one half-ulp of the output dtype times |exact|) of the fp64 oracle on
    the dequantized pages, fp16 and bf16 queries, windows and sinks, invalid page ids,
    garbage (NaN included) codes past the context;
  * the fused append + attend op on FP8 pages: pools and factors byte-identical to
    the oracle's append of the new rows (inf, NaN and out-of-range rows included, on
    each walk), output within the same bound;
  * chunked prefill over FP8 pages vs the oracle's prefill on the dequantized pages.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as orc

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
OUT_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.uint8).numpy()


def fp8_case(iva, lengths, hkv, d, src_dtype, seed, extra_pages=3, decades=6.0):
    """Rows of magnitude 10^U(-decades/2, decades/2) (decades=0: N(0, 1/d) rows, the
    scale of the other attention tests), written over garbage codes and factors."""
    gen = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(n / 16) for n in lengths)
    num_pages = need + extra_pages
    layout = iva.workloads.permuted_layout(lengths, num_pages, gen)
    ks, vs = iva.pool_shapes(num_pages, hkv, d, 16, FP8)
    k_pool = torch.randint(0, 256, ks, dtype=torch.uint8, generator=gen)  # garbage codes
    v_pool = torch.randint(0, 256, vs, dtype=torch.uint8, generator=gen)
    k_scale = torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5
    v_scale = torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5
    n_tok = sum(lengths)
    mag = 10.0 ** ((torch.rand(n_tok, hkv, 1, generator=gen) - 0.5) * decades) if decades \
        else torch.full((n_tok, hkv, 1), d ** -0.5)
    k_new = (torch.randn(n_tok, hkv, d, generator=gen) * mag).to(src_dtype)
    v_new = (torch.randn(n_tok, hkv, d, generator=gen) * mag).to(src_dtype)
    if n_tok > 5:
        k_new[5] = 0
    slots = torch.cat([layout.slots(b, torch.arange(n)) for b, n in enumerate(lengths)])
    return dict(layout=layout, k_pool=k_pool, v_pool=v_pool, k_scale=k_scale, v_scale=v_scale,
                k_new=k_new, v_new=v_new, slots=slots, num_pages=num_pages)


def append_both(iva, dev, c, slots=None):
    """The same append on the GPU and in the oracle; returns (gpu tensors, oracle arrays)."""
    slots = c["slots"] if slots is None else slots
    g = {k: c[k].clone().to(dev) for k in ("k_pool", "v_pool", "k_scale", "v_scale")}
    g["k_pool"], g["v_pool"] = g["k_pool"].view(FP8), g["v_pool"].view(FP8)
    iva.kv_append(c["k_new"].to(dev), c["v_new"].to(dev), g["k_pool"], g["v_pool"],
                  slots.to(dev), k_scale=g["k_scale"], v_scale=g["v_scale"])
    o = dict(k_pool=c["k_pool"].numpy().copy(), v_pool=c["v_pool"].numpy().copy(),
             k_scale=c["k_scale"].numpy().copy(), v_scale=c["v_scale"].numpy().copy())
    orc.append_fp8(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"],
                   c["k_new"].float().numpy(), c["v_new"].float().numpy(), slots.numpy())
    return g, o


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
def test_append_fp8_bit_exact(iva, dev, src, d):
    c = fp8_case(iva, [17, 40, 3], 4, d, src, seed=d)
    slots = c["slots"].clone()
    slots[7] = -1
    slots[9] = c["num_pages"] * 16 + 3  # outside the pool: skipped
    g, o = append_both(iva, dev, c, slots)
    torch.cuda.synchronize()
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"])
    assert np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
def test_append_fp8_whole_pages_bit_exact(iva, dev, src, d):
    """Chunk appends whose 16-token groups each fill one page in slot order, mixed with
    groups that do not (a sequence of 20 tokens, a group spanning two sequences), on 5 kv
    heads: codes and factors equal the oracle's."""
    c = fp8_case(iva, [32, 48, 20, 12, 16], 5, d, src, seed=d + 3)
    g, o = append_both(iva, dev, c)
    torch.cuda.synchronize()
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"])
    assert np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])


@pytest.mark.parametrize("n_groups", [12, 160], ids=["few_tokens", "many_tokens"])
def test_append_fp8_groups_that_only_look_page_aligned(iva, dev, n_groups):
    """Token groups whose first slot starts a page and whose last slot ends it, with
    anything in between: the rows of that page permuted, a skipped slot, rows of other
    pages, and a duplicate-free mix with plain page-order groups and groups that start
    mid-page. Codes and factors equal the oracle's (the kernel picks its lane layout
    from a group's first and last slot; the result must not depend on it). 12 groups
    take the one-head-per-wave launch, 160 the every-head-per-workgroup one."""
    gen = torch.Generator().manual_seed(71 + n_groups)
    hkv, d = 8, 128
    num_pages = 2 * n_groups + 4
    pages = torch.randperm(num_pages, generator=gen)
    rows = []
    for i in range(n_groups):
        p, q = int(pages[2 * i]), int(pages[2 * i + 1])
        kind = i % 4
        if kind == 0:  # page order
            s = p * 16 + torch.arange(16)
        elif kind == 1:  # first and last in place, the rows between permuted
            s = p * 16 + torch.cat([torch.tensor([0]), 1 + torch.randperm(14, generator=gen),
                                    torch.tensor([15])])
        elif kind == 2:  # first and last of one page, the rows between from another page
            s = torch.cat([torch.tensor([p * 16]), q * 16 + 1 + torch.arange(14),
                           torch.tensor([p * 16 + 15])])
        else:  # starts mid-page and runs into the next page
            off = int(torch.randint(1, 16, (1,), generator=gen))
            s = torch.cat([p * 16 + torch.arange(off, 16), q * 16 + torch.arange(off)])
        rows.append(s)
    slots = torch.cat(rows).to(torch.int32)
    slots[16 * 1 + 5] = -1  # a skipped slot inside a permuted group
    n_tok = slots.numel()
    ks, vs = iva.pool_shapes(num_pages, hkv, d, 16, FP8)
    mag = 10.0 ** ((torch.rand(n_tok, hkv, 1, generator=gen) - 0.5) * 6.0)
    c = dict(k_pool=torch.randint(0, 256, ks, dtype=torch.uint8, generator=gen),
             v_pool=torch.randint(0, 256, vs, dtype=torch.uint8, generator=gen),
             k_scale=torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5,
             v_scale=torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5,
             k_new=(torch.randn(n_tok, hkv, d, generator=gen) * mag).half(),
             v_new=(torch.randn(n_tok, hkv, d, generator=gen) * mag).half(), slots=slots)
    g, o = append_both(iva, dev, c)
    torch.cuda.synchronize()
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"])
    assert np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])


@pytest.mark.parametrize("src", [torch.float16, torch.bfloat16], ids=str)
def test_append_fp8_chunks_starting_mid_page(iva, dev, src):
    """One call appends a 512-row chunk to each of 10 sequences that already hold L_b
    rows (most not a multiple of 16), so every chunk starts mid-page and neighbouring
    token groups share pages: codes and factors equal the oracle's; with RoPE fused,
    byte-identical to rope_ followed by the FP8 append of the rotated rows."""
    gen = torch.Generator().manual_seed(23)
    prior = [int(x) for x in torch.randint(1, 900, (10,), generator=gen)]
    prior[0] = 16 * 5
    chunk, hkv, d = 512, 8, 128
    total = [n + chunk for n in prior]
    num_pages = sum(-(-n // 16) for n in total) + 3
    lay = iva.workloads.permuted_layout(total, num_pages, gen)
    k_new = (torch.randn(10 * chunk, hkv, d, generator=gen) * d ** -0.5).to(src)
    v_new = (torch.randn(10 * chunk, hkv, d, generator=gen) * d ** -0.5).to(src)
    slots = torch.cat([lay.slots(b, torch.arange(n, n + chunk)) for b, n in enumerate(prior)])
    ks, vs = iva.pool_shapes(num_pages, hkv, d, 16, FP8)
    base = dict(k_pool=torch.randint(0, 256, ks, dtype=torch.uint8, generator=gen),
                v_pool=torch.randint(0, 256, vs, dtype=torch.uint8, generator=gen),
                k_scale=torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5,
                v_scale=torch.rand(iva.scale_shape(num_pages, hkv), generator=gen) + 0.5,
                k_new=k_new, v_new=v_new, slots=slots)
    g, o = append_both(iva, dev, base)
    torch.cuda.synchronize()
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"]) and np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])
    pos = torch.cat([torch.arange(n, n + chunk) for n in prior]).to(torch.int32).to(dev)
    out = []
    for fused in (True, False):
        t = {k: base[k].clone().to(dev) for k in ("k_pool", "v_pool", "k_scale", "v_scale")}
        t["k_pool"], t["v_pool"] = t["k_pool"].view(FP8), t["v_pool"].view(FP8)
        if fused:
            iva.kv_append(k_new.to(dev), v_new.to(dev), t["k_pool"], t["v_pool"], slots.to(dev),
                          k_scale=t["k_scale"], v_scale=t["v_scale"], rope_positions=pos)
        else:
            k_rot = iva.rope_(k_new.to(dev).clone(), pos)
            iva.kv_append(k_rot, v_new.to(dev), t["k_pool"], t["v_pool"], slots.to(dev),
                          k_scale=t["k_scale"], v_scale=t["v_scale"])
        out.append([u8(t["k_pool"]), u8(t["v_pool"]), t["k_scale"].cpu().numpy(), t["v_scale"].cpu().numpy()])
    for a_, b_ in zip(*out):
        assert np.array_equal(a_, b_)


@pytest.mark.parametrize("src", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("rope", [False, True], ids=["plain", "rope"])
def test_append_fp8_from_unaligned_strided_rows(iva, dev, src, rope):
    """Source rows that start one element into a wider buffer (aligned to the element
    only) and a kv head stride larger than head_dim: codes and factors equal those of the
    same rows appended from a contiguous copy, plain or with RoPE fused (and, plain, the
    oracle's)."""
    d, hkv = 128, 3
    c = fp8_case(iva, [17, 40, 3], hkv, d, src, seed=41, decades=0)
    n = c["k_new"].shape[0]
    wide_k = torch.zeros(n, hkv, d + 8, dtype=src, device=dev)
    wide_v = torch.zeros(n, hkv, d + 8, dtype=src, device=dev)
    k_src, v_src = wide_k[..., 1:d + 1], wide_v[..., 1:d + 1]
    k_src.copy_(c["k_new"].to(dev))
    v_src.copy_(c["v_new"].to(dev))
    assert k_src.data_ptr() % 16 and v_src.data_ptr() % 16
    pos = (torch.arange(n, dtype=torch.int32) * 37).to(dev)
    kw = dict(rope_positions=pos) if rope else {}
    out = []
    for k_in, v_in in ((k_src, v_src), (c["k_new"].to(dev), c["v_new"].to(dev))):
        g = {k: c[k].clone().to(dev) for k in ("k_pool", "v_pool", "k_scale", "v_scale")}
        g["k_pool"], g["v_pool"] = g["k_pool"].view(FP8), g["v_pool"].view(FP8)
        iva.kv_append(k_in, v_in, g["k_pool"], g["v_pool"], c["slots"].to(dev),
                      k_scale=g["k_scale"], v_scale=g["v_scale"], **kw)
        out.append([u8(g["k_pool"]), u8(g["v_pool"]), g["k_scale"].cpu().numpy(),
                    g["v_scale"].cpu().numpy()])
    for a, b in zip(*out):
        assert np.array_equal(a, b)
    if not rope:  # and both equal the oracle's append
        o = dict(k_pool=c["k_pool"].numpy().copy(), v_pool=c["v_pool"].numpy().copy(),
                 k_scale=c["k_scale"].numpy().copy(), v_scale=c["v_scale"].numpy().copy())
        orc.append_fp8(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"],
                       c["k_new"].float().numpy(), c["v_new"].float().numpy(), c["slots"].numpy())
        assert np.array_equal(out[0][0], o["k_pool"]) and np.array_equal(out[0][1], o["v_pool"])


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("out_len,outputs", [(48, "aligned"), (45, "aligned"), (48, "offset")])
def test_gather_fp8_exact(iva, dev, out_dtype, d, out_len, outputs):
    """Dequantized rows equal the oracle's (code / factor in float32, then the output
    cast), zero past the context and on an invalid page; out_len 45 ends inside a page
    (on 5 kv heads: a group of four and a group of one in the chunk kernel's workgroups).
    "offset": outputs that are views 4-8 bytes into a buffer (not 16-byte aligned: the
    element-wise kernel), else the 16-byte chunk kernel."""
    hkv = 5 if out_len == 45 else 2
    c = fp8_case(iva, [17, 40, 3, 0], hkv, d, torch.float16, seed=3 + d)
    g, o = append_both(iva, dev, c)
    lay = c["layout"]
    bt = lay.block_tables.clone()
    bt[1, 1] = -1
    out = None
    if outputs == "offset":
        shape = (4, 2, out_len, d)
        n = 4 * 2 * out_len * d
        bufs = [torch.full((n + 8,), 7.0, dtype=out_dtype, device=dev) for _ in range(2)]
        out = tuple(b_[2:2 + n].view(shape) for b_ in bufs)
        assert all(t.data_ptr() % 16 for t in out)
    ko, vo = iva.kv_gather(g["k_pool"], g["v_pool"], bt.to(dev), lay.context_lens.to(dev),
                           out_len=out_len, out=out, k_scale=g["k_scale"], v_scale=g["v_scale"],
                           out_dtype=out_dtype)
    rk, rv = orc.gather_fp8(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"], bt.numpy(),
                            lay.context_lens.numpy(), out_len=out_len)
    exp_k = torch.from_numpy(rk).to(out_dtype)
    exp_v = torch.from_numpy(rv).to(out_dtype)
    assert torch.equal(ko.cpu(), exp_k) and torch.equal(vo.cpu(), exp_v)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16], ids=str)
def test_gather_fp8_quotients_are_ieee(iva, dev, out_dtype):
    """Every code over factors spread log-uniformly on [2^-120, 2^120] and at chosen
    points (powers of two and their float neighbours, negative factors, 1e-8, 1e8):
    through the 16-byte chunk kernel the gathered values are float32 code / factor
    rounded once, bit for bit, then cast; NaN codes stay NaN."""
    pages, d = 96, 256
    ks, vs = iva.pool_shapes(pages, 1, d, 16, FP8)
    g = torch.Generator().manual_seed(12)
    n = pages * 16 * d
    kb = ((torch.arange(n) * 5 + torch.arange(n) // 4096) % 256).to(torch.uint8).reshape(ks)
    vb = ((torch.arange(n) * 7 + torch.arange(n) // 4096) % 256).to(torch.uint8).reshape(vs)
    sf = (2.0 ** (torch.rand(pages, 1, 16, generator=g, dtype=torch.float64) * 240 - 120)).float()
    edge = np.float32(2.0 ** 100)
    specials = [2.0 ** -100, np.nextafter(np.float32(2.0 ** -100), np.float32(0)), 2.0 ** 100,
                np.nextafter(edge, np.float32(np.inf)), -(2.0 ** -100), -3.0, -(2.0 ** 100),
                1e-8, 1e8, 1.0, 448 / 3.3, 2.0 ** -120, 2.0 ** 120, 0.7, 1.5, 3.0]
    sf[0, 0, :] = torch.tensor(specials, dtype=torch.float32)
    vsf = sf.flip(0).contiguous()
    bt = torch.arange(pages, dtype=torch.int32).reshape(pages, 1)
    ctx = torch.full((pages,), 16, dtype=torch.int32)
    ko, vo = iva.kv_gather(kb.view(FP8).to(dev), vb.view(FP8).to(dev), bt.to(dev), ctx.to(dev),
                           out_len=16, k_scale=sf.to(dev), v_scale=vsf.to(dev),
                           out_dtype=out_dtype)
    rk, rv = orc.gather_fp8(kb.numpy(), vb.numpy(), sf.numpy(), vsf.numpy(), bt.numpy(),
                            ctx.numpy(), out_len=16)
    bits = torch.int32 if out_dtype == torch.float32 else torch.int16
    for got, ref in ((ko.cpu(), rk), (vo.cpu(), rv)):
        exp = torch.from_numpy(ref).to(out_dtype)
        nan = torch.isnan(exp)
        assert torch.equal(torch.isnan(got), nan)
        assert torch.equal(got[~nan].view(bits), exp[~nan].view(bits))


def test_all_codes_decode_as_torch(iva, dev):
    """Every code (each appears 16 times in one page, factor 1) gathers as
    torch.float8_e4m3fn converts it."""
    ks, vs = iva.pool_shapes(1, 1, 256, 16, FP8)
    kb = (torch.arange(4096) % 256).to(torch.uint8).reshape(ks)   # [1, 1, 16, 16, 16]
    vb = (torch.arange(4096) * 7 % 256).to(torch.uint8).reshape(vs)  # [1, 1, 256, 16]
    scale = torch.ones(1, 1, 16)
    ko, vo = iva.kv_gather(kb.view(FP8).to(dev), vb.view(FP8).to(dev),
                           torch.zeros(1, 1, dtype=torch.int32, device=dev),
                           torch.tensor([16], dtype=torch.int32, device=dev), out_len=16,
                           k_scale=scale.to(dev), v_scale=scale.to(dev), out_dtype=torch.float32)
    kref = kb.view(FP8).float()[0, 0].permute(1, 0, 2).reshape(16, 256)  # [row, dim]
    # V bytes are in the FP8 tile order; the oracle's inverse gives (dim, key)
    vnat = torch.from_numpy(orc.fp8_v_from_tiles(vb.numpy()))
    vref = vnat.view(FP8).float()[0, 0].t()
    for got, exp in ((ko[0, 0].cpu(), kref), (vo[0, 0].cpu(), vref)):
        assert torch.equal(torch.isnan(got), torch.isnan(exp))
        assert torch.equal(got[~torch.isnan(got)], exp[~torch.isnan(exp)])


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("window,sink,units", [(0, 0, "few"), (70, 4, "few"), (0, 0, "mid"),
                                                (70, 4, "mid")])
def test_decode_fp8_vs_oracle(iva, dev, qdt, d, window, sink, units):
    """FP8 decode attention against the oracle on the dequantized pages; "mid": 40
    sequences x 8 kv heads on tables of at most 33 pages (one to four units per CU: one
    partition per sequence in a single launch), else a few units (the stream walk)."""
    lengths = [1, 16, 17, 100, 257, 513]
    hq, hkv = 8, 2
    if units == "mid":
        lengths = lengths + torch.randint(2, 60, (34,), generator=torch.Generator().manual_seed(4)).tolist()
        hq, hkv = 32, 8
    c = fp8_case(iva, lengths, hkv, d, torch.float32, seed=11 + d, decades=0)
    g, o = append_both(iva, dev, c)
    lay = c["layout"]
    bt = lay.block_tables.clone()
    bt[4, 3] = -1                     # an invalid page inside a context
    q = (torch.randn(len(lengths), hq, d, generator=torch.Generator().manual_seed(5)) * d ** -0.5).to(qdt)
    out = iva.paged_decode_attention(q.to(dev), g["k_pool"], g["v_pool"], bt.to(dev),
                                     lay.context_lens.to(dev), window=window, n_sink=sink,
                                     k_scale=g["k_scale"], v_scale=g["v_scale"])
    ref = orc.decode_attention_fp8(q.float().numpy(), o["k_pool"], o["v_pool"], o["k_scale"],
                                   o["v_scale"], bt.numpy(), lay.context_lens.numpy(),
                                   window=window, n_sink=sink)
    err = np.abs(out.float().cpu().numpy() - ref)
    bound = 2e-3 + OUT_ULP[qdt] * np.abs(ref)
    assert (err <= bound).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("window,sink,many", [(0, 0, False), (70, 4, False), (0, 0, True),
                                               (0, 0, "mid"), (70, 4, "mid")])
def test_decode_append_fp8_fused_vs_oracle(iva, dev, qdt, d, window, sink, many):
    """The fused op on FP8 pages: pools and factors afterwards byte-identical to the
    oracle's append of the new rows (the same quantization as kv_append), output within
    2e-3 of the oracle's decode over the dequantized pages.  An empty sequence (zero
    row, nothing stored), a sequence of one token (the new token alone) and a new token
    whose page id is invalid (neither stored nor attended).  ``many``: 136 sequences x 8
    kv heads (>= 1024 units: the merge with four output elements per thread); "mid": 40
    sequences x 8 kv heads on tables of at most 33 pages (one to four units per CU: the
    single launch, each unit walked and merged by one workgroup)."""
    lengths = [0, 1, 16, 17, 100, 257, 513]
    hq, hkv = 8, 2
    if many:
        extra = 129 if many is True else 33
        lengths = lengths + torch.randint(2, 60, (extra,), generator=torch.Generator().manual_seed(3)).tolist()
        hq, hkv = 32, 8
    c = fp8_case(iva, lengths, hkv, d, torch.float32, seed=31 + d, decades=0)
    offs = np.cumsum([0] + lengths[:-1]).tolist()
    prev = torch.cat([torch.arange(o, o + n - 1) for o, n in zip(offs, lengths) if n > 1])
    g, o = append_both(iva, dev, dict(c, k_new=c["k_new"][prev], v_new=c["v_new"][prev],
                                      slots=c["slots"][prev]))
    lay = c["layout"]
    bt = lay.block_tables.clone()
    bt[4, (lengths[4] - 1) // 16] = -1          # the new token's page of sequence 4
    ctx = lay.context_lens
    kn = torch.zeros(len(lengths), hkv, d)
    vn = torch.zeros(len(lengths), hkv, d)
    step_slots = torch.full((len(lengths),), -1, dtype=torch.int32)
    for b, (off, n) in enumerate(zip(offs, lengths)):
        if n == 0:
            continue
        kn[b], vn[b] = c["k_new"][off + n - 1], c["v_new"][off + n - 1]
        page = int(bt[b, (n - 1) // 16])
        if page >= 0:
            step_slots[b] = page * 16 + (n - 1) % 16
    kn, vn = kn.to(qdt), vn.to(qdt)
    q = (torch.randn(len(lengths), hq, d, generator=torch.Generator().manual_seed(6)) * d ** -0.5).to(qdt)
    out = iva.paged_decode_append_attention(q.to(dev), kn.to(dev), vn.to(dev), g["k_pool"],
                                            g["v_pool"], bt.to(dev), ctx.to(dev), window=window,
                                            n_sink=sink, k_scale=g["k_scale"],
                                            v_scale=g["v_scale"])
    orc.append_fp8(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"], kn.float().numpy(),
                   vn.float().numpy(), step_slots.numpy())
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"]) and np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])
    ref = orc.decode_attention_fp8(q.float().numpy(), o["k_pool"], o["v_pool"], o["k_scale"],
                                   o["v_scale"], bt.numpy(), ctx.numpy(), window=window,
                                   n_sink=sink)
    err = np.abs(out.float().cpu().numpy() - ref)
    bound = 2e-3 + OUT_ULP[qdt] * np.abs(ref)
    assert (err <= bound).all(), f"max err {err.max():.3e}"
    assert not out[0].any()                      # empty sequence


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("walk", ["stream", "many", "single"])
def test_decode_append_fp8_fused_rows_beyond_the_scaled_range(iva, dev, qdt, walk):
    """New rows that leave e4m3's range under their factor, through the fused op: an inf
    and a -inf element, NaN elements, a row times 1e12 (bf16: factor clamped to 1e-8;
    fp16: the row overflows to inf) and rows times 1e-9, on the last kv head of five
    sequences.  The codes and factors stored equal the oracle's append of the same rows
    (the quantization ivakv_append_fp8 applies); every other (sequence, kv head) unit's
    output stays within 2e-3 of the oracle's decode.  Walks: "stream" (a few units: the
    stream walk and its fused merge), "many" (>= 1024 units: the four-element merge),
    "single" (40 sequences x 8 kv heads on short tables: one launch per step)."""
    lengths = [0, 1, 16, 17, 100, 257, 513]
    hq, hkv = 8, 2
    if walk != "stream":
        extra = 129 if walk == "many" else 33
        lengths = lengths + torch.randint(2, 60, (extra,), generator=torch.Generator().manual_seed(3)).tolist()
        hq, hkv = 32, 8
    c = fp8_case(iva, lengths, hkv, 128, torch.float32, seed=71, decades=0)
    offs = np.cumsum([0] + lengths[:-1]).tolist()
    prev = torch.cat([torch.arange(o, o + n - 1) for o, n in zip(offs, lengths) if n > 1])
    g, o = append_both(iva, dev, dict(c, k_new=c["k_new"][prev], v_new=c["v_new"][prev],
                                      slots=c["slots"][prev]))
    lay = c["layout"]
    bt, ctx = lay.block_tables, lay.context_lens
    kn = torch.zeros(len(lengths), hkv, 128)
    vn = torch.zeros(len(lengths), hkv, 128)
    step_slots = torch.full((len(lengths),), -1, dtype=torch.int32)
    for b, (off, n) in enumerate(zip(offs, lengths)):
        if n:
            kn[b], vn[b] = c["k_new"][off + n - 1], c["v_new"][off + n - 1]
            step_slots[b] = int(bt[b, (n - 1) // 16]) * 16 + (n - 1) % 16
    hx = hkv - 1
    kn[2, hx, 5] = math.inf
    vn[3, hx, 9] = -math.inf
    kn[5, hx, 7] = math.nan
    vn[5, hx, 0] = math.nan
    kn[6, hx] *= 1e12
    vn[6, hx, 3] = math.nan
    kn[1, hx] *= 1e-9
    vn[4, hx] *= 1e-9
    kn, vn = kn.to(qdt), vn.to(qdt)
    q = (torch.randn(len(lengths), hq, 128, generator=torch.Generator().manual_seed(8)) * 128 ** -0.5).to(qdt)
    out = iva.paged_decode_append_attention(q.to(dev), kn.to(dev), vn.to(dev), g["k_pool"],
                                            g["v_pool"], bt.to(dev), ctx.to(dev),
                                            k_scale=g["k_scale"], v_scale=g["v_scale"])
    orc.append_fp8(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"], kn.float().numpy(),
                   vn.float().numpy(), step_slots.numpy())
    assert np.array_equal(u8(g["k_pool"]), o["k_pool"]) and np.array_equal(u8(g["v_pool"]), o["v_pool"])
    assert np.array_equal(g["k_scale"].cpu().numpy(), o["k_scale"])
    assert np.array_equal(g["v_scale"].cpu().numpy(), o["v_scale"])
    with np.errstate(invalid="ignore", over="ignore"):
        ref = orc.decode_attention_fp8(q.float().numpy(), o["k_pool"], o["v_pool"], o["k_scale"],
                                       o["v_scale"], bt.numpy(), ctx.numpy())
    got = out.float().cpu().numpy()
    G = hq // hkv
    checked = np.ones(got.shape[:2], dtype=bool)
    checked[[2, 3, 5, 6], hx * G:(hx + 1) * G] = False   # units whose new rows are not finite
    err = np.abs(got - ref)[checked]
    bound = 2e-3 + OUT_ULP[qdt] * np.abs(ref[checked])
    assert (err <= bound).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("window,sink", [(0, 0), (50, 4)])
def test_prefill_fp8_vs_oracle(iva, dev, qdt, d, window, sink):
    """Chunked prefill over FP8 pages (garbage codes, NaN included, past every context;
    an invalid page id inside one) vs the fp64 oracle's prefill over the dequantized
    pages.  Keys and values are rounded once to the query dtype on their way into LDS,
    so bf16 carries one more 2^-9 relative rounding of K and V than the decode walk."""
    lengths, chunks = [1, 17, 300, 45, 130], [1, 17, 37, 0, 64]
    hq, hkv = 8, 2
    c = fp8_case(iva, lengths, hkv, d, torch.float32, seed=41 + d, decades=0)
    g, o = append_both(iva, dev, c)
    lay = c["layout"]
    bt = lay.block_tables.clone()
    bt[2, 5] = -1                               # an invalid page inside a context
    qs = torch.tensor(np.cumsum([0] + chunks), dtype=torch.int32)
    q = (torch.randn(int(qs[-1]), hq, d, generator=torch.Generator().manual_seed(9)) * d ** -0.5).to(qdt)
    out = iva.paged_prefill_attention(q.to(dev), g["k_pool"], g["v_pool"], bt.to(dev),
                                      lay.context_lens.to(dev), qs.to(dev), window=window,
                                      n_sink=sink, k_scale=g["k_scale"], v_scale=g["v_scale"])
    kd, vd = orc.dequantize_pools(o["k_pool"], o["v_pool"], o["k_scale"], o["v_scale"], np.float64)
    ref = orc.prefill_attention(q.double().numpy(), kd, vd, bt.numpy(), lay.context_lens.numpy(),
                                qs.numpy(), window=window, n_sink=sink)
    err = np.abs(out.float().cpu().numpy() - ref)
    bound = 2e-3 + OUT_ULP[qdt] * np.abs(ref)
    assert (err <= bound).all(), f"max err {err.max():.3e}"


def test_fp8_argument_errors(iva, dev):
    c = fp8_case(iva, [20], 2, 64, torch.float16, seed=1)
    g, _ = append_both(iva, dev, c)
    lay = c["layout"]
    q = torch.randn(1, 4, 64, device=dev).half()
    args = (q, g["k_pool"], g["v_pool"], lay.block_tables.to(dev), lay.context_lens.to(dev))
    with pytest.raises(ValueError, match="k_scale"):
        iva.paged_decode_attention(*args)
    with pytest.raises(TypeError, match="float16 or bfloat16"):
        iva.paged_decode_attention(q.float(), *args[1:], k_scale=g["k_scale"], v_scale=g["v_scale"])
    with pytest.raises(ValueError, match="stream walk"):
        iva.paged_decode_attention(*args, partition_pages=8, k_scale=g["k_scale"], v_scale=g["v_scale"])
    with pytest.raises(ValueError, match="k_scale"):
        iva.kv_append(c["k_new"].to(dev), c["v_new"].to(dev), g["k_pool"], g["v_pool"],
                      c["slots"].to(dev))
    rows = torch.zeros(1, 2, 64, device=dev).half()
    with pytest.raises(ValueError, match="k_scale"):
        iva.paged_decode_append_attention(q, rows, rows, *args[1:])
    with pytest.raises(TypeError, match="float16 or bfloat16"):
        iva.paged_decode_append_attention(q, rows.float(), rows, *args[1:], k_scale=g["k_scale"],
                                          v_scale=g["v_scale"])


def test_append_encodes_every_tie_and_boundary(iva, dev):
    """The device encoder on chosen values: a row whose first element is 448 has scaling
    factor 1, so its other elements are encoded as given.  Every e4m3 code's value, the
    midpoints between neighbouring codes (round-to-nearest-even ties) and the floats one
    ulp either side of them, both signs, subnormal range and the saturation edge up to
    448, plus random floats over the whole range: codes identical to the oracle's (which
    equals torch's float8_e4m3fn cast, tests/test_oracle.py)."""
    vals = orc.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # 0 .. 448
    mids = (vals[:-1] + vals[1:]) / 2
    pts = np.concatenate([vals, mids]).astype(np.float32)
    ulp = np.concatenate([np.nextafter(pts, np.float32(0)), np.nextafter(pts, np.float32(1e9))])
    pts = np.concatenate([pts, ulp.astype(np.float32)])
    pts = pts[(pts >= 0) & (pts <= 448)]
    rng = np.random.default_rng(17)
    rnd = (2.0 ** rng.uniform(-14, np.log2(448), 20000)).astype(np.float32)
    x = np.concatenate([pts, -pts, rnd, -rnd, np.zeros(3, np.float32)])
    d, hkv = 128, 1
    per = d - 1
    n = -(-x.size // per)
    rows = np.zeros((n, hkv, d), np.float32)
    rows[:, :, 0] = 448.0
    flat = np.zeros(n * per, np.float32)
    flat[:x.size] = x
    rows[:, 0, 1:] = flat.reshape(n, per)
    pages = -(-n // 16)
    ks, vs = iva.pool_shapes(pages, hkv, d, 16, FP8)
    kp = torch.zeros(ks, dtype=torch.uint8, device=dev).view(FP8)
    vp = torch.zeros(vs, dtype=torch.uint8, device=dev).view(FP8)
    ksc = torch.zeros(iva.scale_shape(pages, hkv), device=dev)
    vsc = torch.zeros(iva.scale_shape(pages, hkv), device=dev)
    src = torch.from_numpy(rows).to(dev)
    iva.kv_append(src, src, kp, vp, torch.arange(n, dtype=torch.int32, device=dev),
                  k_scale=ksc, v_scale=vsc)
    assert bool((ksc.flatten()[:n] == 1).all()) and bool((vsc.flatten()[:n] == 1).all())
    ok_k, ok_v, os_k, os_v = (orc.empty_pools(pages, hkv, d, 16, np.uint8, fill=0) +
                              (orc.empty_scales(pages, hkv, 16), orc.empty_scales(pages, hkv, 16)))
    orc.append_fp8(ok_k, ok_v, os_k, os_v, rows, rows, np.arange(n))
    assert np.array_equal(u8(kp), ok_k) and np.array_equal(u8(vp), ok_v)


def test_append_rows_beyond_the_scaled_range(iva, dev):
    """Rows whose scaled values would leave +-448 take the integer encoder: an inf element
    (factor 448 / inf clamped to 1e-8), a NaN element, and a max |x| of 1e12 (factor
    clamped to 1e-8, so values up to 1e4 saturate at 448).  Codes and factors equal the
    oracle's, rows of ordinary scale beside them included."""
    d, hkv, n = 64, 2, 6
    rng = np.random.default_rng(3)
    rows = rng.standard_normal((n, hkv, d)).astype(np.float32)
    rows[0, 0, 5] = np.inf
    rows[1, 1, 7] = -np.inf
    rows[2, 0, 9] = np.nan
    rows[3, 1, :] *= 1e12
    rows[4, 0, :] *= 1e-9
    ks, vs = iva.pool_shapes(1, hkv, d, 16, FP8)
    kp = torch.zeros(ks, dtype=torch.uint8, device=dev).view(FP8)
    vp = torch.zeros(vs, dtype=torch.uint8, device=dev).view(FP8)
    ksc = torch.zeros(iva.scale_shape(1, hkv), device=dev)
    vsc = torch.zeros(iva.scale_shape(1, hkv), device=dev)
    src = torch.from_numpy(rows).to(dev)
    iva.kv_append(src, src, kp, vp, torch.arange(n, dtype=torch.int32, device=dev),
                  k_scale=ksc, v_scale=vsc)
    ok_k, ok_v = orc.empty_pools(1, hkv, d, 16, np.uint8, fill=0)
    os_k, os_v = orc.empty_scales(1, hkv, 16), orc.empty_scales(1, hkv, 16)
    os_k[:], os_v[:] = 0, 0
    orc.append_fp8(ok_k, ok_v, os_k, os_v, rows, rows, np.arange(n))
    assert np.array_equal(u8(kp), ok_k) and np.array_equal(u8(vp), ok_v)
    assert np.array_equal(ksc.cpu().numpy(), os_k) and np.array_equal(vsc.cpu().numpy(), os_v)

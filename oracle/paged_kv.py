"""numpy oracle of the paged KV hot path.  TEST INFRASTRUCTURE ONLY.

Restates, on the paged layout, the semantics of the reference's
  - KVCache.update slice-assign            src/core/rope_kv.py:98-110
  - AttentionTorch cache append (torch.cat) src/core/attention.py:61-63
  - KVCache.get_slice                      src/core/rope_kv.py:136-137
  - AttentionTorch math                    src/core/attention.py:77-102
  - masks (causal / window / sink)         src/core/attention.py:79-93,115-148
  - kv_gather / kv_scatter kernels         src/kernels_t/kv_ops_triton.py:18-65,129
  - FP8 pages (e4m3fn, per-row scaling)   configs/quant_infer.yaml:22,52, src/quant/fp8_runtime.py:34,66-76
  - RoPE                                  src/core/rope_kv.py:22-50

Layout (X = 16 // itemsize, BS = block size):
  k_pool [P, Hkv, D/X, BS, X]: K(page, h, t, d) at ((d // X) * BS + t) * X + d % X
  v_pool [P, Hkv, D, BS]:      V(page, h, t, d) at d * BS + t
Slot s -> page s // BS, row s % BS.

Decisions the reference leaves open (fixed here and in the kernels):
  * GQA: query head h reads KV head h // (Hq // Hkv) (repeat_interleave order).
  * Decode positions are absolute: with context length L (the new token already
    appended) the query sits at L - 1 and sees keys 0..L-1 (append-before-score
    order of attention.py:61-77).
  * Window W keeps keys j >= L - W, i.e. [i - W + 1, i] for query i = L - 1
    (attention.py:124-127 at absolute positions).
  * Sinks are the union [0, n_sink) | window, not the reference's AND of masks.
  * An empty context (L == 0) yields a zero output row.
  * Gather keeps the cache dtype.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np


def chunk_elems(itemsize: int) -> int:
    return 16 // itemsize


def empty_pools(num_pages: int, hkv: int, head_dim: int, block_size: int, dtype,
                fill=0) -> Tuple[np.ndarray, np.ndarray]:
    """Pools of one layer filled with ``fill`` (a canary value for untouched slots)."""
    dt = np.dtype(dtype)
    x = chunk_elems(dt.itemsize)
    assert head_dim % x == 0
    k = np.full((num_pages, hkv, head_dim // x, block_size, x), fill, dtype=dt)
    v = np.full((num_pages, hkv, head_dim, block_size), fill, dtype=dt)
    return k, v


def append(k_pool: np.ndarray, v_pool: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
           slot_mapping: np.ndarray) -> None:
    """In place: row ``t`` of ``k_new/v_new`` ([n_tok, Hkv, D]) lands in slot ``slot_mapping[t]``;
    slots outside ``[0, P*BS)`` (e.g. -1) are skipped.  ``KVCache.update`` writes new rows at
    their sequence positions (rope_kv.py:109-110); on the paged cache the position is the slot."""
    num_pages, hkv, nch, bs, x = k_pool.shape
    slots = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    valid = (slots >= 0) & (slots < num_pages * bs)
    ts = np.nonzero(valid)[0]
    if ts.size == 0:
        return
    s = slots[ts]
    page, off = s // bs, s % bs
    k_pool[page, :, :, off, :] = k_new[ts].reshape(ts.size, hkv, nch, x)
    v_pool[page, :, :, off] = v_new[ts]


def gather(k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray, ctx_lens: np.ndarray,
           out_len: Optional[int] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Contiguous ``[B, Hkv, out_len, D]`` K and V of each sequence (``KVCache.get_slice``,
    rope_kv.py:136-137); rows at or past ``ctx_lens[b]`` and rows on invalid pages are zero."""
    num_pages, hkv, nch, bs, x = k_pool.shape
    d = nch * x
    bt = np.asarray(block_tables, dtype=np.int64)
    ctx = np.asarray(ctx_lens, dtype=np.int64).reshape(-1)
    batch, max_blocks = bt.shape
    if out_len is None:
        out_len = max_blocks * bs
    k_out = np.zeros((batch, hkv, out_len, d), dtype=k_pool.dtype)
    v_out = np.zeros((batch, hkv, out_len, d), dtype=v_pool.dtype)
    for b in range(batch):
        lim = min(max(int(ctx[b]), 0), out_len)
        for j in range(min(-(-lim // bs), max_blocks)):
            p = int(bt[b, j])
            if p < 0 or p >= num_pages:
                continue
            n = min(bs, lim - j * bs)
            k_out[b, :, j * bs:j * bs + n, :] = (
                k_pool[p, :, :, :n, :].transpose(0, 2, 1, 3).reshape(hkv, n, d))
            v_out[b, :, j * bs:j * bs + n, :] = v_pool[p, :, :, :n].transpose(0, 2, 1)
    return k_out, v_out


def append_loops(k_flat: np.ndarray, v_flat: np.ndarray, k_new, v_new, slot_mapping,
                 num_pages: int, hkv: int, head_dim: int, bs: int) -> None:
    """Brute-force append on FLAT pools using the address formula of include/ivakv.h."""
    x = chunk_elems(k_flat.dtype.itemsize)
    tile = head_dim * bs
    for t, s in enumerate(list(np.asarray(slot_mapping).reshape(-1))):
        s = int(s)
        if s < 0 or s >= num_pages * bs:
            continue
        page, row = divmod(s, bs)
        for h in range(hkv):
            base = (page * hkv + h) * tile
            for dd in range(head_dim):
                k_flat[base + ((dd // x) * bs + row) * x + dd % x] = k_new[t][h][dd]
                v_flat[base + dd * bs + row] = v_new[t][h][dd]


def gather_loops(k_flat: np.ndarray, v_flat: np.ndarray, block_tables, ctx_lens, num_pages: int,
                 hkv: int, head_dim: int, bs: int, out_len: int):
    """Brute-force gather from FLAT pools using the address formula of include/ivakv.h."""
    x = chunk_elems(k_flat.dtype.itemsize)
    tile = head_dim * bs
    batch = len(ctx_lens)
    k_out = np.zeros((batch, hkv, out_len, head_dim), dtype=k_flat.dtype)
    v_out = np.zeros((batch, hkv, out_len, head_dim), dtype=v_flat.dtype)
    for b in range(batch):
        for pos in range(min(int(ctx_lens[b]), out_len)):
            j, row = divmod(pos, bs)
            if j >= len(block_tables[b]):
                continue
            page = int(block_tables[b][j])
            if page < 0 or page >= num_pages:
                continue
            for h in range(hkv):
                base = (page * hkv + h) * tile
                for dd in range(head_dim):
                    k_out[b, h, pos, dd] = k_flat[base + ((dd // x) * bs + row) * x + dd % x]
                    v_out[b, h, pos, dd] = v_flat[base + dd * bs + row]
    return k_out, v_out


def visible(length: int, window: int = 0, n_sink: int = 0) -> np.ndarray:
    """Keys a decode query at position ``length - 1`` attends to: causal, within the
    sliding window (attention.py:124-127 at absolute positions) or an attention sink."""
    j = np.arange(max(length, 0))
    if window and window > 0:
        return (j >= length - window) | (j < n_sink)
    return np.ones_like(j, dtype=bool)


def expand_gqa(x: np.ndarray, group: int) -> np.ndarray:
    """[Hkv, ...] -> [Hkv * group, ...] with query head h reading KV head h // group
    (torch ``repeat_interleave`` order)."""
    return np.repeat(x, group, axis=0)


def decode_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                     block_tables: np.ndarray, ctx_lens: np.ndarray, scale: Optional[float] = None,
                     window: int = 0, n_sink: int = 0) -> np.ndarray:
    """fp64 single-query attention of ``q`` ([B, Hq, D]) over each sequence's paged K/V:
    ``softmax(q k^T * scale) v`` over the visible keys (attention.py:77-102)."""
    q = np.asarray(q, dtype=np.float64)
    batch, hq, d = q.shape
    hkv = k_pool.shape[1]
    g = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    ctx = np.asarray(ctx_lens, dtype=np.int64).reshape(-1)
    bt = np.asarray(block_tables, dtype=np.int64)
    num_pages, bs = k_pool.shape[0], k_pool.shape[3]
    max_len = int(max(ctx.max(initial=0), 0))
    k_all, v_all = gather(k_pool, v_pool, bt, ctx, out_len=max_len)
    out = np.zeros((batch, hq, d), dtype=np.float64)
    for b in range(batch):
        length = int(ctx[b])
        if length <= 0:
            continue
        # keys on a page id outside the pool (or past the table) are not attended
        page_idx = np.arange(length) // bs
        pid = np.full(length, -1, dtype=np.int64)
        in_table = page_idx < bt.shape[1]
        pid[in_table] = bt[b, page_idx[in_table]]
        vis = visible(length, window, n_sink) & (pid >= 0) & (pid < num_pages)
        if not vis.any():
            continue
        k = expand_gqa(k_all[b, :, :length][:, vis].astype(np.float64), g)
        v = expand_gqa(v_all[b, :, :length][:, vis].astype(np.float64), g)
        scores = np.einsum("hd,had->ha", q[b], k) * scale
        scores -= scores.max(axis=1, keepdims=True)
        p = np.exp(scores)
        p /= p.sum(axis=1, keepdims=True)
        out[b] = np.einsum("ha,had->hd", p, v)
    return out


def decode_attention_loops(q, k_rows, v_rows, ctx_lens, scale: float, window: int = 0,
                           n_sink: int = 0):
    """Pure-Python single-query attention on contiguous rows ``k_rows[b][h][j][d]`` (tiny
    inputs only): the textbook formula evaluated term by term."""
    batch, hq, d = len(q), len(q[0]), len(q[0][0])
    hkv = len(k_rows[0])
    g = hq // hkv
    out = [[[0.0] * d for _ in range(hq)] for _ in range(batch)]
    for b in range(batch):
        length = int(ctx_lens[b])
        keys = [j for j in range(length)
                if not window or window <= 0 or j >= length - window or j < n_sink]
        if not keys:
            continue
        for h in range(hq):
            kh = h // g
            s = [sum(float(q[b][h][i]) * float(k_rows[b][kh][j][i]) for i in range(d)) * scale
                 for j in keys]
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            for i in range(d):
                out[b][h][i] = sum(e[n] * float(v_rows[b][kh][j][i]) for n, j in enumerate(keys)) / z
    return out


def visible_at(pos: int, length: int, window: int = 0, n_sink: int = 0) -> np.ndarray:
    """Keys 0..length-1 a query at absolute position ``pos`` attends to: causal
    (``j <= pos``, attention.py:79-81 at absolute positions), within the sliding window
    ``j > pos - window`` (attention.py:124-127) or an attention sink ``j < n_sink``
    (attention.py:131-148, as a union).  For ``pos = length - 1`` this is
    :func:`visible`."""
    j = np.arange(max(length, 0))
    vis = j <= pos
    if window and window > 0:
        vis &= (j > pos - window) | (j < n_sink)
    return vis


def prefill_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                      block_tables: np.ndarray, ctx_lens: np.ndarray, query_start: np.ndarray,
                      scale: Optional[float] = None, window: int = 0,
                      n_sink: int = 0) -> np.ndarray:
    """fp64 causal multi-query attention over paged K/V (prefill / chunked prefill).

    ``q`` is ``[n_tok, Hq, D]``; sequence b owns rows ``query_start[b] ..
    query_start[b+1]-1``, which sit at absolute positions ``L - n_b .. L - 1``
    (``L = ctx_lens[b]``, the chunk already appended: attention.py:61-63 then
    :77-102).  Each row is ``softmax(q k^T * scale) v`` over :func:`visible_at` keys
    on valid page ids; rows at negative positions or with no visible key are zero."""
    q = np.asarray(q, dtype=np.float64)
    n_tok, hq, d = q.shape
    hkv = k_pool.shape[1]
    g = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    ctx = np.asarray(ctx_lens, dtype=np.int64).reshape(-1)
    qs = np.asarray(query_start, dtype=np.int64).reshape(-1)
    bt = np.asarray(block_tables, dtype=np.int64)
    num_pages, bs = k_pool.shape[0], k_pool.shape[3]
    max_len = int(max(ctx.max(initial=0), 0))
    k_all, v_all = gather(k_pool, v_pool, bt, ctx, out_len=max_len)
    out = np.zeros((n_tok, hq, d), dtype=np.float64)
    for b in range(len(ctx)):
        length, s0, s1 = int(ctx[b]), int(qs[b]), int(qs[b + 1])
        n = s1 - s0
        if length <= 0 or n <= 0:
            continue
        page_idx = np.arange(length) // bs
        pid = np.full(length, -1, dtype=np.int64)
        in_table = page_idx < bt.shape[1]
        pid[in_table] = bt[b, page_idx[in_table]]
        valid = (pid >= 0) & (pid < num_pages)
        k = expand_gqa(k_all[b, :, :length].astype(np.float64), g)  # [Hq, L, D]
        v = expand_gqa(v_all[b, :, :length].astype(np.float64), g)
        for i in range(n):
            pos = length - n + i
            if pos < 0:
                continue
            vis = visible_at(pos, length, window, n_sink) & valid
            if not vis.any():
                continue
            scores = np.einsum("hd,had->ha", q[s0 + i], k[:, vis]) * scale
            scores -= scores.max(axis=1, keepdims=True)
            p = np.exp(scores)
            p /= p.sum(axis=1, keepdims=True)
            out[s0 + i] = np.einsum("ha,had->hd", p, v[:, vis])
    return out


# ---------------------------------------------------------------------------- FP8 pools
#
# kv_cache_dtype "fp8" (configs/quant_infer.yaml:22,52) as OCP e4m3fn codes, the format
# of torch.float8_e4m3fn that the reference's FP8 runtime uses
# (src/quant/fp8_runtime.py:34), with the reference's scaling rule sf = 448 / amax,
# 1 for amax == 0, clamped to [1e-8, 1e8] (fp8_runtime.py:66-76), applied per
# (token, kv head) row: codes = e4m3(x * sf), read back as code / sf.

FP8_MAX = np.float32(448.0)


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3fn codes: round to nearest even, saturating at +-448; NaN -> 0x7F."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = (u >> 24) & 0x80
    au = u & 0x7FFFFFFF
    a = au.astype(np.uint32).view(np.float32)
    sub = a < np.float32(2.0 ** -6)
    code_sub = np.rint(np.where(sub, a, 0) * np.float32(512.0)).astype(np.int64)  # step 2^-9
    r = (au + 0x7FFFF + ((au >> 20) & 1)) >> 20  # 3 mantissa bits, RNE, exponent carried
    code_n = np.where(r >= 960 + 0x7F, 0x7E, r - 960)  # rebias 127 -> 7
    code = np.minimum(np.where(sub, code_sub, code_n), 0x7E)
    code = np.where(au > 0x7F800000, 0x7F, code)
    return (code | sign).astype(np.uint8)


def e4m3_decode(codes) -> np.ndarray:
    """e4m3fn codes -> float32, exactly (0x7F / 0xFF are NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    e, m = (c >> 3) & 0xF, c & 7
    normal = ((e + 120) << 23) | (m << 20)
    v = np.where(e == 0, m.astype(np.float32) * np.float32(2.0 ** -9),
                 normal.astype(np.uint32).view(np.float32))
    v = np.where((e == 15) & (m == 7), np.float32(np.nan), v).astype(np.float32)
    return np.where(c & 0x80, -v, v).astype(np.float32)


def row_scale(amax) -> np.ndarray:
    """Scaling factor of rows with max |x| = amax (float32), fp8_runtime.py:67-76:
    1 for amax == 0, else 448 / amax clamped as ``max(1e-8, min(sf, 1e8))`` evaluates in
    Python, where a NaN sf compares false both times and comes out as 1e-8."""
    amax = np.asarray(amax, dtype=np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sf = FP8_MAX / np.where(amax == 0, np.float32(1), amax)
    sf = np.where(amax == 0, np.float32(1), sf)
    sf = np.where(np.isnan(sf), np.float32(1e-8), np.clip(sf, np.float32(1e-8), np.float32(1e8)))
    return sf.astype(np.float32)


def quantize_rows(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Rows over the last axis: (codes, sf) with codes = e4m3(x * sf) in float32."""
    x = np.asarray(x, dtype=np.float32)
    sf = row_scale(np.abs(x).max(axis=-1))
    return e4m3_encode(x * sf[..., None]), sf


def fp8_v_to_tiles(v_nat: np.ndarray) -> np.ndarray:
    """FP8 V tiles from natural [..., D, 16] (dim, key) order to the pool's byte order
    [d % 16][key / 4][d / 16][key % 4] (same shape): ivakv_internal.h fp8_v_offset, chosen
    so each lane of the decode walk reads whole 16-byte words.  An order of this build,
    not of the reference (whose KV cache is contiguous)."""
    *lead, d, bs = v_nat.shape
    n = len(lead)
    t = v_nat.reshape(*lead, d // 16, 16, bs // 4, 4)          # (d/16, d%16, key/4, key%4)
    t = t.transpose(*range(n), n + 1, n + 2, n, n + 3)        # (d%16, key/4, d/16, key%4)
    return np.ascontiguousarray(t).reshape(*lead, d, bs)


def fp8_v_from_tiles(v_dev: np.ndarray) -> np.ndarray:
    """Inverse of :func:`fp8_v_to_tiles`."""
    *lead, d, bs = v_dev.shape
    n = len(lead)
    t = v_dev.reshape(*lead, 16, bs // 4, d // 16, 4)          # (d%16, key/4, d/16, key%4)
    t = t.transpose(*range(n), n + 2, n, n + 1, n + 3)        # (d/16, d%16, key/4, key%4)
    return np.ascontiguousarray(t).reshape(*lead, d, bs)


def empty_scales(num_pages: int, hkv: int, block_size: int) -> np.ndarray:
    return np.ones((num_pages, hkv, block_size), dtype=np.float32)


def append_fp8(k_pool: np.ndarray, v_pool: np.ndarray, k_scale: np.ndarray, v_scale: np.ndarray,
               k_new: np.ndarray, v_new: np.ndarray, slot_mapping: np.ndarray) -> None:
    """In place: each (token, kv head) row of ``k_new/v_new`` quantized with its own scaling
    factor; K codes go where :func:`append` puts a row, V codes there in the FP8 tile order
    (:func:`fp8_v_to_tiles`), factors to ``[page, head, row]``."""
    kc, ksf = quantize_rows(k_new)
    vc, vsf = quantize_rows(v_new)
    v_nat = fp8_v_from_tiles(v_pool)
    append(k_pool, v_nat, kc, vc, slot_mapping)
    v_pool[...] = fp8_v_to_tiles(v_nat)
    num_pages, hkv, _, bs, _ = k_pool.shape
    slots = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    ok = (slots >= 0) & (slots < num_pages * bs)
    ts = np.nonzero(ok)[0]
    page, off = slots[ts] // bs, slots[ts] % bs
    k_scale[page, :, off] = ksf[ts]
    v_scale[page, :, off] = vsf[ts]


def dequantize_pools(k_pool: np.ndarray, v_pool: np.ndarray, k_scale: np.ndarray,
                     v_scale: np.ndarray, dtype=np.float32) -> Tuple[np.ndarray, np.ndarray]:
    """FP8 pools as pools of ``dtype`` in the 16-bit layout (V back in natural order):
    code / sf (float32 division)."""
    k = e4m3_decode(k_pool) / k_scale[:, :, None, :, None]
    v = e4m3_decode(fp8_v_from_tiles(v_pool)) / v_scale[:, :, None, :]
    return k.astype(dtype), v.astype(dtype)


def gather_fp8(k_pool, v_pool, k_scale, v_scale, block_tables, ctx_lens,
               out_len: Optional[int] = None) -> Tuple[np.ndarray, np.ndarray]:
    """:func:`gather` of the dequantized FP8 pools (float32)."""
    kd, vd = dequantize_pools(k_pool, v_pool, k_scale, v_scale)
    return gather(kd, vd, block_tables, ctx_lens, out_len)


def decode_attention_fp8(q, k_pool, v_pool, k_scale, v_scale, block_tables, ctx_lens,
                         scale: Optional[float] = None, window: int = 0,
                         n_sink: int = 0) -> np.ndarray:
    """:func:`decode_attention` over the dequantized FP8 pools."""
    kd, vd = dequantize_pools(k_pool, v_pool, k_scale, v_scale, np.float64)
    return decode_attention(q, kd, vd, block_tables, ctx_lens, scale, window, n_sink)


# ---------------------------------------------------------------------------- RoPE

def rope_freqs(head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """f_i = 1 / theta^(2i / D) per dim pair, computed in double and stored as float32 as
    RoPE._compute_freqs fills its float32 buffer (src/core/rope_kv.py:22-30)."""
    return np.array([1.0 / (theta ** (i / head_dim)) for i in range(0, head_dim, 2)],
                    dtype=np.float32)


def rope(x: np.ndarray, positions: np.ndarray, theta: float = 10000.0) -> np.ndarray:
    """Rows ``x[t, ..., D]`` rotated at ``positions[t]`` (rope_kv.py:32-50): pair (2i, 2i+1)
    by a = float32(p) * f_i (a float32 product, as the reference's float32 tensors
    compute it), y0 = x0 cos a - x1 sin a, y1 = x0 sin a + x1 cos a, in fp64."""
    x = np.asarray(x, dtype=np.float64)
    pos = np.asarray(positions, dtype=np.int64).reshape(-1)
    f = rope_freqs(x.shape[-1], theta)
    ang = (pos.astype(np.float32)[:, None] * f[None, :]).astype(np.float64)  # [n, D/2]
    shape = (len(pos),) + (1,) * (x.ndim - 2) + (f.size,)
    c, s = np.cos(ang).reshape(shape), np.sin(ang).reshape(shape)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    y = np.empty_like(x)
    y[..., 0::2] = x0 * c - x1 * s
    y[..., 1::2] = x0 * s + x1 * c
    return y


def index_gather(kv: np.ndarray, indices: np.ndarray) -> np.ndarray:
    """``out[b, h, j] = kv[b, h, indices[j]]`` (kv_gather_kernel, kv_ops_triton.py:33-40)."""
    return kv[:, :, np.asarray(indices, dtype=np.int64), :].copy()


def index_scatter(kv: np.ndarray, indices: np.ndarray, values: np.ndarray) -> np.ndarray:
    """Functional scatter: a copy of ``kv`` with ``[:, :, indices[j]] = values[:, :, j]``
    (kv_ops_triton.py:58-65 on the clone made at :129)."""
    out = kv.copy()
    out[:, :, np.asarray(indices, dtype=np.int64), :] = values
    return out

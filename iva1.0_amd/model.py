"""Model-level drop-in of IVA1.0's KV path: ``get_attention`` / ``attn_impl`` dispatch,
the paged attention module, and the ``Transformer`` / ``TransformerBlock`` /
``TransformerConfig`` surface that threads a KV cache through the blocks.

Mirrors src/core of the reference at its interfaces (signatures, argument
meaning, return contracts, errors) for the path ``Transformer.forward(kv_cache=...)``:

  TransformerConfig   src/core/transformer.py:25-78; ``attn_impl`` also admits
                      "hip_paged" (whitelist at :71-72), plus ``n_kv_heads``
                      (grouped-query attention; default = n_heads) and the paged
                      cache geometry (``kv_block_size``, ``kv_num_pages``).
  get_attention       src/core/attention.py:190-194; "hip_paged" -> PagedAttention.
  AttentionTorch      src/core/attention.py:17-148 on a contiguous KVCache (torch.cat
                      append), the reference's default backend.
  PagedAttention      same constructor/forward contract (:37-45,110) on a PagedKVCache:
                      single-token decode appends and attends in one op
                      (ivakv_decode_append_attn); multi-token (prefill) steps append
                      with ivakv_append and run ivakv_prefill_attn.  Builds from the
                      reference's own TransformerConfig (fields it lacks take their
                      defaults) and takes over the reference's contiguous KVCache.
  KVCache             src/core/rope_kv.py:71-137 (contiguous cache of AttentionTorch).
  RMSNorm / FFN       src/core/norms.py:14-36, src/core/ffn.py:16-64 (needed by the
                      dense decoder of config C3; not part of the paged hot path).
  Transformer         src/core/transformer.py:154-320: learned absolute positions
                      from ``kv_cache.seq_len`` (:200-203), the block loop (:229-238),
                      the return dict (:242-255); ``generate`` prefills once and then
                      decodes one token per step through the cache.

Deliberate differences from the reference (each is a defect there, see the tests):
  * masks use absolute positions: a decode query at position L-1 sees keys 0..L-1
    (the reference's tril(ones(S, k_len)) lets it see only key 0, attention.py:80);
    the sliding window is [L-W, L-1]; sink tokens are the UNION with the window;
  * each layer has its own cache pools (the reference threads one cache through
    every layer, transformer.py:229-238, so layer l attends to layers 0..l);
  * the tied LM head uses the token embedding (heads.py:31-41 draws a new random CPU
    weight on every call);
  * ``generate`` decodes incrementally instead of re-running the whole sequence
    every step (transformer.py:285-290).
RoPE stays a no-op inside attention, as in the reference (attention.py:112-113):
positions come from the learned position embedding.  MoE and HRM are out of scope
(``moe_enable`` / ``hrm_enable`` raise).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .ops import (FP8, kv_gather, paged_decode_append_attention,
                  paged_prefill_attention, rope_)
from .paged_cache import PagedKVCache


def _cfg(config: Any, name: str, default: Any) -> Any:
    """A field of the paged backend that the reference's TransformerConfig
    (src/core/transformer.py:25-78) does not have: read with its default, so every module
    here builds from the reference config unchanged (n_kv_heads = n_heads, no sinks, no
    RoPE inside attention, pages of 16 in the model dtype)."""
    value = getattr(config, name, None)
    return default if value is None else value


@dataclass
class TransformerConfig:
    """src/core/transformer.py:25-78 plus the fields of the paged backend."""

    d_model: int = 1024
    n_layers: int = 16
    n_heads: int = 16
    vocab_size: int = 32000
    seq_len: int = 4096

    rope_theta: float = 100000.0

    attn_impl: str = "torch"
    norm_impl: str = "torch"

    moe_enable: bool = False
    hrm_enable: bool = False

    tie_embeddings: bool = True
    sliding_window: Optional[int] = None

    dropout: float = 0.1
    use_flash_attn: bool = False
    causal: bool = True

    norm_eps: float = 1e-6
    elementwise_affine: bool = True

    hidden_mult: int = 4
    activation: str = "swiglu"

    # paged backend
    n_kv_heads: Optional[int] = None     # None = n_heads (the reference has no GQA)
    kv_block_size: int = 16
    kv_num_pages: Optional[int] = None   # None = enough for every sequence at seq_len
    sink_tokens: int = 0                 # attention-sink tokens kept visible with the window
    # The reference computes RoPE state but its attention never applies it
    # (attention.py:57-59,112-113); True rotates q and k as its RoPE module describes
    # (rope_kv.py:22-50), fused into the paged append on the hip_paged backend.
    rope_in_attention: bool = False
    kv_cache_dtype: Optional[str] = None  # None = model dtype; "fp8" = e4m3fn pages
                                          # (configs/quant_infer.yaml:52 memory.kv_cache_dtype)

    def __post_init__(self):
        if self.d_model % self.n_heads != 0:
            raise ValueError(f"d_model ({self.d_model}) must be divisible by n_heads ({self.n_heads})")
        if self.attn_impl not in ["torch", "triton", "hip_paged"]:
            raise ValueError(f"attn_impl must be 'torch', 'triton' or 'hip_paged', got {self.attn_impl}")
        if self.norm_impl not in ["torch", "triton"]:
            raise ValueError(f"norm_impl must be 'torch' or 'triton', got {self.norm_impl}")
        if self.activation not in ["swiglu", "gelu", "relu"]:
            raise ValueError(f"activation must be 'swiglu', 'gelu', or 'relu', got {self.activation}")
        if self.n_kv_heads is None:
            self.n_kv_heads = self.n_heads
        if self.n_heads % self.n_kv_heads != 0:
            raise ValueError(f"n_heads ({self.n_heads}) must be a multiple of n_kv_heads ({self.n_kv_heads})")
        if self.kv_cache_dtype not in (None, "fp8"):
            raise ValueError(f"kv_cache_dtype must be None or 'fp8', got {self.kv_cache_dtype!r}")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


class KVCache:
    """Contiguous cache of the torch backend (src/core/rope_kv.py:71-137)."""

    def __init__(self, batch_size: int, n_heads: int, head_dim: int, seq_len: int,
                 device: torch.device, dtype: torch.dtype = torch.float16):
        self.batch_size = batch_size
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.seq_len = seq_len
        self.device = device
        self.dtype = dtype
        self.k = torch.zeros(batch_size, n_heads, seq_len, head_dim, device=device, dtype=dtype)
        self.v = torch.zeros(batch_size, n_heads, seq_len, head_dim, device=device, dtype=dtype)

    def update(self, new_k: torch.Tensor, new_v: torch.Tensor, start_pos: int) -> None:
        end_pos = start_pos + new_k.size(2)
        if end_pos > self.seq_len:
            self.resize(end_pos)
        self.k[:, :, start_pos:end_pos] = new_k
        self.v[:, :, start_pos:end_pos] = new_v

    def resize(self, new_seq_len: int) -> None:
        if new_seq_len <= self.seq_len:
            return
        new_k = torch.zeros(self.batch_size, self.n_heads, new_seq_len, self.head_dim,
                            device=self.device, dtype=self.dtype)
        new_v = torch.zeros_like(new_k)
        new_k[:, :, :self.seq_len] = self.k
        new_v[:, :, :self.seq_len] = self.v
        self.k, self.v, self.seq_len = new_k, new_v, new_seq_len

    def clear(self) -> None:
        self.k.zero_()
        self.v.zero_()

    def get_slice(self, start: int, end: int) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.k[:, :, start:end], self.v[:, :, start:end]


class LayeredKVCache:
    """Per-layer contiguous caches behind one object, with the same layer cursor as
    PagedKVCache, so the torch backend also keeps separate K/V per layer."""

    def __init__(self, batch_size: int, n_heads: int, head_dim: int, num_layers: int,
                 device: torch.device, dtype: torch.dtype):
        self.batch_size, self.n_heads, self.head_dim = batch_size, n_heads, head_dim
        self.num_layers, self.device, self.dtype = num_layers, device, dtype
        self.layers = [KVCache(batch_size, n_heads, head_dim, 0, device, dtype)
                       for _ in range(num_layers)]
        self.seq_len = 0
        self._cursor = 0

    def next_layer(self) -> KVCache:
        c = self.layers[self._cursor]
        self._cursor += 1
        if self._cursor == self.num_layers:
            self._cursor = 0
        return c

    def commit(self, t: int) -> None:
        if self._cursor == 0:
            self.seq_len += t


def _visible(q_pos: torch.Tensor, k_pos: torch.Tensor, window: Optional[int], n_sink: int
             ) -> torch.Tensor:
    """[..., S, K] visibility at absolute positions: causal, within the window, or a sink."""
    qp = q_pos[..., :, None]
    kp = k_pos[..., None, :]
    ok = kp <= qp
    if window is not None and window > 0:
        ok = ok & ((kp > qp - window) | (kp < n_sink))
    return ok


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
            allowed: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T scale, masked) v in fp32 with GQA; q [B,Hq,S,D], k/v [B,Hkv,K,D],
    allowed [B or 1, 1, S, K].  Rows with no visible key give zeros."""
    g = q.shape[1] // k.shape[1]
    kf = k.float().repeat_interleave(g, dim=1)
    vf = v.float().repeat_interleave(g, dim=1)
    scores = torch.matmul(q.float(), kf.transpose(-2, -1).contiguous()) * scale
    scores = scores.masked_fill(~allowed, float("-inf"))
    w = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
    return torch.matmul(w, vf).to(q.dtype)


def _sink_count(sink_cfg: Optional[Dict[str, Any]], default: int) -> int:
    if sink_cfg is None:
        return default
    return int(sink_cfg.get("sink_tokens", 4))  # attention.py:138 default


def _rope_torch(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """The reference's RoPE.forward (src/core/rope_kv.py:22-50), vectorized: x [B, H, S, D]
    rotated pairwise at positions [S], in float32, returned in x's dtype."""
    d = x.shape[-1]
    f = torch.tensor([1.0 / (theta ** (i / d)) for i in range(0, d, 2)], dtype=torch.float32,
                     device=x.device)
    ang = positions.to(torch.float32)[:, None] * f[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    xf = x.float()
    x0, x1 = xf[..., 0::2], xf[..., 1::2]
    y = torch.empty_like(xf)
    y[..., 0::2] = x0 * c - x1 * s
    y[..., 1::2] = x0 * s + x1 * c
    return y.to(x.dtype)


class _AttentionBase(nn.Module):
    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.config = config
        self.d_model = config.d_model
        self.n_heads = config.n_heads
        self.n_kv_heads = int(_cfg(config, "n_kv_heads", config.n_heads))
        if self.n_heads % self.n_kv_heads:
            raise ValueError(f"n_heads ({self.n_heads}) must be a multiple of n_kv_heads "
                             f"({self.n_kv_heads})")
        self.head_dim = config.d_model // config.n_heads
        self.dropout = config.dropout
        self.causal = config.causal
        self.sink_tokens = int(_cfg(config, "sink_tokens", 0))
        kv_dim = self.n_kv_heads * self.head_dim
        self.q_proj = nn.Linear(self.d_model, self.d_model, bias=False)
        self.k_proj = nn.Linear(self.d_model, kv_dim, bias=False)
        self.v_proj = nn.Linear(self.d_model, kv_dim, bias=False)
        self.o_proj = nn.Linear(self.d_model, self.d_model, bias=False)
        self.dropout_layer = nn.Dropout(self.dropout)
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.rope = bool(_cfg(config, "rope_in_attention", False))
        self.rope_theta = float(config.rope_theta)

    def _project(self, x):
        b, s, _ = x.shape
        q = self.q_proj(x).view(b, s, self.n_heads, self.head_dim)
        k = self.k_proj(x).view(b, s, self.n_kv_heads, self.head_dim)
        v = self.v_proj(x).view(b, s, self.n_kv_heads, self.head_dim)
        return q, k, v

    def _apply_rope(self, x: torch.Tensor, rope_state: Optional[torch.Tensor]) -> torch.Tensor:
        return x  # attention.py:112-113: RoPE is a no-op inside attention

    @staticmethod
    def _key_mask(attention_mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        """The reference's padding mask (src/core/attention.py:95-97): ``attention_mask``
        [B, M] (0 = masked) is broadcast against the scores [B, H, S, K] as
        ``attention_mask.unsqueeze(1).unsqueeze(2)``, so it masks keys when M == K and
        every key of a row when M == 1 (a padded single-token step); other widths fail
        to broadcast, as in the reference.  Returns that [B, 1, 1, M] bool "key kept"
        tensor, or None when there is no mask or nothing is masked."""
        if attention_mask is None or bool(attention_mask.all()):
            return None
        return (attention_mask != 0).unsqueeze(1).unsqueeze(2)


class AttentionTorch(_AttentionBase):
    """The reference's default backend (src/core/attention.py:17-148) with grouped KV
    heads and absolute-position masks, on contiguous per-layer caches."""

    def forward(self, x: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                kv_cache: Optional[Any] = None, rope_state: Optional[torch.Tensor] = None,
                sliding_window: Optional[int] = None,
                sink_cfg: Optional[Dict[str, Any]] = None) -> Tuple[torch.Tensor, Optional[Any]]:
        b, s, _ = x.shape
        q, k, v = self._project(x)
        q = self._apply_rope(q.transpose(1, 2), rope_state)
        k = self._apply_rope(k.transpose(1, 2), rope_state)
        v = v.transpose(1, 2)
        start = kv_cache.seq_len if kv_cache is not None else 0
        if self.rope:
            pos = torch.arange(start, start + s, device=x.device)
            q = _rope_torch(q, pos, self.rope_theta)
            k = _rope_torch(k, pos, self.rope_theta)
        if isinstance(kv_cache, LayeredKVCache):
            layer = kv_cache.next_layer()
            k = torch.cat([layer.k, k], dim=2)  # attention.py:62-63
            v = torch.cat([layer.v, v], dim=2)
            layer.k, layer.v, layer.seq_len = k, v, start + s
            kv_cache.commit(s)
        elif kv_cache is not None:
            k = torch.cat([kv_cache.k, k], dim=2)
            v = torch.cat([kv_cache.v, v], dim=2)
            new = type(kv_cache)(batch_size=kv_cache.batch_size, n_heads=kv_cache.n_heads,
                                 head_dim=kv_cache.head_dim, seq_len=start + s, device=x.device,
                                 dtype=k.dtype)
            new.k, new.v = k, v
            kv_cache = new
        key_ok = self._key_mask(attention_mask)
        q_pos = torch.arange(start, start + s, device=x.device)
        k_pos = torch.arange(k.shape[2], device=x.device)
        if self.causal:
            allowed = _visible(q_pos, k_pos, sliding_window, _sink_count(sink_cfg, self.sink_tokens))
        else:
            allowed = torch.ones(s, k.shape[2], dtype=torch.bool, device=x.device)
        allowed = allowed[None, None] if key_ok is None else allowed[None, None] & key_ok
        out = _attend(q, k, v, self.scale, allowed)
        out = out.transpose(1, 2).contiguous().view(b, s, self.d_model)
        return self.o_proj(out), kv_cache


class PagedAttention(_AttentionBase):
    """``attn_impl="hip_paged"``: the attention module on a PagedKVCache.

    forward(x, attention_mask, kv_cache, rope_state, sliding_window, sink_cfg)
    -> (out, kv_cache), as AttentionTorch (src/core/attention.py:37-45,110); the
    cache is mutated in place and returned.  A single-token step (decode) appends the
    new row and attends over the pages in one op (ivakv_decode_append_attn); a
    multi-token step (prefill / chunked prefill) appends with ivakv_append and runs
    the causal attention of the new tokens over the pages (ivakv_prefill_attn).
    A contiguous ``KVCache`` is taken over as a PagedKVCache (:meth:`_adopt`), which is
    returned in its place.  Without a cache a causal step runs the same kernels on a
    one-layer paged cache of its own tokens, and None is returned, as the reference
    returns (attention.py:74-75).  Non-causal attention (``config.causal`` False) is
    evaluated in torch on the gathered pages: the paged kernels are causal.  With a
    sliding window, once the forward's last layer is enqueued the cache releases the
    pages no later query can see (:meth:`PagedKVCache.release_window`; the sink pages
    stay resident), so a long sequence holds about window + sinks tokens per layer.
    A padding mask (``attention_mask`` with zeros, src/core/attention.py:95-97) is applied
    as the reference broadcasts it (:meth:`_key_mask`): the step's rows are still appended
    and gathered by the kernels, and the masked attention is evaluated on the gathered
    keys in torch.  A row whose every key is masked gives zeros, where the reference's
    softmax over all -inf gives NaN (which its next layer then spreads to every row).
    """

    def forward(self, x: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                kv_cache: Optional[Any] = None, rope_state: Optional[torch.Tensor] = None,
                sliding_window: Optional[int] = None,
                sink_cfg: Optional[Dict[str, Any]] = None) -> Tuple[torch.Tensor, Optional[Any]]:
        if self.training and self.dropout > 0:
            raise NotImplementedError("the paged attention path is for inference (model.eval())")
        if kv_cache is not None and not isinstance(kv_cache, PagedKVCache):
            kv_cache = self._adopt(kv_cache, x)
        key_ok = self._key_mask(attention_mask)
        b, s, _ = x.shape
        returned = kv_cache
        if kv_cache is None and self.causal:
            kv_cache = PagedKVCache(b, self.n_kv_heads, self.head_dim, 0, x.device, x.dtype,
                                    num_layers=1, max_seq_len=s)
        q, k, v = self._project(x)
        n_sink = _sink_count(sink_cfg, self.sink_tokens)
        window = sliding_window if sliding_window and sliding_window > 0 else None
        if kv_cache is not None and kv_cache.current_layer == 0:
            kv_cache.note_window(window, n_sink)
        rope_pos = None  # K rows rotated inside the append instead of separately
        if self.rope:
            # absolute positions of the new tokens, token-major [B * s] int32 on the device
            pos = kv_cache.token_positions(s) if kv_cache is not None else \
                torch.arange(s, dtype=torch.int32, device=x.device).repeat(b)
            rope_(q.reshape(b * s, self.n_heads, self.head_dim), pos, self.rope_theta)
            if kv_cache is None or s == 1:
                rope_(k.reshape(b * s, self.n_kv_heads, self.head_dim), pos, self.rope_theta)
            else:
                rope_pos = pos
        if kv_cache is None:  # non-causal without a cache
            allowed = torch.ones(s, s, dtype=torch.bool, device=x.device)[None, None]
            if key_ok is not None:
                allowed = allowed & key_ok
            out = _attend(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), self.scale,
                          allowed)
            out = out.transpose(1, 2)
        else:
            # a padding mask: the rows are appended (ivakv_append) and gathered
            # (ivakv_gather) by the kernels, and the masked attention evaluated on the
            # gathered keys in torch (the paged attention kernels take no per-key mask)
            decode = s == 1 and self.causal and key_ok is None
            fp8 = kv_cache.pool.fp8
            view = kv_cache.layer_step(k.contiguous(), v.contiguous(), append=not decode,
                                       rope_positions=rope_pos, rope_theta=self.rope_theta)
            if decode:
                # append + attend in one op: the new row lands at position L-1 of each page
                # table and is scored straight from k / v (ivakv_decode_append_attn; on
                # FP8 pages quantized as the append would, ivakv_decode_append_attn_fp8)
                o = paged_decode_append_attention(
                    q.view(b, self.n_heads, self.head_dim), k.view(b, self.n_kv_heads, self.head_dim),
                    v.view(b, self.n_kv_heads, self.head_dim), view.k_pool, view.v_pool,
                    view.block_tables, view.context_lens, scale=self.scale, window=window or 0,
                    n_sink=n_sink if window else 0, **view.scales)
                out = o.view(b, 1, self.n_heads, self.head_dim)
            elif self.causal and key_ok is None and (not fp8 or q.dtype in (torch.float16,
                                                                          torch.bfloat16)):
                # the chunk's rows sit at positions start .. start+s-1 of every sequence
                # (FP8 pages: dequantized inside the kernel, ivakv_prefill_attn_fp8)
                qs = torch.arange(0, (b + 1) * s, s, dtype=torch.int32, device=x.device)
                o = paged_prefill_attention(
                    q.reshape(b * s, self.n_heads, self.head_dim), view.k_pool, view.v_pool,
                    view.block_tables, view.context_lens, qs, scale=self.scale,
                    window=window or 0, n_sink=n_sink if window else 0, max_query_len=s,
                    **view.scales)
                out = o.view(b, s, self.n_heads, self.head_dim)
            else:
                # non-causal, a padding mask, or fp32 queries on FP8 pages: gather
                # (dequantized for FP8) and evaluate the masked attention of the new
                # tokens in torch
                total = view.start + s
                kw = dict(view.scales, out_dtype=q.dtype) if fp8 else {}
                kc, vc = kv_gather(view.k_pool, view.v_pool, view.block_tables,
                                   view.context_lens, out_len=total, **kw)
                q_pos = torch.arange(view.start, total, device=x.device)
                k_pos = torch.arange(total, device=x.device)
                allowed = _visible(q_pos, k_pos, window, n_sink) if self.causal else \
                    torch.ones(s, total, dtype=torch.bool, device=x.device)
                allowed = allowed[None, None] if key_ok is None else allowed[None, None] & key_ok
                out = _attend(q.transpose(1, 2), kc, vc, self.scale, allowed)
                out = out.transpose(1, 2)
        if kv_cache is not None and returned is not None and kv_cache.current_layer == 0:
            # the forward's last layer is enqueued: with a sliding window, the pages no later
            # query can see go back to the pool (sink pages stay)
            kv_cache.release_window()
        out = out.reshape(b, s, self.d_model)
        return self.o_proj(out), (kv_cache if returned is not None else None)

    def _adopt(self, cache: Any, x: torch.Tensor) -> PagedKVCache:
        """Takes over a contiguous cache (the reference's ``KVCache``, src/core/rope_kv.py:
        71-137: ``k`` / ``v`` of ``[B, H, seq_len, D]``), as the reference's
        ``Transformer.generate`` passes one: a new ``KVCache(seq_len=0)`` whose whole
        sequence is fed again on every step (transformer.py:273-290).

        Returns a PagedKVCache with one layer per block of the model (``config.n_layers``),
        every layer starting with the cache's ``seq_len`` rows.  The block returns it in
        place of the contiguous cache, so the following blocks of the same forward take
        their own layers from it through the layer cursor, each layer attending to its own
        keys and values (the reference threads one cache through all blocks,
        transformer.py:229-238).  After the last block the paged cache holds every layer's
        rows and its ``seq_len`` has advanced by the forward's tokens."""
        for name in ("k", "v", "seq_len", "batch_size"):
            if not hasattr(cache, name):
                raise TypeError(f"kv_cache of type {type(cache).__name__} has no {name!r}: "
                                "expected a PagedKVCache or a KVCache")
        b, s, _ = x.shape
        s0 = int(cache.seq_len)
        if int(cache.batch_size) != b:
            raise ValueError(f"kv_cache holds {cache.batch_size} sequences, input has {b}")
        if s0 > 0 and (tuple(cache.k.shape[1:]) != (self.n_kv_heads, s0, self.head_dim)
                       or cache.v.shape != cache.k.shape):
            raise ValueError(f"kv_cache k / v are {tuple(cache.k.shape)}, expected "
                             f"[{b}, {self.n_kv_heads}, {s0}, {self.head_dim}]")
        page_dtype = FP8 if _cfg(self.config, "kv_cache_dtype", None) == "fp8" else x.dtype
        paged = PagedKVCache(b, self.n_kv_heads, self.head_dim, 0, x.device, page_dtype,
                             num_layers=int(getattr(self.config, "n_layers", 1)),
                             block_size=int(_cfg(self.config, "kv_block_size", 16)),
                             max_seq_len=s0 + s, compute_dtype=x.dtype)
        if s0 > 0:
            k0, v0 = cache.k.to(x.dtype), cache.v.to(x.dtype)
            for layer in range(paged.num_layers):
                paged.select_layer(layer)
                paged.update(k0, v0, 0)
            paged.select_layer(0)
        return paged


def get_attention(config: Any) -> nn.Module:
    """src/core/attention.py:190-194 plus the paged backend.  ``"triton"`` gives the torch
    module, as the reference's ``AttentionTriton`` does: its forward copies its weights
    into a new ``AttentionTorch`` and runs that (attention.py:151-187)."""
    if config.attn_impl == "hip_paged":
        return PagedAttention(config)
    return AttentionTorch(config)


class RMSNorm(nn.Module):
    """src/core/norms.py:14-36."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.eps = config.norm_eps
        self.weight = nn.Parameter(torch.ones(config.d_model)) if config.elementwise_affine else None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf / torch.sqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + self.eps)
        y = y.to(x.dtype)
        return y * self.weight if self.weight is not None else y


class FFN(nn.Module):
    """src/core/ffn.py:27-64.  "swiglu" computes silu(up(x)) * gate(x): the reference
    concatenates [gate, up] and its SwiGLU returns silu(second half) * first half
    (ffn.py:21-24,57-60)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.activation = config.activation
        hidden = config.d_model * config.hidden_mult
        self.gate_proj = nn.Linear(config.d_model, hidden, bias=False)
        self.up_proj = nn.Linear(config.d_model, hidden, bias=False)
        self.down_proj = nn.Linear(hidden, config.d_model, bias=False)
        self.dropout_layer = nn.Dropout(config.dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.activation == "swiglu":
            hidden = F.silu(self.up_proj(x)) * self.gate_proj(x)
        else:
            act = F.gelu if self.activation == "gelu" else F.relu
            hidden = self.dropout_layer(act(self.gate_proj(x))) * self.up_proj(x)
        return self.down_proj(hidden)


class TransformerBlock(nn.Module):
    """src/core/transformer.py:81-151 (pre-norm attention and FFN with residuals)."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        if config.moe_enable or config.hrm_enable:
            raise NotImplementedError("MoE and HRM blocks are not part of this build")
        self.config = config
        self.attention = get_attention(config)
        self.ffn = FFN(config)
        self.norm1 = RMSNorm(config)
        self.norm2 = RMSNorm(config)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x, attention_mask=None, kv_cache=None, rope_state=None, sliding_window=None,
                sink_cfg=None, router_temp=None, hrm_state=None):
        attn_out, new_kv_cache = self.attention(self.norm1(x), attention_mask=attention_mask,
                                                kv_cache=kv_cache, rope_state=rope_state,
                                                sliding_window=sliding_window, sink_cfg=sink_cfg)
        x = x + self.dropout(attn_out)
        x = x + self.dropout(self.ffn(self.norm2(x)))
        return x, new_kv_cache, {}


class Transformer(nn.Module):
    """src/core/transformer.py:154-320 at its interfaces."""

    def __init__(self, config: TransformerConfig):
        super().__init__()
        self.config = config
        self.token_embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.position_embedding = nn.Embedding(config.seq_len, config.d_model)
        self.blocks = nn.ModuleList([TransformerBlock(config) for _ in range(config.n_layers)])
        self.norm = RMSNorm(config)
        self.lm_head = (None if config.tie_embeddings
                        else nn.Linear(config.d_model, config.vocab_size, bias=False))
        self.value_head = nn.Sequential(nn.Linear(config.d_model, config.d_model // 2), nn.ReLU(),
                                        nn.Linear(config.d_model // 2, 1))
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        if isinstance(module, nn.Linear):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                torch.nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def new_kv_cache(self, batch_size: int, max_seq_len: int, device=None, dtype=None):
        """An empty cache of the configured backend for ``batch_size`` sequences of up to
        ``max_seq_len`` tokens, one set of K/V per layer."""
        cfg = self.config
        device = device or self.token_embedding.weight.device
        dtype = dtype or self.token_embedding.weight.dtype
        n_kv = int(_cfg(cfg, "n_kv_heads", cfg.n_heads))
        head_dim = cfg.d_model // cfg.n_heads
        if cfg.attn_impl == "hip_paged":
            page_dtype = FP8 if _cfg(cfg, "kv_cache_dtype", None) == "fp8" else dtype
            cache = PagedKVCache(batch_size, n_kv, head_dim, 0, device, page_dtype,
                                 num_layers=cfg.n_layers, block_size=_cfg(cfg, "kv_block_size", 16),
                                 max_seq_len=max_seq_len, num_pages=_cfg(cfg, "kv_num_pages", None),
                                 compute_dtype=dtype)
            cache.resize(max_seq_len)
            return cache
        return LayeredKVCache(batch_size, n_kv, head_dim, cfg.n_layers, device, dtype)

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        w = self.token_embedding.weight if self.lm_head is None else self.lm_head.weight
        return F.linear(x, w)

    def forward(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                kv_cache: Optional[Any] = None, return_logits: bool = True,
                return_value: bool = False, **kwargs) -> Dict[str, torch.Tensor]:
        batch_size, seq_len = input_ids.shape
        device = input_ids.device
        if isinstance(kv_cache, PagedKVCache) and kv_cache.static:
            position_ids = kv_cache.device_positions()  # on the device: graph-replayable
        else:
            start = kv_cache.seq_len if kv_cache is not None else 0
            position_ids = torch.arange(start, start + seq_len, device=device,
                                        dtype=torch.long).unsqueeze(0).expand(batch_size, -1)
        x = self.token_embedding(input_ids) + self.position_embedding(position_ids)
        # attention_mask None means all ones (transformer.py:212-213 builds ones_like)
        sliding_window = self.config.sliding_window
        n_sink = int(_cfg(self.config, "sink_tokens", 0))
        sink_cfg = {"sink_tokens": n_sink} if n_sink else None
        for block in self.blocks:
            x, kv_cache, _ = block(x, attention_mask=attention_mask, kv_cache=kv_cache,
                                   sliding_window=sliding_window, sink_cfg=sink_cfg)
        x = self.norm(x)
        outputs: Dict[str, torch.Tensor] = {}
        if return_logits:
            outputs["logits"] = self.logits(x)
        if return_value:
            outputs["value"] = self.value_head(x)
        return outputs

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_length: int = 100, temperature: float = 1.0,
                 top_p: float = 0.9, top_k: int = 50, do_sample: bool = True,
                 pad_token_id: int = 0, eos_token_id: Optional[int] = 2, **kwargs) -> torch.Tensor:
        """src/core/transformer.py:257-320 with an incremental cache: one prefill
        forward of the prompt, then one single-token forward per new token.

        With ``attn_impl="hip_paged"`` and ``use_graph=True`` (keyword) the decode
        step is captured once as a HIP graph and replayed: the cache's pages are
        reserved up front and its per-step bookkeeping runs on the device.  EOS
        stopping (``eos_token_id``) needs a host read per step; pass None to run
        all ``max_length`` steps without one.
        """
        self.eval()
        batch_size, prompt_len = input_ids.shape
        own_cache = kwargs.get("kv_cache") is None
        cache = kwargs.get("kv_cache") or self.new_kv_cache(batch_size, prompt_len + max_length)
        use_graph = bool(kwargs.get("use_graph", False))
        if use_graph and not isinstance(cache, PagedKVCache):
            raise ValueError("use_graph needs attn_impl='hip_paged'")
        out = torch.empty(batch_size, prompt_len + max_length, dtype=input_ids.dtype,
                          device=input_ids.device)
        out[:, :prompt_len] = input_ids
        n = 0
        try:
            logits = self.forward(input_ids, kv_cache=cache)["logits"][:, -1, :]
            tok = self._sample(logits, temperature, top_p, top_k, do_sample)
            out[:, prompt_len] = tok[:, 0]
            n = 1
            if use_graph and max_length > 1:
                n = self._decode_graph(cache, tok, out, prompt_len, max_length, temperature,
                                       top_p, top_k, do_sample)
            else:
                while n < max_length and not (eos_token_id is not None
                                              and bool((tok == eos_token_id).all())):
                    logits = self.forward(tok, kv_cache=cache)["logits"][:, -1, :]
                    tok = self._sample(logits, temperature, top_p, top_k, do_sample)
                    out[:, prompt_len + n] = tok[:, 0]
                    n += 1
        finally:
            if own_cache and isinstance(cache, PagedKVCache):
                cache.free()
        return out[:, :prompt_len + n]

    def _decode_graph(self, cache: PagedKVCache, tok, out, prompt_len, max_length, temperature,
                      top_p, top_k, do_sample) -> int:
        """Decode steps 2..max_length as replays of one captured HIP graph.  Step 2 runs
        eagerly on the capture stream (warming every kernel and workspace), step 3 is
        captured (capture records without executing), then the graph is replayed."""
        cache.begin_static_decode(max_length - 1)
        static_tok = tok.clone()
        stream = torch.cuda.Stream(device=tok.device)
        stream.wait_stream(torch.cuda.current_stream(tok.device))

        def step():
            logits = self.forward(static_tok, kv_cache=cache)["logits"][:, -1, :]
            static_tok.copy_(self._sample(logits, temperature, top_p, top_k, do_sample))

        n = 1
        try:
            with torch.cuda.stream(stream):
                step()
                cache.advance_host(1)
                out[:, prompt_len + n] = static_tok[:, 0]
                n += 1
                if n < max_length:
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=stream):
                        step()  # recorded, not executed: the device state does not move
                    while n < max_length:
                        graph.replay()
                        cache.advance_host(1)
                        out[:, prompt_len + n] = static_tok[:, 0]
                        n += 1
            torch.cuda.current_stream(tok.device).wait_stream(stream)
        finally:
            cache.end_static_decode()
        return n

    @staticmethod
    def _sample_filtered(logits, temperature, top_p, top_k):
        """Temperature, top-k and top-p filtering, then a multinomial draw."""
        logits = logits / temperature
        if top_k > 0:
            vals, idx = torch.topk(logits, top_k)
            logits = torch.full_like(logits, float("-inf")).scatter_(1, idx, vals)
        if top_p < 1.0:
            sorted_logits, sorted_idx = torch.sort(logits, descending=True)
            cum = torch.cumsum(F.softmax(sorted_logits, dim=-1), dim=-1)
            remove = cum > top_p
            remove[..., 1:] = remove[..., :-1].clone()
            remove[..., 0] = False
            logits = logits.masked_fill(remove.scatter(1, sorted_idx, remove), float("-inf"))
        return torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)

    @staticmethod
    def _sample(logits, temperature, top_p, top_k, do_sample):
        """Top-k / top-p / multinomial or argmax (transformer.py:292-313).  Greedy
        decoding takes the argmax directly: the filters always keep the maximum."""
        if not do_sample:
            return torch.argmax(logits, dim=-1, keepdim=True)
        return Transformer._sample_filtered(logits, temperature, top_p, top_k)

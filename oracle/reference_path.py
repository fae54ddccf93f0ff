"""torch-CPU restatement of the reference's contiguous KV path.  TEST INFRASTRUCTURE ONLY.

The reference package cannot be imported (src/core/rope_kv.py:199-203 does not
parse and src/utils/logging.py:13 needs tensorboard), so its KV path is
restated here operation for operation, in the library it is written in:
  ContiguousKVCache         KVCache (src/core/rope_kv.py:71-137): zero-filled
                            [B, H, S, D] buffers, slice-assign update with
                            grow-by-copy resize, get_slice views.
  cat_append                the cache branch of AttentionTorch.forward
                            (src/core/attention.py:61-63): torch.cat on dim 2.
  attention_math            AttentionTorch.forward scores/masks/softmax/PV
                            (src/core/attention.py:77-102), with the masks at
                            absolute positions and sinks as a union (the build's
                            fix of the reference's misaligned masks), GQA by
                            repeat_interleave.
  reference_decode_step     one decode step of that path on a padded batch: the
                            torch.cat append of one new row per sequence, then
                            the attention math.  bench.py times this on the
                            host cores as the CPU baseline.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


class ContiguousKVCache:
    """Restatement of ``KVCache`` (rope_kv.py:71-137)."""

    def __init__(self, batch_size: int, n_heads: int, head_dim: int, seq_len: int,
                 device="cpu", dtype: torch.dtype = torch.float16):
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

    def get_slice(self, start: int, end: int) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.k[:, :, start:end], self.v[:, :, start:end]


def cat_append(cache_k: torch.Tensor, cache_v: torch.Tensor, k: torch.Tensor,
               v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``torch.cat([kv_cache.k, k], dim=2)`` (attention.py:62-63)."""
    return torch.cat([cache_k, k], dim=2), torch.cat([cache_v, v], dim=2)


def attention_math(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                   key_valid: Optional[torch.Tensor] = None,
                   key_pos: Optional[torch.Tensor] = None,
                   query_pos: Optional[torch.Tensor] = None,
                   window: Optional[int] = None, n_sink: int = 0) -> torch.Tensor:
    """``softmax(q k^T * scale + masks) v`` (attention.py:77-102).

    q [B, Hq, S, D]; k, v [B, Hkv, Lk, D] (GQA by ``repeat_interleave`` on dim 1).
    key_valid [B, Lk] plays the role of ``attention_mask`` (attention.py:95-97).
    key_pos [B, Lk] / query_pos [B, S] are absolute positions for the causal,
    window (attention.py:124-127) and sink masks; when omitted the keys are
    0..Lk-1 and the queries the last S of them.
    """
    batch, hq, s_len, _ = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    g = hq // hkv
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if key_pos is None:
        key_pos = torch.arange(lk).unsqueeze(0).expand(batch, -1)
    if query_pos is None:
        query_pos = torch.arange(lk - s_len, lk).unsqueeze(0).expand(batch, -1)
    kp = key_pos[:, None, None, :]
    qp = query_pos[:, None, :, None]
    allowed = kp <= qp
    if window is not None and window > 0:
        allowed = allowed & ((kp > qp - window) | (kp < n_sink))
    if key_valid is not None:
        allowed = allowed & key_valid[:, None, None, :].bool()
    scores = scores.masked_fill(~allowed, float("-inf"))
    weights = torch.softmax(scores, dim=-1)
    weights = torch.nan_to_num(weights, nan=0.0)  # rows with no visible key -> zero output
    return torch.matmul(weights, v)


def padded_batch(k_rows, v_rows, lengths, dtype=torch.float32):
    """Packs per-sequence contiguous rows ([Hkv, L_b, D] each) into the reference's
    zero-padded [B, Hkv, Lmax, D] cache layout plus the key-valid mask."""
    batch = len(lengths)
    hkv, _, d = k_rows[0].shape
    lmax = max(int(x) for x in lengths)
    k = torch.zeros(batch, hkv, lmax, d, dtype=dtype)
    v = torch.zeros(batch, hkv, lmax, d, dtype=dtype)
    valid = torch.zeros(batch, lmax, dtype=torch.bool)
    for b, length in enumerate(lengths):
        k[b, :, :length] = k_rows[b].to(dtype)
        v[b, :, :length] = v_rows[b].to(dtype)
        valid[b, :length] = True
    return k, v, valid


def reference_decode_step(cache_k: torch.Tensor, cache_v: torch.Tensor, valid: torch.Tensor,
                          lengths: torch.Tensor, q: torch.Tensor, k_new: torch.Tensor,
                          v_new: torch.Tensor, scale: float, window: Optional[int] = None,
                          n_sink: int = 0) -> torch.Tensor:
    """One decode step of the reference path on a padded batch.

    cache_k/v [B, Hkv, Lc, D] hold each sequence's first ``lengths[b] - 1`` rows
    (zero-padded, ``valid`` marks them); q [B, Hq, 1, D]; k_new/v_new [B, Hkv, 1, D]
    are the rows of the token at position ``lengths[b] - 1``.  Appends with torch.cat
    as AttentionTorch does, then evaluates the attention math.  Returns [B, Hq, 1, D].
    """
    batch, _, lc, _ = cache_k.shape
    k, v = cat_append(cache_k, cache_v, k_new, v_new)
    key_valid = torch.cat([valid, torch.ones(batch, 1, dtype=torch.bool)], dim=1)
    key_pos = torch.cat([torch.arange(lc).unsqueeze(0).expand(batch, -1),
                         (lengths.to(torch.long) - 1).unsqueeze(1)], dim=1)
    query_pos = (lengths.to(torch.long) - 1).unsqueeze(1)
    return attention_math(q, k, v, scale, key_valid=key_valid, key_pos=key_pos,
                          query_pos=query_pos, window=window, n_sink=n_sink)


class ReferenceRoPE:
    """The reference's RoPE module (src/core/rope_kv.py:9-50) restated in torch: a float32
    frequency buffer filled pair by pair, cos / sin of position * frequency, and the
    pairwise rotation loop writing into a zeros_like(x) result."""

    def __init__(self, head_dim: int, theta: float = 10000.0):
        self.head_dim = head_dim
        freqs = torch.zeros(head_dim, dtype=torch.float32)
        for i in range(0, head_dim, 2):
            freqs[i] = 1.0 / (theta ** (i / head_dim))
            if i + 1 < head_dim:
                freqs[i + 1] = freqs[i]
        self.freqs = freqs

    def forward(self, x: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
        """x [B, H, S, D], position_ids [B, S]."""
        pos_freqs = position_ids.unsqueeze(-1) * self.freqs.unsqueeze(0).unsqueeze(0)
        cos = torch.cos(pos_freqs).unsqueeze(1).expand(-1, x.shape[1], -1, -1)
        sin = torch.sin(pos_freqs).unsqueeze(1).expand(-1, x.shape[1], -1, -1)
        out = torch.zeros_like(x)
        for i in range(0, self.head_dim, 2):
            if i + 1 < self.head_dim:
                out[..., i] = x[..., i] * cos[..., i] - x[..., i + 1] * sin[..., i]
                out[..., i + 1] = x[..., i] * sin[..., i] + x[..., i + 1] * cos[..., i]
            else:
                out[..., i] = x[..., i]
        return out


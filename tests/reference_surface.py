"""The reference's own model-level surface, restated for the drop-in tests.

The reference package cannot be imported (src/core/rope_kv.py:199-203 is a SyntaxError,
src/utils/logging.py:13 needs tensorboard), so the tests restate the three pieces of it
that a user of the paged backend goes through, each with the two-line patch into src/core
(the whitelist entry and the get_attention branch below):

  RefTransformerConfig   src/core/transformer.py:25-78: exactly the reference's fields,
                         and its __post_init__ with "hip_paged" added to the whitelist
                         (:71-72, the one-line patch).
  patched_get_attention  src/core/attention.py:190-194 with the "hip_paged" branch added.
  reference_generate     src/core/transformer.py:257-320: a contiguous KVCache of length 0,
                         the whole sequence fed again on every step, top-k / top-p
                         filtering, argmax or multinomial, EOS stop.
"""
from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

# The field list of transformer.py:25-65, in order: (name, default).
REFERENCE_FIELDS = [
    ("d_model", 1024), ("n_layers", 16), ("n_heads", 16), ("vocab_size", 32000),
    ("seq_len", 4096), ("rope_theta", 100000.0), ("attn_impl", "torch"),
    ("norm_impl", "torch"), ("moe_enable", False), ("hrm_enable", False),
    ("tie_embeddings", True), ("sliding_window", None), ("n_experts", 4), ("top_k", 2),
    ("capacity_factor", 1.25), ("dropless", False), ("aux_loss_coef", 0.01),
    ("expert_parallel", False), ("max_steps", 8), ("halt_penalty", 0.1),
    ("sink_strength_init", 0.5), ("temp_bounds", (0.1, 2.0)), ("dropout", 0.1),
    ("use_flash_attn", False), ("causal", True), ("norm_eps", 1e-6),
    ("elementwise_affine", True), ("hidden_mult", 4), ("activation", "swiglu"),
]


@dataclass
class RefTransformerConfig:
    """transformer.py:25-78 field for field; only the attn_impl whitelist differs."""

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
    n_experts: int = 4
    top_k: int = 2
    capacity_factor: float = 1.25
    dropless: bool = False
    aux_loss_coef: float = 0.01
    expert_parallel: bool = False
    max_steps: int = 8
    halt_penalty: float = 0.1
    sink_strength_init: float = 0.5
    temp_bounds: Tuple[float, float] = (0.1, 2.0)
    dropout: float = 0.1
    use_flash_attn: bool = False
    causal: bool = True
    norm_eps: float = 1e-6
    elementwise_affine: bool = True
    hidden_mult: int = 4
    activation: str = "swiglu"

    def __post_init__(self):
        if self.d_model % self.n_heads != 0:
            raise ValueError(f"d_model ({self.d_model}) must be divisible by n_heads ({self.n_heads})")
        if self.attn_impl not in ["torch", "triton", "hip_paged"]:  # the patched line
            raise ValueError(f"attn_impl must be 'torch' or 'triton', got {self.attn_impl}")
        if self.norm_impl not in ["torch", "triton"]:
            raise ValueError(f"norm_impl must be 'torch' or 'triton', got {self.norm_impl}")
        if self.activation not in ["swiglu", "gelu", "relu"]:
            raise ValueError(f"activation must be 'swiglu', 'gelu', or 'relu', got {self.activation}")


def field_list():
    return [(f.name, f.default) for f in fields(RefTransformerConfig)]


def patched_get_attention(config):
    """attention.py:190-194 with a first branch for "hip_paged"; AttentionTriton's forward runs
    an AttentionTorch with its weights (attention.py:151-187), so the torch module
    stands in for it."""
    from iva_amd.model import AttentionTorch
    if config.attn_impl == "hip_paged":
        from iva_amd.model import PagedAttention
        return PagedAttention(config)
    return AttentionTorch(config)


@torch.no_grad()
def reference_generate(model, input_ids, max_length=100, temperature=1.0, top_p=0.9, top_k=50,
                       do_sample=True, eos_token_id=2):
    """transformer.py:257-320: one KVCache(seq_len=0) for the call (fp16, the KVCache
    default), the whole sequence fed again every step, filtering, then a draw or argmax."""
    from iva_amd.model import KVCache
    model.eval()
    cfg = model.config
    kv_cache = KVCache(batch_size=input_ids.shape[0], n_heads=cfg.n_heads,
                       head_dim=cfg.d_model // cfg.n_heads, seq_len=0, device=input_ids.device)
    generated = input_ids.clone()
    for _ in range(max_length):
        outputs = model.forward(generated, kv_cache=kv_cache, return_logits=True,
                                return_value=False)
        logits = outputs["logits"][:, -1, :] / temperature
        if top_k > 0:
            vals, idx = torch.topk(logits, top_k)
            logits = torch.full_like(logits, float("-inf"))
            logits.scatter_(1, idx, vals)
        if top_p < 1.0:
            sorted_logits, sorted_idx = torch.sort(logits, descending=True)
            cum = torch.cumsum(F.softmax(sorted_logits, dim=-1), dim=-1)
            remove = cum > top_p
            remove[..., 1:] = remove[..., :-1].clone()
            remove[..., 0] = 0
            logits[remove.scatter(1, sorted_idx, remove)] = float("-inf")
        if do_sample:
            nxt = torch.multinomial(F.softmax(logits, dim=-1), num_samples=1)
        else:
            nxt = torch.argmax(logits, dim=-1, keepdim=True)
        generated = torch.cat([generated, nxt], dim=1)
        if (nxt == eos_token_id).all():
            break
    return generated

"""Model-level parity of two backends with identical weights (teacher-forced logits and
greedy tokens), shared by the GPU model tests.

The argument: if every teacher-forced logit of the paged backend is within ``tol`` of
the torch backend's, the two argmaxes can differ only at a step whose torch top-2 margin
is at most ``2 * tol``.  So the checks are
  1. max |logits_paged - logits_torch| <= tol at every step (teacher-forced along the
     torch backend's own greedy stream, so both see the same inputs);
  2. greedy tokens equal at every step whose torch margin exceeds 2 * tol, and at least
     ``min_compared`` such steps exist (the check cannot pass vacuously);
  3. free-running greedy generation: each sequence's first divergence from the torch
     backend's stream falls on a step whose torch margin is at most 2 * tol (a near-tie,
     which either backend may resolve either way).
"""
from __future__ import annotations

import torch


@torch.no_grad()
def teacher_forced_logits(model, ids: torch.Tensor, prompt_len: int) -> torch.Tensor:
    """fp32 logits ``[B, n, V]`` predicting tokens ``prompt_len .. ids.shape[1]-1`` (one
    prefill forward of the prompt, then one single-token forward per token of ``ids``)."""
    cache = model.new_kv_cache(ids.shape[0], ids.shape[1], device=ids.device)
    outs = [model(ids[:, :prompt_len], kv_cache=cache)["logits"][:, -1:].float()]
    for t in range(prompt_len, ids.shape[1] - 1):
        outs.append(model(ids[:, t:t + 1], kv_cache=cache)["logits"].float())
    if hasattr(cache, "free"):
        cache.free()
    return torch.cat(outs, dim=1)


def top2_margin(logits: torch.Tensor) -> torch.Tensor:
    top = logits.topk(2, dim=-1).values
    return top[..., 0] - top[..., 1]


@torch.no_grad()
def check_greedy_parity(ref, paged, prompts: torch.Tensor, steps: int, tol: float,
                        min_compared: int) -> dict:
    """Runs checks 1-3 of the module docstring; returns the figures behind them."""
    p = prompts.shape[1]
    g_ref = ref.generate(prompts, max_length=steps, do_sample=False, eos_token_id=None)
    g_pag = paged.generate(prompts, max_length=steps, do_sample=False, eos_token_id=None)
    assert g_ref.shape == g_pag.shape == (prompts.shape[0], p + steps)
    l_ref = teacher_forced_logits(ref, g_ref, p)
    l_pag = teacher_forced_logits(paged, g_ref, p)
    diff = (l_ref - l_pag).abs().max().item()
    assert diff <= tol, f"teacher-forced logits differ by {diff} > {tol}"
    margin = top2_margin(l_ref)
    tokens = g_ref[:, p:]
    compared = margin > 2 * tol
    n_compared = int(compared.sum())
    assert n_compared >= min_compared, f"only {n_compared} steps above the 2*tol margin"
    bad = (l_pag.argmax(dim=-1) != tokens) & compared
    assert not bool(bad.any()), f"greedy token differs at steps {bad.nonzero().tolist()}"
    first_div = []
    for b in range(prompts.shape[0]):
        differ = (g_pag[b, p:] != tokens[b]).nonzero()
        if differ.numel():
            t = int(differ[0])
            first_div.append((t, float(margin[b, t])))
            assert margin[b, t] <= 2 * tol, \
                f"sequence {b} diverges at step {t} where the torch margin is {margin[b, t]}"
    return {"max_logit_diff": diff, "compared": n_compared, "first_divergence": first_div,
            "l_ref": l_ref, "l_pag": l_pag, "tokens": g_ref}

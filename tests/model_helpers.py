"""Shared helpers of the model-level GPU tests: teacher-forced logits through the paged cache."""

from __future__ import annotations

import torch


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| in float64 on the host."""
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@torch.no_grad()
def forced_logits(model, prompts: torch.Tensor, forced: torch.Tensor) -> torch.Tensor:
    """Last-position logits of the prefill and of each teacher-forced decode step,
    ``[steps + 1, seq, vocab]`` (float32, host), through a paged cache of 16-token blocks."""
    dev = model.embed_tokens.weight.device
    dtype = model.embed_tokens.weight.dtype
    seqs, plen = prompts.shape
    steps = forced.shape[1]
    per = -(-(plen + steps + 1) // 16)
    cache = model.allocate_cache(seqs * per, 16, dtype, dev)
    table = torch.arange(seqs * per, dtype=torch.int32, device=dev).view(seqs, per)
    out = [model(prompts.to(dev).reshape(-1), torch.arange(plen, device=dev).repeat(seqs), cache=cache,
                 block_ids=table, context_lens=torch.full((seqs,), plen, dtype=torch.int32, device=dev),
                 q_len=plen, last_only=True).last_logits()]
    for i in range(steps):
        pos = torch.full((seqs,), plen + i, dtype=torch.long, device=dev)
        out.append(model(forced[:, i].to(dev), pos, cache=cache, block_ids=table,
                         context_lens=(pos + 1).to(torch.int32), q_len=1, last_only=True).last_logits())
    return torch.stack(out).float().cpu()


def confident_positions(ref: torch.Tensor, margin: float) -> torch.Tensor:
    """Mask of the (step, sequence) rows whose top-1 logit leads the runner-up by more than
    ``margin`` (absolute), where any path within that error must pick the same token."""
    top2 = ref.topk(2, dim=-1).values
    return (top2[..., 0] - top2[..., 1]) > margin

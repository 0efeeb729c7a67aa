"""Last-token logits: the vocabulary projection only where the engine reads it.

The reference's model projects every position of a step onto the vocabulary
(``src/llmopt/model/modeling.py:128-130``), and its model runner then keeps only each
sequence's last position (``src/llmopt/engine/model_runner.py:93-114``, ``last_logits()``).
During prefill that is ``seq * q_len`` rows of a ``[hidden, vocab]`` product (Llama-3-8B:
4096 x 128256, 1.05 GB of bf16 weight) of which ``seq`` rows are used. :func:`last_token_logits`
projects only those rows; each kept row is the same row-wise linear map, so the result equals
the reference's kept logits up to the GEMM's own rounding.
"""

from __future__ import annotations

import torch

__all__ = ["last_token_hidden", "last_token_logits"]


def last_token_hidden(hidden: torch.Tensor, q_len: int) -> torch.Tensor:
    """``hidden [seq * q_len, H]`` (sequence-major, as the model lays a step out) ->
    ``[seq, H]``, the last position of every sequence."""
    if q_len < 1:
        raise ValueError(f"q_len must be >= 1, got {q_len}")
    total, width = int(hidden.shape[0]), int(hidden.shape[-1])
    if total % q_len:
        raise ValueError(f"{total} rows are not a whole number of sequences of {q_len} tokens")
    return hidden.reshape(total // q_len, q_len, width)[:, -1]


def last_token_logits(hidden: torch.Tensor, lm_head: torch.nn.Module, q_len: int) -> torch.Tensor:
    """``[seq, vocab]`` logits of each sequence's last position: ``lm_head`` applied to
    :func:`last_token_hidden` only (the reference applies it to all ``seq * q_len`` rows, then
    keeps ``logits.view(seq, q_len, -1)[:, -1]``)."""
    return lm_head(last_token_hidden(hidden, q_len).contiguous())

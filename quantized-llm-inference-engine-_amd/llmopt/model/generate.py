"""Static-batch greedy generation through the paged KV cache.

The reference's engine (scheduler, block pool, request objects) is out of scope here; this is
the part of its model runner (``src/llmopt/engine/model_runner.py:93-114``) that the
end-to-end measurement needs: one prefill forward over every prompt, then one forward per
decode step, each sequence's next token the argmax of its last-position logits. Blocks are
handed out contiguously, ``ceil((prompt_len + steps) / block_size)`` per sequence.

On HIP devices the decode step -- embedding, every layer's kernels, the final norm,
``lm_head`` on the last positions, the argmax and the advance of positions and context lengths
-- is captured once as a HIP graph and replayed for the remaining steps, so the step costs the
GPU time of its kernels and not their host launch overhead.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import torch

__all__ = ["GenerationResult", "GreedyGenerator"]


@dataclass
class GenerationResult:
    tokens: torch.Tensor          # [seq, steps] generated ids (the first comes from the prefill)
    prefill_seconds: float
    decode_seconds: float         # steps 2 .. steps-1 (step 1 runs eagerly and is then captured)
    prefill_logits: torch.Tensor  # [seq, vocab] last-position logits of the prefill

    @property
    def decode_tokens_per_second(self) -> float:
        seqs, steps = self.tokens.shape
        return seqs * (steps - 2) / self.decode_seconds if steps > 2 and self.decode_seconds > 0 else 0.0


def _argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The greedy choice of each row: the argmax kernel on HIP devices, torch elsewhere; into
    ``out`` (int64 [rows]) when given."""
    if logits.is_cuda and logits.dim() == 2 and logits.dtype in (torch.float32, torch.float16, torch.bfloat16):
        from llmopt.kernels import ops

        return ops.argmax_rows(logits, out=out)
    if out is None:
        return logits.argmax(-1)
    return torch.argmax(logits, -1, out=out)


class GreedyGenerator:
    """Greedy decoding of a batch of equal-length prompts with ``model``.

    Args:
        model: a :class:`DecoderOnlyModel` (any device).
        block_size: cache block size in tokens.
        cache_dtype: KV cache dtype (default: the embedding's dtype).
        use_graph: capture the decode step as a HIP graph (HIP devices only).
    """

    def __init__(self, model: torch.nn.Module, block_size: int = 16, cache_dtype: torch.dtype | None = None,
                 use_graph: bool = True) -> None:
        self.model = model
        self.block_size = block_size
        weight = model.embed_tokens.weight
        self.device = weight.device
        self.cache_dtype = cache_dtype or weight.dtype
        self.use_graph = use_graph and self.device.type == "cuda"

    def _sync(self) -> None:
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)

    @torch.no_grad()
    def generate(self, prompts: torch.Tensor, steps: int, forced: torch.Tensor | None = None) -> GenerationResult:
        """Generate ``steps`` tokens per prompt (``prompts [seq, prompt_len]``). With ``forced
        [seq, steps]`` the step inputs are those tokens instead of the argmax (teacher forcing);
        ``tokens`` then still holds the argmax of every step."""
        if steps < 1:
            raise ValueError("steps must be >= 1")
        dev = self.device
        seqs, plen = int(prompts.shape[0]), int(prompts.shape[1])
        per_seq = -(-(plen + steps) // self.block_size)
        cache = self.model.allocate_cache(seqs * per_seq, self.block_size, self.cache_dtype, dev)
        table = torch.arange(seqs * per_seq, dtype=torch.int32, device=dev).view(seqs, per_seq)
        out = torch.empty(seqs, steps, dtype=torch.long, device=dev)

        # ---- prefill ----
        ids = prompts.to(dev).reshape(-1)
        pos = torch.arange(plen, device=dev).repeat(seqs)
        lens = torch.full((seqs,), plen, dtype=torch.int32, device=dev)
        self._sync()
        t0 = time.perf_counter()
        logits = self.model(ids, pos, cache=cache, block_ids=table, context_lens=lens,
                            token_offsets=torch.zeros(seqs, dtype=torch.int32, device=dev), q_len=plen,
                            last_only=True).last_logits()
        out[:, 0] = _argmax(logits)
        self._sync()
        prefill_s = time.perf_counter() - t0
        prefill_logits = logits.float()

        # ---- decode: static buffers advanced in place ----
        tok = (forced[:, 0].to(dev) if forced is not None else out[:, 0]).contiguous().clone()
        pos = torch.full((seqs,), plen, dtype=torch.long, device=dev)
        lens = torch.full((seqs,), plen + 1, dtype=torch.int32, device=dev)
        nxt = torch.empty(seqs, dtype=torch.long, device=dev)

        # Without teacher forcing the step's argmax is the next step's input: written straight
        # into tok (the embedding gather has read tok before the argmax writes it).
        sink = nxt if forced is not None else tok

        def step() -> None:
            lg = self.model(tok, pos, cache=cache, block_ids=table, context_lens=lens, q_len=1,
                            last_only=True).last_logits()
            _argmax(lg, out=sink)
            pos.add_(1)
            lens.add_(1)

        def feed(i: int) -> None:  # after step i: record its token, set the next input
            out[:, i].copy_(sink)
            if forced is not None:
                tok.copy_(forced[:, i].to(dev))

        if steps > 1:
            step()
            feed(1)
        graph = None
        if self.use_graph and steps > 2:
            side = torch.cuda.Stream(dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side), torch.cuda.graph(graph, stream=side):
                step()
            torch.cuda.current_stream(dev).wait_stream(side)
        self._sync()
        t0 = time.perf_counter()
        for i in range(2, steps):
            if graph is not None:
                graph.replay()
            else:
                step()
            feed(i)
        self._sync()
        decode_s = time.perf_counter() - t0
        return GenerationResult(tokens=out, prefill_seconds=prefill_s, decode_seconds=decode_s,
                                prefill_logits=prefill_logits)

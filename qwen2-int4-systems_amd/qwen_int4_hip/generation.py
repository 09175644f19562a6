"""Cached greedy generation over the HIP W4G64 model.

``CachedGenerationState`` and ``greedy_generate_cached`` restate
src/qwen_int4/generation.py:10-111 (prefill, greedy decode with the growing
per-layer cache, request selection, close).  ``StaticGreedyDecoder`` is the
serving form of the same loop for a batch of unpadded prompts of one length:
the cache is preallocated, each decode step has fixed shapes and runs as one
replay of a HIP graph captured after a warm-up step.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .decode import FusedDecodeStep, FusedPrefill


@dataclass
class CachedGenerationState:
    """Owned KV cache and mask state for one left-padded generation batch."""

    model: torch.nn.Module
    generated_ids: torch.Tensor
    attention_mask: torch.Tensor
    logits: torch.Tensor
    past_key_values: tuple
    active: bool = True

    def _require_active(self) -> None:
        if not self.active:
            raise RuntimeError("cached generation state is closed")

    @classmethod
    def prefill(cls, model, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None):
        if input_ids.ndim != 2 or input_ids.shape[1] == 0:
            raise ValueError("input_ids must have shape [batch, non_empty_sequence]")
        if attention_mask is None:
            attention_mask = torch.ones_like(input_ids, dtype=torch.bool)
        if attention_mask.shape != input_ids.shape:
            raise ValueError("attention_mask must have the same shape as input_ids")
        mask = attention_mask.to(dtype=torch.bool)
        # left padding only: every row is some padding followed by a non-empty valid run
        valid = mask.long()
        first = torch.where(mask.any(dim=1), valid.argmax(dim=1), torch.full_like(valid[:, 0], mask.shape[1]))
        tail_valid = torch.arange(mask.shape[1], device=mask.device).view(1, -1) >= first.view(-1, 1)
        if bool((first >= mask.shape[1]).any()) or not bool(torch.equal(tail_valid, mask)):
            raise ValueError("cached batching supports only non-empty left-padded attention masks")
        with torch.inference_mode():
            logits, cache = model(input_ids, attention_mask=mask, use_cache=True)
        if not isinstance(cache, tuple):
            raise RuntimeError("cache-enabled model did not return per-layer key/value tensors")
        return cls(model, input_ids, mask, logits, cache)

    def next_greedy_tokens(self) -> torch.Tensor:
        self._require_active()
        return self.logits[:, -1].argmax(dim=-1, keepdim=True)

    def decode(self, next_tokens: torch.Tensor) -> torch.Tensor:
        self._require_active()
        if next_tokens.ndim != 2 or next_tokens.shape != (self.generated_ids.shape[0], 1):
            raise ValueError("next_tokens must have shape [batch, 1]")
        with torch.inference_mode():
            self.generated_ids = torch.cat((self.generated_ids, next_tokens), dim=1)
            self.attention_mask = torch.cat((self.attention_mask, torch.ones_like(next_tokens, dtype=torch.bool)),
                                            dim=1)
            self.logits, self.past_key_values = self.model(next_tokens, attention_mask=self.attention_mask,
                                                           past_key_values=self.past_key_values, use_cache=True)
        return self.logits

    def select_requests(self, indices) -> None:
        """Reorder or remove requests while preserving cache ownership."""
        self._require_active()
        selected = torch.as_tensor(indices, dtype=torch.long, device=self.generated_ids.device)
        if selected.ndim != 1 or selected.numel() == 0:
            raise ValueError("request indices must be a non-empty one-dimensional sequence")
        batch = self.generated_ids.shape[0]
        if int(selected.min()) < 0 or int(selected.max()) >= batch:
            raise IndexError("request index is outside the cached batch")
        if selected.unique().numel() != selected.numel():
            raise ValueError("duplicate request indices require explicit beam-cache semantics")
        self.generated_ids = self.generated_ids.index_select(0, selected)
        self.attention_mask = self.attention_mask.index_select(0, selected)
        self.logits = self.logits.index_select(0, selected)
        self.past_key_values = tuple((k.index_select(0, selected), v.index_select(0, selected))
                                     for k, v in self.past_key_values)

    def close(self) -> None:
        """Release owned cache tensors and make further use fail closed."""
        self.past_key_values = ()
        self.logits = torch.empty(0, device=self.generated_ids.device)
        self.active = False


def greedy_generate_cached(model, input_ids: torch.Tensor, *, max_new_tokens: int,
                           attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """One prefill, then ``max_new_tokens`` cached greedy decode steps."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative")
    state = CachedGenerationState.prefill(model, input_ids, attention_mask)
    for _ in range(max_new_tokens):
        state.decode(state.next_greedy_tokens())
    return state.generated_ids


class StaticGreedyDecoder:
    """Greedy decoding of ``batch`` unpadded prompts of one length with a
    preallocated cache of ``max_length`` positions.  The prompt runs as
    ``decode.FusedPrefill`` and every decode step is one HIP graph replay
    (``use_graph``) of ``decode.FusedDecodeStep``; with ``fused=False``, the
    module-level forward and ``model.decode_static`` instead."""

    def __init__(self, model, batch: int, max_length: int, *, use_graph: bool = True, fused: bool = True) -> None:
        self.model = model
        self.fused = FusedDecodeStep(model, batch, max_length) if fused else None
        self.fused_prefill = FusedPrefill(model) if fused else None
        self.batch = batch
        self.max_length = max_length
        device = model.lm_head.weight.device
        self.caches = model.new_static_cache(batch, max_length, device)
        self.token = torch.zeros((batch, 1), dtype=torch.long, device=device)
        self.position = torch.zeros(1, dtype=torch.long, device=device)
        self.use_graph = use_graph
        self.graph = None
        self._stream = None
        self.logits = None
        self.length = 0

    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Prompt logits [B, T, V]; fills cache positions [0, T)."""
        batch, length = input_ids.shape
        if batch != self.batch or length >= self.max_length:
            raise ValueError("prompt batch or length does not fit this decoder")
        with torch.inference_mode():
            if self.fused_prefill is not None:
                logits = self.fused_prefill(input_ids, self.caches)
            else:
                logits, caches = self.model(input_ids, use_cache=True)
                for (ks, vs), (k, v) in zip(self.caches, caches):
                    ks[:, :, :length].copy_(k)
                    vs[:, :, :length].copy_(v)
        self.length = length
        self.token.copy_(logits[:, -1].argmax(dim=-1, keepdim=True))
        return logits

    def _run(self, next_token: torch.Tensor | None) -> torch.Tensor:
        """One decode step; the fused step also writes the greedy choice into
        ``next_token`` (the module path leaves that to ``step``)."""
        if self.fused is not None:
            return self.fused(self.token, self.position, self.caches, next_token)
        return self.model.decode_static(self.token, self.position, self.caches)

    def step(self, token: torch.Tensor | None = None) -> torch.Tensor:
        """Decode the pending token -- the previous step's greedy choice, or
        ``token`` [B, 1] when given -- at the next position; returns its
        logits [B, 1, V] and picks the next greedy token."""
        if self.length >= self.max_length:
            raise RuntimeError("static cache is full")
        if token is not None:
            self.token.copy_(token)
        self.position.fill_(self.length)
        fused = self.fused is not None
        with torch.inference_mode():
            if not self.use_graph:
                self.logits = self._run(self.token if fused else None)
            elif self.graph is None:
                # the capture stream lives as long as the graph: its workspace is keyed by it
                self._stream = stream = torch.cuda.Stream()
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    # warm-up outside capture (allocates workspaces); its greedy
                    # choice goes to a scratch tensor so the replay below reads
                    # the same input token
                    self._run(torch.empty_like(self.token) if fused else None)
                torch.cuda.current_stream().wait_stream(stream)
                torch.cuda.synchronize()
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph, stream=stream):  # same stream: same workspaces
                    self.logits = self._run(self.token if fused else None)
                self.graph.replay()
            else:
                self.graph.replay()
            self.length += 1
            if not fused:
                self.token.copy_(self.logits[:, -1].argmax(dim=-1, keepdim=True))
        return self.logits

    def generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Prompt plus ``max_new_tokens`` greedy tokens [B, T + max_new_tokens]."""
        self.prefill(input_ids)
        out = [input_ids, self.token.clone()]
        for _ in range(max_new_tokens - 1):
            self.step()
            out.append(self.token.clone())
        return torch.cat(out, dim=1)[:, : input_ids.shape[1] + max_new_tokens]

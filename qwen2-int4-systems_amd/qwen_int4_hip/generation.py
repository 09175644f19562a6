"""Cached greedy generation over the HIP W4G64 model.

``CachedGenerationState`` and ``greedy_generate_cached`` provide the
reference's cached-generation interface (src/qwen_int4/generation.py:10-115:
the same names, attributes, arguments, exception types and the message
fragments its tests match): one prefill of a left-padded batch, then one
cached greedy step at a time, with request selection and an explicit close.
``StaticGreedyDecoder`` is the serving form of the same loop for a batch of
unpadded prompts of one length: the cache is preallocated, each decode step
has fixed shapes and runs as one replay of a HIP graph captured after a
warm-up step.
"""

from __future__ import annotations

import torch

from .decode import FusedDecodeStep, FusedPrefill, check_token_range


def _is_left_padded(mask: torch.Tensor) -> bool:
    """Every row is zero or more padding positions followed by a non-empty run
    of valid ones: along a row the mask never falls from valid to padding,
    and its last position is valid."""
    m = mask.to(torch.int8)
    never_falls = bool((m[:, 1:] >= m[:, :-1]).all()) if m.shape[1] > 1 else True
    return never_falls and bool(m[:, -1].all())


class CachedGenerationState:
    """A left-padded batch under cached greedy decoding.

    Holds the model, every token so far (``generated_ids``), the attention
    mask over them, the logits of the last forward and the per-layer
    key/value caches, which it owns: ``select_requests`` reorders or drops
    rows of all of them together, and ``close`` releases the caches, after
    which every use raises."""

    def __init__(self, model, generated_ids: torch.Tensor, attention_mask: torch.Tensor, logits: torch.Tensor,
                 past_key_values: tuple, active: bool = True) -> None:
        self.model = model
        self.generated_ids = generated_ids
        self.attention_mask = attention_mask
        self.logits = logits
        self.past_key_values = past_key_values
        self.active = active

    @classmethod
    def prefill(cls, model, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None):
        """Run the prompt batch once with the cache enabled."""
        if input_ids.ndim != 2 or input_ids.shape[1] == 0:
            raise ValueError("input_ids must have shape [batch, non_empty_sequence]")
        mask = torch.ones_like(input_ids, dtype=torch.bool) if attention_mask is None else attention_mask
        if mask.shape != input_ids.shape:
            raise ValueError("attention_mask must have the same shape as input_ids")
        mask = mask.to(dtype=torch.bool)
        if not _is_left_padded(mask):
            raise ValueError("cached batching supports only non-empty left-padded attention masks")
        with torch.inference_mode():
            logits, caches = model(input_ids, attention_mask=mask, use_cache=True)
        if not isinstance(caches, tuple):
            raise RuntimeError("cache-enabled model did not return per-layer key/value tensors")
        return cls(model, input_ids, mask, logits, caches)

    def _check_open(self) -> None:
        if not self.active:
            raise RuntimeError("cached generation state is closed")

    def next_greedy_tokens(self) -> torch.Tensor:
        """[batch, 1]: the argmax of each row's last logits."""
        self._check_open()
        return self.logits[:, -1].argmax(dim=-1, keepdim=True)

    def decode(self, next_tokens: torch.Tensor) -> torch.Tensor:
        """Append one token per row and run it against the cache; returns the
        new logits [batch, 1, vocab]."""
        self._check_open()
        if next_tokens.ndim != 2 or next_tokens.shape != (self.generated_ids.shape[0], 1):
            raise ValueError("next_tokens must have shape [batch, 1]")
        grown = torch.cat((self.attention_mask, torch.ones_like(next_tokens, dtype=torch.bool)), dim=1)
        with torch.inference_mode():
            logits, caches = self.model(next_tokens, attention_mask=grown, past_key_values=self.past_key_values,
                                        use_cache=True)
        self.generated_ids = torch.cat((self.generated_ids, next_tokens), dim=1)
        self.attention_mask, self.logits, self.past_key_values = grown, logits, caches
        return self.logits

    def select_requests(self, indices) -> None:
        """Keep only the rows ``indices`` (in that order), in every owned tensor."""
        self._check_open()
        rows = torch.as_tensor(indices, dtype=torch.long, device=self.generated_ids.device)
        if rows.ndim != 1 or rows.numel() == 0:
            raise ValueError("request indices must be a non-empty one-dimensional sequence")
        lo, hi = int(rows.min()), int(rows.max())
        if lo < 0 or hi >= self.generated_ids.shape[0]:
            raise IndexError("request index is outside the cached batch")
        if rows.unique().numel() != rows.numel():
            raise ValueError("duplicate request indices require explicit beam-cache semantics")

        def pick(t: torch.Tensor) -> torch.Tensor:
            return t.index_select(0, rows)

        self.generated_ids, self.attention_mask, self.logits = map(pick, (self.generated_ids, self.attention_mask,
                                                                          self.logits))
        self.past_key_values = tuple(tuple(map(pick, pair)) for pair in self.past_key_values)

    def close(self) -> None:
        """Drop the caches and logits; later calls raise RuntimeError."""
        self.past_key_values = ()
        self.logits = torch.empty(0, device=self.generated_ids.device)
        self.active = False


def greedy_generate_cached(model, input_ids: torch.Tensor, *, max_new_tokens: int,
                           attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Prompt plus ``max_new_tokens`` greedy tokens per row, [batch, T + max_new_tokens]."""
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
        self.vocab = model.model.embed_tokens.weight.shape[0]
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
        check_token_range(input_ids, self.vocab)
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
            if not isinstance(token, torch.Tensor) or tuple(token.shape) != tuple(self.token.shape):
                raise ValueError(f"token must have shape {list(self.token.shape)}")
            check_token_range(token, self.vocab)
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

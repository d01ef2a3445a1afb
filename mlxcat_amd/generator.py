"""Host-side mirror of mlxcat's generator / scheduler interface over the HIP step.

Names, argument meaning and error behaviour follow the reference (local-ai-cat/mlxcat):
  SpeculativeDecodingConfiguration  Sources/MLXCat/TrackB/BatchGenerator.swift:10-29
  SpeculativeDecodingStats          BatchGenerator.swift:31-38
  FinishReason / Response           BatchGenerator.swift:40-66
  ContinuousBatchGenerator          BatchGenerator.swift:144-600 (insert/remove/next)
  Scheduler.submit / step           Sources/MLXCat/TrackB/Scheduler.swift:310-434
Every decode step runs on the GPU through mc_step (propose, verify forward, accept,
rollback, history append, finish detection) with one host synchronisation.
"""
from __future__ import annotations

import enum
from collections import deque
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L


@dataclass
class SpeculativeDecodingConfiguration:
    enabled: bool = False
    max_proposal_tokens: int = 4
    max_suffix_tokens: int = 16
    min_context_tokens: int = 8
    # beyond the reference: acceptance rule and the reference's single-row / greedy gates
    acceptance: int = L.ACCEPT_ALL_OR_NOTHING
    single_row_only: bool = True
    greedy_only: bool = True

    def __post_init__(self):  # the Swift initialiser's clamps (BatchGenerator.swift:23-25)
        self.max_proposal_tokens = max(0, self.max_proposal_tokens)
        self.max_suffix_tokens = max(1, self.max_suffix_tokens)
        self.min_context_tokens = max(2, self.min_context_tokens)

    @classmethod
    def disabled(cls) -> "SpeculativeDecodingConfiguration":
        return cls(enabled=False)

    @classmethod
    def batched(cls, k: int, max_suffix: int = 16, min_context: int = 8) -> "SpeculativeDecodingConfiguration":
        """n-gram speculation for every row, prefix acceptance, sampled rows allowed."""
        return cls(enabled=True, max_proposal_tokens=k, max_suffix_tokens=max_suffix, min_context_tokens=min_context,
                   acceptance=L.ACCEPT_PREFIX, single_row_only=False, greedy_only=False)

    def as_c(self) -> dict:
        return dict(enabled=int(self.enabled), max_proposal_tokens=self.max_proposal_tokens,
                    max_suffix_tokens=self.max_suffix_tokens, min_context_tokens=self.min_context_tokens,
                    acceptance=self.acceptance, single_row_only=int(self.single_row_only),
                    greedy_only=int(self.greedy_only))


@dataclass
class SpeculativeDecodingStats:
    proposed_token_count: int = 0
    accepted_token_count: int = 0
    proposal_batch_count: int = 0
    rejected_batch_count: int = 0


class FinishReason(enum.Enum):
    STOP = "stop"
    LENGTH = "length"
    CANCELLED = "cancelled"
    FAILED = "failed"


@dataclass
class Response:
    uid: str
    token: int
    finish_reason: FinishReason | None = None


@dataclass
class SamplingParameters:
    """SamplingParameters (Sampling.swift:139-194) minus the grammar, XTC and thinking-budget
    options, which the step does not implement."""
    temperature: float = 0.0
    top_p: float = 0.0
    top_k: int = 0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    min_tokens: int = 0
    logit_bias: dict = field(default_factory=dict)
    seed: int | None = None
    eos_token_ids: tuple = ()
    tool_call_start_token_id: int | None = None

    def as_c(self) -> L.Sampling:
        return L.make_sampling(self.temperature, self.top_p, self.seed, tuple(self.eos_token_ids),
                               -1 if self.tool_call_start_token_id is None else self.tool_call_start_token_id,
                               top_k=self.top_k, min_p=self.min_p, repetition_penalty=self.repetition_penalty,
                               presence_penalty=self.presence_penalty, frequency_penalty=self.frequency_penalty,
                               min_tokens=self.min_tokens, logit_bias=self.logit_bias)


_FIN = {0: None, 1: FinishReason.STOP, 2: FinishReason.LENGTH}


class ContinuousBatchGenerator:
    def __init__(self, model: L.Model, max_rows: int, max_context: int,
                 speculative_decoding: SpeculativeDecodingConfiguration | None = None):
        self.model = model
        self.speculative_decoding = speculative_decoding or SpeculativeDecodingConfiguration()
        self.batch = L.Batch(model, max_rows, max_context, self.speculative_decoding.as_c())
        self.row_uid: list[str | None] = [None] * max_rows

    @property
    def is_empty(self) -> bool:
        return all(u is None for u in self.row_uid)

    @property
    def has_free_row(self) -> bool:
        return any(u is None for u in self.row_uid)

    def insert(self, uid: str, prompt, sampling: SamplingParameters, max_tokens: int) -> Response:
        """Prefill + first token; returns the first token's Response (finished rows are not kept)."""
        if uid in self.row_uid:
            raise ValueError(f"duplicate batch uid '{uid}'")  # BatchGenerator.swift:357
        row = self.row_uid.index(None)
        tok, fin = self.batch.insert(row, prompt, max_tokens, sampling.as_c())
        if fin == 0:
            self.row_uid[row] = uid
        return Response(uid, tok, _FIN[fin])

    def remove(self, uid: str) -> None:
        if uid in self.row_uid:
            r = self.row_uid.index(uid)
            self.batch.remove(r)
            self.row_uid[r] = None

    def next(self, forced_accept=None) -> list[Response]:
        """ContinuousBatchGenerator.next(): one speculative (or plain) step for every row."""
        if self.is_empty:
            return []
        toks, cnts, fins = self.batch.step(forced_accept)
        out: list[Response] = []
        for r, uid in enumerate(self.row_uid):
            if uid is None:
                continue
            n = int(cnts[r])
            for j in range(n):
                fin = _FIN[int(fins[r])] if j == n - 1 else None
                out.append(Response(uid, int(toks[r, j]), fin))
            if fins[r]:
                self.row_uid[r] = None
        return out

    @property
    def speculation_stats(self) -> SpeculativeDecodingStats:
        s = self.batch.stats()
        return SpeculativeDecodingStats(s["proposed"], s["accepted"], s["proposal_batches"], s["rejected_batches"])


@dataclass
class Request:
    uid: str
    prompt: list
    max_tokens: int
    sampling: SamplingParameters = field(default_factory=SamplingParameters)


class Scheduler:
    """Scheduler.submit / step / isIdle over one ContinuousBatchGenerator."""

    def __init__(self, model: L.Model, max_concurrent_requests: int, max_context: int,
                 speculative_decoding: SpeculativeDecodingConfiguration | None = None):
        self.generator = ContinuousBatchGenerator(model, max_concurrent_requests, max_context, speculative_decoding)
        self.waiting: deque[Request] = deque()

    def submit(self, request: Request) -> None:
        self.waiting.append(request)

    @property
    def is_idle(self) -> bool:
        return not self.waiting and self.generator.is_empty

    def _admit(self) -> list[Response]:
        out = []
        while self.waiting and self.generator.has_free_row:
            rq = self.waiting.popleft()
            out.append(self.generator.insert(rq.uid, rq.prompt, rq.sampling, rq.max_tokens))
        return out

    def step(self) -> list[Response]:
        was_empty = self.generator.is_empty
        processed = self._admit()
        if self.generator.is_empty:
            return processed
        if was_empty and any(r.token >= 0 for r in processed):  # Scheduler.swift:350-353
            return processed
        processed.extend(self.generator.next())
        if self.generator.is_empty:
            processed.extend(self._admit())
        return processed

    @property
    def speculative_decoding_stats(self) -> SpeculativeDecodingStats:
        return self.generator.speculation_stats


def generate(scheduler: Scheduler, requests: list[Request]) -> dict[str, list[int]]:
    """MLXCatEngine.generate: submit everything, step until idle, collect tokens per uid."""
    for rq in requests:
        scheduler.submit(rq)
    toks: dict[str, list[int]] = {rq.uid: [] for rq in requests}
    while not scheduler.is_idle:
        for r in scheduler.step():
            if r.token >= 0:
                toks[r.uid].append(r.token)
    return toks


def as_numpy(tokens) -> np.ndarray:
    return np.asarray(tokens, dtype=np.int32)

"""CPU restatement of flarellm's Generator loop (flare-core/src/generate.rs).

TEST INFRASTRUCTURE ONLY: the checker for the product's generation loop
(flarellm_amd/csrc/generate.cpp).  The model is any object with
forward_greedy(token, pos) -> (token, value) and forward_logits(token, pos)
-> logits, normally oracle.OracleModel.  Prefill is sequential forward steps
over the prompt: Model::forward_prefill is asserted equal to them by the
reference's own test_batched_prefill_matches_sequential (generate.rs:657).
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import oracle as O

NGRAM_MAX_ENTRIES = 10_000  # generate.rs:7
MAX_DRAFT_TOKENS = 5        # generate.rs:10
NGRAM_SIZES = (2, 3, 4)     # generate.rs:13


class NgramCache:
    """generate.rs:37-103."""

    def __init__(self):
        self.table: dict[tuple, list] = {}
        self.total_entries = 0

    def record(self, tokens):  # generate.rs:55-75
        for n in NGRAM_SIZES:
            if len(tokens) < n + 1:
                continue
            start = len(tokens) - n - 1
            self.table.setdefault(tuple(tokens[start:start + n]), []).append(tokens[-1])
            self.total_entries += 1
        if self.total_entries > NGRAM_MAX_ENTRIES:
            self.evict()

    def record_all(self, tokens):  # record_prompt_ngrams, generate.rs:166-182
        for n in NGRAM_SIZES:
            if len(tokens) < n + 1:
                continue
            for i in range(len(tokens) - n):
                self.table.setdefault(tuple(tokens[i:i + n]), []).append(tokens[i + n])
                self.total_entries += 1
        if self.total_entries > NGRAM_MAX_ENTRIES:
            self.evict()

    def lookup(self, tokens):  # lookup_drafts, generate.rs:79-92
        for n in reversed(NGRAM_SIZES):
            if len(tokens) < n:
                continue
            cont = self.table.get(tuple(tokens[len(tokens) - n:]))
            if cont is not None:
                return list(cont[max(0, len(cont) - MAX_DRAFT_TOKENS):])
        return []

    def evict(self):  # generate.rs:96-102
        self.table.clear()
        self.total_entries = 0


@dataclass
class Params:
    """SamplingParams (sampling.rs:19-70) without self-speculation."""
    temperature: float = 0.7
    top_p: float = 0.9
    top_k: int = 40
    repeat_penalty: float = 1.1
    min_p: float = 0.0
    speculative: bool = True


@dataclass
class Stats:
    attempts: int = 0
    drafted: int = 0
    accepted: int = 0


@dataclass
class Generator:
    model: object
    params: Params
    tokens: list = field(default_factory=list)
    position: int = 0
    ngram: NgramCache = field(default_factory=NgramCache)
    stats: Stats = field(default_factory=Stats)

    def speculative(self):  # generate.rs:128-130
        return self.params.speculative and self.params.temperature == 0.0

    def prefill(self, prompt):  # generate.rs:139-163
        if not len(prompt):
            return
        for i, t in enumerate(prompt):
            self.model.forward_greedy(int(t), self.position + i)
        self.tokens.extend(int(t) for t in prompt)
        self.position += len(prompt)
        if self.speculative():
            self.ngram.record_all(self.tokens)

    def _forward_next(self, u):
        last = self.tokens[-1] if self.tokens else 0
        p = self.params
        if p.temperature == 0.0 and p.repeat_penalty == 1.0:
            return self.model.forward_greedy(last, self.position)[0]
        logits = self.model.forward_logits(last, self.position)
        return O.sample(logits, p.temperature, p.top_p, p.top_k, p.repeat_penalty, p.min_p, self.tokens, u)

    def _push(self, t):
        self.tokens.append(int(t))
        self.position += 1
        if self.speculative():
            self.ngram.record(self.tokens)

    def step(self, u):  # generate.rs:186-238
        t = self._forward_next(u)
        self._push(t)
        return t

    def speculative_step(self):  # generate.rs:244-312 (sequential verification)
        drafts = self.ngram.lookup(self.tokens)
        if not drafts:
            return []
        self.stats.attempts += 1
        self.stats.drafted += len(drafts)
        out = []
        for d in drafts:
            v = self._forward_next(0.0)
            self._push(v)
            out.append(v)
            if v != d:
                break
            self.stats.accepted += 1
        return out

    def generate(self, prompt, max_tokens, eos=None, rng=lambda: 0.5, on_token=lambda t, s: True):
        """generate.rs:409-531 (n-gram speculation only)."""
        self.prefill(prompt)
        gen, step = [], 0
        spec = self.speculative()
        while step < max_tokens:
            if spec and step > 0:
                res = self.speculative_step()
                if res:
                    stop = False
                    for t in res:
                        gen.append(t)
                        if eos is not None and t == eos:
                            stop = True
                            break
                        if not on_token(t, step):
                            stop = True
                            break
                        step += 1
                        if step >= max_tokens:
                            stop = True
                            break
                    if stop:
                        break
                    continue
            t = self.step(rng())
            gen.append(t)
            if eos is not None and t == eos:
                break
            if not on_token(t, step):
                break
            step += 1
        return gen

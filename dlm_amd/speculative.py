"""Speculative decoding over the paged path: a draft proposes gamma tokens, the
target verifies all of them in ONE batched pass, rejected tokens are rolled
back in the block-table books.

Mirrors dlm's ``SpeculativeSession`` / ``SpeculativeDecoder``
(src/speculative.rs:56-185) by name and by the greedy acceptance rule
(:145-185): accept each draft token while it equals the target's greedy
choice; at the first mismatch emit the target's token and end the round; if
all ``gamma`` are accepted, emit the target's bonus token unless that would
exceed the round's budget.  The output is exactly target-greedy decoding
(tests/speculative.rs:77-171).

What differs is the cost, which is the point of the paged path: dlm re-runs
the whole sequence through the target once per verified position
(``target_next``, speculative.rs:133-141).  Here every generator keeps its
KV in paged pools; a round runs ``[last, d1 .. d_gamma]`` through every
target layer at once (``dlmk_verify_block_paged``: weights read once per
round, gamma + 1 causal queries over the pools) and then truncates the books
to the accepted prefix (``PagedKvCache.truncate_sequence``).  The draft's
cache is truncated the same way.

Invariant between rounds, for both generators: the sequence's cache holds
the K/V of every token of ``seq`` but the last one.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import numpy as np
import torch

from .block import PagedGpuKernel
from .cache import KvCacheConfig, PagedKvCache
from .ops import BLOCK_SIZE


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """rmsnorm (src/forward/cpu.rs:934-942), rows of x, f32."""
    x = np.asarray(x, np.float32)
    mean_sq = (x * x).sum(axis=-1, keepdims=True, dtype=np.float32) / np.float32(x.shape[-1])
    inv = np.float32(1.0) / np.sqrt(mean_sq + np.float32(eps))
    return (x * inv * np.asarray(weight, np.float32)).astype(np.float32)


def argmax(logits: np.ndarray) -> int:
    """Greedy pick, first maximum wins; NaN never wins (src/generate.rs:21-31)."""
    v = np.where(np.isnan(logits), -np.inf, logits)
    return int(np.argmax(v))


class PagedGenerator:
    """``Generator`` (src/generate.rs:236-300) over the paged GPU path: token
    embedding, the decode blocks of a ``PagedGpuKernel`` over this
    generator's own paged pools and books, final rmsnorm and the LM head.
    Embedding, final norm and LM head run on the host, as dlm's do
    (generate.rs:315-331); the hidden states come back from the device."""

    def __init__(self, kernel: PagedGpuKernel, embedding: np.ndarray, final_norm: np.ndarray,
                 lm_head: np.ndarray, vocab_size: int, rms_eps: float, total_blocks: int,
                 seed: int = 0):
        c = kernel.cfg
        self.kernel = kernel
        self.vocab_size = vocab_size
        self.hidden_size = c.hidden_size
        self.embedding = np.asarray(embedding, np.float32).reshape(vocab_size, c.hidden_size)
        self.final_norm = np.asarray(final_norm, np.float32)
        self.lm_head = np.asarray(lm_head, np.float32).reshape(vocab_size, c.hidden_size)
        self.rms_eps = rms_eps
        self.cache = PagedKvCache.with_seeded_shuffle(
            KvCacheConfig(kernel.num_layers(), c.num_kv_heads, c.head_dim, BLOCK_SIZE),
            total_blocks, seed)
        shape = (total_blocks, c.num_kv_heads, c.head_dim * BLOCK_SIZE)
        dev = kernel.device
        self.pools = [(torch.zeros(shape, dtype=torch.float32, device=dev),
                       torch.zeros(shape, dtype=torch.float32, device=dev))
                      for _ in range(kernel.num_layers())]
        self._next_seq = 1

    def new_sequence(self) -> int:
        s = self._next_seq
        self._next_seq += 1
        return s

    def embed(self, tokens: Sequence[int]) -> np.ndarray:
        ids = np.asarray(tokens, np.int64)
        if ids.size and (ids.min() < 0 or ids.max() >= self.vocab_size):
            raise ValueError(f"token out of vocab range {self.vocab_size}")
        return self.embedding[ids]

    def logits(self, hidden: np.ndarray) -> np.ndarray:
        """final rmsnorm + LM head (generate.rs:328-331), rows of hidden."""
        normed = rmsnorm(hidden, self.final_norm, self.rms_eps)
        return (normed[..., None, :] * self.lm_head).sum(axis=-1, dtype=np.float32)

    def forward(self, seq_id: int, tokens: Sequence[int]) -> np.ndarray:
        """Run ``tokens`` through every layer at the sequence's next positions
        (reserved in the books first, as decode_token does); returns their
        final hidden states [n, hidden].  One token uses the decode block,
        several the batched verify block."""
        n = len(tokens)
        start = self.cache.sequence_len(seq_id)
        self.cache.append_tokens(seq_id, n)
        tables, _ = self.cache.block_tables([seq_id], self.kernel.max_blocks)
        dev = self.kernel.device
        table = torch.from_numpy(np.ascontiguousarray(tables[0], np.int32)).to(dev)
        h = torch.from_numpy(np.ascontiguousarray(self.embed(tokens))).to(dev)
        for layer in range(self.kernel.num_layers()):
            if n == 1:
                self.kernel.run_block(layer, h[0], self.pools[layer], table, start, start)
            else:
                self.kernel.run_tokens(layer, h, self.pools[layer], table, start, start)
        return h.cpu().numpy()

    def prefill(self, seq_id: int, tokens: Sequence[int], chunk: int = 8) -> None:
        for i in range(0, len(tokens), chunk):
            self.forward(seq_id, tokens[i:i + chunk])

    def generate(self, prompt: Sequence[int], max_new_tokens: int) -> List[int]:
        """Plain greedy decoding (Generator::generate, generate.rs:338-380,
        greedy sampler, no EOS): the reference speculative output must equal."""
        if not prompt:
            raise ValueError("prompt must be non-empty")
        s = self.new_sequence()
        try:
            self.prefill(s, prompt[:-1])
            out: List[int] = []
            last = prompt[-1]
            for _ in range(max_new_tokens):
                last = argmax(self.logits(self.forward(s, [last]))[0])
                out.append(last)
            return out
        finally:
            self.cache.free_sequence(s)


class SpeculativeSession:
    """One draft-propose / batched target-verify round per ``step``
    (SpeculativeSession, src/speculative.rs:102-185)."""

    def __init__(self, target: PagedGenerator, draft: PagedGenerator, gamma: int,
                 prompt: Sequence[int]):
        if not prompt:
            raise ValueError("prompt must be non-empty")
        self.target, self.draft = target, draft
        self.gamma = max(int(gamma), 1)
        self.seq: List[int] = list(prompt)
        self.proposed = 0
        self.accepted = 0
        self.t_seq = target.new_sequence()
        self.d_seq = draft.new_sequence()
        # Both caches hold every token but the last.
        target.prefill(self.t_seq, self.seq[:-1])
        draft.prefill(self.d_seq, self.seq[:-1])

    def close(self) -> None:
        self.target.cache.free_sequence(self.t_seq)
        self.draft.cache.free_sequence(self.d_seq)

    def step(self, budget: int) -> List[int]:
        """Emit 1..=gamma+1 tokens (at most ``budget``), exactly the target's
        greedy continuation of the sequence."""
        if budget <= 0:
            return []
        gamma = min(self.gamma, budget)
        held = len(self.seq) - 1  # cached positions, both generators
        # Draft proposes gamma tokens, one decode step each.
        drafts: List[int] = []
        tok = self.seq[-1]
        for _ in range(gamma):
            tok = argmax(self.draft.logits(self.draft.forward(self.d_seq, [tok]))[0])
            drafts.append(tok)
        self.proposed += len(drafts)
        # Target verifies [last, d1 .. d_gamma] in one pass: row j is the
        # target's greedy choice after d_j (after `last` for j = 0).
        choice = [argmax(r) for r in
                  self.target.logits(self.target.forward(self.t_seq, [self.seq[-1]] + drafts))]
        emitted: List[int] = []
        all_accepted = True
        for j, dt in enumerate(drafts):
            if choice[j] == dt:
                emitted.append(dt)
                self.accepted += 1
            else:
                emitted.append(choice[j])  # the target's correction ends the round
                all_accepted = False
                break
        if all_accepted and len(emitted) < budget:
            emitted.append(choice[gamma])  # bonus token
        self.seq.extend(emitted)
        # Roll back to "every token but the last": the target ran gamma + 1
        # positions, the draft gamma.
        keep = held + len(emitted)
        self.target.cache.truncate_sequence(self.t_seq, keep)
        if keep <= held + gamma:
            self.draft.cache.truncate_sequence(self.d_seq, keep)
        else:  # the bonus round: the draft has not seen d_gamma yet
            self.draft.forward(self.d_seq, [drafts[-1]])
        return emitted


class SpeculativeDecoder:
    """``prompt -> tokens`` over ``SpeculativeSession`` (speculative.rs:56-93)."""

    def __init__(self, target: PagedGenerator, draft: PagedGenerator, gamma: int):
        self.target, self.draft, self.gamma = target, draft, max(int(gamma), 1)
        self.proposed = self.accepted = 0

    def generate(self, prompt: Sequence[int], max_new_tokens: int) -> List[int]:
        session = SpeculativeSession(self.target, self.draft, self.gamma, prompt)
        try:
            out: List[int] = []
            while len(out) < max_new_tokens:
                emitted = session.step(max_new_tokens - len(out))
                if not emitted:
                    break
                out.extend(emitted)
            self.proposed, self.accepted = session.proposed, session.accepted
            return out[:max_new_tokens]
        finally:
            session.close()

    def acceptance_rate(self) -> float:
        return 0.0 if self.proposed == 0 else self.accepted / self.proposed


class SpeculativeScheduler:
    """``BatchScheduler::with_speculative`` (src/batching.rs:189-401): at most
    ``max_batch`` requests in flight, each a ``SpeculativeSession`` advanced by
    one round per tick; a round's tokens are emitted in order and the request
    stops at its length cap or at an EOS token (inclusive), discarding the
    rest of that round, as plain decoding would have stopped there
    (batching.rs:337-378).  Finished requests release their blocks."""

    def __init__(self, target: PagedGenerator, draft: PagedGenerator, max_batch: int,
                 gamma: int):
        self.target, self.draft = target, draft
        self.max_batch = max(int(max_batch), 1)
        self.gamma = max(int(gamma), 1)
        self.pending: List[tuple] = []
        self.active: List[dict] = []
        self.proposed = self.accepted = 0

    def submit(self, req_id: int, prompt: Sequence[int], max_new_tokens: int,
               eos: Sequence[int] = ()) -> None:
        if not prompt:
            raise ValueError("prompt must be non-empty")
        self.pending.append((req_id, list(prompt), int(max_new_tokens), list(eos)))

    def speculative_stats(self):
        """(proposed, accepted) over every finished request."""
        return self.proposed, self.accepted

    def has_work(self) -> bool:
        return bool(self.pending or self.active)

    def _admit(self) -> List[int]:
        zero = []
        while len(self.active) < self.max_batch and self.pending:
            req_id, prompt, n, eos = self.pending.pop(0)
            if n == 0:
                zero.append(req_id)
                continue
            self.active.append({"id": req_id, "eos": eos, "remaining": n,
                                "session": SpeculativeSession(self.target, self.draft,
                                                              self.gamma, prompt)})
        return zero

    def step(self):
        """One tick: returns (produced [(id, token)], finished ids)."""
        finished = self._admit()
        produced = []
        still = []
        for a in self.active:
            s = a["session"]
            done = False
            for tok in s.step(a["remaining"]):
                produced.append((a["id"], tok))
                a["remaining"] -= 1
                if a["remaining"] == 0 or tok in a["eos"]:
                    done = True
                    break
            if done:
                self.proposed += s.proposed
                self.accepted += s.accepted
                s.close()
                finished.append(a["id"])
            else:
                still.append(a)
        self.active = still
        return produced, finished

    def run(self):
        """Ticks until every request completes: [(id, tokens)] in completion order."""
        outputs, results = {}, []
        while self.has_work():
            produced, finished = self.step()
            for req_id, tok in produced:
                outputs.setdefault(req_id, []).append(tok)
            for req_id in finished:
                results.append((req_id, outputs.pop(req_id, [])))
        return results

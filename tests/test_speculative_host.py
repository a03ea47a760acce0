"""Host logic of the speculative round (dlm_amd.speculative) on the CPU.

The generators here are stand-ins with the PagedGenerator surface whose
"model" is a hash of the cached token prefix: the hidden state of the token
at position p depends on the tokens the generator's books hold at positions
0..p.  A round that rolled the books back to the wrong length would shift
positions and change every later choice, so token equality with plain greedy
decoding (the property of tests/speculative.rs:77-171) checks the
propose / verify / accept / truncate bookkeeping, not only the acceptance
rule.  The accept rule and budget handling follow src/speculative.rs:145-185.
"""
import numpy as np
import pytest

from dlm_amd import KvCacheConfig, PagedKvCache
from dlm_amd.speculative import SpeculativeDecoder, SpeculativeSession, argmax, rmsnorm

VOCAB = 11


class HashGenerator:
    """PagedGenerator surface over a prefix-hash model; ``agree`` makes the
    draft copy the target's choice with that probability (per prefix)."""

    def __init__(self, seed, total_blocks=64, agree_with=None, agree=0.0):
        self.seed = seed
        self.cache = PagedKvCache.with_seeded_shuffle(KvCacheConfig(1, 1, 4, 16), total_blocks,
                                                      seed)
        self.hist = {}  # seq -> {position: token}, the "pools"
        self.agree_with, self.agree = agree_with, agree
        self._next = 1
        self.calls = []  # (seq, start, n) of every forward

    def new_sequence(self):
        s = self._next
        self._next += 1
        self.hist[s] = {}
        return s

    def next_token(self, prefix):
        h = hash((self.seed,) + tuple(prefix)) & 0xFFFFFFFF
        if self.agree_with is not None and (h % 1000) < self.agree * 1000:
            return self.agree_with.next_token(prefix)
        return h % VOCAB

    def forward(self, seq, tokens):
        start = self.cache.sequence_len(seq)
        self.cache.append_tokens(seq, len(tokens))
        self.calls.append((seq, start, len(tokens)))
        out = np.zeros((len(tokens), VOCAB), np.float32)
        for j, t in enumerate(tokens):
            self.hist[seq][start + j] = t
            prefix = [self.hist[seq][p] for p in range(start + j + 1)]
            out[j, self.next_token(prefix)] = 1.0
        return out

    def logits(self, hidden):
        return hidden

    def prefill(self, seq, tokens, chunk=8):
        for i in range(0, len(tokens), chunk):
            self.forward(seq, tokens[i:i + chunk])

    def greedy(self, prompt, n):
        seq, out = list(prompt), []
        for _ in range(n):
            seq.append(self.next_token(seq))
            out.append(seq[-1])
        return out


@pytest.mark.parametrize("gamma", [1, 2, 4, 7])
@pytest.mark.parametrize("agree", [0.0, 0.5, 0.9, 1.0])
def test_speculative_equals_target_greedy(gamma, agree):
    target = HashGenerator(1)
    draft = HashGenerator(2, agree_with=target, agree=agree)
    for prompt, n in (([1, 2, 3], 8), ([7], 5), ([4, 5], 40), (list(range(10)) * 3, 25)):
        dec = SpeculativeDecoder(target, draft, gamma)
        assert dec.generate(prompt, n) == target.greedy(prompt, n)
        assert dec.accepted <= dec.proposed
        if agree == 1.0:
            assert dec.accepted == dec.proposed and dec.acceptance_rate() == 1.0
    # Every session freed its sequences: the books are empty again.
    assert target.cache.num_sequences() == 0 and draft.cache.num_sequences() == 0
    assert target.cache.free_blocks() == target.cache.total_blocks()


def test_session_round_by_round_budget_and_invariant():
    """tests/speculative.rs:109-131: rounds capped by the tokens still wanted;
    between rounds both caches hold every token of the sequence but the last."""
    target = HashGenerator(1)
    draft = HashGenerator(2, agree_with=target, agree=0.6)
    prompt, n = [1, 2, 3], 30
    s = SpeculativeSession(target, draft, 4, prompt)
    out = []
    while len(out) < n:
        emitted = s.step(n - len(out))
        assert 1 <= len(emitted) <= min(5, n - len(out))
        out.extend(emitted)
        held = len(s.seq) - 1
        assert target.cache.sequence_len(s.t_seq) == held
        assert draft.cache.sequence_len(s.d_seq) == held
        # The cached tokens are exactly the sequence's (rolled back, not stale).
        assert [target.hist[s.t_seq][p] for p in range(held)] == s.seq[:-1]
        assert [draft.hist[s.d_seq][p] for p in range(held)] == s.seq[:-1]
    assert out == target.greedy(prompt, n)
    assert s.step(0) == []
    s.close()


def test_verify_is_one_batched_target_pass_per_round():
    """The target runs gamma + 1 tokens in one forward per round (dlm runs one
    full re-prefill per verified position)."""
    target = HashGenerator(1)
    draft = HashGenerator(2)  # disagrees: every round ends at its first token
    s = SpeculativeSession(target, draft, 4, [3, 1, 4, 1, 5])
    target.calls.clear()
    for _ in range(3):
        s.step(100)
    assert [c[2] for c in target.calls] == [5, 5, 5]
    s.close()


def test_rmsnorm_and_argmax_follow_the_reference():
    # cpu.rs:1289-1293: x=[3,4] -> [0.8485, 1.1314]
    np.testing.assert_allclose(rmsnorm(np.array([3.0, 4.0]), np.ones(2), 0.0),
                               [0.848528, 1.131371], atol=1e-4)
    # generate.rs:21-31: first maximum wins; NaN never wins; all -inf -> 0.
    assert argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert argmax(np.array([np.nan, 1.0, 0.5], np.float32)) == 1
    assert argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


def test_scheduler_matches_greedy_across_requests():
    """tests/speculative.rs:133-155: max_batch 2 forces staggered admission;
    every request equals its own target greedy; stats add up."""
    from dlm_amd.speculative import SpeculativeScheduler
    target = HashGenerator(1)
    draft = HashGenerator(2, agree_with=target, agree=0.7)
    reqs = [(1, [1, 2, 3], 7), (2, [7], 5), (3, [4, 5], 6), (4, [9, 9, 9, 9], 0)]
    sched = SpeculativeScheduler(target, draft, 2, 4)
    for rid, prompt, n in reqs:
        sched.submit(rid, prompt, n)
    results = dict(sched.run())
    assert set(results) == {1, 2, 3, 4}
    for rid, prompt, n in reqs:
        assert results[rid] == target.greedy(prompt, n), rid
    proposed, accepted = sched.speculative_stats()
    assert 0 < proposed and accepted <= proposed
    assert target.cache.num_sequences() == 0 and draft.cache.num_sequences() == 0


def test_scheduler_respects_eos():
    """tests/speculative.rs:157-171: stop at EOS (included) before the cap,
    matching plain decoding, even mid-round."""
    from dlm_amd.speculative import SpeculativeScheduler
    target = HashGenerator(1)
    draft = HashGenerator(1)  # identical draft: full rounds
    plain = target.greedy([1, 2], 10)
    eos = plain[2]  # first reached mid-way through the first 5-token round
    assert eos not in plain[:2]
    sched = SpeculativeScheduler(target, draft, 4, 4)
    sched.submit(1, [1, 2], 10, [eos])
    (rid, toks), = sched.run()
    assert rid == 1 and toks == plain[:3]
    assert target.cache.num_sequences() == 0

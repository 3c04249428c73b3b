"""Token-level view of a byte DFA (automaton.py of the reference): a token is
allowed from a state when its bytes never reach the dead state and end in a
state that can still reach an accepting state; EOS only from accepting
states."""

from __future__ import annotations

from .regex.compile import DFA
from .tokenizer import Vocabulary

DEAD = -1


class TokenDFA:
    def __init__(self, dfa: DFA, vocab: Vocabulary) -> None:
        self.dfa = dfa
        self.vocab = vocab
        self._live = dfa.live_states()
        self._step_cache: dict[tuple[int, int], int] = {}
        self._allowed_cache: dict[int, frozenset[int]] = {}

    @property
    def start(self) -> int:
        return self.dfa.start

    def is_accepting(self, state: int) -> bool:
        return state in self.dfa.accept

    def step(self, state: int, token_id: int) -> int:
        if token_id == self.vocab.eos_id:
            return state if self.is_accepting(state) else DEAD
        key = (state, token_id)
        hit = self._step_cache.get(key)
        if hit is None:
            cur = state
            for byte in self.vocab.token_bytes[token_id]:
                cur = self.dfa.step(cur, byte)
                if cur == self.dfa.dead:
                    cur = DEAD
                    break
            if cur != DEAD and cur not in self._live:
                cur = DEAD
            hit = self._step_cache[key] = cur
        return hit

    def allowed(self, state: int) -> frozenset[int]:
        hit = self._allowed_cache.get(state)
        if hit is None:
            ids = {t for t in range(self.vocab.size) if self.step(state, t) != DEAD}
            if self.vocab.eos_id is not None and self.is_accepting(state):
                ids.add(self.vocab.eos_id)
            hit = self._allowed_cache[state] = frozenset(ids)
        return hit

    def mask(self, state: int, out=None) -> list[bool]:
        allowed = self.allowed(state)
        if out is None:
            out = [False] * self.vocab.size
        for i in range(self.vocab.size):
            out[i] = i in allowed
        return out

"""Per-sequence CPU constraint for context-free grammars (the ``"cpu"``
backend of :class:`~bpdecode_amd.hf.GrammarLogitsProcessor`; grammar/constraint.py
of the reference).  Allowed sets come from a token-trie walk of the unbounded
host PDA and are memoised per config-set on the compiled grammar."""

from __future__ import annotations

from ..interface import BaseConstraint
from ..tokenizer import Vocabulary
from .gbnf import parse_gbnf
from .ir import Grammar
from .pda import PDA, CompiledGrammar
from .tokentrie import token_trie


class CFGConstraint(BaseConstraint):
    def __init__(self, grammar: str | Grammar, vocab: Vocabulary, *, root: str = "root",
                 max_depth: int = 64) -> None:
        g = grammar if isinstance(grammar, Grammar) else parse_gbnf(grammar, root)
        self._setup(CompiledGrammar.build(g), vocab, max_depth)

    def _setup(self, compiled, vocab, max_depth) -> None:
        self._compiled = compiled
        self._vocab = vocab
        self._max_depth = max_depth
        self._pda = PDA(compiled, max_depth=max_depth)
        self._token_bytes = vocab.token_bytes
        self._history: list[int] = []

    @classmethod
    def from_compiled(cls, compiled: CompiledGrammar, vocab: Vocabulary, *, max_depth: int = 64):
        obj = cls.__new__(cls)
        obj._setup(compiled, vocab, max_depth)
        return obj

    @property
    def vocab_size(self) -> int:
        return self._vocab.size

    def reset(self) -> None:
        self._pda = PDA(self._compiled, max_depth=self._max_depth)
        self._history.clear()

    def is_complete(self) -> bool:
        return self._pda.is_complete()

    def _feeds_ok(self, data: bytes) -> bool:
        snap = self._pda.configs
        try:
            return all(self._pda.advance_byte(b) for b in data) and not self._pda.dead()
        finally:
            self._pda.set_configs(snap)

    def accepts(self, token_id: int) -> bool:
        if token_id == self._vocab.eos_id:
            return self.is_complete()
        return self._feeds_ok(self._token_bytes[token_id])

    def advance(self, token_id: int) -> None:
        if token_id == self._vocab.eos_id:
            if not self.is_complete():
                raise ValueError("EOS is not valid: the string is not a complete match")
            self._history.append(token_id)
            return
        for b in self._token_bytes[token_id]:
            if not self._pda.advance_byte(b):
                raise ValueError(f"token {token_id} is not accepted from the current state")
        self._history.append(token_id)

    def allowed_ids(self) -> frozenset[int]:
        memo = self._compiled.mask_memo
        key = (id(self._vocab), self._pda.configs)
        hit = memo.get(key)
        if hit is None:
            hit = memo[key] = frozenset(token_trie(self._vocab).allowed(self._pda))
        return hit

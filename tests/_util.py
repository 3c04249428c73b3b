"""Shared helpers of the test-suite (not a test module)."""

from __future__ import annotations

import numpy as np
import torch

from bpdecode_amd.grammar.ir import Alt, CharSet, Concat, Empty, Opt, Plus, Ref
from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
from oracle import dense as OD

TOY_VOCAB = Vocabulary.from_tokens(
    ["a", "b", "c", "ab", "ba", "0", "1", "12", "-", ".", "aa", "", "caf", "\xc3", "\xe9", "é", "<eos>"],
    eos_id=16,
)
TOY_PATTERNS = ["[01]+", "a+b*", "(ab)+", "-?[0-9]+(\\.[0-9]+)?", "a|bc|12", "[a-c]*", "caf(e|é)"]

PDA_VOCAB = Vocabulary.from_tokens(
    ["(", ")", "x", "y", "{", "}", "a", "b", ":", "0", "1", ",", "<eos>", "((", "x)", "", "{a", ":0,",
     "\"", "[1", "[", "]", "tr", "ue", "nul", "l", "-", "2.5", "e9", " ", "\"ab\"", "\\n"],
    eos_id=12,
)


def oracle_table(fsa: FsaTensors) -> np.ndarray:
    """tok_next from the oracle's restatement of build_token_transitions."""
    return OD.build_token_transitions(
        fsa.trans.cpu().numpy(), fsa.accept.cpu().numpy(), fsa.live.cpu().numpy(), fsa.num_symbols,
        fsa.offsets.cpu().numpy(), fsa.symbols.cpu().numpy(), fsa.eos_id,
    )


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32).numpy().copy()


class OracleWalk:
    """One sequence walked through the oracle's tok_next table of a regex
    bundle: the allowed token ids, the commit, and completeness (EOS
    allowed)."""

    def __init__(self, fsa: FsaTensors) -> None:
        self.fsa = fsa
        self.rows: dict[int, np.ndarray] = {}  # oracle tok_next rows, built as states are met
        self.accept = fsa.accept.cpu().numpy().astype(bool)
        self.state = fsa.start

    def _row(self, s: int) -> np.ndarray:
        if s not in self.rows:
            f = self.fsa
            self.rows[s] = OD.build_token_transitions(
                f.trans.cpu().numpy(), f.accept.cpu().numpy(), f.live.cpu().numpy(), f.num_symbols,
                f.offsets.cpu().numpy(), f.symbols.cpu().numpy(), f.eos_id, rows=[s])[0]
        return self.rows[s]

    def allowed(self) -> set[int]:
        if self.state < 0:
            return set()
        return set(np.nonzero(self._row(self.state) != -1)[0].tolist())

    def advance(self, token: int) -> None:
        if self.state >= 0:
            self.state = int(OD.advance(self._row(self.state)[None], [0], [token])[0])

    def is_complete(self) -> bool:
        return self.state >= 0 and bool(self.accept[self.state])


def reachable(tok_next: np.ndarray, start: int) -> list[int]:
    seen, todo = {start}, [start]
    while todo:
        for d in np.unique(tok_next[todo.pop()]):
            if d >= 0 and int(d) not in seen:
                seen.add(int(d))
                todo.append(int(d))
    return sorted(seen)


def member(grammar, text):
    """Is ``text`` in the language of ``grammar``?  An independent recursive
    matcher over the grammar IR (no NFA, no PDA): the set of end positions."""
    rules = grammar.rules
    busy = set()

    def m(e, pos):
        if isinstance(e, Empty):
            return {pos}
        if isinstance(e, CharSet):
            return {pos + 1} if pos < len(text) and e.matches(ord(text[pos])) else set()
        if isinstance(e, Ref):
            key = (e.name, pos)
            if key in busy:
                return set()
            busy.add(key)
            try:
                return m(rules[e.name], pos)
            finally:
                busy.discard(key)
        if isinstance(e, Concat):
            cur = {pos}
            for p in e.parts:
                cur = set().union(*(m(p, q) for q in cur)) if cur else set()
            return cur
        if isinstance(e, Alt):
            return set().union(*(m(o, pos) for o in e.options))
        if isinstance(e, Opt):
            return {pos} | m(e.node, pos)
        reached = set() if isinstance(e, Plus) else {pos}
        frontier = {pos}
        while frontier:
            nxt = set()
            for p in frontier:
                for q in m(e.node, p):
                    if q not in reached:
                        reached.add(q)
                        nxt.add(q)
            frontier = nxt
        return reached

    return len(text) in m(rules[grammar.root], 0)

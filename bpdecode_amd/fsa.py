"""Host FSA tables in the layout the native library consumes (fsa.py:31-218 of
the reference): a dense symbol-class transition table, reachability
(``live``), and each token's symbol-class sequence.

The scalar :func:`step` is the semantic definition of one ``tok_next`` entry
(fsa.py:155-174): walk the token's classes from ``state``; the result is ``-1``
when the walk reaches ``dead`` or ends in a state from which no accepting
state is reachable.  EOS is decided by id: it maps an accepting state to
itself and everything else to ``-1``.
"""

from __future__ import annotations

from collections import deque
from collections.abc import Sequence
from dataclasses import dataclass, field

from .regex.compile import DFA
from .tokenizer import Vocabulary


@dataclass(frozen=True)
class FsaTable:
    num_states: int
    num_symbols: int
    start: int
    dead: int
    trans: tuple[int, ...]
    accept: tuple[int, ...]
    live: tuple[int, ...]
    symbols: tuple[tuple[int, int], ...] = ()

    def target(self, state: int, sym: int) -> int:
        return self.trans[state * self.num_symbols + sym]


@dataclass
class TokenSymbols:
    vocab_size: int
    eos_id: int
    offsets: Sequence[int] = field(default_factory=lambda: [0])  # list or int32 array
    symbols: bytes = b""


def build_reachability(num_states, num_symbols, trans, accept) -> list[int]:
    """``live[s] = 1`` iff an accepting state is reachable from ``s``: a reverse
    breadth-first search from the accepting set (fsa.py:70-104)."""
    preds: list[list[int]] = [[] for _ in range(num_states)]
    for s in range(num_states):
        row = trans[s * num_symbols : (s + 1) * num_symbols]
        for t in row:
            if 0 <= t < num_states:
                preds[t].append(s)
    live = [1 if accept[s] else 0 for s in range(num_states)]
    todo = deque(s for s in range(num_states) if accept[s])
    while todo:
        for p in preds[todo.popleft()]:
            if not live[p]:
                live[p] = 1
                todo.append(p)
    return live


def fsa_from_dfa(dfa: DFA, with_live: bool = True) -> FsaTable:
    """The DFA as flat tables; ``with_live=False`` leaves ``live`` empty for
    a builder that computes it elsewhere (the device)."""
    n = len(dfa.trans)
    m = len(dfa.symbols)
    flat = tuple(t for row in dfa.trans for t in row)
    accept = tuple(1 if s in dfa.accept else 0 for s in range(n))
    return FsaTable(
        num_states=n,
        num_symbols=m,
        start=dfa.start,
        dead=dfa.dead,
        trans=flat,
        accept=accept,
        live=tuple(build_reachability(n, m, flat, accept)) if with_live else (),
        symbols=tuple(dfa.symbols),
    )


def token_symbols(dfa: DFA, vocab: Vocabulary) -> TokenSymbols:
    lut = bytes(dfa.symbol_of(b) for b in range(256))
    data, offsets = vocab.packed
    return TokenSymbols(
        vocab_size=vocab.size,
        eos_id=vocab.eos_id if vocab.eos_id is not None else -1,
        offsets=offsets,
        symbols=data.translate(lut),
    )


def step(fsa: FsaTable, toks: TokenSymbols, state: int, token_id: int) -> int:
    if token_id == toks.eos_id:
        return state if state >= 0 and fsa.accept[state] else -1
    if state < 0:
        return -1
    cur = state
    for i in range(toks.offsets[token_id], toks.offsets[token_id + 1]):
        sym = toks.symbols[i]
        if sym < 0 or sym >= fsa.num_symbols:
            return -1
        cur = fsa.trans[cur * fsa.num_symbols + sym]
        if cur == fsa.dead:
            return -1
    return cur if fsa.live[cur] else -1


def compute_mask(fsa: FsaTable, toks: TokenSymbols, state: int) -> list[bool]:
    out = [step(fsa, toks, state, t) != -1 for t in range(toks.vocab_size)]
    if toks.eos_id >= 0 and state >= 0 and fsa.accept[state]:
        out[toks.eos_id] = True
    return out


def advance_state_batch(fsa, toks, states, token_ids) -> list[int]:
    return [step(fsa, toks, s, t) for s, t in zip(states, token_ids, strict=True)]


def apply_mask(fsa, toks, states, logits, neg_inf: float = float("-inf")):
    for row, s in zip(logits, states, strict=True):
        for t in range(toks.vocab_size):
            if step(fsa, toks, s, t) == -1:
                row[t] = neg_inf
    return logits

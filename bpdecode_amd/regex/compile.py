"""Regex AST -> complete byte DFA over symbol classes.

Thompson construction followed by subset construction, as in the reference
(regex/compile.py:53-255).  Both steps are replicated in their observable
details because committed DFA state ids are part of the API: states are
numbered in breadth-first discovery order from the start closure, symbol
classes are visited in increasing byte order, an explicit absorbing ``dead``
state is appended last, and the NFA has the same shape node for node (the
subset construction is not minimised, so the NFA's shape decides the DFA).
"""

from __future__ import annotations

from dataclasses import dataclass

from .parser import Alt, CharSet, Concat, Empty, Opt, Plus, Star, parse
from .utf8 import utf8_sequences

BYTE_LIMIT = 256


class ThompsonNFA:
    """Byte NFA: ``edges[s]`` lists ``(lo, hi, dst)`` with ``lo = -1`` for an
    epsilon move (``hi`` unused)."""

    def __init__(self) -> None:
        self.edges: list[list[tuple[int, int, int]]] = []
        self.start = 0
        self.accept = 0

    def state(self) -> int:
        self.edges.append([])
        return len(self.edges) - 1

    def eps(self, a: int, b: int) -> None:
        self.edges[a].append((-1, 0, b))

    def byte(self, a: int, lo: int, hi: int, b: int) -> None:
        self.edges[a].append((lo, hi, b))

    def build(self, node) -> tuple[int, int]:
        if isinstance(node, Empty):
            s, e = self.state(), self.state()
            self.eps(s, e)
            return s, e
        if isinstance(node, CharSet):
            s, e = self.state(), self.state()
            for lo, hi in node.ranges:
                for seq in utf8_sequences(lo, hi):
                    cur = s
                    for j, (blo, bhi) in enumerate(seq):
                        nxt = e if j == len(seq) - 1 else self.state()
                        self.byte(cur, blo, bhi, nxt)
                        cur = nxt
            return s, e
        if isinstance(node, Concat):
            if not node.parts:
                return self.build(Empty())
            s, e = self.build(node.parts[0])
            for part in node.parts[1:]:
                ps, pe = self.build(part)
                self.eps(e, ps)
                e = pe
            return s, e
        if isinstance(node, Alt):
            s, e = self.state(), self.state()
            for opt in node.options:
                os_, oe = self.build(opt)
                self.eps(s, os_)
                self.eps(oe, e)
            return s, e
        if isinstance(node, (Star, Plus, Opt)):
            ins, ine = self.build(node.node)
            s, e = self.state(), self.state()
            self.eps(s, ins)
            self.eps(ine, e)
            if not isinstance(node, Plus):
                self.eps(s, e)
            if not isinstance(node, Opt):
                self.eps(ine, ins)
            return s, e
        raise TypeError(f"unhandled AST node: {type(node).__name__}")

    def closure(self, seeds) -> frozenset[int]:
        seen = set(seeds)
        todo = list(seeds)
        while todo:
            for lo, _, dst in self.edges[todo.pop()]:
                if lo < 0 and dst not in seen:
                    seen.add(dst)
                    todo.append(dst)
        return frozenset(seen)


@dataclass(frozen=True)
class DFA:
    """Complete DFA over half-open byte classes ``symbols[k] = [lo, hi)``.

    ``trans[s][k]`` is the target of class ``k``; ``dead`` is absorbing and
    non-accepting.
    """

    symbols: tuple[tuple[int, int], ...]
    trans: tuple[tuple[int, ...], ...]
    accept: frozenset[int]
    start: int
    dead: int

    def symbol_of(self, byte: int) -> int:
        lo, hi = 0, len(self.symbols)
        while lo < hi:
            mid = (lo + hi) // 2
            a, b = self.symbols[mid]
            if byte < a:
                hi = mid
            elif byte >= b:
                lo = mid + 1
            else:
                return mid
        return -1

    def step(self, state: int, byte: int) -> int:
        if state < 0:
            return self.dead
        k = self.symbol_of(byte)
        return self.dead if k < 0 else self.trans[state][k]

    def live_states(self) -> frozenset[int]:
        """States from which an accepting state is reachable."""
        preds: dict[int, set[int]] = {}
        for s, row in enumerate(self.trans):
            for t in row:
                if t >= 0:
                    preds.setdefault(t, set()).add(s)
        seen = set(self.accept)
        todo = list(self.accept)
        while todo:
            for p in preds.get(todo.pop(), ()):
                if p not in seen:
                    seen.add(p)
                    todo.append(p)
        return frozenset(seen)


def subset_construct(nfa: ThompsonNFA, symbols, sample) -> DFA:
    """Breadth-first subset construction; ``sample[k]`` is a byte of class k."""
    first = nfa.closure([nfa.start])
    index = {first: 0}
    queue = [first]
    rows: list[list[int]] = []
    head = 0
    while head < len(queue):
        cur = queue[head]
        head += 1
        row = []
        for b in sample:
            moved = {dst for s in cur for lo, hi, dst in nfa.edges[s] if lo >= 0 and lo <= b <= hi}
            if not moved:
                row.append(-1)
                continue
            key = nfa.closure(moved)
            idx = index.get(key)
            if idx is None:
                idx = len(queue)
                index[key] = idx
                queue.append(key)
            row.append(idx)
        rows.append(row)
    dead = len(queue)
    table = [tuple(dead if t < 0 else t for t in row) for row in rows]
    table.append((dead,) * len(symbols))
    accept = frozenset(i for key, i in index.items() if nfa.accept in key)
    return DFA(tuple(symbols), tuple(table), accept, 0, dead)


def compile_ast(ast) -> DFA:
    nfa = ThompsonNFA()
    nfa.start, nfa.accept = nfa.build(ast)
    cuts = {0, BYTE_LIMIT}
    for out in nfa.edges:
        for lo, hi, _ in out:
            if lo >= 0:
                cuts.add(lo)
                cuts.add(hi + 1)
    cuts = sorted(cuts)
    symbols = tuple((cuts[i], cuts[i + 1]) for i in range(len(cuts) - 1))
    return subset_construct(nfa, symbols, [a for a, _ in symbols])


def compile_regex(pattern: str) -> DFA:
    """Compile ``pattern`` to a :class:`DFA` (regex/compile.py:194-196)."""
    return compile_ast(parse(pattern))

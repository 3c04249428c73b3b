"""Per-rule byte NFAs with ``call`` edges (grammar/nfa.py:20-108 of the
reference).

Edge labels: ``None`` (epsilon), ``("byte", lo, hi)``, ``("call", rule)``.
State numbering and per-state edge order follow the Thompson construction
node for node: the flattened PDA table (and so every stack frame value and the
order in which closures append configurations) depends on both.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..regex.utf8 import utf8_sequences
from .ir import Alt, CharSet, Concat, Empty, Opt, Plus, Ref, Star


@dataclass
class RuleNFA:
    start: int
    accept: int
    num_states: int
    edges: dict = field(default_factory=dict)

    def out(self, s: int) -> list:
        return self.edges.get(s, [])


class _RuleBuilder:
    def __init__(self) -> None:
        self.edges: dict[int, list] = {}

    def state(self) -> int:
        s = len(self.edges)
        self.edges[s] = []
        return s

    def link(self, a: int, label, b: int) -> None:
        self.edges[a].append((label, b))

    def build(self, e) -> tuple[int, int]:
        if isinstance(e, (Empty, Ref)):
            s, t = self.state(), self.state()
            self.link(s, None if isinstance(e, Empty) else ("call", e.name), t)
            return s, t
        if isinstance(e, CharSet):
            s, t = self.state(), self.state()
            for lo, hi in e.ranges:
                for seq in utf8_sequences(lo, hi):
                    cur = s
                    for j, (blo, bhi) in enumerate(seq):
                        nxt = t if j == len(seq) - 1 else self.state()
                        self.link(cur, ("byte", blo, bhi), nxt)
                        cur = nxt
            return s, t
        if isinstance(e, Concat):
            if not e.parts:
                return self.build(Empty())
            s, t = self.build(e.parts[0])
            for p in e.parts[1:]:
                ps, pt = self.build(p)
                self.link(t, None, ps)
                t = pt
            return s, t
        if isinstance(e, Alt):
            s, t = self.state(), self.state()
            for o in e.options:
                os_, ot = self.build(o)
                self.link(s, None, os_)
                self.link(ot, None, t)
            return s, t
        if isinstance(e, (Star, Plus, Opt)):
            ins, int_ = self.build(e.node)
            s, t = self.state(), self.state()
            self.link(s, None, ins)
            self.link(int_, None, t)
            if not isinstance(e, Plus):
                self.link(s, None, t)
            if not isinstance(e, Opt):
                self.link(int_, None, ins)
            return s, t
        raise TypeError(f"unhandled grammar node: {type(e).__name__}")


def compile_rule(expr) -> RuleNFA:
    b = _RuleBuilder()
    s, t = b.build(expr)
    return RuleNFA(start=s, accept=t, num_states=len(b.edges), edges=b.edges)


def compile_rules(grammar) -> dict[str, RuleNFA]:
    return {name: compile_rule(e) for name, e in grammar.rules.items()}

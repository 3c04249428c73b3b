"""Compiled grammar: per-rule byte NFAs and their coreachable states
(grammar/pda.py:32-108 of the reference).

``CompiledGrammar.coreachable[rule]`` is the set of states from which the
rule's accept state is reachable, a ``call`` edge counting as passable iff its
callee can derive some string; it becomes the ``live`` prune of the flattened
device table (grammar/device.py).  ``regular`` names the rules with no
recursion through calls (their frames can be replaced by a byte DFA).
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .ir import Grammar
from .nfa import RuleNFA, compile_rules

def _passable(label, ok: dict) -> bool:
    return not (label is not None and label[0] == "call" and not ok.get(label[1]))


def rule_nonempty(rules: dict[str, RuleNFA]) -> dict[str, bool]:
    """Fixpoint: can each rule derive some string (the empty one included)?"""
    ok = dict.fromkeys(rules, False)
    changed = True
    while changed:
        changed = False
        for name, nfa in rules.items():
            if ok[name]:
                continue
            seen = {nfa.start}
            todo = [nfa.start]
            while todo:
                s = todo.pop()
                for label, dst in nfa.out(s):
                    if _passable(label, ok) and dst not in seen:
                        seen.add(dst)
                        todo.append(dst)
            if nfa.accept in seen:
                ok[name] = changed = True
    return ok


def coreachable_sets(rules: dict[str, RuleNFA], ok: dict) -> dict[str, frozenset[int]]:
    out = {}
    for name, nfa in rules.items():
        preds: dict[int, list[int]] = {}
        for s in range(nfa.num_states):
            for label, dst in nfa.out(s):
                if _passable(label, ok):
                    preds.setdefault(dst, []).append(s)
        seen = {nfa.accept}
        todo = [nfa.accept]
        while todo:
            for p in preds.get(todo.pop(), ()):
                if p not in seen:
                    seen.add(p)
                    todo.append(p)
        out[name] = frozenset(seen)
    return out


@dataclass
class CompiledGrammar:
    rules: dict
    root: str
    coreachable: dict
    regular: frozenset = frozenset()
    residual_memo: dict = field(default_factory=dict)

    @classmethod
    def build(cls, grammar: Grammar) -> CompiledGrammar:
        from .regular import regular_rules

        rules = compile_rules(grammar)
        obj = cls(rules, grammar.root, coreachable_sets(rules, rule_nonempty(rules)))
        obj.regular = regular_rules(obj)
        return obj

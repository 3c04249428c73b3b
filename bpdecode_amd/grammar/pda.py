"""Compiled grammar (rule NFAs + coreachability) and the unbounded host PDA
(grammar/pda.py:32-234 of the reference).

``CompiledGrammar.coreachable[rule]`` is the set of states from which the
rule's accept state is reachable, a ``call`` edge counting as passable iff its
callee can derive some string; it becomes the ``live`` prune of the flattened
device table.  :class:`PDA` is the unbounded, set-based automaton the
CPU-side :class:`~bpdecode_amd.grammar.constraint.CFGConstraint` uses.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .ir import Grammar
from .nfa import RuleNFA, compile_rules

DEFAULT_MAX_DEPTH = 64
DEFAULT_MAX_CONFIGS = 4096


class PDAOverflow(RuntimeError):
    """The config-set or the stack depth exceeded its cap."""


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
    transition_memo: dict = field(default_factory=dict)
    mask_memo: dict = field(default_factory=dict)
    residual_memo: dict = field(default_factory=dict)

    @classmethod
    def build(cls, grammar: Grammar) -> CompiledGrammar:
        from .regular import regular_rules

        rules = compile_rules(grammar)
        obj = cls(rules, grammar.root, coreachable_sets(rules, rule_nonempty(rules)))
        obj.regular = regular_rules(obj)
        return obj


class PDA:
    """Unbounded set-of-stacks automaton; a frame is ``(rule, nfa_state)``."""

    def __init__(self, compiled: CompiledGrammar, *, max_depth: int = DEFAULT_MAX_DEPTH,
                 max_configs: int = DEFAULT_MAX_CONFIGS) -> None:
        self.g = compiled
        self.max_depth = max_depth
        self.max_configs = max_configs
        self._memo = compiled.transition_memo
        root = compiled.rules[compiled.root]
        self._configs = self._close(frozenset({((compiled.root, root.start),)}))

    @property
    def configs(self) -> frozenset:
        return self._configs

    def set_configs(self, configs: frozenset) -> None:
        self._configs = configs

    def dead(self) -> bool:
        return not self._configs

    def _close(self, configs: frozenset) -> frozenset:
        hit = self._memo.get(("c", configs))
        if hit is None:
            hit = self._close_uncached(configs)
            self._memo[("c", configs)] = hit
        return hit

    def _close_uncached(self, configs: frozenset) -> frozenset:
        done: set = set()
        todo = list(configs)
        while todo:
            cfg = todo.pop()
            if cfg in done:
                continue
            done.add(cfg)
            if not cfg:
                continue
            rule, st = cfg[-1]
            nfa = self.g.rules[rule]
            if st == nfa.accept and len(cfg) > 1:
                todo.append(cfg[:-1])
            for label, dst in nfa.out(st):
                if label is None:
                    todo.append(cfg[:-1] + ((rule, dst),))
                elif label[0] == "call" and len(cfg) < self.max_depth:
                    callee = label[1]
                    todo.append(cfg[:-1] + ((rule, dst), (callee, self.g.rules[callee].start)))
            if len(done) > self.max_configs:
                raise PDAOverflow(f"config-set exceeded {self.max_configs}")
        co = self.g.coreachable
        return frozenset(c for c in done if not c or c[-1][1] in co[c[-1][0]])

    def advance_byte(self, b: int) -> bool:
        key = ("t", self._configs, b)
        nxt = self._memo.get(key)
        if nxt is None:
            moved = set()
            for cfg in self._configs:
                if not cfg:
                    continue
                rule, st = cfg[-1]
                for label, dst in self.g.rules[rule].out(st):
                    if label is not None and label[0] == "byte" and label[1] <= b <= label[2]:
                        moved.add(cfg[:-1] + ((rule, dst),))
            nxt = self._close(frozenset(moved))
            self._memo[key] = nxt
        self._configs = nxt
        return bool(nxt)

    def first_byte_ranges(self) -> list[tuple[int, int]]:
        spans = []
        for cfg in self._configs:
            if cfg:
                rule, st = cfg[-1]
                for label, _ in self.g.rules[rule].out(st):
                    if label is not None and label[0] == "byte":
                        spans.append((label[1], label[2]))
        from ..regex.parser import merge_ranges

        return list(merge_ranges(spans))

    def is_complete(self) -> bool:
        root = self.g.rules[self.g.root]
        return ((self.g.root, root.accept),) in self._configs

"""Residual byte DFA of a regular PDA frame (grammar/regular.py:22-199 of the
reference).

A frame ``(rule, state)`` whose reachable part calls only regular rules has a
regular residual language until it pops; inlining the regular callees gives
one byte NFA, and a subset construction over the 256 single-byte classes
gives its DFA, with the rule's accept state marking the DFA accept set.  The
flat JSON-Schema document DFA is the residual of the root rule at its start.
"""

from __future__ import annotations

from ..regex.compile import DFA, ThompsonNFA, subset_construct

_BYTE_CLASSES = tuple((b, b + 1) for b in range(256))


def regular_rules(compiled) -> frozenset[str]:
    """Rules that transitively call only regular rules."""
    calls = {
        name: {lbl[1] for s in range(nfa.num_states) for lbl, _ in nfa.out(s)
               if lbl is not None and lbl[0] == "call"}
        for name, nfa in compiled.rules.items()
    }
    regular = {n for n, c in calls.items() if not c}
    grew = True
    while grew:
        grew = False
        for n, c in calls.items():
            if n not in regular and c <= regular:
                regular.add(n)
                grew = True
    return frozenset(regular)


def _reachable(nfa, start: int) -> set[int]:
    seen = {start}
    todo = [start]
    while todo:
        for _, dst in nfa.out(todo.pop()):
            if dst not in seen:
                seen.add(dst)
                todo.append(dst)
    return seen


def frame_is_regular(compiled, regular, rule: str, state: int) -> bool:
    nfa = compiled.rules[rule]
    return all(
        lbl is None or lbl[0] != "call" or lbl[1] in regular
        for s in _reachable(nfa, state)
        for lbl, _ in nfa.out(s)
    )


def _inline(compiled, out: ThompsonNFA, rule: str, entry: int) -> tuple[int, int]:
    """Copy ``rule``'s NFA into ``out`` (callees inlined recursively)."""
    nfa = compiled.rules[rule]
    local: dict[int, int] = {}

    def at(s: int) -> int:
        if s not in local:
            local[s] = out.state()
        return local[s]

    for s in range(nfa.num_states):
        src = at(s)
        for lbl, dst in nfa.out(s):
            if lbl is None:
                out.eps(src, at(dst))
            elif lbl[0] == "byte":
                out.byte(src, lbl[1], lbl[2], at(dst))
            else:
                cs, ce = _inline(compiled, out, lbl[1], compiled.rules[lbl[1]].start)
                out.eps(src, cs)
                out.eps(ce, at(dst))
    return at(entry), at(nfa.accept)


def _eps_closure_in_rule(nfa, state: int) -> frozenset[int]:
    seen = {state}
    todo = [state]
    while todo:
        for lbl, dst in nfa.out(todo.pop()):
            if lbl is None and dst not in seen:
                seen.add(dst)
                todo.append(dst)
    return frozenset(seen)


def residual_dfa(compiled, rule: str, state: int) -> DFA:
    """Byte DFA of frame ``(rule, state)``'s residual language (cached per
    epsilon-closure of the frame's state)."""
    key = ("dfa", (rule, _eps_closure_in_rule(compiled.rules[rule], state)))
    hit = compiled.residual_memo.get(key)
    if hit is None:
        nfa = ThompsonNFA()
        nfa.start, nfa.accept = _inline(compiled, nfa, rule, state)
        hit = subset_construct(nfa, _BYTE_CLASSES, list(range(256)))
        compiled.residual_memo[key] = hit
    return hit

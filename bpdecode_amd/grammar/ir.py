"""Grammar IR: named rules whose bodies are regex AST nodes plus :class:`Ref`
(grammar/ir.py:30-92 of the reference)."""

from __future__ import annotations

from dataclasses import dataclass

from ..regex.parser import Alt, CharSet, Concat, Empty, Opt, Plus, Star

__all__ = ["Alt", "CharSet", "Concat", "Empty", "Grammar", "Opt", "Plus", "Ref", "Star", "Expr"]


@dataclass(frozen=True)
class Ref:
    """A reference to another rule by name."""

    name: str


Expr = Empty | CharSet | Concat | Alt | Star | Plus | Opt | Ref


def _children(e):
    if isinstance(e, Concat):
        return e.parts
    if isinstance(e, Alt):
        return e.options
    if isinstance(e, (Star, Plus, Opt)):
        return (e.node,)
    return ()


def refs_in(e) -> set[str]:
    out: set[str] = set()
    todo = [e]
    while todo:
        x = todo.pop()
        if isinstance(x, Ref):
            out.add(x.name)
        todo.extend(_children(x))
    return out


@dataclass(frozen=True)
class Grammar:
    """Rules in definition order (the order fixes PDA state ids) + root name."""

    rules: dict
    root: str = "root"

    def __post_init__(self) -> None:
        if self.root not in self.rules:
            raise KeyError(f"root rule {self.root!r} is not defined")
        missing = set().union(*(refs_in(e) for e in self.rules.values())) - set(self.rules)
        if missing:
            raise KeyError(f"undefined rule(s): {', '.join(sorted(missing))}")

    def is_regular(self) -> bool:
        return not any(refs_in(e) for e in self.rules.values())

"""Regex source -> AST.

Accepted syntax (the reference's, regex/parser.py:1-15): literals with ``\\``
escapes, ``.``, ``* + ?``, ``{m}`` ``{m,}`` ``{m,n}``, ``|``, ``( )`` and
``[...]`` / ``[^...]`` classes, plus the ``\\d \\w \\s`` shorthands and their
negations outside classes.  Anchors, backreferences and lookaround raise
:class:`RegexSyntaxError`.

The AST shape is part of the contract: the NFA built from it, and therefore
the DFA state numbering that committed states are reported in, follows the
tree node for node.  Counted repetition ``x{m,n}`` expands to ``m`` copies of
``x`` followed by ``n - m`` optional copies (a trailing ``x*`` when unbounded),
as regex/parser.py:129-148 does.
"""

from __future__ import annotations

from dataclasses import dataclass

UNICODE_MAX = 0x10FFFF


class RegexSyntaxError(ValueError):
    """A construct the parser does not implement, or malformed input."""


@dataclass(frozen=True)
class Empty:
    """Matches the empty string."""


@dataclass(frozen=True)
class CharSet:
    """Inclusive code-point ranges, sorted and non-overlapping."""

    ranges: tuple[tuple[int, int], ...]

    def matches(self, cp: int) -> bool:
        return any(lo <= cp <= hi for lo, hi in self.ranges)


@dataclass(frozen=True)
class Concat:
    parts: tuple


@dataclass(frozen=True)
class Alt:
    options: tuple


@dataclass(frozen=True)
class Star:
    node: object


@dataclass(frozen=True)
class Plus:
    node: object


@dataclass(frozen=True)
class Opt:
    node: object


Node = Empty | CharSet | Concat | Alt | Star | Plus | Opt

_SHORTHAND = {
    "d": ((0x30, 0x39),),
    "w": ((0x30, 0x39), (0x41, 0x5A), (0x5F, 0x5F), (0x61, 0x7A)),
    "s": ((0x09, 0x0D), (0x20, 0x20)),
}
_CONTROL = {"n": "\n", "t": "\t", "r": "\r", "f": "\f", "v": "\v"}


def merge_ranges(ranges) -> tuple[tuple[int, int], ...]:
    """Sort and coalesce overlapping or touching inclusive ranges."""
    out: list[list[int]] = []
    for lo, hi in sorted(ranges):
        if out and lo <= out[-1][1] + 1:
            if hi > out[-1][1]:
                out[-1][1] = hi
        else:
            out.append([lo, hi])
    return tuple((a, b) for a, b in out)


def complement(ranges) -> tuple[tuple[int, int], ...]:
    """Complement of ``ranges`` within ``[0, UNICODE_MAX]``."""
    out = []
    nxt = 0
    for lo, hi in sorted(ranges):
        if lo > nxt:
            out.append((nxt, lo - 1))
        nxt = max(nxt, hi + 1)
    if nxt <= UNICODE_MAX:
        out.append((nxt, UNICODE_MAX))
    return tuple(out)


def _seq(nodes: list) -> object:
    if not nodes:
        return Empty()
    return nodes[0] if len(nodes) == 1 else Concat(tuple(nodes))


def repeat(node, lo: int, hi: int | None):
    """``node{lo,hi}`` (``hi=None`` = unbounded) as a Concat of copies."""
    parts = [node] * lo
    if hi is None:
        parts.append(Star(node))
    else:
        parts.extend([Opt(node)] * (hi - lo))
    return _seq(parts)


class _Reader:
    def __init__(self, text: str) -> None:
        self.text = text
        self.i = 0

    def peek(self) -> str | None:
        return self.text[self.i] if self.i < len(self.text) else None

    def take(self) -> str:
        c = self.text[self.i]
        self.i += 1
        return c

    # alternation := sequence ('|' sequence)*
    def alternation(self):
        branches = [self.sequence()]
        while self.peek() == "|":
            self.i += 1
            branches.append(self.sequence())
        return branches[0] if len(branches) == 1 else Alt(tuple(branches))

    def sequence(self):
        items = []
        while self.peek() is not None and self.peek() not in "|)":
            items.append(self.quantified())
        return _seq(items)

    def quantified(self):
        node = self.atom()
        while True:
            c = self.peek()
            if c == "*":
                self.i += 1
                node = Star(node)
            elif c == "+":
                self.i += 1
                node = Plus(node)
            elif c == "?":
                self.i += 1
                node = Opt(node)
            elif c == "{":
                node = self.counted(node)
            else:
                return node

    def number(self) -> int:
        j = self.i
        while self.i < len(self.text) and self.text[self.i].isdigit():
            self.i += 1
        if j == self.i:
            raise RegexSyntaxError("expected a number in counted repetition")
        return int(self.text[j : self.i])

    def counted(self, node):
        self.i += 1  # '{'
        lo = self.number()
        hi: int | None = lo
        if self.peek() == ",":
            self.i += 1
            hi = None if self.peek() == "}" else self.number()
        if self.peek() != "}":
            raise RegexSyntaxError("expected '}' to close counted repetition")
        self.i += 1
        if hi is not None and hi < lo:
            raise RegexSyntaxError("counted repetition {m,n} has n < m")
        return repeat(node, lo, hi)

    def atom(self):
        c = self.peek()
        if c is None:
            return Empty()
        if c == "(":
            self.i += 1
            inner = self.alternation()
            if self.peek() != ")":
                raise RegexSyntaxError("unbalanced '('")
            self.i += 1
            return inner
        if c == "[":
            return self.char_class()
        if c == ".":
            self.i += 1
            return CharSet(((0, UNICODE_MAX),))
        if c in "*+?":
            raise RegexSyntaxError(f"nothing to repeat before {c!r}")
        if c in "^$":
            raise RegexSyntaxError("anchors are not supported")
        if c == ")":
            raise RegexSyntaxError("unbalanced ')'")
        self.i += 1
        if c == "\\":
            if self.peek() is None:
                raise RegexSyntaxError("trailing backslash")
            e = self.take()
            if e in _SHORTHAND:
                return CharSet(_SHORTHAND[e])
            if e in "DWS":
                return CharSet(complement(_SHORTHAND[e.lower()]))
            cp = ord(_CONTROL.get(e, e))
            return CharSet(((cp, cp),))
        return CharSet(((ord(c), ord(c)),))

    def class_member(self) -> int:
        c = self.take()
        if c == "\\":
            e = self.take()
            return ord(_CONTROL.get(e, e))
        return ord(c)

    def char_class(self):
        self.i += 1  # '['
        negate = self.peek() == "^"
        if negate:
            self.i += 1
        spans = []
        first = True
        while True:
            c = self.peek()
            if c is None:
                raise RegexSyntaxError("unterminated character class")
            if c == "]" and not first:
                self.i += 1
                break
            first = False
            lo = self.class_member()
            after = self.text[self.i + 1 : self.i + 2]
            if self.peek() == "-" and after not in ("]", ""):
                self.i += 1
                hi = self.class_member()
                if hi < lo:
                    raise RegexSyntaxError("character class range is out of order")
                spans.append((lo, hi))
            else:
                spans.append((lo, lo))
        merged = merge_ranges(spans)
        return CharSet(complement(merged) if negate else merged)


def parse(pattern: str):
    """Parse ``pattern`` to an AST (regex/parser.py:262-268)."""
    r = _Reader(pattern)
    node = r.alternation()
    if r.peek() is not None:
        raise RegexSyntaxError(
            f"unexpected character at position {r.i}: {r.text[r.i]!r}"
        )
    return node

"""GBNF (llama.cpp grammar format) -> :class:`Grammar` (grammar/gbnf.py:1-276 of
the reference).

``name ::= body`` rules; ``|`` alternation; juxtaposition concatenates;
``"strings"``, ``[...]`` / ``[^...]`` classes, rule references, ``( )``, one
postfix ``* + ?`` or ``{m,n}`` per atom, ``#`` comments and ``\\xHH``
``\\uHHHH`` ``\\UHHHHHHHH`` escapes.  Redefining a rule replaces its body but
keeps its original position, as a Python dict assignment does; the position
fixes the rule's state-id offset in the flattened PDA table.
"""

from __future__ import annotations

from ..regex.parser import complement, merge_ranges, repeat
from .ir import Alt, CharSet, Concat, Empty, Grammar, Opt, Plus, Ref, Star

_NAME0 = set("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ")
_NAME = _NAME0 | set("0123456789-_")
_ESC = {"n": 0x0A, "t": 0x09, "r": 0x0D, "f": 0x0C, "v": 0x0B, "0": 0x00}


class GBNFSyntaxError(ValueError):
    """Malformed GBNF."""


class _Lexer:
    def __init__(self, src: str) -> None:
        self.s = src
        self.i = 0

    def fail(self, msg: str) -> GBNFSyntaxError:
        return GBNFSyntaxError(f"{msg} at position {self.i}")

    def skip(self) -> None:
        s, n = self.s, len(self.s)
        while self.i < n:
            c = s[self.i]
            if c in " \t\r\n":
                self.i += 1
            elif c == "#":
                while self.i < n and s[self.i] != "\n":
                    self.i += 1
            else:
                return

    def peek(self) -> str:
        self.skip()
        return self.s[self.i] if self.i < len(self.s) else ""

    def name(self) -> str:
        self.skip()
        j = self.i
        if j >= len(self.s) or self.s[j] not in _NAME0:
            raise self.fail("expected a rule name")
        self.i += 1
        while self.i < len(self.s) and self.s[self.i] in _NAME:
            self.i += 1
        return self.s[j : self.i]

    def rule_starts_here(self) -> bool:
        """Is the upcoming text ``NAME ::=`` (a new rule, not a reference)?"""
        self.skip()
        j, s, n = self.i, self.s, len(self.s)
        if j >= n or s[j] not in _NAME0:
            return False
        j += 1
        while j < n and s[j] in _NAME:
            j += 1
        while j < n and s[j] in " \t\r\n":
            j += 1
        return s.startswith("::=", j)

    # --- grammar ------------------------------------------------------
    def grammar(self) -> dict:
        rules: dict = {}
        while self.peek():
            name = self.name()
            self.skip()
            if not self.s.startswith("::=", self.i):
                raise self.fail(f"expected '::=' after rule {name!r}")
            self.i += 3
            rules[name] = self.alternatives()
        if not rules:
            raise self.fail("empty grammar")
        return rules

    def alternatives(self):
        opts = [self.sequence()]
        while self.peek() == "|":
            self.i += 1
            opts.append(self.sequence())
        return opts[0] if len(opts) == 1 else Alt(tuple(opts))

    def sequence(self):
        parts = []
        while True:
            c = self.peek()
            if c in ("", "|", ")") or (c in _NAME0 and self.rule_starts_here()):
                break
            parts.append(self.postfix())
        if not parts:
            return Empty()
        return parts[0] if len(parts) == 1 else Concat(tuple(parts))

    def postfix(self):
        node = self.atom()
        c = self.peek()
        if c in ("*", "+", "?"):
            self.i += 1
            return {"*": Star, "+": Plus, "?": Opt}[c](node)
        if c == "{":
            self.i += 1
            lo = self.integer()
            hi: int | None = lo
            if self.peek() == ",":
                self.i += 1
                self.skip()
                hi = None if self.s[self.i] == "}" else self.integer()
            if self.peek() != "}":
                raise self.fail("expected '}' to close repetition")
            self.i += 1
            if hi is not None and hi < lo:
                raise self.fail("repetition {m,n} has n < m")
            return repeat(node, lo, hi)
        return node

    def integer(self) -> int:
        self.skip()
        j = self.i
        while self.i < len(self.s) and self.s[self.i].isdigit():
            self.i += 1
        if j == self.i:
            raise self.fail("expected an integer")
        return int(self.s[j : self.i])

    def atom(self):
        c = self.peek()
        if c == "(":
            self.i += 1
            inner = self.alternatives()
            if self.peek() != ")":
                raise self.fail("unbalanced '('")
            self.i += 1
            return inner
        if c == '"':
            return self.literal()
        if c == "[":
            return self.char_class()
        if c and c in _NAME0:
            return Ref(self.name())
        raise self.fail(f"unexpected character {c!r}")

    def literal(self):
        self.i += 1  # opening quote
        cps = []
        while self.i < len(self.s) and self.s[self.i] != '"':
            cps.append(self.char())
        if self.i >= len(self.s):
            raise self.fail("unterminated string")
        self.i += 1
        if not cps:
            return Empty()
        parts = [CharSet(((cp, cp),)) for cp in cps]
        return parts[0] if len(parts) == 1 else Concat(tuple(parts))

    def char_class(self):
        self.i += 1  # '['
        neg = self.i < len(self.s) and self.s[self.i] == "^"
        if neg:
            self.i += 1
        spans = []
        n = len(self.s)
        while self.i < n and self.s[self.i] != "]":
            lo = self.char()
            if self.i + 1 < n and self.s[self.i] == "-" and self.s[self.i + 1] != "]":
                self.i += 1
                hi = self.char()
                if hi < lo:
                    raise self.fail("char class range out of order")
                spans.append((lo, hi))
            else:
                spans.append((lo, lo))
        if self.i >= n:
            raise self.fail("unterminated char class")
        self.i += 1
        merged = merge_ranges(spans)
        return CharSet(complement(merged) if neg else merged)

    def char(self) -> int:
        c = self.s[self.i]
        self.i += 1
        if c != "\\":
            return ord(c)
        if self.i >= len(self.s):
            raise self.fail("trailing backslash")
        e = self.s[self.i]
        self.i += 1
        if e in _ESC:
            return _ESC[e]
        width = {"x": 2, "u": 4, "U": 8}.get(e)
        if width is None:
            return ord(e)
        if self.i + width > len(self.s):
            raise self.fail(f"expected {width} hex digits")
        chunk = self.s[self.i : self.i + width]
        try:
            v = int(chunk, 16)
        except ValueError as exc:
            raise self.fail(f"bad hex escape {chunk!r}") from exc
        self.i += width
        return v


def parse_gbnf(text: str, root: str = "root") -> Grammar:
    """Parse GBNF source into a :class:`Grammar`."""
    return Grammar(rules=_Lexer(text).grammar(), root=root)


__all__ = ["GBNFSyntaxError", "parse_gbnf", "Alt", "CharSet", "Concat", "Empty", "Opt", "Plus", "Ref", "Star"]

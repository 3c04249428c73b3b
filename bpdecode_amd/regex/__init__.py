"""Regex front-end: pattern -> AST -> UTF-8 byte DFA over symbol classes."""

from .compile import DFA, compile_ast, compile_regex
from .parser import RegexSyntaxError, parse

__all__ = ["DFA", "RegexSyntaxError", "compile_ast", "compile_regex", "parse"]

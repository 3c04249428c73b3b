"""Context-free grammars: GBNF / JSON Schema front-ends, the compiled rule
NFAs, the flattened device tables and the batched PDA step."""

from __future__ import annotations

from .constraint import CFGConstraint
from .gbnf import GBNFSyntaxError, parse_gbnf
from .ir import Grammar, Ref
from .json_schema import JsonSchemaError, json_schema_to_grammar
from .pda import PDA, CompiledGrammar, PDAOverflow

__all__ = [
    "CFGConstraint", "CompiledGrammar", "GBNFSyntaxError", "Grammar", "JsonSchemaError",
    "PDA", "PDAOverflow", "Ref", "json_schema_to_grammar", "parse_gbnf",
]

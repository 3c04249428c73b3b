"""Context-free grammars: GBNF / JSON Schema front-ends, the compiled rule
NFAs, the flattened device tables and the batched PDA step."""

from __future__ import annotations

from .gbnf import GBNFSyntaxError, parse_gbnf
from .ir import Grammar, Ref
from .json_schema import JsonSchemaError, json_schema_to_grammar
from .pda import CompiledGrammar

__all__ = [
    "CompiledGrammar", "GBNFSyntaxError", "Grammar", "JsonSchemaError", "Ref",
    "json_schema_to_grammar", "parse_gbnf",
]

"""JSON Schema subset -> :class:`Grammar` (grammar/json_schema.py:42-223 of the
reference).

Supported: ``type`` (object/array/string/number/integer/boolean/null),
``properties``/``required``/``additionalProperties``, ``items`` with
``minItems``/``maxItems``, ``enum``, ``const``, string ``pattern`` and
``minLength``/``maxLength``, ``anyOf``/``oneOf``, and local ``$ref`` into
``$defs``/``definitions``.  Objects are emitted in schema property order.
The primitive rules come first, then ``$ref`` targets in resolution order,
then the root rule: that order fixes the flattened PDA's state ids.
"""

from __future__ import annotations

import json
from typing import Any

from ..regex.parser import parse as parse_regex
from .ir import Alt, CharSet, Concat, Empty, Grammar, Opt, Ref, Star

__all__ = ["json_schema_to_grammar", "JsonSchemaError"]


class JsonSchemaError(ValueError):
    """Unsupported or malformed schema."""


def _text(s: str):
    parts = [CharSet(((ord(c), ord(c)),)) for c in s]
    if not parts:
        return Empty()
    return parts[0] if len(parts) == 1 else Concat(tuple(parts))


def _json_text(value: Any):
    return _text(json.dumps(value, separators=(",", ":")))


# Same rule set and rule order as the reference's primitive block.
_PRIMITIVES = r"""
ws        ::= [ \t\n\r]*
json-value ::= json-object | json-array | json-string | json-number | "true" | "false" | "null"
json-object ::= "{" ws (json-member (ws "," ws json-member)*)? ws "}"
json-member ::= json-string ws ":" ws json-value
json-array ::= "[" ws (json-value (ws "," ws json-value)*)? ws "]"
json-string ::= "\"" json-char* "\""
json-char  ::= [^"\\\x00-\x1F] | "\\" (["\\/bfnrt] | "u" hex hex hex hex)
hex        ::= [0-9a-fA-F]
json-number ::= "-"? json-int json-frac? json-exp?
json-int   ::= "0" | [1-9] [0-9]*
json-frac  ::= "." [0-9]+
json-exp   ::= [eE] [+-]? [0-9]+
"""


class _SchemaCompiler:
    def __init__(self, defs: dict) -> None:
        self.rules: dict = {}
        self.defs = defs
        self.ref_names: dict[str, str] = {}

    def compile(self, schema: Any):
        if schema is True or schema == {}:
            return Ref("json-value")
        if schema is False:
            raise JsonSchemaError("schema `false` matches nothing")
        if not isinstance(schema, dict):
            raise JsonSchemaError(f"schema must be an object, got {type(schema).__name__}")
        if "$ref" in schema:
            return Ref(self.resolve(schema["$ref"]))
        if "const" in schema:
            return _json_text(schema["const"])
        if "enum" in schema:
            return Alt(tuple(_json_text(v) for v in schema["enum"]))
        for key in ("anyOf", "oneOf"):
            if key in schema:
                return Alt(tuple(self.compile(s) for s in schema[key]))
        t = schema.get("type")
        if isinstance(t, list):
            return Alt(tuple(self.compile({**schema, "type": one}) for one in t))
        if t is None:
            return Ref("json-value")
        if t == "object":
            return self.obj(schema)
        if t == "array":
            return self.array(schema)
        if t == "string":
            return self.string(schema)
        if t == "number":
            return Ref("json-number")
        if t == "integer":
            return Concat((Opt(_text("-")), Ref("json-int")))
        if t == "boolean":
            return Alt((_text("true"), _text("false")))
        if t == "null":
            return _text("null")
        raise JsonSchemaError(f"unsupported type {t!r}")

    def resolve(self, ref: str) -> str:
        if ref in self.ref_names:
            return self.ref_names[ref]
        for prefix in ("#/$defs/", "#/definitions/"):
            if ref.startswith(prefix):
                key = ref[len(prefix):]
                if key not in self.defs:
                    raise JsonSchemaError(f"$ref target not found: {ref}")
                name = f"_def_{key}"
                self.ref_names[ref] = name
                self.rules[name] = Empty()  # placeholder: breaks reference cycles
                self.rules[name] = self.compile(self.defs[key])
                return name
        raise JsonSchemaError(f"unsupported $ref: {ref}")

    def obj(self, schema: dict):
        props = list(schema.get("properties", {}).items())
        required = set(schema.get("required", []))
        extra = schema.get("additionalProperties", True)

        def tail(i: int, seen: bool):
            if i == len(props):
                return self.extra_members(extra, seen)
            name, sub = props[i]
            kv = Concat((_json_text(name), Ref("ws"), _text(":"), Ref("ws"), self.compile(sub)))
            head = Concat((Ref("ws"), _text(","), Ref("ws"), kv)) if seen else kv
            present = Concat((head, tail(i + 1, True)))
            return present if name in required else Alt((tail(i + 1, seen), present))

        return Concat((_text("{"), Ref("ws"), tail(0, False), Ref("ws"), _text("}")))

    def extra_members(self, extra: Any, seen: bool):
        if extra is False:
            return Empty()
        value = Ref("json-value") if extra is True else self.compile(extra)
        member = Concat((Ref("json-string"), Ref("ws"), _text(":"), Ref("ws"), value))
        more = Concat((Ref("ws"), _text(","), Ref("ws"), member))
        return Star(more) if seen else Opt(Concat((member, Star(more))))

    def array(self, schema: dict):
        item = self.compile(schema.get("items", True))
        lo = int(schema.get("minItems", 0))
        hi = schema.get("maxItems")
        more = Concat((Ref("ws"), _text(","), Ref("ws"), item))
        if hi is None:
            if lo == 0:
                body = Opt(Concat((item, Star(more))))
            elif lo == 1:
                body = Concat((item, Star(more)))
            else:
                body = Concat((item, Concat((*([more] * (lo - 1)), Star(more)))))
        else:
            hi = int(hi)
            if hi < lo:
                raise JsonSchemaError("maxItems < minItems")
            opts = [Empty() if n == 0 else Concat((item, *([more] * (n - 1))))
                    for n in range(lo, hi + 1)]
            body = opts[0] if len(opts) == 1 else Alt(tuple(opts))
        return Concat((_text("["), Ref("ws"), body, Ref("ws"), _text("]")))

    def string(self, schema: dict):
        if "pattern" in schema:
            inner = parse_regex(schema["pattern"])
            return Concat((_text('"'), inner if inner is not None else Empty(), _text('"')))
        lo, hi = schema.get("minLength"), schema.get("maxLength")
        if lo is None and hi is None:
            return Ref("json-string")
        lo = int(lo or 0)
        ch = Ref("json-char")
        parts = [ch] * lo
        if hi is None:
            parts.append(Star(ch))
        else:
            parts.extend([Opt(ch)] * (int(hi) - lo))
        body = Empty() if not parts else (parts[0] if len(parts) == 1 else Concat(tuple(parts)))
        return Concat((_text('"'), body, _text('"')))


def json_schema_to_grammar(schema: Any, *, root: str = "root") -> Grammar:
    from .gbnf import parse_gbnf

    prims = dict(parse_gbnf(_PRIMITIVES + '\nroot ::= "x"').rules)
    del prims["root"]
    defs = {}
    if isinstance(schema, dict):
        defs = schema.get("$defs") or schema.get("definitions") or {}
    c = _SchemaCompiler(defs)
    c.rules.update(prims)
    body = c.compile(schema)
    c.rules[root] = body
    return Grammar(rules=c.rules, root=root)

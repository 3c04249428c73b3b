"""The C declarations of include/bpdecode_hip.h, the ctypes table the package
binds them with (``_lib._SIGNATURES`` and the structure classes) and the
ctypes stub INTEGRATION.md shows a maintainer agree argument for argument:
same count, same kind and width in every position, and every call in the
stub passes as many arguments as its ``argtypes`` declare.  No device call."""

from __future__ import annotations

import ast
import ctypes as C
import re
from pathlib import Path

import pytest

from bpdecode_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "bpdecode_hip.h"
INTEGRATION = ROOT / "INTEGRATION.md"

# C scalar spellings -> the category ctypes must use for them
_C_SCALARS = {
    "int": "i32", "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64",
    "size_t": "u64", "double": "f64", "float": "f32", "void": "void",
}


def _ctype_kind(t) -> str:
    if t is None:
        return "void"
    if t in (C.c_void_p, C.c_char_p) or (isinstance(t, type) and issubclass(t, C._Pointer)):
        return "ptr"
    size = C.sizeof(t)
    if t in (C.c_float, C.c_double):
        return f"f{8 * size}"
    signed = t(-1).value < 0
    return f"{'i' if signed else 'u'}{8 * size}"


def _c_kind(decl: str) -> str:
    decl = decl.strip()
    if "*" in decl:
        return "ptr"
    words = [w for w in re.findall(r"\w+", decl) if w not in ("const", "struct", "unsigned")]
    if not words:
        raise ValueError(f"cannot read C declaration {decl!r}")
    return _C_SCALARS[words[0]]


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def header_functions() -> dict[str, tuple[str, list[str]]]:
    """name -> (return kind, parameter kinds) of every ``bpd_*`` prototype."""
    text = _strip_comments(HEADER.read_text())
    text = re.sub(r"#[^\n]*", " ", text)
    out = {}
    for ret, name, params in re.findall(r"([\w\s\*]+?)\b(bpd_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = ret.split(";")[-1].split("}")[-1]
        params = params.strip()
        kinds = [] if params in ("", "void") else [
            _c_kind(re.sub(r"\b\w+\s*$", "", p.strip()) if "*" not in p.split()[-1] else p)
            for p in params.split(",")]
        out[name] = (_c_kind(ret), kinds)
    return out


def header_structs() -> dict[str, list[str]]:
    """struct name -> field kinds in declaration order."""
    text = _strip_comments(HEADER.read_text())
    out = {}
    for body, name in re.findall(r"typedef\s+struct\s+\w*\s*\{(.*?)\}\s*(\w+)\s*;", text, re.S):
        kinds = []
        for line in body.split(";"):
            line = line.strip()
            if not line:
                continue
            m = re.match(r"((?:const\s+)?[\w]+\s*\*?)\s*(.*)$", line)
            base, names = m.group(1), m.group(2)
            for n in names.split(","):
                kinds.append("ptr" if ("*" in base or n.strip().startswith("*")) else _c_kind(base))
        out[name] = kinds
    return out


def _struct_kinds(cls) -> list[str]:
    return [_ctype_kind(t) for _, t in cls._fields_]


def test_header_prototypes_match_the_binding_table():
    decl = header_functions()
    assert len(decl) >= 40
    assert set(decl) == set(_lib._SIGNATURES), (sorted(set(decl) ^ set(_lib._SIGNATURES)))
    for name, (ret, params) in decl.items():
        res, args = _lib._SIGNATURES[name]
        assert _ctype_kind(res) == ret, f"{name}: return {ret} in the header, {res} bound"
        got = [_ctype_kind(a) for a in args]
        assert got == params, f"{name}: header {params} != bound {got}"


def test_header_structs_match_the_binding_classes():
    structs = header_structs()
    pairs = {"BpdPdaTable": _lib.PdaTableC, "BpdPdaFrames": _lib.PdaFramesC,
             "BpdTokenBytes": _lib.TokenBytesC, "BpdFsaTable": _lib.FsaTableC,
             "BpdSoftClasses": _lib.SoftClassesC}
    assert set(structs) == set(pairs)
    for name, cls in pairs.items():
        assert _struct_kinds(cls) == structs[name], name


def _integration_blocks() -> list[str]:
    return re.findall(r"```python\n(.*?)```", INTEGRATION.read_text(), re.S)


def test_integration_stub_matches_the_header():
    """Every ``argtypes`` the INTEGRATION.md stub sets equals the header's
    parameter list, its structure classes equal the header's layouts, and
    each call passes as many arguments as the function takes."""
    decl = header_functions()
    structs = header_structs()
    ns = {"C": C, "vp": C.c_void_p, "i32": C.c_int32, "i64": C.c_int64, "f64": C.c_double,
          "f32": C.c_float, "sz": C.c_size_t}
    seen = 0
    calls = 0
    for block in _integration_blocks():
        tree = ast.parse(block)
        for node in ast.walk(tree):
            if isinstance(node, ast.ClassDef) and any(
                    isinstance(b, ast.Attribute) and b.attr == "Structure" for b in node.bases):
                exec(compile(ast.Module([node], []), "<stub>", "exec"), ns)
                cname = {"FsaTableC": "BpdFsaTable", "PdaTableC": "BpdPdaTable",
                         "SoftClassesC": "BpdSoftClasses", "TokenBytesC": "BpdTokenBytes",
                         "PdaFramesC": "BpdPdaFrames"}[node.name]
                assert _struct_kinds(ns[node.name]) == structs[cname], node.name
        for node in ast.walk(tree):
            if (isinstance(node, ast.Assign) and isinstance(node.targets[0], ast.Attribute)
                    and node.targets[0].attr == "argtypes"):
                name = node.targets[0].value.attr
                kinds = [_ctype_kind(t) for t in eval(compile(ast.Expression(node.value), "<stub>", "eval"), ns)]
                assert kinds == decl[name][1], f"INTEGRATION.md {name}: {kinds} != header {decl[name][1]}"
                seen += 1
            if (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute)
                    and node.func.attr.startswith("bpd_") and not node.keywords):
                name = node.func.attr
                assert len(node.args) == len(decl[name][1]), (
                    f"INTEGRATION.md calls {name} with {len(node.args)} arguments, "
                    f"the header declares {len(decl[name][1])}")
                calls += 1
    assert seen >= 3 and calls >= 3


@pytest.mark.parametrize("decl,kind", [("const int32_t* p", "ptr"), ("int64_t rows", "i64"),
                                       ("double neg_inf", "f64"), ("size_t n", "u64"),
                                       ("BpdSoftClasses* out", "ptr"), ("int dtype", "i32")])
def test_c_kind_reader(decl, kind):
    base = decl if "*" in decl else re.sub(r"\b\w+\s*$", "", decl)
    assert _c_kind(base) == kind

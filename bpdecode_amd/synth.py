"""Seeded synthetic workloads of the constraint step: vocabularies, grammars,
starting states / config-sets and logits.  Every generator takes an explicit
seed so the same workload can be rebuilt on any machine.

Vocabularies: ids 0-255 are the single bytes 0x00-0xFF, ids 256..V-2 random
printable strings, id V-1 is EOS (bytes ``</s>``; EOS is decided by id).
"""

from __future__ import annotations

import string

import numpy as np
import torch

from .tokenizer import Vocabulary

IPV4 = r"([0-9]{1,3}\.){3}[0-9]{1,3}"
EMAIL = r"[a-z0-9._]{1,32}@[a-z0-9-]{1,24}\.(com|org|net|io)"

FLAT_SCHEMA = {
    "type": "object",
    "properties": {
        "name": {"type": "string", "maxLength": 24},
        "year": {"type": "integer"},
        "compiled": {"type": "boolean"},
    },
    "required": ["name", "year", "compiled"],
    "additionalProperties": False,
}

# Recursive JSON values.  Whitespace is an inline character class (no rule
# frame), so an object nesting level costs three frames (value, object,
# member) and an array level two.
JSON_GBNF = r"""
root   ::= value
value  ::= object | array | string | number | "true" | "false" | "null"
object ::= "{" [ \t\n]* ( member ( [ \t\n]* "," [ \t\n]* member )* [ \t\n]* )? "}"
member ::= string [ \t\n]* ":" [ \t\n]* value
array  ::= "[" [ \t\n]* ( value ( [ \t\n]* "," [ \t\n]* value )* [ \t\n]* )? "]"
string ::= "\"" ( [^"\\\x00-\x1F] | "\\" ["\\/bfnrt] )* "\""
number ::= "-"? ( "0" | [1-9] [0-9]* ) ( "." [0-9]+ )? ( [eE] [+-]? [0-9]+ )?
"""

_LOWER = string.ascii_lowercase
_UPPER = string.ascii_uppercase
_DIGITS = string.digits
_PUNCT = '{}[]:,."@'


def _other(exclude: str) -> str:
    return "".join(chr(c) for c in range(0x21, 0x7F) if chr(c) not in exclude)


# (class chars, probability) per vocabulary family
MIX_IPV4 = [(_DIGITS, 0.20), (".", 0.10), (_LOWER, 0.40), (" ", 0.10),
            (_other(_DIGITS + "." + _LOWER), 0.20)]
MIX_SERVING = [(_LOWER, 0.40), (_DIGITS, 0.10), (_PUNCT, 0.15), (" ", 0.10), (_UPPER, 0.10),
               (_other(_LOWER + _DIGITS + _PUNCT + _UPPER), 0.15)]


def synthetic_vocab(size: int, seed: int, min_len: int, max_len: int, mix) -> Vocabulary:
    """``size`` tokens: 256 single bytes, random strings with lengths uniform
    in [min_len, max_len] whose characters draw a class by ``mix`` weight
    then a character uniformly within it, and EOS last."""
    rng = np.random.default_rng(seed)
    n = size - 257
    lens = rng.integers(min_len, max_len + 1, size=n)
    total = int(lens.sum())
    probs = np.array([p for _, p in mix], dtype=np.float64)
    cls = rng.choice(len(mix), size=total, p=probs / probs.sum())
    out = np.empty(total, dtype=np.uint8)
    for k, (chars, _) in enumerate(mix):
        pick = np.nonzero(cls == k)[0]
        table = np.frombuffer(chars.encode(), dtype=np.uint8)
        out[pick] = table[rng.integers(0, len(table), size=pick.size)]
    raw = out.tobytes()
    ends = np.cumsum(lens)
    starts = ends - lens
    toks = [bytes([b]) for b in range(256)]
    toks += [raw[s:e] for s, e in zip(starts.tolist(), ends.tolist())]
    toks.append(b"</s>")
    return Vocabulary(tuple(toks), eos_id=size - 1)


def ipv4_vocab(size: int = 32_000, seed: int = 0) -> Vocabulary:
    return synthetic_vocab(size, seed, 2, 8, MIX_IPV4)


def serving_vocab(size: int = 151_936, seed: int = 1) -> Vocabulary:
    return synthetic_vocab(size, seed, 2, 12, MIX_SERVING)


def random_walk_states(tok_next: torch.Tensor, start: int, eos_id: int, rows: int,
                       max_steps: int, seed: int) -> torch.Tensor:
    """Per row: ``U[0, max_steps]`` uniformly random allowed non-EOS tokens
    from ``start`` (stopping early where nothing but EOS is allowed)."""
    rng = np.random.default_rng(seed)
    tn = tok_next.cpu().numpy()
    allowed = {}
    out = np.empty(rows, dtype=np.int32)
    for r in range(rows):
        s = start
        for _ in range(int(rng.integers(0, max_steps + 1))):
            ids = allowed.get(s)
            if ids is None:
                ids = np.nonzero(tn[s] >= 0)[0]
                ids = allowed[s] = ids[ids != eos_id]
            if ids.size == 0:
                break
            s = int(tn[s, ids[int(rng.integers(0, ids.size))]])
        out[r] = s
    return torch.from_numpy(out)


def random_byte_walk_states(tok_next: torch.Tensor, start: int, rows: int, max_bytes: int,
                            seed: int) -> torch.Tensor:
    """Per row: the state after a random valid partial document of
    ``U[0, max_bytes]`` bytes -- each byte drawn uniformly among the
    single-byte tokens (ids 0-255) the current state allows (stopping early
    where none is allowed)."""
    rng = np.random.default_rng(seed)
    tn = tok_next.cpu().numpy()[:, :256]
    allowed = {}
    out = np.empty(rows, dtype=np.int32)
    for r in range(rows):
        s = start
        for _ in range(int(rng.integers(0, max_bytes + 1))):
            ids = allowed.get(s)
            if ids is None:
                ids = allowed[s] = np.nonzero(tn[s] >= 0)[0]
            if ids.size == 0:
                break
            s = int(tn[s, ids[int(rng.integers(0, ids.size))]])
        out[r] = s
    return torch.from_numpy(out)


def logits(rows: int, vocab: int, std: float, dtype: torch.dtype, seed: int, device="cpu") -> torch.Tensor:
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, vocab, generator=g) * std
    return x.to(dtype).to(device)


def json_prefix(rng: np.random.Generator, depth: int, max_len: int = 200) -> bytes:
    """A valid prefix of a JSON document with ``depth`` containers open at its
    end, at most ``max_len`` bytes."""
    ws = lambda: rng.choice(["", "", " ", "\n"])  # noqa: E731
    word = lambda: "".join(rng.choice(list(_LOWER + _DIGITS), size=int(rng.integers(1, 7))))  # noqa: E731
    scalar = lambda: str(rng.choice([f'"{word()}"', str(int(rng.integers(-999, 9999))), "true",  # noqa: E731
                                     "false", "null", f"{rng.integers(0, 99)}.{rng.integers(0, 99)}"]))
    parts: list[str] = []
    for _ in range(depth):
        if rng.random() < 0.5:
            parts.append("[" + ws())
            for _ in range(int(rng.integers(0, 3))):
                parts.append(scalar() + ws() + "," + ws())
        else:
            parts.append("{" + ws())
            for _ in range(int(rng.integers(0, 3))):
                parts.append(f'"{word()}"' + ws() + ":" + ws() + scalar() + ws() + "," + ws())
            parts.append(f'"{word()}"' + ws() + ":" + ws())
    tail = rng.choice(["", f'"{word()[:3]}', str(int(rng.integers(0, 99))), "tr", "nu", ""])
    text = "".join(parts) + str(tail)
    data = text.encode()
    if len(data) > max_len:
        data = data[:max_len]
    return data

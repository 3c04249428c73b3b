"""Code-point ranges -> UTF-8 byte-range sequences.

A range ``[lo, hi]`` of scalars becomes a list of sequences of inclusive byte
ranges whose concatenations decode to exactly those scalars (surrogates
excluded).  The order of the sequences is fixed because the NFA builders
create one state chain per sequence, in list order, and the flattened PDA
table's state ids and edge order depend on it.  The order is the one of
regex/utf8.py:333-392: for each surrogate-free piece and each equal-length
split, the byte positions are refined left to right; at a position where the
two endpoints differ, the low-edge branch comes first, then the high-edge
branch, then the interior span.
"""

from __future__ import annotations

UNICODE_MAX = 0x10FFFF
_LEN_LIMITS = (0x7F, 0x7FF, 0xFFFF)
_CONT_LO, _CONT_HI = 0x80, 0xBF


def encode(cp: int) -> list[int]:
    """UTF-8 bytes of scalar ``cp``."""
    return list(chr(cp).encode("utf-8", "surrogatepass"))


def _without_surrogates(lo: int, hi: int) -> list[tuple[int, int]]:
    lo, hi = max(lo, 0), min(hi, UNICODE_MAX)
    if lo > hi:
        return []
    pieces = []
    if lo < 0xD800:
        pieces.append((lo, min(hi, 0xD7FF)))
    if hi > 0xDFFF:
        pieces.append((max(lo, 0xE000), hi))
    return pieces


def _same_length_pieces(lo: int, hi: int) -> list[tuple[int, int]]:
    pieces = []
    for limit in _LEN_LIMITS:
        if lo <= limit < hi:
            pieces.append((lo, limit))
            lo = limit + 1
    pieces.append((lo, hi))
    return pieces


def _refine(lo_b, hi_b, pos, pin_lo, pin_hi, prefix, out) -> None:
    n = len(lo_b)
    if not pin_lo and not pin_hi:
        out.append(prefix + ((_CONT_LO, _CONT_HI),) * (n - pos))
        return
    a = lo_b[pos] if pin_lo else _CONT_LO
    b = hi_b[pos] if pin_hi else _CONT_HI
    if pos == n - 1:
        out.append(prefix + ((a, b),))
        return
    if a == b:
        _refine(lo_b, hi_b, pos + 1, pin_lo, pin_hi, prefix + ((a, a),), out)
        return
    # an endpoint whose remaining bytes already cover the full continuation
    # span merges into the interior instead of getting its own branch
    lo_whole = pin_lo and all(x == _CONT_LO for x in lo_b[pos + 1 :])
    hi_whole = pin_hi and all(x == _CONT_HI for x in hi_b[pos + 1 :])
    if not lo_whole:
        _refine(lo_b, hi_b, pos + 1, pin_lo, False, prefix + ((a, a),), out)
    if not hi_whole:
        _refine(lo_b, hi_b, pos + 1, False, pin_hi, prefix + ((b, b),), out)
    mid_lo = a if lo_whole else a + 1
    mid_hi = b if hi_whole else b - 1
    if mid_lo <= mid_hi:
        out.append(prefix + ((mid_lo, mid_hi),) + ((_CONT_LO, _CONT_HI),) * (n - 1 - pos))


def utf8_sequences(lo: int, hi: int) -> list[tuple[tuple[int, int], ...]]:
    """Byte-range sequences matching exactly the scalars in ``[lo, hi]``."""
    out: list[tuple[tuple[int, int], ...]] = []
    for a, b in _without_surrogates(lo, hi):
        for x, y in _same_length_pieces(a, b):
            _refine(encode(x), encode(y), 0, True, True, (), out)
    return out

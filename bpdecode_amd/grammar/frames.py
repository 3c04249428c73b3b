"""Stack-relative config lists of the PDA mask's fast path (no counterpart in
the reference; an acceleration of pda_try_token, pda.hpp:248-258).

A config-set whose configs all sit on one common stack ``P`` is the ordered
list of the configs' *suffixes* above ``P`` (each at least one frame).  As
long as no config pops into ``P`` (a suffix of one frame whose top state
accepts) the bounded step, the closure and the compaction act on the
suffixes alone: a byte step takes each top's byte edges in config and edge
order, the closure takes epsilon edges, pushes callees and pops accepting
tops inside the suffix, all of them skipping configs already in the list and
stopping at 8 configs (the ones a full set drops), and the compaction drops
configs whose top is not live.  Suffixes are kept to ``MAX_SUFFIX`` frames
(a push beyond ends the list's knowledge) and every absolute depth stays
below the set limit when ``|P| + MAX_SUFFIX <= 32``.

:func:`frame_lists` enumerates such lists breadth-first from the closure of
every single state, with their byte transitions, and classifies every token
from every list as *inside* (each byte keeps the list non-empty without a
pop into ``P`` or a push beyond ``MAX_SUFFIX``: allowed), *dead* (the list
empties first: rejected) or *boundary* (it needs ``P``: the device walks it
through the real sets; EOS and the empty tokens, whose verdicts depend on
the whole set, are boundary too).  The device matches a set against the
lists at its longest common stack and at up to ``MAX_SUFFIX - 1`` frames
below it (most specific first), through a hash table of the keys.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

MAX_SUFFIX = 4  # frames of a suffix
SLOTS = 1024  # hash-table slots (staged in LDS by the mask kernel)
MAX_LISTS = 700  # at most 0.7 * SLOTS keys
KEY_WORDS = 48  # n, 8 suffix lengths, 8 x MAX_SUFFIX frames, padding
SAT = 0x10000  # transition flag: the step dropped a config at the 8-config cap
EMPTY = 0xFFFFFFFF
_EPS, _BYTE, _CALL = 0, 1, 2
_DEAD, _BOUNDARY = -1, -2
_CAP = 8  # configs per set
_MAXD = 32  # frames per config


@dataclass
class FrameLists:
    keys: np.ndarray  # int32 [L, KEY_WORDS]
    slots: np.ndarray  # uint32 [SLOTS]: list id | fingerprint << 12, EMPTY
    trans: np.ndarray  # int32 [L, 256]: list reached (| SAT), -1 empty, -2 boundary
    allowed: np.ndarray  # uint32 [L, ceil(V/32)]
    seed_off: np.ndarray  # int32 [L + 1]
    seeds: np.ndarray  # int32 walk positions

    @property
    def num_lists(self) -> int:
        return int(self.keys.shape[0])


# ------------------------------------------------------------------ hash --
def _mix32(x: int) -> int:
    x &= 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x


def list_hash(lst) -> int:
    """Hash of a list of suffixes, as the device computes it: a sum of
    per-word mixes salted by (config, position), so lanes can add their
    words in any order."""
    h = _mix32(0xC2B2AE35 ^ len(lst))
    for i, sfx in enumerate(lst):
        h += _mix32((((i << 8) | 0xFF) * 0x85EBCA6B) ^ len(sfx))
        for k, f in enumerate(sfx):
            h += _mix32((((i << 8) | k) * 0x9E3779B1) ^ (f & 0xFFFFFFFF))
    return _mix32(h & 0xFFFFFFFF)


# ------------------------------------------------------------- the steps --
class _Tables:
    def __init__(self, g) -> None:
        c = lambda t: t.cpu().numpy()  # noqa: E731
        self.accept = c(g.accept).astype(bool)
        self.live = c(g.live).astype(bool)
        off = c(g.edge_offsets).astype(np.int64)
        kind, lo, hi = c(g.edge_kind), c(g.edge_lo), c(g.edge_hi)
        dst, callee = c(g.edge_dst), c(g.edge_callee)
        n = len(self.accept)
        # per state: byte edges (lo, hi, dst) and closure edges (kind, dst, callee), in edge order
        self.byte = [[(int(lo[e]), int(hi[e]), int(dst[e])) for e in range(off[s], off[s + 1])
                      if kind[e] == _BYTE] for s in range(n)]
        self.clos = [[(int(kind[e]), int(dst[e]), int(callee[e])) for e in range(off[s], off[s + 1])
                      if kind[e] != _BYTE] for s in range(n)]


def _add(nxt: list, x: tuple) -> bool:
    """Append x unless present; False when the list is full (x dropped)."""
    if x in nxt:
        return True
    if len(nxt) >= _CAP:
        return False
    nxt.append(x)
    return True


def _close(t: _Tables, nxt: list, sat: bool, lmax: int):
    """Closure and compaction of a suffix list (close() and prune_dead() of
    pda_core.hpp over the suffixes), and whether a config was dropped at the
    cap; BOUNDARY when a config pops into the common stack or pushes beyond
    ``lmax`` frames, DEAD when no config is left."""
    i = 0
    while i < len(nxt):
        sfx = nxt[i]
        top = sfx[-1]
        if t.accept[top]:
            if len(sfx) == 1:
                return _BOUNDARY, sat
            sat = not _add(nxt, sfx[:-1]) or sat
        for kind, dst, callee in t.clos[top]:
            if kind == _EPS:
                sat = not _add(nxt, sfx[:-1] + (dst,)) or sat
            else:
                if len(sfx) + 1 > lmax:
                    return _BOUNDARY, sat
                sat = not _add(nxt, sfx[:-1] + (dst, callee)) or sat
        i += 1
    out = tuple(s for s in nxt if t.live[s[-1]])
    return (out if out else _DEAD), sat


def _step(t: _Tables, lst: tuple, byte: int, lmax: int):
    nxt: list = []
    sat = False
    for sfx in lst:
        for lo, hi, dst in t.byte[sfx[-1]]:
            if lo <= byte <= hi:
                sat = not _add(nxt, sfx[:-1] + (dst,)) or sat
    return _close(t, nxt, sat, lmax)


def _enumerate(t: _Tables, lmax: int, limit: int) -> tuple[list, np.ndarray]:
    """Lists reachable from the closure of every single state (breadth
    first, at most ``limit``) and their byte transitions."""
    lists: list = []
    index: dict = {}
    for s in range(len(t.accept)):
        r, _ = _close(t, [(s,)], False, lmax)
        if isinstance(r, tuple) and r not in index and len(lists) < limit:
            index[r] = len(lists)
            lists.append(r)
    rows = []
    head = 0
    while head < len(lists):
        row = []
        memo: dict = {}
        lst = lists[head]
        for byte in range(256):
            # bytes over the same byte edges step alike
            sig = tuple(lo <= byte <= hi for sfx in lst for lo, hi, _ in t.byte[sfx[-1]])
            if sig in memo:
                row.append(memo[sig])
                continue
            nx, sat = _step(t, lst, byte, lmax)
            if isinstance(nx, tuple):
                if nx not in index:
                    if len(lists) >= limit:
                        memo[sig] = _BOUNDARY
                        row.append(_BOUNDARY)
                        continue
                    index[nx] = len(lists)
                    lists.append(nx)
                code = index[nx] | (SAT if sat else 0)
            else:
                code = nx
            memo[sig] = code
            row.append(code)
        rows.append(row)
        head += 1
    return lists, np.array(rows, dtype=np.int32).reshape(len(lists), 256)


def _classify(codes: np.ndarray, g, order: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Inside-token bitmaps, seed offsets and seeds of every list, from the
    native classifier (every token walked from every list)."""
    import ctypes as C
    import os

    from .. import _lib

    L, V = codes.shape[0], g.vocab_size
    off = np.ascontiguousarray(g.tok_offsets.cpu().numpy().astype(np.int32))
    tb = np.ascontiguousarray(g.tok_bytes.cpu().numpy().astype(np.uint8))
    if tb.size == 0:
        tb = np.zeros(1, np.uint8)
    order = np.ascontiguousarray(order.astype(np.int32))
    codes = np.ascontiguousarray(codes.astype(np.int32))
    allowed = np.zeros((L, (V + 31) // 32), dtype=np.uint32)
    count = np.zeros(L, dtype=np.int32)
    threads = min(16, os.cpu_count() or 1)
    p = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    lib = _lib.lib()
    _lib.check(lib.bpd_host_frame_classify(p(codes), L, p(off), p(tb), V, g.eos_id, p(order), p(allowed),
                                           p(count), None, None, threads))
    seed_off = np.zeros(L + 1, dtype=np.int32)
    np.cumsum(count, out=seed_off[1:])
    seeds = np.zeros(max(int(seed_off[-1]), 1), dtype=np.int32)
    _lib.check(lib.bpd_host_frame_classify(p(codes), L, p(off), p(tb), V, g.eos_id, p(order), p(allowed),
                                           p(count), p(seed_off), p(seeds), threads))
    return allowed, seed_off, seeds[:int(seed_off[-1])]


def frame_lists(g, order: np.ndarray, limit: int = MAX_LISTS) -> FrameLists | None:
    """Keys, hash table, transitions, inside-token bitmaps and boundary seeds
    (walk positions of ``order``) of the stack-relative lists of ``g`` (a
    :class:`~bpdecode_amd.grammar.device.PdaTensors`)."""
    if g.num_states == 0 or g.vocab_size == 0:
        return None
    t = _Tables(g)
    lists, codes = _enumerate(t, MAX_SUFFIX, min(limit, MAX_LISTS))
    if not lists:
        return None
    L = len(lists)
    allowed, seed_off, seeds = _classify(codes, g, order)
    keys = np.zeros((L, KEY_WORDS), dtype=np.int32)
    slots = np.full(SLOTS, EMPTY, dtype=np.uint32)
    for i, lst in enumerate(lists):
        keys[i, 0] = len(lst)
        for c, sfx in enumerate(lst):
            keys[i, 1 + c] = len(sfx)
            keys[i, 9 + c * MAX_SUFFIX:9 + c * MAX_SUFFIX + len(sfx)] = sfx
        h = list_hash(lst)
        s = h & (SLOTS - 1)
        while slots[s] != EMPTY:
            s = (s + 1) & (SLOTS - 1)
        slots[s] = np.uint32(i | (((h >> 10) & 0xFFFFF) << 12))
    return FrameLists(
        keys=keys,
        slots=slots,
        trans=np.ascontiguousarray(codes),
        allowed=allowed,
        seed_off=seed_off,
        seeds=seeds,
    )


def frame_match(cfg: np.ndarray, fl: FrameLists) -> tuple[int, int]:
    """The list a flat config-set takes on the device and the depth of the
    common stack it is taken over ((-1, -1): none).  The common stack is
    tried at the configs' longest common prefix below every top and up to
    ``MAX_SUFFIX - 1`` frames shorter, shortest first (longest suffixes),
    each with every suffix at most ``MAX_SUFFIX`` frames and the stack plus
    ``MAX_SUFFIX`` frames within the depth limit."""
    n = int(cfg[0])
    if n < 1 or n > _CAP:
        return -1, -1
    depth = [int(cfg[2 + i]) for i in range(n)]
    if min(depth) < 1 or max(depth) > _MAXD:
        return -1, -1
    frames = cfg[2 + _CAP:].reshape(_CAP, _MAXD)
    p = 0
    while p < min(depth) - 1 and all(frames[i, p] == frames[0, p] for i in range(n)):
        p += 1
    for j in range(min(p, MAX_SUFFIX - 1), -1, -1):
        b = p - j
        if b + MAX_SUFFIX > _MAXD or max(depth) - b > MAX_SUFFIX:
            continue
        lst = tuple(tuple(int(x) for x in frames[i, b:depth[i]]) for i in range(n))
        h = list_hash(lst)
        s = h & (SLOTS - 1)
        while fl.slots[s] != EMPTY:
            e = int(fl.slots[s])
            if (e >> 12) == ((h >> 10) & 0xFFFFF):
                key = fl.keys[e & 0xFFF]
                if int(key[0]) == n and all(
                        int(key[1 + i]) == len(lst[i]) and
                        list(key[9 + i * MAX_SUFFIX:9 + i * MAX_SUFFIX + len(lst[i])]) == list(lst[i])
                        for i in range(n)):
                    return e & 0xFFF, b
            s = (s + 1) & (SLOTS - 1)
    return -1, -1


def frame_list_of(cfg: np.ndarray, fl: FrameLists) -> int:
    """The list a flat config-set takes on the device (-1: none)."""
    return frame_match(cfg, fl)[0]

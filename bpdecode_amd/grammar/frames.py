"""Frame lists of the PDA mask's fast path (no counterpart in the reference;
an acceleration of pda_try_token, pda.hpp:248-258, for one kind of row).

A row whose config-set has every config inside one call-free rule R, all
over the same stack below the top frame, walks a token exactly like the
ordered list of its top states does under the bounded step restricted to R:
a byte step takes each top's byte edges in config and edge order, the
closure takes epsilon edges in the same order, both skip states already in
the list and stop appending at 8 (the configs a full set drops), and the
compaction drops states that are not live -- the stack below never matters
until some top reaches R's accept state, where the set pops into the caller.

For each list reachable from the entry of every call-free rule (and each
token), :func:`frame_lists` therefore classifies the token as *inside*
(every byte keeps the list non-empty and never reaches R's accept: allowed),
*dead* (the list empties first: rejected) or *boundary* (it reaches R's
accept at some byte: the device walks it through the real sets).  The mask
kernel matches a row's list against these keys, takes the inside tokens from
the list's bitmap and walks only the boundary tokens (plus EOS and empty
tokens, whose verdicts depend on the whole set).  A row with another list,
or any config outside R, takes the ordinary walk.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

MAX_LISTS = 64  # the kernel matches a row against all keys with one wave
KEY_WORDS = 9  # n, then up to 8 top states
SAT = 0x10000  # transition flag: the step dropped a state at the 8-config cap
_EPS, _BYTE, _CALL = 0, 1, 2
_DEAD, _BOUNDARY = -1, -2
_CAP = 8  # configs per set


@dataclass
class FrameLists:
    keys: np.ndarray  # int32 [L, 9]
    trans: np.ndarray  # int32 [L, 256]: list reached (| SAT), -1 empty, -2 reaches the accept state
    allowed: np.ndarray  # uint32 [L, ceil(V/32)]
    seed_off: np.ndarray  # int32 [L + 1]
    seeds: np.ndarray  # int32 walk positions

    @property
    def num_lists(self) -> int:
        return int(self.keys.shape[0])


class _Tables:
    def __init__(self, g) -> None:
        c = lambda t: t.cpu().numpy()  # noqa: E731
        self.accept = c(g.accept).astype(bool)
        self.live = c(g.live).astype(bool)
        self.off = c(g.edge_offsets).astype(np.int64)
        self.kind = c(g.edge_kind)
        self.lo = c(g.edge_lo)
        self.hi = c(g.edge_hi)
        self.dst = c(g.edge_dst)

    def edges(self, s: int) -> range:
        return range(int(self.off[s]), int(self.off[s + 1]))


def _add(nxt: list[int], x: int) -> bool:
    """Append x unless present; False when the list is full (x dropped)."""
    if x in nxt:
        return True
    if len(nxt) >= _CAP:
        return False
    nxt.append(x)
    return True


def _close(t: _Tables, nxt: list[int], sat: bool):
    """Closure and compaction of a list inside a call-free rule, and whether
    some state was dropped at the cap; BOUNDARY when some state accepts (its
    config pops into the caller)."""
    i = 0
    while i < len(nxt):
        s = nxt[i]
        if t.accept[s]:
            return _BOUNDARY, sat
        for e in t.edges(s):
            k = int(t.kind[e])
            if k == _CALL:
                return _BOUNDARY, sat  # not call-free after all: leave it to the real walk
            if k == _EPS:
                sat = not _add(nxt, int(t.dst[e])) or sat
        i += 1
    out = tuple(s for s in nxt if t.live[s])
    return (out if out else _DEAD), sat


def _step(t: _Tables, lst: tuple, byte: int):
    nxt: list[int] = []
    sat = False
    for s in lst:
        for e in t.edges(s):
            if int(t.kind[e]) == _BYTE and int(t.lo[e]) <= byte <= int(t.hi[e]):
                sat = not _add(nxt, int(t.dst[e])) or sat
    return _close(t, nxt, sat)


def _rule_lists(t: _Tables, start: int, limit: int) -> tuple[list[tuple], dict]:
    """Lists reachable from the rule's entry by steps that stay inside, in
    breadth-first order (at most ``limit``), and their byte transitions."""
    entry, _ = _close(t, [start], False)
    if not isinstance(entry, tuple):
        return [], {}
    lists = [entry]
    index = {entry: 0}
    trans: dict[int, list[int]] = {}
    head = 0
    while head < len(lists):
        row = []
        for byte in range(256):
            nx, sat = _step(t, lists[head], byte)
            if isinstance(nx, tuple):
                if nx not in index:
                    if len(lists) >= limit:
                        nx = None  # beyond the table: that byte makes the token a boundary one
                    else:
                        index[nx] = len(lists)
                        lists.append(nx)
            if nx is None:
                row.append(_BOUNDARY)
            elif isinstance(nx, tuple):
                row.append(index[nx] | (SAT if sat else 0))
            else:
                row.append(nx)
        trans[head] = row
        head += 1
    return lists, trans


def frame_lists(g, order: np.ndarray, limit: int = MAX_LISTS) -> FrameLists | None:
    """Keys, inside-token bitmaps and boundary seeds (walk positions of
    ``order``) of the lists of every call-free, non-root rule of ``g``
    (a :class:`~bpdecode_amd.grammar.device.PdaTensors` with ``rules``)."""
    if not g.rules:
        return None
    t = _Tables(g)
    keys: list[tuple] = []
    trans_rows: list[list[int]] = []
    for base, n_states, start, _acc, has_calls, is_root in g.rules:
        if has_calls or is_root or len(keys) >= limit:
            continue
        lists, trans = _rule_lists(t, base + start, limit - len(keys))
        shift = len(keys)
        for i, lst in enumerate(lists):
            keys.append(lst)
            trans_rows.append([x + shift if x >= 0 else x for x in trans[i]])  # (SAT is above the ids)
    if not keys:
        return None
    L, V = len(keys), g.vocab_size
    codes = np.array(trans_rows, dtype=np.int32)  # [L, 256]
    table = np.where(codes >= 0, codes & (SAT - 1), codes)
    off = g.tok_offsets.cpu().numpy().astype(np.int64)
    tb = g.tok_bytes.cpu().numpy()
    lens = off[1:] - off[:-1]
    special = lens == 0
    if 0 <= g.eos_id < V:
        special[g.eos_id] = True
    # walk every (list, token) pair one byte position at a time
    state = np.tile(np.arange(L, dtype=np.int32)[:, None], (1, V))  # >= 0 inside, else code
    for p in range(int(lens.max()) if V else 0):
        act = np.nonzero(lens > p)[0]
        if act.size == 0:
            break
        b = tb[off[act] + p].astype(np.int64)
        cur = state[:, act]
        going = cur >= 0
        nxt = np.where(going, table[np.maximum(cur, 0), b[None, :]], cur)
        state[:, act] = nxt
    inside = (state >= 0) & ~special[None, :]
    boundary = (state == _BOUNDARY) | special[None, :]
    words = (V + 31) // 32
    bits = np.zeros((L, words * 32), dtype=bool)
    bits[:, :V] = inside
    allowed = np.packbits(bits, axis=1, bitorder="little").view("<u4")  # bit t of word t >> 5
    pos = np.empty(V, dtype=np.int64)
    pos[order.astype(np.int64)] = np.arange(V)
    seed_parts, seed_off = [], [0]
    for i in range(L):
        s = np.sort(pos[np.nonzero(boundary[i])[0]]).astype(np.int32)
        seed_parts.append(s)
        seed_off.append(seed_off[-1] + s.size)
    key_arr = np.full((L, KEY_WORDS), -1, dtype=np.int32)
    for i, lst in enumerate(keys):
        key_arr[i, 0] = len(lst)
        key_arr[i, 1:1 + len(lst)] = lst
    return FrameLists(
        keys=key_arr,
        trans=np.ascontiguousarray(codes),
        allowed=np.ascontiguousarray(allowed.astype(np.uint32)),
        seed_off=np.array(seed_off, dtype=np.int32),
        seeds=np.concatenate(seed_parts) if seed_parts else np.zeros(0, np.int32),
    )

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

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib

MAX_SUFFIX = 5  # frames of a suffix (BPD_PDA_FRAME_SUFFIX)
SLOTS = 2048  # hash-table slots (staged in LDS by the mask kernel)
MAX_LISTS = 1400  # at most 0.7 * SLOTS keys
KEY_WORDS = 56  # n, 8 suffix lengths, 8 x MAX_SUFFIX frames, padding
SAT = 0x10000  # transition flag: the step dropped a config at the 8-config cap
RAW = 0x20000  # transition flag: the compaction dropped none (stepped words = composed words)
EMPTY = 0xFFFFFFFF
_CAP = 8  # configs per set
_MAXD = 32  # frames per config


@dataclass
class FrameLists:
    """The lists on the tables' device: ``keys`` int32 [L, KEY_WORDS],
    ``slots`` int32 [SLOTS] (uint32 words: list id | fingerprint << 12, or
    EMPTY), ``trans`` int32 [L, 256] (list reached | SAT | RAW, -1 empty, -2
    boundary), ``allowed`` int32 [L, ceil(V/32)] (uint32 words), ``seed_off``
    int32 [L + 1] and ``seeds`` int32 walk positions."""

    keys: torch.Tensor
    slots: torch.Tensor
    trans: torch.Tensor
    allowed: torch.Tensor
    seed_off: torch.Tensor
    seeds: torch.Tensor

    @property
    def num_lists(self) -> int:
        return int(self.keys.shape[0])

    def host(self) -> dict:
        """numpy copies of the arrays (slots and allowed as uint32)."""
        h = self.__dict__.get("_host")
        if h is None:
            h = {n: getattr(self, n).cpu().numpy() for n in ("keys", "slots", "trans", "allowed", "seed_off", "seeds")}
            h["slots"] = h["slots"].view(np.uint32)
            h["allowed"] = h["allowed"].view(np.uint32)
            self.__dict__["_host"] = h
        return h


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


# ------------------------------------------------------------ the build --
def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _classify_host(trans: np.ndarray, g, order: np.ndarray):
    """Inside-token bitmaps, seed offsets and seeds from the native host
    classifier (every token walked from every list, 16 threads at most)."""
    L, V = trans.shape[0], g.vocab_size
    off = np.ascontiguousarray(g.tok_offsets.cpu().numpy().astype(np.int32))
    tb = np.ascontiguousarray(g.tok_bytes.cpu().numpy().astype(np.uint8))
    if tb.size == 0:
        tb = np.zeros(1, np.uint8)
    order = np.ascontiguousarray(order.astype(np.int32))
    allowed = np.zeros((L, (V + 31) // 32), dtype=np.uint32)
    count = np.zeros(L, dtype=np.int32)
    threads = min(16, os.cpu_count() or 1)
    lib = _lib.lib()
    _lib.check(lib.bpd_host_frame_classify(_np_ptr(trans), L, _np_ptr(off), _np_ptr(tb), V, g.eos_id, _np_ptr(order),
                                           _np_ptr(allowed), _np_ptr(count), None, None, threads))
    seed_off = np.zeros(L + 1, dtype=np.int32)
    np.cumsum(count, out=seed_off[1:])
    seeds = np.zeros(max(int(seed_off[-1]), 1), dtype=np.int32)
    _lib.check(lib.bpd_host_frame_classify(_np_ptr(trans), L, _np_ptr(off), _np_ptr(tb), V, g.eos_id, _np_ptr(order),
                                           _np_ptr(allowed), _np_ptr(count), _np_ptr(seed_off), _np_ptr(seeds),
                                           threads))
    t = torch.from_numpy
    return t(allowed.view(np.int32)), t(seed_off), t(seeds[:int(seed_off[-1])])


def _classify_device(trans: torch.Tensor, g, order: torch.Tensor):
    """The same on the tables' device: a counting pass (bitmaps and seeds
    per block of walk positions), prefix sums, a filling pass."""
    dev = g.device
    L, V = int(trans.shape[0]), g.vocab_size
    lib = _lib.lib()
    blocks = int(lib.bpd_frame_classify_blocks(V))
    off = g.tok_offsets.to(dev, torch.int32).contiguous()
    tb = g.tok_bytes.contiguous()
    if tb.numel() == 0:
        tb = torch.zeros(1, dtype=torch.uint8, device=dev)
    order = order.to(dev, torch.int32).contiguous()
    allowed = torch.zeros((L, (V + 31) // 32), dtype=torch.int32, device=dev)
    counts = torch.empty((L, blocks), dtype=torch.int32, device=dev)
    stream = _lib.stream_of(dev)
    p = _lib.ptr
    _lib.check(lib.bpd_frame_classify(p(trans), L, p(off), p(tb), V, g.eos_id, p(order), p(allowed), p(counts),
                                      None, None, stream))
    flat = counts.view(-1).to(torch.int64)
    offsets = torch.cumsum(flat, 0) - flat
    total = int(flat.sum().item())
    seeds = torch.empty(max(total, 1), dtype=torch.int32, device=dev)
    _lib.check(lib.bpd_frame_classify(p(trans), L, p(off), p(tb), V, g.eos_id, p(order), p(allowed), p(counts),
                                      p(offsets), p(seeds), stream))
    seed_off = torch.empty(L + 1, dtype=torch.int32, device=dev)
    seed_off[:L] = offsets.view(L, blocks)[:, 0].to(torch.int32)
    seed_off[L] = total
    return allowed, seed_off, seeds[:total]


def frame_lists(g, order, limit: int = MAX_LISTS) -> FrameLists | None:
    """Keys, hash table, transitions, inside-token bitmaps and boundary seeds
    (walk positions of ``order``) of the stack-relative lists of ``g`` (a
    :class:`~bpdecode_amd.grammar.device.PdaTensors`), on its device: the
    lists are enumerated on the host, the tokens classified where the tables
    are."""
    if g.num_states == 0 or g.vocab_size == 0:
        return None
    host = g if g.device.type == "cpu" else g.to("cpu")
    limit = min(limit, MAX_LISTS)
    keys = np.zeros((limit, KEY_WORDS), dtype=np.int32)
    trans = np.zeros((limit, 256), dtype=np.int32)
    slots = np.zeros(SLOTS, dtype=np.uint32)
    L = int(_lib.lib().bpd_host_frame_lists(C.byref(host.c_table()), limit, _np_ptr(keys), _np_ptr(trans),
                                            _np_ptr(slots)))
    if L < 0:
        _lib.check(-L)
    if L == 0:
        return None
    keys, trans = np.ascontiguousarray(keys[:L]), np.ascontiguousarray(trans[:L])
    order_t = torch.as_tensor(order)
    if g.device.type == "cpu":
        allowed, seed_off, seeds = _classify_host(trans, g, order_t.numpy())
        dev_t = torch.from_numpy
    else:
        trans_d = torch.from_numpy(trans).to(g.device)
        allowed, seed_off, seeds = _classify_device(trans_d, g, order_t)
        dev_t = lambda a: torch.from_numpy(a).to(g.device)  # noqa: E731
    return FrameLists(keys=dev_t(keys), slots=dev_t(slots.view(np.int32)), trans=dev_t(trans),
                      allowed=allowed, seed_off=seed_off, seeds=seeds)


def frame_match(cfg: np.ndarray, fl: FrameLists) -> tuple[int, int]:
    """The list a flat config-set takes on the device and the depth of the
    common stack it is taken over ((-1, -1): none).  The common stack is
    tried at the configs' longest common prefix below every top and up to
    ``MAX_SUFFIX - 1`` frames shorter, shortest first (longest suffixes),
    each with every suffix at most ``MAX_SUFFIX`` frames and the stack plus
    ``MAX_SUFFIX`` frames within the depth limit."""
    h = fl.host()
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
        hv = list_hash(lst)
        s = hv & (SLOTS - 1)
        while h["slots"][s] != EMPTY:
            e = int(h["slots"][s])
            if (e >> 12) == ((hv >> 10) & 0xFFFFF):
                key = h["keys"][e & 0xFFF]
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

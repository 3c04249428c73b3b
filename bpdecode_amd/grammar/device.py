"""Flattened PDA tables, the PDA operators and :class:`CFGConstraintBatch`
(grammar/device.py of the reference).

:func:`build_pda_tensors` concatenates every rule's NFA into one global state
space (rules in grammar order, each rule's states in its NFA numbering) with a
CSR edge list (per state, edges in NFA insertion order); this is the table
layout the reference's kernels consume (device.py:79-158), reproduced so that
config-sets and their raw words are comparable across implementations.

``eps_reduce=True`` first removes epsilon moves inside every rule NFA: each
state gets the byte/call edges of its epsilon-closure (closure in
breadth-first order, duplicates dropped) plus one epsilon edge to the rule's
accept state when the closure contains it, so completion still pops.  The
language is unchanged and the bounded PDA semantics are untouched; closures
hold far fewer intermediate configurations, which keeps grammars such as
nested JSON under the 8-configuration cap.
"""

from __future__ import annotations

import ctypes as C
import hashlib
from collections.abc import Hashable, Sequence
from dataclasses import dataclass, field, replace

import numpy as np
import torch

from .. import _lib
from .._lib import PDA_CONFIG_WORDS, PDA_MAX_CONFIGS, PDA_MAX_DEPTH, check, lib, ptr
from ..tokenizer import Vocabulary
from .nfa import RuleNFA
from .frames import frame_lists
from .pda import CompiledGrammar, coreachable_sets, rule_nonempty

PDA_CONFIG_FLAT = PDA_CONFIG_WORDS
_EPS, _BYTE, _CALL = 0, 1, 2


_WALK_ORDERS: dict = {}  # walk orders by the content of the token tables (a few vocabularies)


def _walk_order(off: torch.Tensor, tb: torch.Tensor, vocab: int, eos_id: int):
    """Walk order of the memoised device mask and its first-byte runs (kept
    for the token tables' content: every grammar over one vocabulary shares
    them).

    Tokens are ordered by first byte, then byte length, then their next 15
    bytes; EOS and empty tokens come last (group 256).  Consecutive lanes of
    a wave take consecutive positions, so they walk equally long tokens that
    share prefixes: they reach the same table entries and leave the walk
    together.  ``runs[c]`` is the first position of group ``c`` (257
    entries; group 256 ends at ``vocab``), so a row skips at once every
    group whose first byte empties its config-set."""
    o32 = off.cpu().numpy()
    b = tb.cpu().numpy()
    h = hashlib.blake2b(digest_size=16)
    h.update(np.int64([vocab, eos_id]).tobytes())
    h.update(np.ascontiguousarray(o32[: vocab + 1]).tobytes())
    h.update(np.ascontiguousarray(b).tobytes())
    key = h.digest()
    hit = _WALK_ORDERS.get(key)
    if hit is not None:
        return hit[0].clone(), hit[1].clone()
    o = o32.astype(np.int64)
    start, length = o[:vocab], o[1 : vocab + 1] - o[:vocab]
    lead = b[np.minimum(start, max(b.size - 1, 0))].astype(np.int64) if b.size else np.zeros(vocab, np.int64)
    group = np.where(length > 0, lead, 256).astype(np.int64)
    if 0 <= eos_id < vocab:
        group[eos_id] = 256
    keys = []
    for i in range(15, 0, -1):
        idx = np.minimum(start + i, max(b.size - 1, 0))
        keys.append(np.where(i < length, b[idx] if b.size else 0, 0).astype(np.int16))
    keys.append(length)
    keys.append(group)  # primary key last
    order = np.lexsort(keys).astype(np.int32)
    runs = np.searchsorted(group[order], np.arange(257), side="left").astype(np.int32)
    if len(_WALK_ORDERS) >= 8:
        _WALK_ORDERS.pop(next(iter(_WALK_ORDERS)))
    _WALK_ORDERS[key] = (torch.from_numpy(order), torch.from_numpy(runs))
    return torch.from_numpy(order.copy()), torch.from_numpy(runs.copy())


@dataclass
class PdaTensors:
    num_states: int
    root_start: int
    root_accept: int
    accept: torch.Tensor  # uint8 [num_states]
    live: torch.Tensor  # uint8 [num_states]
    edge_offsets: torch.Tensor  # int32 [num_states + 1]
    edge_kind: torch.Tensor  # int32 [nnz]
    edge_lo: torch.Tensor
    edge_hi: torch.Tensor
    edge_dst: torch.Tensor
    edge_callee: torch.Tensor
    tok_offsets: torch.Tensor  # int32 [vocab_size + 1]
    tok_bytes: torch.Tensor  # uint8 [tok_offsets[-1]]
    vocab_size: int
    eos_id: int
    # per rule in flattening order: (first state, states, start, accept,
    # has call edges, is the root rule); host metadata of the frame lists
    rules: tuple = ()
    _c: dict = field(default_factory=dict, repr=False, compare=False)

    _TENSORS = ("accept", "live", "edge_offsets", "edge_kind", "edge_lo", "edge_hi",
                "edge_dst", "edge_callee", "tok_offsets", "tok_bytes")

    @property
    def device(self) -> torch.device:
        return self.accept.device

    def to(self, device) -> PdaTensors:
        if self.accept.device == torch.device(device):
            return self
        return replace(self, _c={}, **{f: getattr(self, f).to(device) for f in self._TENSORS})

    # --- native views ---------------------------------------------------
    def _validate(self) -> None:
        n = self.num_states
        off = self.edge_offsets.cpu()
        nnz = int(self.edge_kind.numel())
        if self.accept.numel() != n or self.live.numel() != n or off.numel() != n + 1:
            raise RuntimeError("PDA table arrays disagree on num_states")
        if n > 65536:
            raise RuntimeError("PDA tables above 65536 states are not supported")
        if int(off[0]) != 0 or int(off[-1]) != nnz or bool((off[1:] < off[:-1]).any()):
            raise RuntimeError("edge_offsets is not a CSR offset array")
        for name in ("edge_lo", "edge_hi", "edge_dst", "edge_callee"):
            if getattr(self, name).numel() != nnz:
                raise RuntimeError(f"{name} has the wrong length")
        kind = self.edge_kind.cpu()
        if nnz and (int(kind.min()) < 0 or int(kind.max()) > 2):
            raise RuntimeError("edge_kind values must be 0, 1 or 2")
        dst = self.edge_dst.cpu()
        callee = self.edge_callee.cpu()[kind == _CALL]
        for arr in (dst, callee):
            if arr.numel() and (int(arr.min()) < 0 or int(arr.max()) >= n):
                raise RuntimeError("edge target state out of range")
        if not (0 <= self.root_start < n and 0 <= self.root_accept < n):
            raise RuntimeError("root_start / root_accept out of range")
        toff = self.tok_offsets.cpu()
        if toff.numel() != self.vocab_size + 1 or int(toff[0]) != 0 or int(toff[-1]) != self.tok_bytes.numel():
            raise RuntimeError("tok_offsets does not describe tok_bytes")
        if bool((toff[1:] < toff[:-1]).any()):
            raise RuntimeError("tok_offsets must be non-decreasing")

    def c_table(self) -> _lib.PdaTableC:
        t = self._c.get("table")
        if t is None:
            self._validate()
            keep = [x.contiguous() for x in (self.accept, self.live, self.edge_offsets, self.edge_kind,
                                             self.edge_lo, self.edge_hi, self.edge_dst, self.edge_callee)]
            t = _lib.PdaTableC(self.num_states, self.root_start, self.root_accept,
                               int(self.edge_kind.numel()), *(ptr(x) for x in keep))
            self._c["table"] = t
            self._c["table_keep"] = keep
        return t

    def mask_workspace(self, rows: int, device: torch.device, stream: int) -> tuple[torch.Tensor, int]:
        """Workspace of the memoised device mask (interned config-sets and
        transition scratch per row), kept per stream so a step allocates
        nothing once it has run at this size."""
        need = int(lib().bpd_pda_workspace_bytes(rows, self.vocab_size))
        key = ("ws", device, stream)
        ws = self._c.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
            ws[:256].zero_()  # header: no token records packed yet
            self._c[key] = ws
        return ws, need

    def c_tokens(self) -> _lib.TokenBytesC:
        """Token tables of the device mask: bytes, the walk order, its
        first-byte runs and the stack-relative frame lists."""
        t = self._c.get("tokens")
        if t is None:
            off = self.tok_offsets.contiguous()
            tb = self.tok_bytes.contiguous()
            if tb.numel() == 0:
                tb = torch.zeros(1, dtype=torch.uint8, device=self.device)
            order, runs = _walk_order(off, tb, self.vocab_size, self.eos_id)
            keep = [off, tb, order.to(off.device), runs.to(off.device)]
            frames = None
            fl = frame_lists(self, order)
            if fl is not None and fl.num_lists > 0:
                dev = off.device
                seeds = fl.seeds if fl.seeds.numel() else torch.zeros(1, dtype=torch.int32)
                arrs = [a.to(dev).contiguous() for a in (fl.keys, fl.slots, fl.trans, fl.allowed, fl.seed_off, seeds)]
                keep += arrs
                frames = _lib.PdaFramesC(fl.num_lists, fl.allowed.shape[1], *(ptr(a) for a in arrs))
                self._c["frames"] = frames
                self._c["frame_lists"] = fl
            t = _lib.TokenBytesC(self.vocab_size, self.eos_id, ptr(off), ptr(tb), ptr(keep[2]), ptr(keep[3]),
                                 C.pointer(frames) if frames is not None else None,
                                 _pack_tag(off, tb, order, self.vocab_size))
            self._c["tokens"] = t
            self._c["tokens_keep"] = keep
        return t

    def init_config(self) -> torch.Tensor:
        """One freshly initialised config-set ``[PDA_CONFIG_FLAT]`` int32 (built
        on the host, then moved to the tables' device)."""
        out = self._c.get("init")
        if out is None:
            host = self if self.device.type == "cpu" else self.to("cpu")
            buf = torch.zeros(PDA_CONFIG_FLAT, dtype=torch.int32)
            check(lib().bpd_pda_init(host.c_table(), ptr(buf)))
            out = buf.to(self.device)
            self._c["init"] = out
        return out.clone()

    def feed(self, config: torch.Tensor, data: bytes) -> bool:
        """Consume raw bytes into one host config-set in place; False (config
        untouched) when a byte empties it."""
        if config.device.type != "cpu" or config.dtype != torch.int32 or not config.is_contiguous():
            raise RuntimeError("feed works on a contiguous int32 CPU config-set")
        host = self if self.device.type == "cpu" else self.to("cpu")
        rc = lib().bpd_pda_feed(host.c_table(), ptr(config), bytes(data), len(data))
        if rc < 0:
            check(-rc)
        return rc == 1

    def init_batch(self, batch: int) -> torch.Tensor:
        return self.init_config().unsqueeze(0).expand(batch, -1).contiguous()


def _pack_tag(off: torch.Tensor, tb: torch.Tensor, order: torch.Tensor, vocab: int) -> int:
    """Content tag of the token tables (never 0): the device mask packs its
    token records into a workspace once per tag instead of once per call."""
    h = hashlib.blake2b(digest_size=8)
    h.update(int(vocab).to_bytes(8, "little"))
    for x in (off, tb, order):
        h.update(x.detach().cpu().contiguous().numpy().tobytes())
        h.update(b"|")
    return int.from_bytes(h.digest(), "little") or 1


# ------------------------------------------------------------ flattening --
def _eps_reduced(nfa: RuleNFA) -> RuleNFA:
    edges: dict[int, list] = {}
    for s in range(nfa.num_states):
        order = [s]
        seen = {s}
        head = 0
        while head < len(order):
            u = order[head]
            head += 1
            for label, dst in nfa.out(u):
                if label is None and dst not in seen:
                    seen.add(dst)
                    order.append(dst)
        out: list = []
        have = set()
        for u in order:
            for label, dst in nfa.out(u):
                if label is not None and (label, dst) not in have:
                    have.add((label, dst))
                    out.append((label, dst))
        if nfa.accept in seen and s != nfa.accept:
            out.append((None, nfa.accept))
        edges[s] = out
    return RuleNFA(start=nfa.start, accept=nfa.accept, num_states=nfa.num_states, edges=edges)


def eps_reduce(compiled: CompiledGrammar) -> CompiledGrammar:
    rules = {name: _eps_reduced(nfa) for name, nfa in compiled.rules.items()}
    return CompiledGrammar(rules, compiled.root, coreachable_sets(rules, rule_nonempty(rules)),
                           compiled.regular)


def build_pda_tensors(compiled: CompiledGrammar, vocab: Vocabulary, device="cpu", *,
                      eps_reduce: bool = False) -> PdaTensors:
    if eps_reduce:
        compiled = globals()["eps_reduce"](compiled)
    names = list(compiled.rules)
    base: dict[str, int] = {}
    total = 0
    for name in names:
        base[name] = total
        total += compiled.rules[name].num_states
    accept = [0] * total
    live = [0] * total
    offsets = [0] * (total + 1)
    kind: list[int] = []
    lo: list[int] = []
    hi: list[int] = []
    dst_l: list[int] = []
    callee_l: list[int] = []
    for name in names:
        nfa = compiled.rules[name]
        b = base[name]
        accept[b + nfa.accept] = 1
        for s in compiled.coreachable[name]:
            live[b + s] = 1
        for s in range(nfa.num_states):
            offsets[b + s] = len(kind)
            for label, dst in nfa.out(s):
                if label is None:
                    row = (_EPS, 0, 0, b + dst, -1)
                elif label[0] == "byte":
                    row = (_BYTE, label[1], label[2], b + dst, -1)
                else:
                    c = compiled.rules[label[1]]
                    row = (_CALL, 0, 0, b + dst, base[label[1]] + c.start)
                kind.append(row[0])
                lo.append(row[1])
                hi.append(row[2])
                dst_l.append(row[3])
                callee_l.append(row[4])
    offsets[total] = len(kind)
    root = compiled.rules[compiled.root]
    rules = tuple(
        (base[n], compiled.rules[n].num_states, compiled.rules[n].start, compiled.rules[n].accept,
         any(lbl is not None and lbl[0] == "call" for s in range(compiled.rules[n].num_states)
             for lbl, _ in compiled.rules[n].out(s)), n == compiled.root)
        for n in names)
    raw, tok_offsets = vocab.packed
    i32 = lambda xs: torch.tensor(xs, dtype=torch.int32)  # noqa: E731
    g = PdaTensors(
        num_states=total,
        root_start=base[compiled.root] + root.start,
        root_accept=base[compiled.root] + root.accept,
        accept=torch.tensor(accept, dtype=torch.uint8),
        live=torch.tensor(live, dtype=torch.uint8),
        edge_offsets=i32(offsets),
        edge_kind=i32(kind),
        edge_lo=i32(lo),
        edge_hi=i32(hi),
        edge_dst=i32(dst_l),
        edge_callee=i32(callee_l),
        tok_offsets=torch.from_numpy(tok_offsets.copy()),
        tok_bytes=torch.frombuffer(bytearray(raw or b"\0"), dtype=torch.uint8)[: len(raw)].clone(),
        vocab_size=vocab.size,
        eos_id=vocab.eos_id if vocab.eos_id is not None else -1,
        rules=rules,
    )
    g._validate()
    return g.to(device)


# ------------------------------------------------------------- operators --
def _check_configs(configs: torch.Tensor) -> None:
    if configs.dtype != torch.int32:
        raise RuntimeError("configs must be int32")
    if configs.dim() != 2 or configs.size(1) != PDA_CONFIG_FLAT:
        raise RuntimeError(f"configs must be [batch, {PDA_CONFIG_FLAT}]")
    if not configs.is_contiguous():
        raise RuntimeError("configs must be contiguous")


def _same_device(g: PdaTensors, *ts) -> torch.device:
    devs = {g.device} | {t.device for t in ts if t is not None}
    if len(devs) != 1:
        raise RuntimeError("for a call every grammar/config tensor must be on the same device")
    return g.device


def pda_mask_(logits, g: PdaTensors, configs, slots=None, broken=None, neg_inf=float("-inf")):
    """Mask ``logits`` in place: row b against config-set
    ``configs[slots[b]]`` (``configs[b]`` without slots); rows whose
    ``broken`` flag is set are masked entirely."""
    _check_configs(configs)
    dev = _same_device(g, logits, configs, slots, broken)
    if logits.dim() != 2:
        raise RuntimeError("logits must be [batch, vocab]")
    B, V = logits.shape
    if V != g.vocab_size:
        raise RuntimeError("tok_offsets imply a different vocab size")
    if slots is None and configs.size(0) != B:
        raise RuntimeError("one config-set per logits row")
    work = logits if logits.stride(1) == 1 else logits.contiguous()
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    br = None if broken is None else broken.contiguous()
    code = _lib.dtype_code(work.dtype)
    ld = work.stride(0) if B > 1 else V
    if dev.type == "cuda":
        stream = _lib.stream_of(dev)
        ws, ws_bytes = g.mask_workspace(B, dev, stream)
        check(lib().bpd_pda_apply_mask(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl), ptr(br), B,
                                       ptr(work), code, ld, float(neg_inf), ptr(ws), ws_bytes,
                                       stream))
    else:
        check(lib().bpd_host_pda_apply_mask(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl),
                                            ptr(br), B, ptr(work), code, ld, float(neg_inf)))
    if work is not logits:
        logits.copy_(work)
    return logits


def pda_apply_mask_(logits, g: PdaTensors, configs, neg_inf: float = float("-inf")):
    """torch_ops.cpp:326-376 / device.py:161-169: mask one row per config-set."""
    return pda_mask_(logits, g, configs, neg_inf=neg_inf)


def pda_compute_mask(g: PdaTensors, configs, slots=None) -> torch.Tensor:
    """Packed allow bits ``[batch, ceil(vocab/32)]`` (int32 storage of uint32)."""
    _check_configs(configs)
    dev = _same_device(g, configs, slots)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    B = configs.size(0) if sl is None else sl.numel()
    out = torch.empty((B, (g.vocab_size + 31) // 32), dtype=torch.int32, device=dev)
    if dev.type == "cuda":
        stream = _lib.stream_of(dev)
        ws, ws_bytes = g.mask_workspace(B, dev, stream)
        check(lib().bpd_pda_compute_mask(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl), B,
                                         ptr(out), ptr(ws), ws_bytes, stream))
    else:
        check(lib().bpd_host_pda_compute_mask(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl), B,
                                              ptr(out)))
    return out


def pda_step(configs, g: PdaTensors, token_ids, slots=None, broken=None, err=None, low32=False):
    """Advance ``configs[slots[b]]`` by ``token_ids[b]`` in place; returns
    ``(ok uint8 [B], status int32 [B])``.  ``low32`` reads int64 ids by their
    low 32 bits (the ``tokens.to(torch.int32)`` of device.py:278)."""
    _check_configs(configs)
    tk = token_ids.contiguous()
    if tk.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("token_ids must be int32")
    if tk.device != g.device and tk.device.type == "cpu":
        vals = tk.to(torch.int32) if (low32 and tk.dtype == torch.int64) else tk
        if vals.numel() and (int(vals.min()) < 0 or int(vals.max()) >= g.vocab_size):
            bad = int(vals.max()) if int(vals.max()) >= g.vocab_size else int(vals.min())
            raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {g.vocab_size}")
        tk = tk.to(g.device)
    dev = _same_device(g, configs, tk, slots, broken)
    B = tk.numel()
    if slots is None and configs.size(0) != B:
        raise RuntimeError("token_ids must be int32, one per config-set")
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    ok = torch.empty(B, dtype=torch.uint8, device=dev)
    status = torch.empty(B, dtype=torch.int32, device=dev)
    code = _lib.index_code(tk.dtype, low32=low32)
    if dev.type == "cuda":
        stream = _lib.stream_of(dev)
        ws, ws_bytes = g.mask_workspace(B, dev, stream)
        check(lib().bpd_pda_advance(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl), ptr(tk), code, B,
                                    ptr(ok), ptr(broken), ptr(status), ptr(err), ptr(ws), ws_bytes,
                                    stream))
    else:
        check(lib().bpd_host_pda_advance(g.c_table(), g.c_tokens(), ptr(configs), ptr(sl), ptr(tk),
                                         code, B, ptr(ok), ptr(broken), ptr(status)))
    return ok, status


def pda_advance_state(configs, g: PdaTensors, token_ids):
    """torch_ops.cpp:378-425 / device.py:172-183: advance in place, return
    uint8 ``ok`` (0 where the token was rejected; that config-set is left
    unchanged)."""
    if token_ids.dtype != torch.int32:
        raise RuntimeError("token_ids must be int32, one per config-set")
    return pda_step(configs, g, token_ids)[0]


def config_is_complete(g: PdaTensors, config: torch.Tensor) -> bool:
    """pda_is_complete (pda.hpp:238-244) of one flat config-set."""
    c = config.to("cpu").tolist()
    n = c[0]
    return any(c[2 + i] == 1 and c[2 + PDA_MAX_CONFIGS + i * PDA_MAX_DEPTH] == g.root_accept
               for i in range(max(0, min(n, PDA_MAX_CONFIGS))))


_BROKEN = -1


class CFGConstraintBatch:
    """Fixed-capacity pool of PDA config-sets sharing one :class:`PdaTensors`
    (device.py:189-300 of the reference); mask and commit are one kernel
    launch each and neither synchronises with the host."""

    def __init__(self, g: PdaTensors, capacity: int, device=None) -> None:
        self.g = g if device is None else g.to(device)
        self.device = self.g.device
        self.capacity = capacity
        self._configs = self.g.init_batch(capacity)
        self._broken = torch.zeros(capacity, dtype=torch.bool, device=self.device)
        self._slot_of: dict[Hashable, int] = {}
        self._recycled: list[int] = []  # evicted slots, reused last-in first-out
        self._fresh = 0  # slots [fresh, capacity) were never handed out
        self._version = 0
        self._slot_key = None
        self._slot_tensor = None
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device) if self.device.type == "cuda" else None

    def _take_slot(self) -> int:
        if self._recycled:
            return self._recycled.pop()
        if self._fresh >= self.capacity:
            raise RuntimeError(f"CFGConstraintBatch is at capacity ({self.capacity} sequences)")
        self._fresh += 1
        return self._fresh - 1

    def add(self, seq_id: Hashable) -> int:
        """Give ``seq_id`` a slot holding the grammar's initial config-set."""
        if seq_id in self._slot_of:
            raise KeyError(f"sequence {seq_id!r} is already in the batch")
        slot = self._slot_of[seq_id] = self._take_slot()
        self._configs[slot] = self.g.init_config()
        self._broken[slot] = False
        self._version += 1
        return slot

    def evict(self, seq_id: Hashable) -> None:
        self._recycled.append(self._slot_of.pop(seq_id))
        self._version += 1

    def reset(self, seq_id: Hashable) -> None:
        slot = self._slot_of[seq_id]
        self._configs[slot] = self.g.init_config()
        self._broken[slot] = False

    def __len__(self) -> int:
        return len(self._slot_of)

    def __contains__(self, seq_id: Hashable) -> bool:
        return seq_id in self._slot_of

    def _slots(self, seq_ids: Sequence[Hashable]) -> torch.Tensor:
        from ..batch import index_tensor

        key = (self._version, tuple(seq_ids))
        if key != self._slot_key:
            self._slot_tensor = index_tensor([self._slot_of[s] for s in seq_ids], self.device)
            self._slot_key = key
        return self._slot_tensor

    def apply_mask(self, seq_ids, logits, neg_inf: float = float("-inf")):
        slots = self._slots(seq_ids)
        return pda_mask_(logits, self.g, self._configs, slots, self._broken, neg_inf)

    def commit(self, seq_ids, tokens):
        slots = self._slots(seq_ids)
        tk = tokens if tokens.dtype in (torch.int32, torch.int64) else tokens.to(torch.int32)
        _, status = pda_step(self._configs, self.g, tk, slots, self._broken, self._err, low32=True)
        return status

    def is_complete(self, seq_id: Hashable) -> bool:
        slot = self._slot_of[seq_id]
        if self.g.eos_id < 0 or bool(self._broken[slot]):
            return False
        return config_is_complete(self.g, self._configs[slot])

    def is_broken(self, seq_id: Hashable) -> bool:
        return bool(self._broken[self._slot_of[seq_id]])

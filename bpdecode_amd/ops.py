"""Operator layer of the constraint step (ops.py of the reference).

:class:`FsaTensors` is the grammar bundle; the functions below are the
reference's operator API with the same signatures and results.  Every
computation runs in ``libbpdecode_hip.so``: device tensors go to its HIP
kernels on torch's current stream, CPU tensors to its host entry points.
torch only allocates outputs and supplies the stream.

Dense ``tok_next`` semantics (ops.py:143-197, 262-311):

* ``tok_next[s, t]`` is the state after token ``t`` from ``s`` or ``-1`` (the
  walk reaches ``dead`` or ends in a non-live state); the EOS column holds
  ``s`` for an accepting ``s`` and ``-1`` otherwise.
* ``apply_mask_``: ``logits[b, t] = neg_inf`` iff ``states[b] < 0`` or
  ``tok_next[states[b], t] == -1``; all other entries keep their bits.
* ``advance_state``: ``-1`` for a negative state, else ``tok_next[s, t]``
  (a negative ``t`` indexes from the end, as torch indexing does).

A bundle without ``tok_next`` (mask_cpu.cpp:53-71 ``step`` semantics) runs
the symbol-class walking kernels on the device; on the host its rows are
walked by the table builder, entry for entry the same ``step``.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, replace

import numpy as np
import torch

from . import _lib
from ._lib import check, lib, ptr
from .fsa import FsaTable, TokenSymbols, fsa_from_dfa, token_symbols
from .regex import compile_regex
from .regex.compile import DFA
from .tokenizer import Vocabulary

HAVE_NATIVE = True  # the library is required; loading failures raise at first use

DENSE_AUTO_LIMIT = 32_000_000  # S * V at or below which build() densifies (ops.py:137-139)
# A device bundle without tok_next gets a packed allow-bit table (S rows of
# ceil(V/32) words, built from trans by the walking kernel) when it takes at
# most this many bytes; above it, masks walk every token per call.
ALLOW_BITS_LIMIT = 256 << 20


_SOFT_ARRAYS = ("class_off", "class_tok", "class_piece", "piece_off", "state_off", "pair_class",
                "pair_next", "token_class")


@dataclass
class SoftClasses:
    """Tokens grouped by equal ``tok_next`` columns, for the prior-weighted
    lookahead: class ``c`` is ``class_tok[class_off[c]:class_off[c + 1]]``
    (cut into pieces of at most 256 members, ``piece_off``, the pieces of
    ``c`` being ``class_piece[c]:class_piece[c + 1]``); the (class, next
    state) pairs of state ``s`` are
    ``pair_class/pair_next[state_off[s]:state_off[s + 1]]``; ``token_class``
    maps each token to its class (-1: rejected in every state), and
    ``token_class16`` is the same map as int16 (-1 read as 0xFFFF) when
    there are fewer than 65535 classes; ``chunk_members`` lists the classed
    tokens of each 4096-token chunk in ``chunk_cap`` slots per chunk
    (offset << 16 | class, -1 padded) when no chunk has more than 1024."""

    class_off: torch.Tensor
    class_tok: torch.Tensor
    class_piece: torch.Tensor
    piece_off: torch.Tensor
    state_off: torch.Tensor
    pair_class: torch.Tensor
    pair_next: torch.Tensor
    token_class: torch.Tensor
    num_members: int = 0
    num_pairs: int = 0
    token_class16: torch.Tensor | None = None
    chunk_members: torch.Tensor | None = None
    chunk_cap: int = 0

    def __post_init__(self) -> None:
        self._c: _lib.SoftClassesC | None = None
        self._ws: dict = {}

    @property
    def num_classes(self) -> int:
        return int(self.class_off.numel() - 1)

    @property
    def num_pieces(self) -> int:
        return int(self.piece_off.numel() - 1)

    def to(self, device) -> SoftClasses:
        return SoftClasses(*(getattr(self, n).to(device) for n in _SOFT_ARRAYS),
                           num_members=self.num_members, num_pairs=self.num_pairs,
                           token_class16=None if self.token_class16 is None else self.token_class16.to(device),
                           chunk_members=None if self.chunk_members is None else self.chunk_members.to(device),
                           chunk_cap=self.chunk_cap)

    def c_struct(self) -> _lib.SoftClassesC:
        if self._c is None:
            self._c = _lib.SoftClassesC(self.num_classes, self.num_members, self.num_pieces,
                                        self.num_pairs, *(ptr(getattr(self, n)) for n in _SOFT_ARRAYS),
                                        ptr(self.token_class16), ptr(self.chunk_members),
                                        self.chunk_cap if self.chunk_members is not None else 0)
        return self._c

    def workspace(self, rows: int, device: torch.device, stream: int) -> tuple[torch.Tensor, int]:
        """Workspace for ``rows`` rows, kept per stream so a step allocates
        nothing once it has run at this size."""
        vocab = int(self.token_class.numel())
        need = int(lib().bpd_soft_prior_workspace_bytes(rows, vocab, self.num_classes, self.num_pieces))
        key = (device, stream)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
            self._ws[key] = ws
        return ws, need

    @classmethod
    def build(cls, tok_next: torch.Tensor) -> SoftClasses:
        tn = tok_next.to("cpu", torch.int32).contiguous()
        S, V = tn.shape
        c = _lib.SoftClassesC()
        check(lib().bpd_host_soft_classes(ptr(tn), S, V, C.byref(c)))
        sizes = {"class_off": c.num_classes + 1, "class_tok": c.num_members,
                 "class_piece": c.num_classes + 1, "piece_off": c.num_pieces + 1,
                 "state_off": S + 1, "pair_class": c.num_pairs, "pair_next": c.num_pairs,
                 "token_class": V}
        arrays = {n: torch.empty(max(k, 1), dtype=torch.int32) for n, k in sizes.items()}
        for n in _SOFT_ARRAYS:
            setattr(c, n, ptr(arrays[n]))
        tc16 = torch.empty(V, dtype=torch.int16) if c.num_classes < 65535 else None
        c.token_class16 = ptr(tc16)
        chunks = (V + _lib.SOFT_MEMBER_CHUNK - 1) // _lib.SOFT_MEMBER_CHUNK
        members = torch.empty(chunks * _lib.SOFT_MEMBER_CAP_MAX, dtype=torch.int32)
        c.chunk_members = ptr(members)
        check(lib().bpd_host_soft_classes(ptr(tn), S, V, C.byref(c)))
        cap = int(c.chunk_cap)
        return cls(*(arrays[n][:sizes[n]] for n in _SOFT_ARRAYS), num_members=c.num_members,
                   num_pairs=c.num_pairs, token_class16=tc16,
                   chunk_members=members[:chunks * cap].clone() if cap else None, chunk_cap=cap)


@dataclass
class FsaTensors:
    """FSA + token tables as tensors (field-for-field the reference's bundle)."""

    trans: torch.Tensor  # int32 [num_states * num_symbols]
    accept: torch.Tensor  # uint8 [num_states]
    live: torch.Tensor  # uint8 [num_states]
    num_symbols: int
    dead: int
    offsets: torch.Tensor  # int32 [vocab_size + 1]
    symbols: torch.Tensor  # int32 [offsets[-1]]
    eos_id: int
    start: int = 0
    accepting: frozenset = frozenset()
    tok_next: torch.Tensor | None = None  # int32 [num_states, vocab]
    lookahead: torch.Tensor | None = None  # float32 [num_states, vocab]
    # packed allow bits derived from tok_next: int32 [num_states, ceil(vocab/32)],
    # bit t of row s set iff tok_next[s, t] != -1 (the device mask reads these)
    allow_bits: torch.Tensor | None = None
    # token classes of the prior-weighted lookahead (built once from tok_next)
    soft_classes: SoftClasses | None = None

    @property
    def device(self) -> torch.device:
        return self.trans.device

    @property
    def num_states(self) -> int:
        return int(self.accept.numel())

    @property
    def vocab_size(self) -> int:
        return int(self.offsets.numel() - 1)

    def to(self, device) -> FsaTensors:
        if self.trans.device == torch.device(device):
            return self
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return FsaTensors(
            mv(self.trans), mv(self.accept), mv(self.live), self.num_symbols, self.dead,
            mv(self.offsets), mv(self.symbols), self.eos_id, self.start, self.accepting,
            mv(self.tok_next), mv(self.lookahead), mv(self.allow_bits),
            None if self.soft_classes is None else self.soft_classes.to(device),
        )

    def densify(self) -> FsaTensors:
        if self.tok_next is not None:
            return self
        return replace(self, tok_next=build_token_transitions(self))

    def c_fsa_table(self) -> _lib.FsaTableC:
        """The C view of this bundle for the walking kernels, built once and
        kept with it: symbols whose ``trans`` columns are equal are merged
        into one class (a walk cannot tell them apart), so the table the
        kernels read shrinks to [states, classes]; symbol ids at or above
        ``num_symbols`` stay invalid (mapped past the last class).  With it,
        for the fused commit: the merged table as uint16 with every entry
        that cannot lead to acceptance (outside the table, ``dead``, or a
        state off the live set) set to 0xFFFF, and per token a 16-byte record
        of its first 15 classes and its length."""
        c = self.__dict__.get("_c_fsa")
        if c is None:
            S, M, V = self.num_states, self.num_symbols, self.vocab_size
            sym8 = _symbols_u8(self).cpu()
            table = self.trans.to("cpu", torch.int32).reshape(S, M)
            cols, cls = torch.unique(table.t().contiguous(), dim=0, return_inverse=True)
            ncls = int(cols.shape[0])
            remap = torch.full((256,), ncls, dtype=torch.int32)
            remap[:M] = cls.to(torch.int32)
            merged = cols.t().contiguous().reshape(-1)
            sym_cls = remap[sym8.long()].to(torch.uint8)
            trans = merged.to(self.device)
            sym = sym_cls.to(self.device)
            offs = _i32(self.offsets)
            acc, live = self.accept.contiguous(), self.live.contiguous()
            eos = self.eos_id if self.eos_id is not None and 0 <= self.eos_id < self.vocab_size else -1
            t16 = rec = None
            tab = merged.numpy()
            live_np = live.cpu().numpy().astype(bool)
            inside = (tab >= 0) & (tab < S)
            src_live = np.repeat(live_np, ncls)
            # rejecting at a non-live state mid-walk equals the final live
            # check only when no non-live state steps to a live one (true of
            # the reachability set; a caller's other live array keeps the
            # int32 walk)
            closed = not np.any(inside & ~src_live & live_np[np.where(inside, tab, 0)])
            if S < 0xFFFF and closed:
                ok_state = live_np.copy()
                ok_state[self.dead] = False
                keep = inside.copy()
                keep[keep] = ok_state[tab[keep]]
                t16 = torch.from_numpy(np.where(keep, tab, 0xFFFF).astype(np.uint16).view(np.int16)).to(self.device)
            if V:
                o = self.offsets.to("cpu", torch.int64).numpy()
                lens = o[1:] - o[:-1]
                cls_np = sym_cls.numpy()
                r = np.zeros((V, 16), dtype=np.uint8)
                for j in range(15):
                    m = lens > j
                    r[m, j] = cls_np[o[:-1][m] + j]
                r[:, 15] = np.minimum(lens, 255)
                rec = torch.from_numpy(r.reshape(-1)).to(self.device)
            c = _lib.FsaTableC(ptr(trans), S, ncls, self.dead, ptr(acc), ptr(live), ptr(offs),
                               ptr(sym), V, eos, ptr(t16), ptr(rec))
            self.__dict__["_c_fsa"] = c
            self.__dict__["_c_fsa_keep"] = (sym, trans, offs, acc, live, t16, rec)
        return c

    def ensure_allow_bits(self) -> torch.Tensor:
        """The packed allow-bit table (built once and kept on this bundle;
        derived data, so sharing bundles is unaffected): from tok_next when
        the bundle has it, else, on the device, straight from ``trans`` by
        the walking kernel (every state's row; no [states, vocab] int32
        table).  A host bundle without tok_next is densified first."""
        if self.allow_bits is None:
            st = torch.arange(self.num_states, dtype=torch.int32, device=self.device)
            if self.tok_next is None and self.device.type == "cuda":
                self.allow_bits = fsa_compute_mask(self, st)
            else:
                base = self.densify()
                self.tok_next = base.tok_next
                self.allow_bits = dense_compute_mask(base.tok_next, st)
        return self.allow_bits

    def allow_bits_or_none(self) -> torch.Tensor | None:
        """The allow-bit table of a device bundle (built on first use), or
        None for a bundle without tok_next whose table would exceed
        ``ALLOW_BITS_LIMIT`` bytes (its masks walk the tokens instead)."""
        if self.allow_bits is None and self.tok_next is None:
            if self.device.type != "cuda":
                return None
            if self.num_states * ((self.vocab_size + 31) // 32) * 4 > ALLOW_BITS_LIMIT:
                return None
        return self.ensure_allow_bits()

    def ensure_soft_classes(self) -> SoftClasses:
        """Token classes of the prior-weighted lookahead (built once on the
        host from tok_next and kept on this bundle, like the allow bits)."""
        if self.soft_classes is None:
            base = self.densify()
            self.tok_next = base.tok_next
            self.soft_classes = SoftClasses.build(base.tok_next).to(self.device)
        return self.soft_classes

    def with_lookahead(self, k: int = 3) -> FsaTensors:
        base = self.densify()
        return replace(base, lookahead=build_lookahead(base, k))

    @classmethod
    def from_tables(cls, fsa: FsaTable, toks: TokenSymbols) -> FsaTensors:
        return cls(
            trans=torch.tensor(fsa.trans, dtype=torch.int32),
            accept=torch.tensor(fsa.accept, dtype=torch.uint8),
            live=torch.tensor(fsa.live, dtype=torch.uint8),
            num_symbols=fsa.num_symbols,
            dead=fsa.dead,
            offsets=torch.from_numpy(np.asarray(toks.offsets, dtype=np.int32).copy()),
            symbols=torch.frombuffer(bytearray(toks.symbols or b"\x00"), dtype=torch.uint8)[
                : len(toks.symbols)
            ].to(torch.int32),
            eos_id=toks.eos_id,
            start=fsa.start,
            accepting=frozenset(i for i, a in enumerate(fsa.accept) if a),
        )

    @classmethod
    def build(cls, pattern: str | DFA, vocab: Vocabulary, *, dense: bool | str = "auto",
              device=None) -> FsaTensors:
        """Compile ``pattern`` for ``vocab`` (ops.py:127-140).  With a device,
        the tables go there first and the live set and the dense table are
        built by the device kernels."""
        dfa = pattern if isinstance(pattern, DFA) else compile_regex(pattern)
        dev = torch.device(device) if device is not None else torch.device("cpu")
        on_dev = dev.type == "cuda"
        fsa = cls.from_tables(fsa_from_dfa(dfa, with_live=not on_dev), token_symbols(dfa, vocab))
        if on_dev:
            fsa = fsa.to(dev)
            fsa = replace(fsa, live=build_reachability(fsa.trans, fsa.accept, fsa.num_symbols))
        elif dev.type != "cpu":
            fsa = fsa.to(dev)
        want = dense is True or (dense == "auto" and fsa.num_states * fsa.vocab_size <= DENSE_AUTO_LIMIT)
        return fsa.densify() if want else fsa


# --------------------------------------------------------------- helpers --
def _same_device(*ts: torch.Tensor | None) -> torch.device:
    devs = {t.device for t in ts if t is not None}
    if len(devs) != 1:
        raise RuntimeError(f"all tensors of one call must be on the same device, got {sorted(map(str, devs))}")
    return devs.pop()


def _i32(t: torch.Tensor) -> torch.Tensor:
    t = t if t.dtype == torch.int32 else t.to(torch.int32)
    return t.contiguous()


def _unit_stride_rows(logits: torch.Tensor) -> tuple[torch.Tensor, bool]:
    """A view with unit column stride (a copy when needed, flagged)."""
    if logits.dim() != 2:
        raise RuntimeError("logits must be [batch, vocab]")
    if logits.stride(1) == 1 and logits.stride(0) >= max(logits.size(1), 1):
        return logits, False
    return logits.contiguous(), True


def _symbols_u8(fsa: FsaTensors) -> torch.Tensor:
    sym = fsa.symbols
    if sym.numel() and (int(sym.min()) < 0 or int(sym.max()) > 255):
        raise RuntimeError("symbol-class ids must lie in [0, 255]")
    return sym.to(torch.uint8).contiguous() if sym.numel() else torch.zeros(1, dtype=torch.uint8, device=sym.device)


def build_reachability(trans: torch.Tensor, accept: torch.Tensor, num_symbols: int) -> torch.Tensor:
    """``live`` (uint8, on the tables' device): 1 where an accepting state is
    reachable (fsa.py:70-104); the reachability kernel on the device, the
    library's reverse search on the host."""
    tr = _i32(trans)
    ac = accept.to(torch.uint8).contiguous()
    S = int(ac.numel())
    if S and tr.numel() != S * int(num_symbols):
        raise RuntimeError("trans must hold num_states * num_symbols entries")
    live = torch.empty(S, dtype=torch.uint8, device=tr.device)
    if S == 0:
        return live
    if tr.device.type == "cuda":
        check(lib().bpd_build_reachability(ptr(tr), S, int(num_symbols), ptr(ac), ptr(live),
                                           _lib.stream_of(tr.device)))
    else:
        check(lib().bpd_host_build_reachability(ptr(tr), S, int(num_symbols), ptr(ac), ptr(live)))
    return live


def build_token_transitions(fsa: FsaTensors, rows=None) -> torch.Tensor:
    """Dense ``[num_states, vocab]`` int32 next-state table (``[len(rows), vocab]``
    for the given start states), built by the table-builder kernel / host
    routine (ops.py:143-197)."""
    S, M, V = fsa.num_states, fsa.num_symbols, fsa.vocab_size
    dev = fsa.device
    row_states = None
    n = S
    if rows is not None:
        row_states = torch.as_tensor(rows, dtype=torch.int32, device=dev).contiguous()
        n = int(row_states.numel())
        if dev.type != "cuda" and n and (int(row_states.min()) < 0 or int(row_states.max()) >= S):
            raise IndexError(f"row state out of range [0, {S})")
    out = torch.empty((n, V), dtype=torch.int32, device=dev)
    if n == 0 or V == 0:
        return out
    trans = _i32(fsa.trans)
    acc = fsa.accept.contiguous()
    live = fsa.live.contiguous()
    offs = _i32(fsa.offsets)
    sym = _symbols_u8(fsa)
    eos = fsa.eos_id if fsa.eos_id is not None else -1
    args = (ptr(trans), S, M, fsa.dead, ptr(acc), ptr(live), ptr(offs), ptr(sym), V, eos,
            ptr(row_states), n, ptr(out))
    if dev.type == "cuda":
        check(lib().bpd_build_tok_next(*args, _lib.stream_of(dev)))
    else:
        check(lib().bpd_host_build_tok_next(*args))
    return out


def build_lookahead(fsa: FsaTensors, k: int) -> torch.Tensor:
    """Uniform-count soft-lookahead table ``[num_states, vocab]`` float32
    (ops.py:200-236): ``out[s, t] = logZ_{k-1}(tok_next[s, t])`` with the
    backward recurrence ``logZ_{j+1}(s) = logsumexp_t logZ_j(tok_next[s, t])``
    (``⊕ 0`` for accepting ``s``, ``-inf`` off the live set), ``-inf`` on
    rejected tokens and 0 / ``-inf`` in the EOS column."""
    if fsa.tok_next is None:
        fsa = fsa.densify()
    tn = fsa.tok_next.contiguous()
    S, V = tn.shape
    dev = tn.device
    out = torch.empty((S, V), dtype=torch.float32, device=dev)
    eos = fsa.eos_id if fsa.eos_id is not None and 0 <= fsa.eos_id < V else -1
    acc, live = fsa.accept.contiguous(), fsa.live.contiguous()
    if dev.type == "cuda":
        ws_bytes = int(lib().bpd_soft_workspace_bytes(0, S, 0))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        check(lib().bpd_soft_build_lookahead(ptr(tn), S, V, ptr(acc), ptr(live), eos, int(k),
                                             ptr(out), ptr(ws), ws_bytes, _lib.stream_of(dev)))
    else:
        check(lib().bpd_host_soft_build_lookahead(ptr(tn), S, V, ptr(acc), ptr(live), eos, int(k),
                                                  ptr(out)))
    return out


# ------------------------------------------------- dense kernels (+slots) --
def _pending_args(pending: torch.Tensor | None) -> tuple[int | None, int]:
    """(pointer, count) of a queued-writes tensor: int64 [2 * n] on the
    device, n slots followed by their values."""
    if pending is None or pending.numel() == 0:
        return None, 0
    return pending.data_ptr(), pending.numel() // 2


def dense_mask_(logits, tok_next, states, slots=None, neg_inf=float("-inf"), err=None, pending=None):
    """``logits`` masked in place against ``tok_next`` rows; the state of row
    b is ``states[slots[b]]`` when ``slots`` is given (int64), else
    ``states[b]``.  Any float dtype (float64 included).  ``pending``: queued
    pool writes applied by the same launch (device only)."""
    dev = _same_device(logits, tok_next, states, slots)
    work, copied = _unit_stride_rows(logits)
    B, V = work.shape
    S, TV = tok_next.shape
    if TV != V:
        raise RuntimeError(f"logits have {V} columns but tok_next has {TV}")
    nb = B if slots is None else slots.numel()
    if nb != B:
        raise RuntimeError("one slot per logits row")
    st = states if (pending is not None and states.dtype == torch.int32) else _i32(states)
    if slots is None and st.numel() != B:
        raise RuntimeError(f"one state per logits row (got {st.numel()} states for {B} rows)")
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    tn = tok_next if tok_next.dtype == torch.int32 and tok_next.is_contiguous() else _i32(tok_next)
    code = _lib.dtype_code(work.dtype, dense=True)
    ld = work.stride(0) if B > 1 else V
    if dev.type == "cuda":
        pp, np_ = _pending_args(pending)
        check(lib().bpd_dense_apply_mask(ptr(work), code, B, V, ld, ptr(tn), S, ptr(st), ptr(sl),
                                         pp, np_, float(neg_inf), ptr(err), _lib.stream_of(dev)))
    else:
        if pending is not None and pending.numel():
            raise RuntimeError("queued writes are applied by device launches only")
        check(lib().bpd_host_dense_apply_mask(ptr(work), code, B, V, ld, ptr(tn), S, ptr(st),
                                              ptr(sl), float(neg_inf)))
    if copied:
        logits.copy_(work)
    return logits


def dense_mask_bits_(logits, allow_bits, states, slots=None, neg_inf=float("-inf"), err=None,
                     pending=None):
    """Mask from the packed allow-bit table (same result as
    :func:`dense_mask_`), on the device or on the host."""
    dev = _same_device(logits, allow_bits, states, slots)
    work, copied = _unit_stride_rows(logits)
    B, V = work.shape
    S, W = allow_bits.shape
    if W != (V + 31) // 32:
        raise RuntimeError(f"logits have {V} columns but the allow-bit table has {W} words per row")
    if slots is not None and slots.numel() != B:
        raise RuntimeError("one slot per logits row")
    st = states if (pending is not None and states.dtype == torch.int32) else _i32(states)
    if slots is None and st.numel() != B:
        raise RuntimeError(f"one state per logits row (got {st.numel()} states for {B} rows)")
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    code = _lib.dtype_code(work.dtype, dense=True)
    ld = work.stride(0) if B > 1 else V
    if dev.type == "cuda":
        pp, np_ = _pending_args(pending)
        check(lib().bpd_dense_apply_mask_bits(ptr(work), code, B, V, ld, ptr(allow_bits), W, S,
                                              ptr(st), ptr(sl), pp, np_, float(neg_inf), ptr(err),
                                              _lib.stream_of(dev)))
    else:
        if pending is not None and pending.numel():
            raise RuntimeError("queued writes are applied by device launches only")
        check(lib().bpd_host_dense_apply_mask_bits(ptr(work), code, B, V, ld, ptr(allow_bits), W, S,
                                                   ptr(st), ptr(sl), float(neg_inf)))
    if copied:
        logits.copy_(work)
    return logits


def dense_advance(tok_next, states, tokens, slots=None, write_back=False, err=None, pending=None,
                  low32=False):
    """Next state per row; with ``write_back`` the pool ``states`` is updated
    at the rows' slots as well.  int64 ids are indexed in full (ops.py:301-306
    indexes with ``token_ids.long()``), or by their low 32 bits with
    ``low32`` (the ``tokens.to(torch.int32)`` of batch.py:213).  Host-side
    token ids for a device table are range-checked on the host (raising as
    torch indexing does) and copied over; device-side ids out of range yield
    ``-1`` and set ``BPD_FLAG_TOKEN_RANGE`` in ``err``."""
    S, V = tok_next.shape
    tk = tokens.contiguous()
    if tk.dtype not in (torch.int32, torch.int64):
        tk = tk.to(torch.int64)
    if tk.device != tok_next.device and tk.device.type == "cpu":
        if tk.numel():
            vals = tk.to(torch.int32) if (low32 and tk.dtype == torch.int64) else tk
            lo, hi = int(vals.min()), int(vals.max())
            bad = hi if hi >= V else (lo if lo < -V else None)
            if bad is not None:
                raise IndexError(f"index {bad} is out of bounds for dimension 1 with size {V}")
        tk = tk.to(tok_next.device, non_blocking=True)
    dev = _same_device(tok_next, states, tk, slots)
    B = tk.numel()
    if slots is None and states.numel() != B:
        raise RuntimeError("one token id per state")
    if slots is not None and slots.numel() != B:
        raise RuntimeError("one token id per slot")
    if write_back and (states.dtype != torch.int32 or not states.is_contiguous()):
        raise RuntimeError("write_back needs a contiguous int32 state pool")
    st = states if write_back else _i32(states)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    tn = tok_next if tok_next.dtype == torch.int32 and tok_next.is_contiguous() else _i32(tok_next)
    out = torch.empty(B, dtype=torch.int32, device=dev)
    code = _lib.index_code(tk.dtype, low32=low32)
    if dev.type == "cuda":
        pp, np_ = _pending_args(pending)
        check(lib().bpd_dense_advance(ptr(tn), S, V, ptr(st), ptr(sl), pp, np_, ptr(tk), code, B,
                                      ptr(out), int(write_back), ptr(err), _lib.stream_of(dev)))
    else:
        if pending is not None and pending.numel():
            raise RuntimeError("queued writes are applied by device launches only")
        check(lib().bpd_host_dense_advance(ptr(tn), S, V, ptr(st), ptr(sl), ptr(tk), code, B,
                                           ptr(out), int(write_back)))
    return out.view(tokens.shape) if tokens.dim() else out.reshape(())


def dense_compute_mask(tok_next, states, slots=None, err=None):
    dev = _same_device(tok_next, states, slots)
    S, V = tok_next.shape
    st = _i32(states)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    B = st.numel() if sl is None else sl.numel()
    out = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=dev)
    tn = _i32(tok_next)
    if dev.type == "cuda":
        check(lib().bpd_dense_compute_mask(ptr(tn), S, V, ptr(st), ptr(sl), B, ptr(out), ptr(err),
                                           _lib.stream_of(dev)))
    else:
        check(lib().bpd_host_dense_compute_mask(ptr(tn), S, V, ptr(st), ptr(sl), B, ptr(out)))
    return out


def fsa_mask_(logits, fsa: FsaTensors, states, slots=None, neg_inf=float("-inf"), err=None):
    """Device mask of a bundle without ``tok_next``: every token walked from
    the row's state (``states[slots[b]]`` with ``slots``) by the symbol-class
    kernel; rows whose state is out of range are masked and flagged in
    ``err``."""
    dev = _same_device(logits, fsa.trans, states, slots)
    if dev.type != "cuda":
        raise RuntimeError("the walking kernels run on the device")
    work, copied = _unit_stride_rows(logits)
    B, V = work.shape
    if V != fsa.vocab_size:
        raise RuntimeError(f"logits have {V} columns but the vocabulary has {fsa.vocab_size} tokens")
    if slots is not None and slots.numel() != B:
        raise RuntimeError("one slot per logits row")
    st = _i32(states)
    if slots is None and st.numel() != B:
        raise RuntimeError(f"one state per logits row (got {st.numel()} states for {B} rows)")
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    ld = work.stride(0) if B > 1 else V
    check(lib().bpd_fsa_apply_mask(C.byref(fsa.c_fsa_table()), ptr(work), _lib.dtype_code(work.dtype), B, ld,
                                   ptr(st), ptr(sl), float(neg_inf), ptr(err), _lib.stream_of(dev)))
    if copied:
        logits.copy_(work)
    return logits


def fsa_compute_mask(fsa: FsaTensors, states, slots=None, err=None) -> torch.Tensor:
    dev = _same_device(fsa.trans, states, slots)
    st = _i32(states)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    B = st.numel() if sl is None else sl.numel()
    out = torch.empty((B, (fsa.vocab_size + 31) // 32), dtype=torch.int32, device=dev)
    check(lib().bpd_fsa_compute_mask(C.byref(fsa.c_fsa_table()), ptr(st), ptr(sl), B, ptr(out), ptr(err),
                                     _lib.stream_of(dev)))
    return out


def fsa_advance(fsa: FsaTensors, states, tokens, slots=None, write_back=False, err=None, pending=None):
    """Next state per row by the walking kernel; with ``write_back`` the
    pool ``states`` is updated at the rows' slots as well.  ``pending``:
    queued pool writes applied by the same launch (as in
    :func:`dense_advance`)."""
    tk = tokens.contiguous()
    if tk.dtype not in (torch.int32, torch.int64):
        tk = tk.to(torch.int64)
    if tk.device != fsa.trans.device and tk.device.type == "cpu":
        tk = tk.to(fsa.trans.device, non_blocking=True)
    dev = _same_device(fsa.trans, states, tk, slots)
    B = tk.numel()
    if slots is None and states.numel() != B:
        raise RuntimeError("one token id per state")
    if slots is not None and slots.numel() != B:
        raise RuntimeError("one token id per slot")
    if write_back and (states.dtype != torch.int32 or not states.is_contiguous()):
        raise RuntimeError("write_back needs a contiguous int32 state pool")
    st = states if write_back else _i32(states)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    out = torch.empty(B, dtype=torch.int32, device=dev)
    pp, np_ = _pending_args(pending)
    check(lib().bpd_fsa_advance(C.byref(fsa.c_fsa_table()), ptr(st), ptr(sl), pp, np_, ptr(tk),
                                _lib.index_code(tk.dtype), B, ptr(out), int(write_back), ptr(err),
                                _lib.stream_of(dev)))
    return out.view(tokens.shape) if tokens.dim() else out.reshape(())


def _walked_rows(fsa: FsaTensors, states: torch.Tensor):
    """For a bundle without ``tok_next``: each row's table row, walked now,
    plus the per-row state index into it (negative states kept)."""
    st = _i32(states).view(-1)
    if st.numel() and int(st.max()) >= fsa.num_states:
        raise IndexError(f"index {int(st.max())} is out of bounds for dimension 0 with size {fsa.num_states}")
    rows = build_token_transitions(fsa, rows=st.clamp(min=0))
    idx = torch.where(st < 0, st, torch.arange(st.numel(), dtype=torch.int32, device=st.device))
    return rows, idx


# ------------------------------------------------------------- public API --
def apply_soft_(logits: torch.Tensor, fsa: FsaTensors, states: torch.Tensor, alpha: float = 1.0):
    """In place: ``logits += alpha * lookahead[states]`` on the finite part,
    ``-inf`` where the lookahead is ``-inf`` or the state is negative
    (ops.py:239-259)."""
    if fsa.lookahead is None:
        raise ValueError("fsa has no lookahead table; build with dense + with_lookahead")
    return soft_apply_(logits, fsa.lookahead, states, alpha=alpha)


def soft_apply_(logits, lookahead, states, slots=None, alpha: float = 1.0):
    dev = _same_device(logits, lookahead, states, slots)
    work, copied = _unit_stride_rows(logits)
    B, V = work.shape
    S, LV = lookahead.shape
    if LV != V:
        raise RuntimeError(f"logits have {V} columns but the lookahead table has {LV}")
    st = _i32(states)
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    la = lookahead.contiguous()
    code = _lib.dtype_code(work.dtype)
    ld = work.stride(0) if B > 1 else V
    if dev.type == "cuda":
        check(lib().bpd_soft_apply(ptr(work), code, B, V, ld, ptr(la), S, ptr(st), ptr(sl),
                                   float(alpha), None, _lib.stream_of(dev)))
    else:
        check(lib().bpd_host_soft_apply(ptr(work), code, B, V, ld, ptr(la), S, ptr(st), ptr(sl),
                                        float(alpha)))
    if copied:
        logits.copy_(work)
    return logits


def apply_soft_prior_(logits: torch.Tensor, fsa: FsaTensors, states: torch.Tensor, k: int = 4,
                      alpha: float = 1.0, slots: torch.Tensor | None = None, err=None):
    """In place, float32 ``logits`` [B, vocab]: the prior-weighted soft
    lookahead.  ``logpi = log_softmax(logits)`` per row; k-1 rounds of
    ``logZ(s) = logsumexp_t [logpi(t) + logZ(tok_next[s, t])]`` (``⊕ logpi(eos)``
    for accepting ``s``, ``-inf`` off the live set) from ``logZ = 0`` on live
    states; then ``logpi(t) + alpha * logZ(tok_next[s_b, t])`` on allowed
    tokens, ``logpi(eos)`` in the EOS column of accepting rows and ``-inf``
    elsewhere.  ``logpi == 0`` gives the uniform recurrence of
    build_lookahead (ops.py:200-236)."""
    if logits.dtype != torch.float32:
        raise TypeError("the prior-weighted lookahead takes float32 logits")
    if k < 1:
        raise ValueError("k must be >= 1")
    base = fsa if fsa.tok_next is not None else fsa.densify()
    tn = base.tok_next.contiguous()
    dev = _same_device(logits, tn, states, slots)
    work, copied = _unit_stride_rows(logits)
    B, V = work.shape
    S, TV = tn.shape
    if TV != V:
        raise RuntimeError(f"logits have {V} columns but tok_next has {TV}")
    if slots is not None and slots.numel() != B:
        raise RuntimeError("one slot per logits row")
    st = _i32(states)
    if slots is None and st.numel() != B:
        raise RuntimeError(f"one state per logits row (got {st.numel()} states for {B} rows)")
    sl = None if slots is None else slots.to(torch.int64).contiguous()
    acc, live = base.accept.contiguous(), base.live.contiguous()
    eos = base.eos_id if base.eos_id is not None and 0 <= base.eos_id < V else -1
    ld = work.stride(0) if B > 1 else V
    if dev.type == "cuda":
        sc = base.ensure_soft_classes()
        stream = _lib.stream_of(dev)
        ws, ws_bytes = sc.workspace(B, dev, stream)
        check(lib().bpd_soft_prior(ptr(work), B, V, ld, S, ptr(acc), ptr(live), eos, ptr(st),
                                   ptr(sl), C.byref(sc.c_struct()), int(k), float(alpha), ptr(ws),
                                   ws_bytes, ptr(err), stream))
    else:
        check(lib().bpd_host_soft_prior(ptr(work), B, V, ld, ptr(tn), S, ptr(acc), ptr(live), eos,
                                        ptr(st), ptr(sl), int(k), float(alpha)))
    if copied:
        logits.copy_(work)
    return logits


def apply_mask_(logits: torch.Tensor, fsa: FsaTensors, states: torch.Tensor,
                neg_inf: float = float("-inf")) -> torch.Tensor:
    """In place: every disallowed logit of ``logits`` [batch, vocab] becomes
    ``neg_inf``, one grammar state per row (ops.py:262-281)."""
    if fsa.tok_next is not None:
        if logits.device.type == "cuda" or fsa.allow_bits is not None:
            return dense_mask_bits_(logits, fsa.ensure_allow_bits(), states, neg_inf=neg_inf)
        return dense_mask_(logits, fsa.tok_next, states, neg_inf=neg_inf)
    if logits.device.type == "cuda":
        bits = fsa.allow_bits_or_none()
        if bits is not None:
            return dense_mask_bits_(logits, bits, states, neg_inf=neg_inf)
        return fsa_mask_(logits, fsa, states, neg_inf=neg_inf)
    rows, idx = _walked_rows(fsa, states)
    return dense_mask_(logits, rows, idx, neg_inf=neg_inf)


def compute_mask(fsa: FsaTensors, states: torch.Tensor) -> torch.Tensor:
    """Packed allow-mask, uint32 bits in an int32 tensor [batch, ceil(vocab/32)],
    LSB-first (ops.py:284-292)."""
    if fsa.tok_next is not None:
        return dense_compute_mask(fsa.tok_next, states)
    if states.device.type == "cuda":
        return fsa_compute_mask(fsa, states)
    rows, idx = _walked_rows(fsa, states)
    return dense_compute_mask(rows, idx)


def advance_state(fsa: FsaTensors, states: torch.Tensor, token_ids: torch.Tensor) -> torch.Tensor:
    """Next state per request after ``token_ids``; ``-1`` off a valid path
    (ops.py:295-311)."""
    if fsa.tok_next is not None:
        return dense_advance(fsa.tok_next, states, token_ids)
    if states.device.type == "cuda":
        return fsa_advance(fsa, states, token_ids)
    rows, idx = _walked_rows(fsa, states)
    return dense_advance(rows, idx, token_ids)


# registers torch.ops.bpdecode.* (the reference loads its extension at this point)
from . import torch_ops as _torch_ops  # noqa: E402,F401

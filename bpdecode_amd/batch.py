"""Continuous-batching constraint state (batch.py of the reference).

:class:`ConstraintBatch` keeps one int32 DFA state per slot in a device pool.
On the device, ``apply_mask`` and ``commit`` are one kernel launch each: the
slot gather ``pool[slots]`` is fused into the mask kernel, and the commit
kernel gathers, advances and scatters back in one pass.  Slot writes from
``add`` / ``evict`` / ``reset`` are queued on the host; the next mask or
commit launch carries them (uploaded with the slot list in one copy) and
applies them itself, so per-request churn costs no launch of its own.
"""

from __future__ import annotations

import array
import ctypes as C
import operator
from collections.abc import Hashable, Sequence

import torch

from . import _lib, ops
from ._lib import check, lib
from .ops import FsaTensors, advance_state, apply_mask_, apply_soft_
from .tokenizer import Vocabulary

FREE = -2  # slot holds no sequence
BROKEN = -1  # a committed token left the grammar (matches step() == -1)


class _RecencyMap:
    """A bounded map that forgets its least recently used key: a dict's
    insertion order is its recency order (a hit is popped and re-inserted at
    the end), so the oldest key is always the first one."""

    __slots__ = ("_d", "_cap")

    def __init__(self, capacity: int) -> None:
        self._d: dict = {}
        self._cap = capacity

    def lookup(self, key):
        val = self._d.pop(key, None)
        if val is not None:
            self._d[key] = val
        return val

    def insert(self, key, val) -> None:
        self._d[key] = val
        while len(self._d) > self._cap:
            del self._d[next(iter(self._d))]

    def __len__(self) -> int:
        return len(self._d)


class MaskCache:
    """Allowed-token ids per DFA state, kept for the ``max_states`` most
    recently asked states (the API of batch.py:35-86 of the reference).  A
    state's ids are read from the packed allow bits of that state; the
    device mask does not need them (it masks every row in one launch from
    the grammar's allow-bit table)."""

    def __init__(self, fsa: FsaTensors, max_states: int = 512) -> None:
        self._fsa = fsa
        self._vocab = fsa.vocab_size
        self._ids = _RecencyMap(max_states)

    def _compute(self, state: int) -> torch.Tensor:
        dev = self._fsa.device
        if state < 0:
            return torch.empty(0, dtype=torch.long, device=dev)
        words = ops.compute_mask(self._fsa, torch.tensor([state], dtype=torch.int32, device=dev))[0]
        shifts = torch.arange(32, dtype=torch.int64, device=dev)
        flags = (words.to(torch.int64).unsqueeze(1) >> shifts) & 1  # [words, 32], LSB first
        return flags.reshape(-1)[: self._vocab].nonzero().view(-1)

    def allowed_ids(self, state: int) -> torch.Tensor:
        ids = self._ids.lookup(state)
        if ids is None:
            ids = self._compute(state)
            self._ids.insert(state, ids)
        return ids

    def __len__(self) -> int:
        return len(self._ids)

    def apply(self, states: torch.Tensor, logits: torch.Tensor, neg_inf: float = float("-inf")):
        """In place: mask ``logits`` [n, vocab] given one state per row.  On
        the device the grammar's packed allow-bit table (every state's mask,
        built once) or the walking kernel masks all rows in one launch, with
        no host round trip.  On the host each distinct state's cached ids
        set its row of a keep table, and one ``masked_fill_`` through the
        rows' index into that table masks the batch."""
        if logits.device.type == "cuda":
            return ops.apply_mask_(logits, self._fsa, states.to(logits.device), neg_inf)
        uniq, row_of = torch.unique(states.reshape(-1).cpu(), return_inverse=True)
        keep = torch.zeros((uniq.numel(), logits.shape[1]), dtype=torch.bool)
        for i, st in enumerate(uniq.tolist()):
            keep[i, self.allowed_ids(st).cpu()] = True
        logits.masked_fill_(~keep[row_of].to(logits.device), neg_inf)
        return logits


def build_bundle(pattern, vocab: Vocabulary, device: torch.device) -> FsaTensors:
    """Grammar bundle of a regex (or DFA) on ``device`` by the reference's
    density rule (ops.py:137-139): dense when states * vocab <= 32e6, the
    symbol-class walk above it.  The live set and the table are built where
    the bundle lives (the device kernels on a device)."""
    return FsaTensors.build(pattern, vocab, device=device)


class GrammarCache:
    """Compiled grammars of one vocabulary on one device, keyed by pattern;
    the ``max_size`` most recently used are kept (batch.py:89-115 of the
    reference)."""

    def __init__(self, vocab: Vocabulary, device: torch.device | str = "cpu", max_size: int = 128) -> None:
        self._vocab = vocab
        self._device = torch.device(device)
        self._bundles = _RecencyMap(max_size)

    def get(self, pattern: str) -> FsaTensors:
        fsa = self._bundles.lookup(pattern)
        if fsa is None:
            fsa = build_bundle(pattern, self._vocab, self._device)
            self._bundles.insert(pattern, fsa)
        return fsa

    def __len__(self) -> int:
        return len(self._bundles)


def _stage(values: array.array, device: torch.device) -> torch.Tensor:
    """int64 device tensor holding ``values`` (one native staged copy on the
    current stream; ``values`` may change once this returns)."""
    out = torch.empty(len(values), dtype=torch.int64, device=device)
    if len(values):
        addr, n = values.buffer_info()
        check(lib().bpd_stage_int64(out.data_ptr(), addr, n, _lib.stream_of(device)))
    return out


def index_tensor(values: Sequence[int], device: torch.device) -> torch.Tensor:
    """int64 tensor of ``values`` on ``device``."""
    if device.type != "cuda":
        return torch.tensor(values, dtype=torch.long)
    return _stage(array.array("q", values), device)


_DENSE_CODES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16,
                torch.bfloat16: _lib.DTYPE_BF16, torch.float64: _lib.DTYPE_F64}
_TOKEN_CODES = {torch.int32: _lib.INDEX_I32, torch.int64: _lib.INDEX_I64_LOW32}
_COMMIT_FUSED_ROWS = 4096  # the one-block commit kernel takes queued writes up to this many rows


class ConstraintBatch:
    """Fixed-capacity pool of grammar states sharing one :class:`FsaTensors`
    (batch.py:118-226 of the reference)."""

    def __init__(self, fsa: FsaTensors, capacity: int, device=None,
                 mask_cache: bool | MaskCache = False) -> None:
        self.fsa = fsa if device is None else fsa.to(device)
        self.device = self.fsa.device
        self.capacity = capacity
        self._pool = torch.full((capacity,), FREE, dtype=torch.int32, device=self.device)
        self._pending: dict[int, int] = {}
        self._slot_of: dict[Hashable, int] = {}
        self._recycled: list[int] = []  # evicted slots, reused last-in first-out
        self._fresh = 0  # slots [fresh, capacity) were never handed out
        self._version = 0
        self._ids: list | None = None  # seq ids the cached slot list holds
        self._ids_version = -1
        self._slot_vals: list[int] = []
        # the slot list of _ids on the device: its address, the buffer that
        # holds it (the upload buffer of a stream, or a tensor of its own)
        # and, made on first use, a tensor view of it
        self._slot_ptr = 0
        self._slot_buf: torch.Tensor | None = None
        self._slot_tensor: torch.Tensor | None = None
        self._ubufs: dict[int, torch.Tensor] = {}  # stream -> upload buffer (int64)
        # an upload staged by prepare(): (slot list address, queued-writes
        # address, count) and the queued writes it carries (still visible to
        # state_of)
        self._staged: tuple | None = None
        self._staged_pending: dict[int, int] = {}
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device) if self.device.type == "cuda" else None
        if mask_cache is True:
            mask_cache = MaskCache(self.fsa)
        self.cache: MaskCache | None = mask_cache or None
        # the device fast path: the mask from the packed allow-bit table, the
        # commit from tok_next or, for a bundle without it, by the fused
        # walking kernel; both apply the queued pool writes themselves
        bits = self.fsa.allow_bits_or_none() if self.device.type == "cuda" else None
        self._fast = bits is not None
        if self.device.type == "cpu" and self.fsa.tok_next is not None:
            self.fsa.ensure_allow_bits()  # the host mask reads V/8 bytes per row from it
        if self._fast:
            tn = self.fsa.tok_next
            if tn is not None and (tn.dtype != torch.int32 or not tn.is_contiguous()):
                self.fsa.tok_next = tn = tn.to(torch.int32).contiguous()
            self._S, self._V = self.fsa.num_states, self.fsa.vocab_size
            self._W = int(bits.shape[1])
            self._bits_ptr = bits.data_ptr()
            self._pool_ptr, self._err_ptr = self._pool.data_ptr(), self._err.data_ptr()
            self._f_mask = lib().bpd_dense_apply_mask_bits
            if tn is not None:
                self._tn_ptr = tn.data_ptr()
                self._f_advance = lib().bpd_dense_advance
                self._walk_table = None
            else:
                self._walk_table = C.byref(self.fsa.c_fsa_table())
                self._f_advance = lib().bpd_fsa_advance

    # --- pool -----------------------------------------------------------
    def _unstage(self) -> None:
        """Return staged queued writes to the queue (newer writes win)."""
        if self._staged is not None:
            if self._staged_pending:
                merged = dict(self._staged_pending)
                merged.update(self._pending)
                self._pending = merged
            self._staged = None
            self._staged_pending = {}

    def _flush(self) -> None:
        self._unstage()
        if self._pending:
            idx = index_tensor(list(self._pending.keys()), self.device)
            val = torch.tensor(list(self._pending.values()), dtype=torch.int32)
            self._pool.index_put_((idx,), val.to(self.device, non_blocking=True))
            self._pending.clear()

    @property
    def _state(self) -> torch.Tensor:
        """The state pool (pending slot writes applied)."""
        self._flush()
        return self._pool

    # --- lifecycle -------------------------------------------------------
    def _take_slot(self) -> int:
        if self._recycled:
            return self._recycled.pop()
        if self._fresh >= self.capacity:
            raise RuntimeError(f"ConstraintBatch is at capacity ({self.capacity} sequences)")
        self._fresh += 1
        return self._fresh - 1

    def add(self, seq_id: Hashable) -> int:
        """Give ``seq_id`` a slot at the grammar's start state."""
        if seq_id in self._slot_of:
            raise KeyError(f"sequence {seq_id!r} is already in the batch")
        slot = self._slot_of[seq_id] = self._take_slot()
        self._pending[slot] = self.fsa.start
        self._version += 1
        return slot

    def evict(self, seq_id: Hashable) -> None:
        slot = self._slot_of.pop(seq_id)
        self._pending[slot] = FREE
        self._recycled.append(slot)
        self._version += 1

    def reset(self, seq_id: Hashable) -> None:
        self._pending[self._slot_of[seq_id]] = self.fsa.start

    def move(self, src: Hashable, dst: Hashable) -> None:
        """Sequence ``src`` continues as ``dst`` in the same slot (its state
        is kept; nothing is written on the device)."""
        if dst in self._slot_of:
            raise KeyError(f"sequence {dst!r} already in the batch")
        self._slot_of[dst] = self._slot_of.pop(src)
        self._version += 1

    def __len__(self) -> int:
        return len(self._slot_of)

    def __contains__(self, seq_id: Hashable) -> bool:
        return seq_id in self._slot_of

    # --- per step ----------------------------------------------------------
    def _same_ids(self, seq_ids: Sequence[Hashable]) -> bool:
        if self._ids_version != self._version or self._ids is None:
            return False
        return self._ids == (seq_ids if type(seq_ids) is list else list(seq_ids))

    def _upload(self, values: array.array) -> tuple[int, torch.Tensor]:
        """(device address, buffer) holding ``values`` (int64) after one
        staged copy on the current stream, into this batch's upload buffer
        for that stream.  Reusing it is safe: the copy is ordered after every
        launch already enqueued on the stream, the readers of what it held."""
        stream = _lib.stream_of(self.device)
        n = len(values)
        buf = self._ubufs.get(stream)
        if buf is None or buf.numel() < n:
            buf = torch.empty(max(n, self.capacity + 2 * _lib.MAX_FUSED_PENDING), dtype=torch.int64,
                              device=self.device)
            self._ubufs[stream] = buf
        addr, cnt = values.buffer_info()
        ptr = buf.data_ptr()
        if cnt:
            check(lib().bpd_stage_int64(ptr, addr, cnt, stream))
        return ptr, buf

    def _remember(self, seq_ids: Sequence[Hashable], slot_vals, ptr: int, buf: torch.Tensor | None,
                  tensor: torch.Tensor | None = None) -> None:
        self._ids = list(seq_ids)
        self._ids_version = self._version
        self._slot_vals = slot_vals
        self._slot_ptr, self._slot_buf, self._slot_tensor = ptr, buf, tensor

    def _slot_ptr_of(self, seq_ids: Sequence[Hashable]) -> int:
        """Device address of the int64 slot list of ``seq_ids`` (uploaded
        when the ids or the slot map changed)."""
        if not self._same_ids(seq_ids):
            vals = self._lookup(seq_ids)
            if self.device.type == "cuda":
                ptr, buf = self._upload(array.array("q", vals))
                self._remember(seq_ids, vals, ptr, buf)
            else:
                t = torch.tensor(vals, dtype=torch.long)
                self._remember(seq_ids, vals, t.data_ptr(), t, t)
        return self._slot_ptr

    def _slots(self, seq_ids: Sequence[Hashable]) -> torch.Tensor:
        """int64 slot per row on the device, as a tensor."""
        self._slot_ptr_of(seq_ids)
        if self._slot_tensor is None:
            self._slot_tensor = self._slot_buf[:len(self._slot_vals)]
        return self._slot_tensor

    def _lookup(self, seq_ids: Sequence[Hashable]) -> list | tuple:
        """Slot of each id (one C-level pass over the ids)."""
        n = len(seq_ids)
        if n > 1:
            return operator.itemgetter(*seq_ids)(self._slot_of)
        return [self._slot_of[s] for s in seq_ids]

    def _slots_fused(self, seq_ids: Sequence[Hashable], fuse: bool):
        """(slot address, queued-writes address or None, count) for a
        device launch.  With ``fuse`` the queued pool writes travel in the
        slot upload (one pinned copy) and the launch applies them; the caller
        then calls :meth:`_launched`.  Otherwise they are flushed first.  An
        upload staged by :meth:`prepare` for the same ids, with nothing
        queued since, is used as it is."""
        staged = self._staged
        if staged is not None:
            if fuse and not self._pending and self._same_ids(seq_ids):
                return staged
            self._unstage()
        n = len(self._pending)
        if n == 0:
            return self._slot_ptr_of(seq_ids), None, 0
        if not fuse or n > _lib.MAX_FUSED_PENDING or len(seq_ids) == 0:
            self._flush()
            return self._slot_ptr_of(seq_ids), None, 0
        vals = self._slot_vals if self._same_ids(seq_ids) else self._lookup(seq_ids)
        B = len(vals)
        # one upload of [slots | queued slots | queued values]
        arr = array.array("q", vals)
        arr.extend(self._pending.keys())
        arr.extend(self._pending.values())
        ptr, buf = self._upload(arr)
        self._remember(seq_ids, vals, ptr, buf)
        self._staged = (ptr, ptr + 8 * B, n)
        self._staged_pending = self._pending
        self._pending = {}
        return self._staged

    def _launched(self) -> None:
        """The staged queued writes were applied by a launch."""
        self._staged = None
        self._staged_pending = {}

    def prepare(self, seq_ids: Sequence[Hashable]) -> None:
        """Stage the device-side inputs of the next ``apply_mask`` /
        ``commit`` for ``seq_ids``: the slot list and the queued pool writes
        go to the device in one copy now (e.g. while the model computes the
        logits), and the next launch for the same ids applies them.  Calling
        it is optional; later add / evict / reset calls are merged in."""
        if self._fast:
            self._slots_fused(seq_ids, True)
        else:
            self._slots(seq_ids)

    def apply_mask(self, seq_ids: Sequence[Hashable], logits: torch.Tensor,
                   neg_inf: float = float("-inf")) -> torch.Tensor:
        """In place: every grammar-disallowed logit of ``logits``
        [len(seq_ids), vocab] becomes ``neg_inf``."""
        if self._fast and self.cache is None and self._fast_logits(logits, len(seq_ids)):
            code = _DENSE_CODES.get(logits.dtype)
            if code is None:
                raise RuntimeError(f"logits dtype {logits.dtype} is not supported")
            B = len(seq_ids)
            slots, pend, n = self._slots_fused(seq_ids, True)
            ld = logits.stride(0) if B > 1 else self._V
            check(self._f_mask(
                logits.data_ptr(), code, B, self._V, ld, self._bits_ptr, self._W, self._S,
                self._pool_ptr, slots, pend, n, float(neg_inf), self._err_ptr,
                _lib.stream_of(self.device)))
            if n:
                self._launched()
            return logits
        slots = self._slots(seq_ids)
        pool = self._state
        if self.cache is not None:
            self.cache.apply(pool[slots], logits, neg_inf)
        elif self.fsa.allow_bits is not None and logits.device == pool.device:
            ops.dense_mask_bits_(logits, self.fsa.allow_bits, pool, slots, neg_inf, self._err)
        elif self.fsa.tok_next is not None:
            ops.dense_mask_(logits, self.fsa.tok_next, pool, slots, neg_inf, self._err)
        elif logits.device.type == "cuda":
            ops.fsa_mask_(logits, self.fsa, pool, slots, neg_inf, self._err)
        else:
            apply_mask_(logits, self.fsa, pool[slots], neg_inf)
        return logits

    def _fast_logits(self, logits: torch.Tensor, rows: int) -> bool:
        """Logits the device dense path takes as they are: [rows, vocab] on
        this device with unit column stride."""
        if logits.dim() != 2 or logits.device != self.device:
            return False
        B, V = logits.shape
        return B == rows and V == self._V and (logits.stride(1) == 1 or V <= 1) and (
            B <= 1 or logits.stride(0) >= V)

    def apply_soft(self, seq_ids: Sequence[Hashable], logits: torch.Tensor, alpha: float = 1.0):
        """In place: ``logits += alpha * lookahead[state]`` (and mask)."""
        if self.fsa.lookahead is None:
            raise ValueError("fsa has no lookahead table; build with dense + with_lookahead")
        slots = self._slots(seq_ids)
        ops.soft_apply_(logits, self.fsa.lookahead, self._state, slots, alpha)
        return logits

    def apply_soft_prior(self, seq_ids: Sequence[Hashable], logits: torch.Tensor, k: int = 4,
                         alpha: float = 1.0) -> torch.Tensor:
        """In place, float32 ``logits``: each row becomes its log-softmax
        plus ``alpha`` times the log-probability, under the row's own
        softmax, of staying on a live path for ``k - 1`` further tokens
        (``-inf`` on grammar-disallowed tokens)."""
        slots = self._slots(seq_ids)
        ops.apply_soft_prior_(logits, self.fsa, self._state, k, alpha, slots=slots, err=self._err)
        return logits

    def commit(self, seq_ids: Sequence[Hashable], tokens: torch.Tensor) -> torch.Tensor:
        """Advance each sequence by its sampled token; returns the new states
        (``BROKEN`` where the token was off a valid path).  int64 ids count
        by their low 32 bits, as the reference's ``tokens.to(torch.int32)``
        does."""
        B = len(seq_ids)
        if (self._fast and tokens.device == self.device and tokens.dim() == 1
                and tokens.numel() == B and tokens.is_contiguous()):
            code = _TOKEN_CODES.get(tokens.dtype)
            if code is not None:
                slots, pend, n = self._slots_fused(seq_ids, B <= _COMMIT_FUSED_ROWS)
                out = torch.empty(B, dtype=torch.int32, device=self.device)
                if self._walk_table is None:
                    check(self._f_advance(
                        self._tn_ptr, self._S, self._V, self._pool_ptr, slots, pend, n,
                        tokens.data_ptr(), code, B, out.data_ptr(), 1, self._err_ptr,
                        _lib.stream_of(self.device)))
                else:
                    check(self._f_advance(
                        self._walk_table, self._pool_ptr, slots, pend, n, tokens.data_ptr(),
                        code, B, out.data_ptr(), 1, self._err_ptr, _lib.stream_of(self.device)))
                if n:
                    self._launched()
                return out
        slots = self._slots(seq_ids)
        pool = self._state
        if self.fsa.tok_next is not None:
            return ops.dense_advance(self.fsa.tok_next, pool, tokens, slots, True, self._err, low32=True)
        tk = tokens.to(torch.int32) if tokens.dtype == torch.int64 else tokens
        if pool.device.type == "cuda":
            return ops.fsa_advance(self.fsa, pool, tk, slots, True, self._err)
        nxt = advance_state(self.fsa, pool[slots], tk)
        pool[slots] = nxt
        return nxt

    def check_errors(self) -> None:
        """Raise if a device kernel met an out-of-range state or token since
        the last check (synchronises with the device)."""
        if self._err is None:
            return
        flags = int(self._err.item())
        if flags:
            self._err.zero_()
            raise IndexError(f"out-of-range index in a device constraint kernel (flags {flags})")

    # --- queries -----------------------------------------------------------
    def state_of(self, seq_id: Hashable) -> int:
        slot = self._slot_of[seq_id]
        if slot in self._pending:
            return self._pending[slot]
        if slot in self._staged_pending:
            return self._staged_pending[slot]
        return int(self._pool[slot])

    def is_complete(self, seq_id: Hashable) -> bool:
        return self.state_of(seq_id) in self.fsa.accepting

    def is_broken(self, seq_id: Hashable) -> bool:
        return self.state_of(seq_id) == BROKEN

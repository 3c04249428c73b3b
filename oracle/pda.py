"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

ctypes wrapper of ``liboracle_pda.so`` (oracle/pda_oracle.c).  Tables are
passed as numpy arrays; config-sets are int32 ``[batch, 266]``."""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_pda.so"
WORDS = 266
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "liboracle_pda.so"], check=True)
        _lib = C.CDLL(str(LIB))
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Table:
    """numpy copy of a PdaTensors bundle."""

    def __init__(self, g) -> None:
        a = lambda t, dt: np.ascontiguousarray(t.cpu().numpy().astype(dt))  # noqa: E731
        self.n, self.rs, self.ra = g.num_states, g.root_start, g.root_accept
        self.accept = a(g.accept, np.uint8)
        self.live = a(g.live, np.uint8)
        self.off = a(g.edge_offsets, np.int32)
        nnz = max(int(self.off[-1]), 1)
        pad = lambda t: np.ascontiguousarray(np.resize(t.cpu().numpy().astype(np.int32), nnz))  # noqa: E731
        self.kind, self.lo, self.hi = pad(g.edge_kind), pad(g.edge_lo), pad(g.edge_hi)
        self.dst, self.callee = pad(g.edge_dst), pad(g.edge_callee)
        self.vocab, self.eos = g.vocab_size, g.eos_id
        self.toff = a(g.tok_offsets, np.int32)
        tb = g.tok_bytes.cpu().numpy().astype(np.uint8)
        self.tb = np.ascontiguousarray(tb if tb.size else np.zeros(1, np.uint8))

    def args(self):
        return (C.c_int32(self.n), C.c_int32(self.rs), C.c_int32(self.ra), _p(self.accept),
                _p(self.live), _p(self.off), _p(self.kind), _p(self.lo), _p(self.hi), _p(self.dst),
                _p(self.callee))


def init(t: Table) -> np.ndarray:
    out = np.zeros(WORDS, dtype=np.int32)
    lib().oracle_pda_init(*t.args(), _p(out))
    return out


def advance_byte(t: Table, cfg: np.ndarray, byte: int) -> bool:
    assert cfg.dtype == np.int32 and cfg.flags.c_contiguous
    return bool(lib().oracle_pda_advance_byte(*t.args(), _p(cfg), C.c_int32(byte)))


def compute_mask(t: Table, configs: np.ndarray) -> np.ndarray:
    configs = np.ascontiguousarray(configs, dtype=np.int32)
    B = configs.shape[0]
    out = np.zeros((B, (t.vocab + 31) // 32), dtype=np.uint32)
    lib().oracle_pda_compute_mask(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff),
                                  _p(t.tb), _p(configs), C.c_int32(B), _p(out))
    return out


def apply_mask(t: Table, configs: np.ndarray, logits: np.ndarray, neg_inf: float = float("-inf")):
    configs = np.ascontiguousarray(configs, dtype=np.int32)
    assert logits.dtype == np.float32 and logits.flags.c_contiguous
    lib().oracle_pda_apply_mask(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff),
                                _p(t.tb), _p(configs), C.c_int32(configs.shape[0]), _p(logits),
                                C.c_float(neg_inf))
    return logits


def advance(t: Table, configs: np.ndarray, tokens) -> np.ndarray:
    assert configs.dtype == np.int32 and configs.flags.c_contiguous
    tk = np.ascontiguousarray(tokens, dtype=np.int32)
    ok = np.zeros(tk.size, dtype=np.uint8)
    lib().oracle_pda_advance(*t.args(), C.c_int32(t.eos), _p(t.toff), _p(t.tb), _p(configs),
                             _p(tk), C.c_int32(tk.size), _p(ok))
    return ok


def compute_mask_threads(t: Table, configs: np.ndarray, threads: int) -> np.ndarray:
    """:func:`compute_mask` with the rows split over host threads (the C call
    releases the GIL); the same bits."""
    from concurrent.futures import ThreadPoolExecutor

    configs = np.ascontiguousarray(configs, dtype=np.int32)
    B = configs.shape[0]
    threads = max(1, min(threads, B))
    cuts = np.linspace(0, B, threads + 1).astype(int)
    parts = [configs[a:b] for a, b in zip(cuts[:-1], cuts[1:]) if b > a]
    with ThreadPoolExecutor(max_workers=len(parts)) as ex:
        out = list(ex.map(lambda c: compute_mask(t, c), parts))
    return np.concatenate(out, axis=0)

"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

ctypes wrapper of ``_ref/libbpd_ref.so``: the reference's own
csrc/src/mask_cpu.cpp and csrc/src/pda_cpu.cpp compiled from its sources by
``make -C oracle ref``.  :func:`available` is False where the build is absent
(the reference checkout only exists in the development container)."""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from .pda import Table, WORDS, _p

LIB = Path(__file__).resolve().parent / "_ref" / "libbpd_ref.so"
_lib = None


def available() -> bool:
    return LIB.exists()


def lib():
    global _lib
    if _lib is None:
        _lib = C.CDLL(str(LIB))
        _lib.ref_fsa_step.restype = C.c_int32
    return _lib


def pda_init(t: Table) -> np.ndarray:
    out = np.zeros(WORDS, dtype=np.int32)
    lib().ref_pda_init(*t.args(), _p(out))
    return out


def pda_advance_byte(t: Table, cfg: np.ndarray, byte: int) -> bool:
    return bool(lib().ref_pda_advance_byte(*t.args(), _p(cfg), C.c_int32(byte)))


def pda_compute_mask(t: Table, configs: np.ndarray) -> np.ndarray:
    configs = np.ascontiguousarray(configs, dtype=np.int32)
    out = np.zeros((configs.shape[0], (t.vocab + 31) // 32), dtype=np.uint32)
    lib().ref_pda_compute_mask(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff),
                               _p(t.tb), _p(configs), C.c_int32(configs.shape[0]), _p(out))
    return out


def pda_apply_mask(t: Table, configs: np.ndarray, logits: np.ndarray, neg_inf=float("-inf")):
    configs = np.ascontiguousarray(configs, dtype=np.int32)
    lib().ref_pda_apply_mask(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff),
                             _p(t.tb), _p(configs), C.c_int32(configs.shape[0]), _p(logits),
                             C.c_float(neg_inf))
    return logits


def pda_apply_mask_threads(t: Table, configs: np.ndarray, logits: np.ndarray, threads: int,
                           neg_inf=float("-inf")):
    """apply_mask_pda_batch over `threads` host threads, rows split evenly."""
    configs = np.ascontiguousarray(configs, dtype=np.int32)
    lib().ref_pda_apply_mask_threads(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff),
                                     _p(t.tb), _p(configs), C.c_int32(configs.shape[0]), _p(logits),
                                     C.c_float(neg_inf), C.c_int32(threads))
    return logits


def pda_advance(t: Table, configs: np.ndarray, tokens) -> np.ndarray:
    tk = np.ascontiguousarray(tokens, dtype=np.int32)
    ok = np.zeros(tk.size, dtype=np.uint8)
    lib().ref_pda_advance(*t.args(), C.c_int32(t.vocab), C.c_int32(t.eos), _p(t.toff), _p(t.tb),
                          _p(configs), _p(tk), C.c_int32(tk.size), _p(ok))
    return ok


class Fsa:
    """Flat numpy copy of an FSA bundle for the reference's mask_cpu.cpp."""

    def __init__(self, trans, accept, live, num_symbols, dead, offsets, symbols, eos) -> None:
        f = lambda x, dt: np.ascontiguousarray(np.asarray(x, dtype=dt))  # noqa: E731
        self.trans, self.accept, self.live = f(trans, np.int32), f(accept, np.uint8), f(live, np.uint8)
        self.m, self.dead, self.eos = int(num_symbols), int(dead), int(eos)
        self.off = f(offsets, np.int32)
        sym = f(symbols, np.int32)
        self.sym = sym if sym.size else np.zeros(1, np.int32)
        self.n = self.accept.size
        self.vocab = self.off.size - 1

    def head(self):
        return (C.c_int32(self.n), C.c_int32(self.m), C.c_int32(self.dead), _p(self.trans),
                _p(self.accept), _p(self.live), C.c_int32(self.vocab), C.c_int32(self.eos),
                _p(self.off), _p(self.sym))


def fsa_build_reachability(trans, accept, num_symbols) -> np.ndarray:
    tr = np.ascontiguousarray(np.asarray(trans, dtype=np.int32))
    ac = np.ascontiguousarray(np.asarray(accept, dtype=np.uint8))
    live = np.zeros(ac.size, dtype=np.uint8)
    lib().ref_fsa_build_reachability(C.c_int32(ac.size), C.c_int32(num_symbols), _p(tr), _p(ac), _p(live))
    return live


def fsa_step_table(f: Fsa, states) -> np.ndarray:
    st = np.ascontiguousarray(np.asarray(states, dtype=np.int32))
    out = np.zeros((st.size, f.vocab), dtype=np.int32)
    lib().ref_fsa_step_table(*f.head(), _p(st), C.c_int32(st.size), _p(out))
    return out


def fsa_compute_mask(f: Fsa, states) -> np.ndarray:
    st = np.ascontiguousarray(np.asarray(states, dtype=np.int32))
    out = np.zeros((st.size, (f.vocab + 31) // 32), dtype=np.uint32)
    lib().ref_fsa_compute_mask_batch(*f.head(), _p(st), C.c_int32(st.size), _p(out))
    return out


def fsa_apply_mask(f: Fsa, states, logits: np.ndarray, neg_inf=float("-inf")) -> np.ndarray:
    st = np.ascontiguousarray(np.asarray(states, dtype=np.int32))
    lib().ref_fsa_apply_mask_batch(*f.head(), _p(st), C.c_int32(st.size), _p(logits), C.c_float(neg_inf))
    return logits

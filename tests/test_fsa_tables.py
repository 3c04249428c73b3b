"""The derived arrays the fused walking commit reads (built once per bundle
by FsaTensors.c_fsa_table), pinned on the host against the oracle's
tok_next: walking every (state, token) through the live-filtered uint16
table and the 16-byte token records gives the oracle's next state, and the
records hold each token's first 15 symbol classes and its length.  No
device call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import synth
from bpdecode_amd.ops import FsaTensors
from tests._util import TOY_PATTERNS, TOY_VOCAB, oracle_table


def _walk_all(f: FsaTensors) -> np.ndarray:
    """tok_next as the InLds walk of the fused commit computes it."""
    c = f.c_fsa_table()
    sym, trans, offs, acc, live, t16, rec = f.__dict__["_c_fsa_keep"]
    S, ncls, V = f.num_states, c.num_symbols, f.vocab_size
    t16 = t16.numpy().view(np.uint16).reshape(S, ncls).astype(np.int64)
    rec = rec.numpy().reshape(V, 16)
    o = f.offsets.numpy().astype(np.int64)
    symn = sym.numpy()
    lens = o[1:] - o[:-1]
    assert np.array_equal(rec[:, 15], np.minimum(lens, 255))
    cur = np.tile(np.arange(S, dtype=np.int64)[:, None], (1, V))
    ok = np.ones((S, V), dtype=bool)
    for j in range(int(lens.max(initial=0))):
        active = lens > j
        k = np.where(j < 15, rec[:, min(j, 14)].astype(np.int64),
                     symn[np.clip(o[:-1] + j, 0, len(symn) - 1)].astype(np.int64))
        step = active & (k < ncls)
        bad_sym = active & (k >= ncls)
        nxt = t16[cur[:, step], k[step]] if step.any() else None
        ok[:, bad_sym] = False
        if nxt is not None:
            cur[:, step] = np.where(ok[:, step], nxt, cur[:, step])
            ok[:, step] &= nxt != 0xFFFF
            cur[:, step] = np.where(nxt == 0xFFFF, 0, cur[:, step])
    live_np = live.numpy().astype(bool)
    out = np.where(ok, cur, -1)
    empty = lens == 0
    out[:, empty] = np.where(live_np, np.arange(S), -1)[:, None]
    if 0 <= f.eos_id < V:
        out[:, f.eos_id] = np.where(acc.numpy().astype(bool), np.arange(S), -1)
    return out


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
def test_filtered_table_and_records_walk_like_the_oracle_toy(pattern):
    f = FsaTensors.build(pattern, TOY_VOCAB, dense=False)
    assert np.array_equal(_walk_all(f), oracle_table(f))


def test_filtered_table_and_records_walk_like_the_oracle_email():
    f = FsaTensors.build(synth.EMAIL, synth.serving_vocab(4096, seed=2), dense=False)
    assert f.__dict__.get("_c_fsa") is None
    assert np.array_equal(_walk_all(f), oracle_table(f))


def test_unclosed_live_array_keeps_the_int32_walk():
    """A caller's live array that is not closed under successors (a live
    state reached from a non-live one) gets no filtered table, so the
    commit falls back to the exact walk with the final live check."""
    f = FsaTensors.build("ab|c", TOY_VOCAB, dense=False)
    live = f.live.clone()
    S = f.num_states
    tr = f.trans.reshape(S, f.num_symbols)
    src = next(s for s in range(S) if (tr[s] >= 0).any() and s != f.dead)
    live[src] = 0  # src steps somewhere live but is marked non-live
    g = FsaTensors(f.trans, f.accept, live, f.num_symbols, f.dead, f.offsets, f.symbols, f.eos_id,
                   f.start, f.accepting)
    c = g.c_fsa_table()
    assert not c.trans16 and c.tok_records
    assert torch.equal(f.live, FsaTensors.build("ab|c", TOY_VOCAB, dense=False).live)

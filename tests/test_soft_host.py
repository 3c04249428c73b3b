"""Host side of the prior-weighted lookahead: the token-class builder and the
host form of the kernel against the float64 oracle (relative error 1e-5 with
an absolute floor of 1e-5; -inf pattern exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.ops import FsaTensors, SoftClasses
from oracle import soft as OS
from tests._util import TOY_PATTERNS, TOY_VOCAB, reachable

RTOL, ATOL = 1e-5, 1e-5


def close(got: np.ndarray, want: np.ndarray) -> bool:
    inf_ok = np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    return inf_ok and bool(np.all(np.abs(got[fin] - want[fin]) <= RTOL * np.abs(want[fin]) + ATOL))


def check_classes(tn: np.ndarray, sc: SoftClasses) -> None:
    S, V = tn.shape
    off, mem = sc.class_off.numpy(), sc.class_tok.numpy()
    norm = np.where((tn >= 0) & (tn < S), tn, -1)
    cls = np.full(V, -1)
    for c in range(sc.num_classes):
        members = mem[off[c]:off[c + 1]]
        assert len(members) > 0 and np.all(np.diff(members) > 0)
        cls[members] = c
        assert (norm[:, members] == norm[:, members[:1]]).all()
    reps = mem[off[:-1]]
    assert np.all(np.diff(reps) > 0)  # numbered by smallest member
    assert len(np.unique(norm[:, reps], axis=1).T) == sc.num_classes  # distinct columns
    assert (norm[:, cls < 0] == -1).all() and (cls[(norm >= 0).any(axis=0)] >= 0).all()
    assert np.array_equal(sc.token_class.numpy(), cls)
    assert sc.token_class16 is not None and np.array_equal(sc.token_class16.numpy().astype(np.int64), cls)
    # member lists per 4096-token chunk: (offset << 16 | class) in token order, -1 padded
    chunks = [np.nonzero(cls[g:g + 4096] >= 0)[0] for g in range(0, V, 4096)]
    most = max(len(m) for m in chunks)
    cap = next((c for c in (256, 512, 1024) if most <= c), 0)
    assert sc.chunk_cap == cap
    if cap == 0:
        assert sc.chunk_members is None
    else:
        got = sc.chunk_members.numpy().view(np.uint32).reshape(len(chunks), cap)
        for g, m in enumerate(chunks):
            want = (m.astype(np.uint64) << 16) | cls[g * 4096 + m].astype(np.uint64)
            assert np.array_equal(got[g, :len(m)], want.astype(np.uint32))
            assert (got[g, len(m):] == 0xFFFFFFFF).all()
    po, cp = sc.piece_off.numpy(), sc.class_piece.numpy()
    assert po[0] == 0 and po[-1] == len(mem) and np.all(np.diff(po) > 0) and np.all(np.diff(po) <= 256)
    for c in range(sc.num_classes):
        cuts = po[cp[c]:cp[c + 1] + 1]
        assert cuts[0] == off[c] and cuts[-1] == off[c + 1]
    so, pc, pn = sc.state_off.numpy(), sc.pair_class.numpy(), sc.pair_next.numpy()
    for s in range(S):
        want = [(c, norm[s, reps[c]]) for c in range(sc.num_classes) if norm[s, reps[c]] >= 0]
        assert list(zip(pc[so[s]:so[s + 1]], pn[so[s]:so[s + 1]])) == want


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
def test_classes_toy(pattern):
    fsa = FsaTensors.build(pattern, TOY_VOCAB).densify()
    check_classes(fsa.tok_next.numpy(), SoftClasses.build(fsa.tok_next))


@pytest.mark.parametrize("per_chunk", [0, 1, 300, 1024, 1025, 4096])
def test_chunk_member_capacity(per_chunk):
    """Chunks holding up to 1024 classed tokens get member lists with 256,
    512 or 1024 slots; a chunk with more turns the lists off."""
    V = 9000
    rng = np.random.default_rng(per_chunk)
    tn = np.full((2, V), -1, dtype=np.int32)
    for g in range(0, V, 4096):
        n = min(per_chunk, min(V, g + 4096) - g)
        pick = g + rng.choice(min(V, g + 4096) - g, size=n, replace=False)
        tn[0, pick] = rng.integers(0, 2, size=n)
        tn[1, pick] = 1
    sc = SoftClasses.build(torch.from_numpy(tn))
    check_classes(tn, sc)


def test_classes_out_of_range_entries_read_as_rejected():
    tn = torch.tensor([[0, 5, -7, 1, -1], [1, -1, -1, 1, 9]], dtype=torch.int32)
    sc = SoftClasses.build(tn)
    check_classes(tn.numpy(), sc)
    assert sc.class_tok.tolist() == [0, 3]  # tokens 1, 2 and 4 lead nowhere in range
    assert sc.num_classes == 2


def test_classes_email_serving():
    vocab = synth.serving_vocab(151_936, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    sc = SoftClasses.build(fsa.tok_next)
    check_classes(fsa.tok_next.numpy(), sc)


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("k", [1, 2, 4])
@pytest.mark.parametrize("alpha", [0.0, 1.0, -0.5])
def test_host_prior_matches_oracle(pattern, k, alpha):
    fsa = FsaTensors.build(pattern, TOY_VOCAB).densify()
    S, V = fsa.tok_next.shape
    states = torch.tensor(reachable(fsa.tok_next.numpy(), fsa.start) + [-1], dtype=torch.int32)
    g = torch.Generator().manual_seed(k * 7 + len(pattern))
    x = torch.randn(len(states), V, generator=g) * 3
    got = x.clone()
    ops.apply_soft_prior_(got, fsa, states, k, alpha)
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, states.numpy(), k, alpha)
    assert close(got.double().numpy(), want)


def test_host_prior_slots_and_range_error():
    fsa = FsaTensors.build("a[012]+|b0", TOY_VOCAB).densify()
    S, V = fsa.tok_next.shape
    pool = torch.tensor([-2, 0, 1, 2, -1], dtype=torch.int32)
    slots = torch.tensor([3, 1, 4, 2])
    x = torch.randn(4, V)
    got = x.clone()
    ops.apply_soft_prior_(got, fsa, pool, 3, 1.0, slots=slots)
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, pool[slots].numpy(), 3, 1.0)
    assert close(got.double().numpy(), want)
    with pytest.raises(IndexError):
        ops.apply_soft_prior_(x[:2].clone(), fsa, torch.tensor([0, S], dtype=torch.int32), 3, 1.0)
    with pytest.raises(TypeError):
        ops.apply_soft_prior_(x.to(torch.bfloat16), fsa, pool[:4], 3, 1.0)


def test_host_prior_non_contiguous_rows():
    fsa = FsaTensors.build("[a-c]*", TOY_VOCAB).densify()
    S, V = fsa.tok_next.shape
    wide = torch.randn(3, V + 5)
    view = wide[:, :V]
    st = torch.tensor([0, 0, -1], dtype=torch.int32)
    want = OS.prior_lookahead(view.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, st.numpy(), 3, 0.5)
    ops.apply_soft_prior_(view, fsa, st, 3, 0.5)
    assert close(wide[:, :V].double().numpy(), want)

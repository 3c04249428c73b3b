"""Dense tok_next path through the library's host entry points (CPU
tensors) against the oracle, plus the ConstraintBatch lifecycle scenarios of
the reference's test_batch.py / test_dense.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import BROKEN, FREE, ConstraintBatch, GrammarCache, MaskCache
from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
from oracle import dense as OD
from tests._util import TOY_PATTERNS, TOY_VOCAB, OracleWalk, bits_of, oracle_table

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
def test_table_matches_oracle(pattern):
    fsa = FsaTensors.build(pattern, TOY_VOCAB, dense=True)
    assert np.array_equal(fsa.tok_next.numpy(), oracle_table(fsa))
    rows = [fsa.num_states - 1, 0, 0]
    part = ops.build_token_transitions(fsa, rows=rows)
    assert np.array_equal(part.numpy(), oracle_table(fsa)[rows])


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_apply_mask_and_advance_match_oracle(pattern, dtype):
    fsa = FsaTensors.build(pattern, TOY_VOCAB)
    tn = oracle_table(fsa)
    rng = np.random.default_rng(0)
    B = 64
    states = rng.integers(-2, fsa.num_states, size=B).astype(np.int32)
    base = torch.from_numpy(rng.standard_normal((B, TOY_VOCAB.size)).astype(np.float32)).to(dtype)
    got = base.clone()
    ops.apply_mask_(got, fsa, torch.from_numpy(states))
    want = OD.apply_mask(base.clone(), tn, states)
    assert np.array_equal(bits_of(got), bits_of(want))
    toks = rng.integers(-TOY_VOCAB.size, TOY_VOCAB.size, size=B)
    for tdt in (torch.int32, torch.int64):
        nxt = ops.advance_state(fsa, torch.from_numpy(states), torch.from_numpy(toks).to(tdt))
        assert nxt.dtype == torch.int32
        assert nxt.tolist() == OD.advance(tn, states, toks).tolist()
    bits = ops.compute_mask(fsa, torch.from_numpy(states))
    assert np.array_equal(bits.numpy().view(np.uint32), OD.compute_mask_bits(tn, states))


@pytest.mark.parametrize("neg_inf", [-1e4, -3.0e38, float("nan"), 5.0])
@pytest.mark.parametrize("dtype", DTYPES)
def test_fill_value_conversion(neg_inf, dtype):
    fsa = FsaTensors.build("[01]+", TOY_VOCAB)
    st = torch.tensor([0, 1, -1], dtype=torch.int32)
    base = torch.randn(3, TOY_VOCAB.size).to(dtype)
    try:
        want = OD.apply_mask(base.clone(), oracle_table(fsa), st.numpy(), neg_inf)
    except RuntimeError:
        with pytest.raises(RuntimeError, match="overflow"):
            ops.apply_mask_(base.clone(), fsa, st, neg_inf)
        return
    got = ops.apply_mask_(base.clone(), fsa, st, neg_inf)
    assert np.array_equal(bits_of(got), bits_of(want))


def test_strided_logits_and_dense_vs_walked():
    fsa = FsaTensors.build("-?[0-9]+(\\.[0-9]+)?", TOY_VOCAB, dense=False)
    dense = fsa.densify()
    st = torch.tensor([0, 1, 2, 3, -2], dtype=torch.int32)
    wide = torch.randn(5, TOY_VOCAB.size + 7)
    view = wide[:, 3:3 + TOY_VOCAB.size]
    want = view.clone()
    ops.apply_mask_(want, dense, st)
    ops.apply_mask_(view, fsa, st)  # walked rows, strided logits
    assert torch.equal(view, want)
    col_major = torch.randn(TOY_VOCAB.size, 5).t()
    ref = col_major.clone().contiguous()
    ops.apply_mask_(ref, dense, st)
    ops.apply_mask_(col_major, dense, st)
    assert torch.equal(col_major, ref)


def test_out_of_range_indices_raise():
    fsa = FsaTensors.build("[01]+", TOY_VOCAB)
    with pytest.raises(IndexError):
        ops.apply_mask_(torch.zeros(1, TOY_VOCAB.size), fsa, torch.tensor([fsa.num_states], dtype=torch.int32))
    with pytest.raises(IndexError):
        ops.advance_state(fsa, torch.tensor([0], dtype=torch.int32), torch.tensor([TOY_VOCAB.size]))
    with pytest.raises(IndexError):
        ops.advance_state(fsa, torch.tensor([0], dtype=torch.int32), torch.tensor([-TOY_VOCAB.size - 1]))
    with pytest.raises(RuntimeError):
        ops.apply_mask_(torch.zeros(1, TOY_VOCAB.size + 1), fsa, torch.tensor([0], dtype=torch.int32))


def test_auto_dense_threshold():
    assert FsaTensors.build("[01]+", TOY_VOCAB).tok_next is not None
    assert FsaTensors.build("[01]+", TOY_VOCAB, dense=False).tok_next is None


# ----------------------------------------------------- ConstraintBatch ----
TOKENS = ["a", "b", "c", "ab", "0", "1", "12", "-", ".", "<eos>"]
VOCAB = Vocabulary.from_tokens(TOKENS, eos_id=9)


def test_grammar_cache_dedups_and_evicts_lru():
    cache = GrammarCache(VOCAB, max_size=2)
    a1 = cache.get("[01]+")
    assert cache.get("[01]+") is a1
    cache.get("a+")
    cache.get("[01]+")
    cache.get("b+")
    assert len(cache) == 2 and cache.get("[01]+") is a1


def test_lifecycle_slots_are_reused():
    batch = ConstraintBatch(GrammarCache(VOCAB).get("[01]+"), capacity=2)
    s0, s1 = batch.add("r0"), batch.add("r1")
    assert {s0, s1} == {0, 1}
    with pytest.raises(RuntimeError):
        batch.add("r2")
    batch.evict("r0")
    assert batch._state[s0] == FREE
    assert batch.add("r2") == s0
    assert "r0" not in batch and "r2" in batch and len(batch) == 2
    with pytest.raises(KeyError):
        batch.add("r2")


@pytest.mark.parametrize("mask_cache", [False, True], ids=["kernel", "cached"])
@pytest.mark.parametrize("pattern,seq", [
    ("[01]+", [4, 5, 4, 9]), ("-?[0-9]+(\\.[0-9]+)?", [7, 4, 8, 5]), ("(ab)+", [3, 3, 9]),
    ("a+b*", [0, 0, 1, 9]),
])
def test_matches_single_sequence_reference(pattern, seq, mask_cache):
    batch = ConstraintBatch(GrammarCache(VOCAB).get(pattern), capacity=4, mask_cache=mask_cache)
    ref = OracleWalk(FsaTensors.build(pattern, VOCAB))
    batch.add("s")
    for tok in seq:
        logits = torch.zeros(1, VOCAB.size)
        batch.apply_mask(["s"], logits)
        got = {i for i in range(VOCAB.size) if logits[0, i].item() == 0.0}
        assert got == ref.allowed()
        batch.commit(["s"], torch.tensor([tok], dtype=torch.int32))
        ref.advance(tok)
        assert batch.is_complete("s") == ref.is_complete()


def test_rows_independent_and_broken():
    batch = ConstraintBatch(GrammarCache(VOCAB).get("[01]+"), capacity=3)
    for r in "abc":
        batch.add(r)
    batch.commit(list("abc"), torch.tensor([4, 5, 4], dtype=torch.int32))
    batch.commit(["b"], torch.tensor([5], dtype=torch.int32))
    logits = torch.zeros(3, VOCAB.size)
    batch.apply_mask(list("abc"), logits)
    assert (logits[:, TOKENS.index("0")] == 0).all() and (logits[:, VOCAB.eos_id] == 0).all()
    assert torch.isneginf(logits[:, TOKENS.index("a")]).all()
    out = batch.commit(["a"], torch.tensor([TOKENS.index("a")], dtype=torch.int64))
    assert out.tolist() == [BROKEN] and batch.is_broken("a")
    logits = torch.zeros(1, VOCAB.size)
    batch.apply_mask(["a"], logits)
    assert torch.isneginf(logits).all()
    batch.reset("a")
    assert batch.state_of("a") == batch.fsa.start


@pytest.mark.parametrize("pattern", ["[01]+", "-?[0-9]+(\\.[0-9]+)?", "(ab)+", "a|b|12"])
def test_mask_cache_matches_uncached(pattern):
    fsa = GrammarCache(VOCAB).get(pattern)
    states = list(range(fsa.num_states)) * 2
    st = torch.tensor(states, dtype=torch.int32)
    mc = MaskCache(fsa)
    base = torch.randn(len(st), VOCAB.size)
    want = base.clone()
    ops.apply_mask_(want, fsa, st)
    got = base.clone()
    mc.apply(st, got)
    assert torch.equal(want, got)
    got2 = base.clone()
    mc.apply(st, got2)
    assert torch.equal(want, got2) and len(mc) == fsa.num_states


def test_mask_cache_bounded_and_negative_states():
    """Rows at FREE / BROKEN are masked whole; with room for two states the
    least recently asked one is dropped and recomputed on its next use."""
    fsa = GrammarCache(VOCAB).get("[01]+")
    st = torch.tensor([FREE, 0, BROKEN, 1, 0], dtype=torch.int32)
    mc = MaskCache(fsa, max_states=2)
    base = torch.randn(len(st), VOCAB.size)
    want = base.clone()
    ops.apply_mask_(want, fsa, st)
    got = mc.apply(st, base.clone())
    assert torch.equal(want, got)
    assert torch.isneginf(got[0]).all() and torch.isneginf(got[2]).all()
    assert len(mc) == 2
    first = mc.allowed_ids(1)
    mc.allowed_ids(0)
    mc.allowed_ids(FREE)  # drops state 1, the least recently asked
    assert len(mc) == 2 and 1 not in mc._ids._d
    assert torch.equal(mc.allowed_ids(1), first)


def test_churn_matches_oracle_replay():
    """Continuous batching (add / evict / commit) vs a numpy replay."""
    fsa = FsaTensors.build("[a-c]*b|a+1", TOY_VOCAB)
    tn = oracle_table(fsa)
    rng = np.random.default_rng(3)
    batch = ConstraintBatch(fsa, capacity=16)
    pool = {}
    nxt_id = 0
    for _ in range(20):
        while len(pool) < 12:
            batch.add(nxt_id)
            pool[nxt_id] = fsa.start
            nxt_id += 1
        ids = list(pool)
        rng.shuffle(ids)
        st = np.array([pool[i] for i in ids], dtype=np.int32)
        logits = torch.randn(len(ids), TOY_VOCAB.size)
        want = OD.apply_mask(logits.clone(), tn, st)
        batch.apply_mask(ids, logits)
        assert torch.equal(logits, want)
        toks = rng.integers(0, TOY_VOCAB.size, size=len(ids))
        out = batch.commit(ids, torch.from_numpy(toks))
        exp = OD.advance(tn, st, toks)
        assert out.tolist() == exp.tolist()
        for i, s in zip(ids, exp.tolist()):
            pool[i] = s
        for i in rng.choice(ids, size=3, replace=False).tolist():
            batch.evict(i)
            del pool[i]
    assert all(batch.state_of(i) == s for i, s in pool.items())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("vocab_size", [300, 320, 2048 + 5])
def test_host_allow_bit_mask_matches_table_mask(dtype, vocab_size):
    """The host mask from the packed allow bits (all-rejected words filled,
    all-allowed words skipped, mixed words element by element) equals the
    tok_next host mask and the oracle, on rows at every state, FREE and
    BROKEN, with a row stride wider than the vocabulary."""
    vocab = synth.serving_vocab(vocab_size, seed=5)
    fsa = FsaTensors.build("[a-z0-9]{1,6}(\\.[a-z]+)?|x*", vocab)
    tn = oracle_table(fsa)
    S, V = tn.shape
    bits = fsa.ensure_allow_bits()
    assert np.array_equal(bits.numpy().view(np.uint32), OD.compute_mask_bits(tn, np.arange(S, dtype=np.int32)))
    st = np.array(list(range(S)) + [FREE, BROKEN] + list(range(S))[::-2], dtype=np.int32)
    wide = (torch.randn(len(st), V + 9) * 3).to(dtype)
    base = wide[:, :V]
    want = OD.apply_mask(base.clone(), tn, st)
    got_bits = base.clone()
    ops.dense_mask_bits_(got_bits, bits, torch.from_numpy(st))
    view = wide.clone()[:, :V]  # stride V + 9
    ops.dense_mask_bits_(view, bits, torch.from_numpy(st))
    got_table = base.clone()
    ops.dense_mask_(got_table, fsa.tok_next, torch.from_numpy(st))
    for got in (got_bits, view, got_table):
        assert torch.equal(got.view(torch.uint8 if dtype != torch.float64 else torch.int64),
                           want.view(torch.uint8 if dtype != torch.float64 else torch.int64))

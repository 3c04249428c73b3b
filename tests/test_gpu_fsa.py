"""Bundles without tok_next (the reference's non-dense operators) on the
device against the oracle: the symbol-class walking kernels (every state of
the toy grammars in every logits dtype, the transition table in LDS and in
global memory) and the allow-bit path that replaces them under a size limit
(the table built from trans by the walking kernel, masks by the dense fill
kernel, commits by the fused walking commit); the flat JSON-Schema DFA at
serving scale (826 states, V = 151,936) through both and through the
default ``auto`` bundle over a 64-step trajectory with churn;
ConstraintBatch with slots and churn, the range flags, and MaskCache without
a host round trip.  Bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import ConstraintBatch, MaskCache
from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.grammar.regular import residual_dfa
from bpdecode_amd.ops import FsaTensors
from oracle import dense as OD
from tests._util import TOY_PATTERNS, TOY_VOCAB, bits_of, oracle_table

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(params=["walk-lds", "walk-global", "bits"])
def nondense_path(request, monkeypatch):
    """walk-*: the walking kernels (no allow-bit table; the table in LDS or
    read from global memory); bits: the allow-bit table built from trans."""
    if request.param.startswith("walk"):
        monkeypatch.setattr(ops, "ALLOW_BITS_LIMIT", 0)
    if request.param == "walk-global":
        monkeypatch.setenv("BPD_FSA_TABLE", "global")
    return request.param


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_toy_every_state(dev, pattern, dtype, nondense_path):
    _log(f"case fsa toy {pattern!r} {dtype} path={nondense_path}")
    f = FsaTensors.build(pattern, TOY_VOCAB, dense=False)
    assert f.tok_next is None
    tn = oracle_table(f)
    S, V = tn.shape
    st = np.array(list(range(S)) + [-1, -2] + list(range(S))[::-1], dtype=np.int32)
    fd = f.to(dev)
    lg = (torch.randn(len(st), V) * 3).to(dtype)
    want = OD.apply_mask(lg.clone(), tn, st)
    got = lg.to(dev)
    ops.apply_mask_(got, fd, torch.from_numpy(st).to(dev))
    assert np.array_equal(bits_of(got), bits_of(want))
    assert (fd.allow_bits is not None) == (nondense_path == "bits")
    if fd.allow_bits is not None:  # the table built from trans: every state's oracle row
        every = np.arange(S, dtype=np.int32)
        assert np.array_equal(fd.allow_bits.cpu().numpy().view(np.uint32), OD.compute_mask_bits(tn, every))
    bits = ops.compute_mask(fd, torch.from_numpy(st).to(dev)).cpu().numpy().view(np.uint32)
    assert np.array_equal(bits, OD.compute_mask_bits(tn, st))
    for k in range(3):
        toks = np.array([(5 * i + 7 * k) % V for i in range(len(st))], dtype=np.int32)
        toks[::4] = f.eos_id
        toks[1::9] = -1  # indexes from the end, like the dense commit
        nxt = ops.advance_state(fd, torch.from_numpy(st).to(dev), torch.from_numpy(toks).to(dev))
        assert nxt.cpu().tolist() == OD.advance(tn, st, toks).tolist()


def test_flat_schema_serving_scale(dev, monkeypatch):
    """The flat JSON-Schema DFA at serving scale (826 states, V = 151,936,
    B = 256, bf16) on the walking kernels (no allow-bit table): one mask,
    packed bits and commit against the oracle, then eight mask + commit
    steps through ConstraintBatch."""
    _log("case fsa walk flat-schema DFA V=151936 B=256 bf16, 9 steps")
    monkeypatch.setattr(ops, "ALLOW_BITS_LIMIT", 0)  # the walking kernels
    vocab = synth.serving_vocab(151_936, seed=1)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    plain = FsaTensors.build(dfa, vocab, dense=False)
    assert plain.tok_next is None
    c = plain.to(dev).c_fsa_table()  # equal symbol columns merged: 256 symbols -> fewer classes
    assert c.num_symbols < plain.num_symbols and plain.num_states * c.num_symbols * 4 > 16 * 1024
    fd = plain.to(dev)
    dense_dev = fd.densify()
    tn_dev = dense_dev.tok_next
    starts = synth.random_walk_states(tn_dev.cpu(), plain.start, vocab.eos_id, 256, 20, seed=6)
    st = starts.numpy()
    rows = sorted(set(st.tolist()))[:6]
    want_rows = OD.build_token_transitions(plain.trans.numpy(), plain.accept.numpy(), plain.live.numpy(),
                                           plain.num_symbols, plain.offsets.numpy(), plain.symbols.numpy(),
                                           plain.eos_id, rows=rows)
    assert np.array_equal(tn_dev[rows].cpu().numpy(), want_rows)
    tn = tn_dev.cpu().numpy()
    lg = synth.logits(256, vocab.size, 3.0, torch.bfloat16, seed=8)
    want = OD.apply_mask(lg.clone(), tn, st)
    got = lg.to(dev)
    ops.apply_mask_(got, fd, starts.to(dev))
    assert np.array_equal(bits_of(got), bits_of(want))
    bits = ops.compute_mask(fd, starts.to(dev)).cpu().numpy().view(np.uint32)
    assert np.array_equal(bits, OD.compute_mask_bits(tn, st))
    toks = torch.multinomial(torch.softmax(want.float(), dim=-1), 1,
                             generator=torch.Generator().manual_seed(2)).view(-1)
    nxt = ops.advance_state(fd, starts.to(dev), toks.to(dev))
    assert nxt.cpu().tolist() == OD.advance(tn, st, toks.numpy()).tolist()
    # eight more steps through ConstraintBatch on the walking kernels: the
    # mask against ATen's masked_fill_ over the oracle-checked table, the
    # commit against the oracle's advance
    batch = ConstraintBatch(fd, capacity=256, device=dev)
    assert not batch._fast
    ids = list(range(256))
    for i in ids:
        batch.add(i)
    batch._state[:256] = nxt
    st = nxt.cpu().numpy()
    gen = torch.Generator(device=dev).manual_seed(3)
    for step in range(8):
        lg = torch.randn((256, vocab.size), generator=gen, device=dev).mul_(3.0).to(torch.bfloat16)
        s_ = torch.from_numpy(st).to(dev).long()
        rejected = (tn_dev.index_select(0, s_.clamp(min=0)) == -1) | (s_ < 0)[:, None]
        want = lg.clone().masked_fill_(rejected, float("-inf"))
        got = lg.clone()
        batch.apply_mask(ids, got)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        finite = torch.isfinite(want.float()).any(dim=1)
        probs = torch.softmax(torch.where(finite[:, None], want.float(), torch.zeros_like(want.float())), dim=-1)
        toks = torch.multinomial(probs, 1, generator=gen).view(-1)
        nxt = batch.commit(ids, toks)
        st = OD.advance(tn, st, toks.cpu().numpy())
        assert nxt.cpu().numpy().tolist() == st.tolist(), step
    batch.check_errors()


def test_batch_churn_and_range_flags(dev, nondense_path):
    _log(f"case fsa ConstraintBatch churn path={nondense_path}")
    vocab = synth.serving_vocab(8192, seed=3)
    f = FsaTensors.build(synth.EMAIL, vocab, dense=False)
    tn = OD.build_token_transitions(f.trans.numpy(), f.accept.numpy(), f.live.numpy(), f.num_symbols,
                                    f.offsets.numpy(), f.symbols.numpy(), f.eos_id)
    batch = ConstraintBatch(f, capacity=48, device=dev)
    assert batch.fsa.tok_next is None and batch._fast == (nondense_path == "bits")
    state = {}
    for i in range(32):
        batch.add(i)
        state[i] = f.start
    gen = torch.Generator().manual_seed(4)
    nid = 32
    for step in range(12):
        ids = sorted(state)
        st = np.array([state[i] for i in ids], dtype=np.int32)
        lg = synth.logits(len(ids), vocab.size, 3.0, torch.float32, seed=50 + step)
        want = OD.apply_mask(lg.clone(), tn, st)
        got = lg.to(dev)
        batch.apply_mask(ids, got)
        assert torch.equal(got.cpu(), want), step
        finite = torch.isfinite(want).any(dim=1)
        toks = torch.where(finite, torch.multinomial(torch.softmax(torch.where(
            finite.unsqueeze(1), want, torch.zeros_like(want)), dim=-1), 1, generator=gen).view(-1),
            torch.zeros(len(ids), dtype=torch.long))
        nxt = batch.commit(ids, toks.to(dev)).cpu().tolist()
        ref = OD.advance(tn, st, toks.numpy().astype(np.int32)).tolist()
        assert nxt == ref, step
        for i, s in zip(ids, ref):
            state[i] = s
        for i in ids[step % 5::7]:
            batch.evict(i)
            del state[i]
            batch.add(nid)
            state[nid] = f.start
            nid += 1
    batch.check_errors()
    assert all(batch.state_of(i) == s for i, s in state.items())
    # a state past the table: the row is masked and the flag raised on check
    some = sorted(state)[0]
    batch._state[batch._slot_of[some]] = f.num_states
    got = torch.zeros(1, vocab.size, device=dev)
    batch.apply_mask([some], got)
    assert torch.isneginf(got).all()
    with pytest.raises(IndexError):
        batch.check_errors()


def test_mask_cache_on_device_matches_host(dev):
    _log("case mask cache device vs host")
    for dense in (True, False):
        f = FsaTensors.build("-?[0-9]+(\\.[0-9]+)?", TOY_VOCAB, dense=dense)
        tn = oracle_table(f)
        S, V = tn.shape
        st = torch.tensor(list(range(S)) + [-1, -2, 0], dtype=torch.int32)
        lg = torch.randn(len(st), V)
        host = MaskCache(f).apply(st, lg.clone())
        assert torch.equal(host, OD.apply_mask(lg.clone(), tn, st.numpy()))
        devc = MaskCache(f.to(dev))
        got = devc.apply(st.to(dev), lg.to(dev))
        assert torch.equal(got.cpu(), host)
        assert len(devc) == 0  # no per-state id lists were materialised


def test_flat_schema_auto_mode_churn_64_steps(dev):
    """configs[2] through the default ``auto`` bundle (S * V above the
    density limit, so no tok_next): the allow-bit table is built from trans
    on the device, the mask runs the dense fill kernel over it and the
    commit the fused walking kernel.  B = 512 rows from random valid partial
    documents of 0-80 bytes, bf16 logits N(0, 3), 10 % of the rows evicted
    and re-added at the start state every step (queued writes riding in the
    launches), 64 steps; every mask is compared with ATen's masked_fill_
    over the oracle's whole table (itself equal to the device-built allow
    bits), every commit with the oracle's advance."""
    from bpdecode_amd.batch import build_bundle

    _log("case flat-schema auto bundle V=151936 B=512 bf16 churn 64 steps: oracle table")
    vocab = synth.serving_vocab(151_936, seed=1)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    fsa = build_bundle(dfa, vocab, dev)
    assert fsa.tok_next is None and fsa.num_states * fsa.vocab_size > 32_000_000
    host = fsa.to("cpu")
    tn = OD.build_token_transitions(host.trans.numpy(), host.accept.numpy(), host.live.numpy(),
                                    host.num_symbols, host.offsets.numpy(), host.symbols.numpy(),
                                    host.eos_id)
    B = 512
    batch = ConstraintBatch(fsa, capacity=2 * B, device=dev)
    assert batch._fast and batch._walk_table is not None
    every = np.arange(fsa.num_states, dtype=np.int32)
    assert np.array_equal(fsa.allow_bits.cpu().numpy().view(np.uint32), OD.compute_mask_bits(tn, every))
    _log("case flat-schema auto bundle: trajectory")
    tn_dev = torch.from_numpy(tn).to(dev)
    starts = synth.random_byte_walk_states(torch.from_numpy(tn), fsa.start, B, 80, seed=4).numpy()
    state, active = {}, []
    for i in range(B):
        batch.add(i)
        active.append(i)
        state[i] = int(starts[i])
    batch._state[:B] = torch.from_numpy(starts).to(dev)
    nid = B
    rng = np.random.default_rng(7)
    gen = torch.Generator(device=dev).manual_seed(5)
    for step in range(64):
        ids = list(active)
        st = np.array([state[i] for i in ids], dtype=np.int32)
        lg = torch.randn((B, vocab.size), generator=gen, device=dev).mul_(3.0).to(torch.bfloat16)
        s_ = torch.from_numpy(st).to(dev).long()
        rejected = (tn_dev.index_select(0, s_.clamp(min=0)) == -1) | (s_ < 0)[:, None]
        want = lg.clone().masked_fill_(rejected, float("-inf"))
        got = lg.clone()
        batch.apply_mask(ids, got)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        toks = torch.multinomial(torch.softmax(want.float(), dim=-1), 1, generator=gen).view(-1)
        nxt = batch.commit(ids, toks)
        exp = OD.advance(tn, st, toks.cpu().numpy())
        assert nxt.cpu().numpy().tolist() == exp.tolist(), step
        for i, s in zip(ids, exp.tolist()):
            state[i] = s
        for j in rng.choice(B, size=B // 10, replace=False).tolist():
            batch.evict(active[j])
            del state[active[j]]
            active[j] = nid
            batch.add(nid)
            state[nid] = fsa.start
            nid += 1
    batch.check_errors()
    pool = batch._state.cpu().numpy()
    assert all(pool[batch._slot_of[i]] == s for i, s in state.items())


@pytest.mark.parametrize("rows", [3000, 5000])
def test_fused_walking_commit_large_batches(dev, rows):
    """bpd_fsa_advance at 3,000 rows (one fused launch: four rows per
    thread, queued writes applied) and 5,000 rows (the gather and scatter
    launches, no queued writes) against the oracle's advance."""
    _log(f"case fsa commit rows={rows}")
    vocab = synth.serving_vocab(8192, seed=3)
    f = FsaTensors.build(synth.EMAIL, vocab, dense=False)
    tn = oracle_table(f)
    S, V = tn.shape
    fd = f.to(dev)
    rng = np.random.default_rng(rows)
    st = rng.integers(-2, S, size=rows).astype(np.int32)
    toks = rng.integers(-V, V, size=rows).astype(np.int64)
    pool = torch.from_numpy(st.copy()).to(dev)
    slots = torch.from_numpy(rng.permutation(rows).astype(np.int64)).to(dev)
    want_st = st[slots.cpu().numpy()]
    pending = None
    if rows <= 4096:  # queued writes: 40 slots get a new value first
        qs = rng.choice(rows, size=40, replace=False).astype(np.int64)
        qv = rng.integers(0, S, size=40).astype(np.int64)
        pending = torch.from_numpy(np.concatenate([qs, qv])).to(dev)
        pool_after = st.copy()
        pool_after[qs] = qv
        want_st = pool_after[slots.cpu().numpy()]
    nxt = ops.fsa_advance(fd, pool, torch.from_numpy(toks).to(dev), slots=slots, write_back=True,
                          pending=pending)
    want = OD.advance(tn, want_st, toks)
    assert nxt.cpu().numpy().tolist() == want.tolist()
    expect_pool = (pool_after if pending is not None else st).copy()
    expect_pool[slots.cpu().numpy()] = want
    assert np.array_equal(pool.cpu().numpy(), expect_pool)


def test_walking_commit_with_a_live_array_not_closed(dev):
    """A caller's live array that is not closed under successors (a state
    marked non-live although it steps to a live one): the bundle keeps no
    filtered uint16 table, and the commit walks the int32 table with the
    final live check of mask_cpu.cpp:53-71 -- against the oracle's table
    built with the same live array."""
    _log("case fsa commit, live array not closed")
    f = FsaTensors.build("ab|c|a+1", TOY_VOCAB, dense=False)
    S = f.num_states
    tr = f.trans.reshape(S, f.num_symbols)
    live = f.live.clone()
    src = next(s for s in range(S) if s != f.dead and live[s] and any(
        0 <= int(v) < S and bool(live[int(v)]) for v in tr[s]))
    live[src] = 0
    g = FsaTensors(f.trans, f.accept, live, f.num_symbols, f.dead, f.offsets, f.symbols, f.eos_id,
                   f.start, f.accepting)
    gd = g.to(dev)
    assert not gd.c_fsa_table().trans16
    tn = OD.build_token_transitions(g.trans.numpy(), g.accept.numpy(), live.numpy(), g.num_symbols,
                                    g.offsets.numpy(), g.symbols.numpy(), g.eos_id)
    V = g.vocab_size
    st = np.array([s for s in range(S) for _ in range(V)], dtype=np.int32)
    toks = np.array([t for _ in range(S) for t in range(V)], dtype=np.int64)
    nxt = ops.advance_state(gd, torch.from_numpy(st).to(dev), torch.from_numpy(toks).to(dev))
    assert nxt.cpu().numpy().tolist() == tn[st, toks].tolist()

"""Dense tok_next path on the device (HIP kernels through the C ABI) against
the oracle, at the sizes of the dense workloads: the IPv4 regex over a
32,000-token vocabulary (fp32), the email regex at serving scale (V =
151,936, B = 256, bf16, continuous batching) and the flat JSON-Schema
document DFA (826 states, B = 512, bf16); plus every dtype / fill value /
layout edge case.  Bit-exact throughout."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import ConstraintBatch
from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.grammar.regular import residual_dfa
from bpdecode_amd.ops import FsaTensors
from oracle import dense as OD
from tests._util import TOY_PATTERNS, TOY_VOCAB, bits_of, oracle_table

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def serving_vocab():
    return synth.serving_vocab(151_936, seed=1)


def _sample(logits: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    return torch.multinomial(torch.softmax(logits.float().cpu(), dim=-1), 1, generator=gen).view(-1)


def test_ipv4_32k_fp32_64_steps(dev):
    _log("case ipv4 V=32000 B=8 fp32 64 steps")
    vocab = synth.ipv4_vocab(32_000, seed=0)
    fsa = FsaTensors.build(synth.IPV4, vocab)
    assert fsa.tok_next is not None
    tn = fsa.tok_next.numpy()
    assert np.array_equal(tn, oracle_table(fsa))
    batch = ConstraintBatch(fsa, capacity=8, device=dev)
    start_states = synth.random_walk_states(fsa.tok_next, fsa.start, vocab.eos_id, 8, 3, seed=0)
    for i in range(8):
        batch.add(i)
    batch._state[:8] = start_states.to(dev)
    states = start_states.numpy().copy()
    gen = torch.Generator().manual_seed(0)
    for step in range(64):
        lg = synth.logits(8, vocab.size, 1.0, torch.float32, seed=100 + step)
        want = OD.apply_mask(lg.clone(), tn, states)
        got = lg.to(dev)
        batch.apply_mask(list(range(8)), got)
        assert torch.equal(got.cpu(), want), step
        toks = _sample(want, gen)
        nxt = batch.commit(list(range(8)), toks.to(dev))
        states = OD.advance(tn, states, toks.numpy())
        assert nxt.cpu().numpy().tolist() == states.tolist(), step
    batch.check_errors()


def _aten_mask(logits: torch.Tensor, tok_next: torch.Tensor, states: torch.Tensor,
               neg_inf: float = float("-inf")) -> torch.Tensor:
    """The reference's dense mask as it is written (ops.py:271-276): ATen's
    index_select / compare / masked_fill_, on a copy, on whatever device the
    tensors are on -- the checker for long trajectories, where the numpy
    oracle would take minutes."""
    s = states.long()
    broken = s < 0
    rejected = tok_next.index_select(0, s.clamp(min=0)) == -1
    rejected |= broken[:, None]
    return logits.clone().masked_fill_(rejected, neg_inf)


def _churn_trajectory(dev, serving_vocab, steps):
    V = serving_vocab.size
    fsa_host = FsaTensors.build(synth.EMAIL, serving_vocab)
    fsa = fsa_host.to(dev)
    tn = fsa_host.tok_next.numpy()
    assert np.array_equal(tn, oracle_table(fsa_host))
    gpu_built = FsaTensors.build(synth.EMAIL, serving_vocab, dense=False).to(dev).densify()
    assert torch.equal(gpu_built.tok_next.cpu(), fsa_host.tok_next)
    tn_ref = torch.from_numpy(tn).to(dev)  # the oracle-checked table, for the ATen checker
    B = 256
    batch = ConstraintBatch(fsa, capacity=2 * B, device=dev)
    rng = np.random.default_rng(0)
    state = {}
    nid = 0
    active = []
    for _ in range(B):
        batch.add(nid)
        state[nid] = fsa.start
        active.append(nid)
        nid += 1
    gen = torch.Generator(device=dev).manual_seed(1)
    for step in range(steps):
        ids = list(active)
        st = np.array([state[i] for i in ids], dtype=np.int32)
        lg = torch.randn((B, V), generator=gen, device=dev).mul_(3.0).to(torch.bfloat16)
        want = _aten_mask(lg, tn_ref, torch.from_numpy(st).to(dev))
        if step % 16 == 0:  # the numpy oracle itself, every 16th step
            ref = OD.apply_mask(lg.cpu(), tn, st)
            assert np.array_equal(bits_of(want), bits_of(ref)), step
        got = lg.clone()
        batch.apply_mask(ids, got)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        toks = torch.multinomial(torch.softmax(want.float(), dim=-1), 1, generator=gen).view(-1)
        nxt = batch.commit(ids, toks)
        exp = OD.advance(tn, st, toks.cpu().numpy())
        assert nxt.cpu().numpy().tolist() == exp.tolist(), step
        for i, s in zip(ids, exp.tolist()):
            state[i] = s
        for j in rng.choice(B, size=26, replace=False).tolist():
            batch.evict(active[j])
            del state[active[j]]
            active[j] = nid
            batch.add(nid)
            state[nid] = fsa.start
            nid += 1
    batch.check_errors()
    assert all(batch.state_of(i) == s for i, s in state.items())
    live = batch._state.cpu().numpy()
    for i, s in state.items():
        assert live[batch._slot_of[i]] == s


def test_email_serving_scale_churn_128_steps(dev, serving_vocab):
    """Serving scale, the whole configured trajectory: B = 256, V = 151,936,
    bf16 logits N(0, 3), 10 % of the rows evicted and added every step (the
    queued slot writes ride in the mask launches), 128 steps, tokens sampled
    from the masked softmax; masks, committed states and the pool checked
    every step."""
    _log("case email V=151936 B=256 bf16 churn 128 steps")
    _churn_trajectory(dev, serving_vocab, 128)


def test_flat_schema_dfa_b512_64_steps(dev, serving_vocab):
    """The flat JSON-Schema document DFA (826 states, too large for the auto
    rule, forced dense), B = 512 rows starting from random valid partial
    documents of 0-80 bytes, bf16 logits N(0, 3), 64 mask + commit steps."""
    _log("case flat-schema DFA V=151936 B=512 bf16 64 steps")
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    plain = FsaTensors.build(dfa, serving_vocab, dense=False)
    assert plain.num_states * plain.vocab_size > 32_000_000  # auto would not densify
    dense_dev = plain.to(dev).densify()
    rows = [0, 5, 100, plain.num_states - 1]
    part = ops.build_token_transitions(plain, rows=rows)
    assert np.array_equal(part.numpy(), OD.build_token_transitions(
        plain.trans.numpy(), plain.accept.numpy(), plain.live.numpy(), plain.num_symbols,
        plain.offsets.numpy(), plain.symbols.numpy(), plain.eos_id, rows=rows))
    assert torch.equal(dense_dev.tok_next[rows].cpu(), part)
    tn_dev = dense_dev.tok_next
    tn = tn_dev.cpu().numpy()
    B = 512
    starts = synth.random_byte_walk_states(tn_dev, plain.start, B, 80, seed=4)
    st = starts.numpy().copy()
    assert (st >= 0).all() and len(np.unique(st)) > 20
    batch = ConstraintBatch(dense_dev, capacity=B, device=dev)
    ids = list(range(B))
    for i in ids:
        batch.add(i)
    batch._state[:B] = starts.to(dev)
    gen = torch.Generator(device=dev).manual_seed(5)
    for step in range(64):
        lg = torch.randn((B, serving_vocab.size), generator=gen, device=dev).mul_(3.0).to(torch.bfloat16)
        want = _aten_mask(lg, tn_dev, torch.from_numpy(st).to(dev))
        if step % 16 == 0:
            assert np.array_equal(bits_of(want), bits_of(OD.apply_mask(lg.cpu(), tn, st))), step
        got = lg.clone()
        batch.apply_mask(ids, got)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        toks = torch.multinomial(torch.softmax(want.float(), dim=-1), 1, generator=gen).view(-1)
        nxt = batch.commit(ids, toks)
        st = OD.advance(tn, st, toks.cpu().numpy())
        assert nxt.cpu().numpy().tolist() == st.tolist(), step
    batch.check_errors()


def test_queued_writes_ride_in_launches(dev):
    """add / evict / reset between calls: the mask launch and the commit
    launch apply the queued pool writes themselves (rows read the queued
    value of their slot); more queued writes than one launch takes are
    flushed first.  Masks, returned states and the whole pool against a
    host mirror."""
    vocab = synth.serving_vocab(2048, seed=3)
    fsa = FsaTensors.build(synth.EMAIL, vocab)
    tn = fsa.tok_next.numpy()
    cap = 600
    batch = ConstraintBatch(fsa, capacity=cap, device=dev)
    mirror = np.full(cap, -2, dtype=np.int32)
    rng = np.random.default_rng(4)
    active = []
    nid = 0

    def add():
        nonlocal nid
        slot = batch.add(nid)
        mirror[slot] = fsa.start
        active.append(nid)
        nid += 1

    for _ in range(40):
        add()
    for step in range(30):
        # churn of varying size, including more than one launch applies
        n_ev = [3, 0, 17, 1, 300 if step == 7 else 5][step % 5]
        n_ev = min(n_ev, len(active) - 1)
        for j in sorted(rng.choice(len(active), size=n_ev, replace=False).tolist(), reverse=True):
            sid = active.pop(j)
            mirror[batch._slot_of[sid]] = -2
            batch.evict(sid)
        while len(active) < (40 if step != 7 else 290):
            add()
        if step % 3 == 1 and active:
            sid = active[int(rng.integers(len(active)))]
            batch.reset(sid)
            mirror[batch._slot_of[sid]] = fsa.start
        ids = list(active)
        sl = np.array([batch._slot_of[i] for i in ids])
        st = mirror[sl]
        lg = synth.logits(len(ids), vocab.size, 3.0, torch.float32, seed=step)
        want = OD.apply_mask(lg.clone(), tn, st)
        got = lg.to(dev)
        batch.apply_mask(ids, got)
        assert torch.equal(got.cpu(), want), step
        if step % 4 == 2:  # a write queued between mask and commit reaches the commit launch
            sid = ids[0]
            batch.reset(sid)
            mirror[batch._slot_of[sid]] = fsa.start
            st = mirror[sl]
        toks = torch.from_numpy(rng.integers(0, vocab.size, size=len(ids)))
        nxt = batch.commit(ids, toks.to(dev))
        exp = OD.advance(tn, st, toks.numpy())
        assert nxt.cpu().tolist() == exp.tolist(), step
        mirror[sl] = exp
        assert batch._state.cpu().numpy().tolist() == mirror.tolist(), step
    batch.check_errors()


def test_float64_logits(dev):
    """The dense mask takes float64 logits, as the reference's masked_fill_
    path does (ops.py:271-276): device (allow bits and int32 table) and
    host."""
    vocab = synth.serving_vocab(4099, seed=9)
    fsa = FsaTensors.build(synth.EMAIL, vocab)
    tn = fsa.tok_next.numpy()
    st = np.random.default_rng(2).integers(-2, fsa.num_states, size=19).astype(np.int32)
    base = torch.randn(19, vocab.size, dtype=torch.float64)
    for neg_inf in (float("-inf"), -1e300, 3.25):
        want = OD.apply_mask(base.clone(), tn, st, neg_inf)
        fdev = fsa.to(dev)
        got = base.to(dev)
        ops.apply_mask_(got, fdev, torch.from_numpy(st).to(dev), neg_inf)
        assert np.array_equal(got.cpu().view(torch.int64).numpy(), want.view(torch.int64).numpy())
        got32 = base.to(dev)
        ops.dense_mask_(got32, fdev.tok_next, torch.from_numpy(st).to(dev), neg_inf=neg_inf)
        assert np.array_equal(got32.cpu().view(torch.int64).numpy(), want.view(torch.int64).numpy())
        host = base.clone()
        ops.apply_mask_(host, fsa, torch.from_numpy(st), neg_inf)
        assert np.array_equal(host.view(torch.int64).numpy(), want.view(torch.int64).numpy())
    batch = ConstraintBatch(fsa, capacity=4, device=dev)
    for i in range(4):
        batch.add(i)
    lg = base[:4].to(dev)
    batch.apply_mask(list(range(4)), lg)
    want = OD.apply_mask(base[:4].clone(), tn, np.full(4, fsa.start, np.int32))
    assert np.array_equal(lg.cpu().view(torch.int64).numpy(), want.view(torch.int64).numpy())


def test_int64_token_ids(dev):
    """ConstraintBatch.commit reads int64 ids by their low 32 bits, as the
    reference's ``tokens.to(torch.int32)`` (batch.py:213); ops.advance_state
    indexes with the full int64 (ops.py:301-306): 2**32 + 5 is token 5 for
    the first and out of range for the second."""
    fsa = FsaTensors.build("[01]+", TOY_VOCAB)
    tn = fsa.tok_next.numpy()
    batch = ConstraintBatch(fsa, capacity=2, device=dev)
    batch.add(0)
    batch.add(1)
    one = TOY_VOCAB.token_bytes.index(b"1")
    toks = torch.tensor([2**32 + one, -(2**32) + one], dtype=torch.int64, device=dev)
    nxt = batch.commit([0, 1], toks)
    exp = OD.advance(tn, [fsa.start, fsa.start], toks.cpu().numpy(), low32=True)
    assert nxt.cpu().tolist() == exp.tolist() and exp[0] >= 0
    batch.check_errors()
    st = torch.full((2,), fsa.start, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out = ops.dense_advance(fsa.to(dev).tok_next, st, toks, err=err)
    assert out.cpu().tolist() == [-1, -1] and int(err.item()) & 2
    with pytest.raises(IndexError):
        ops.advance_state(fsa.to(dev), st, toks.cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("neg_inf", [float("-inf"), -1e4, 7.5, float("nan"), -1e9])
@pytest.mark.parametrize("shape", ["aligned", "odd_vocab", "strided", "misaligned"])
def test_edge_cases(dev, dtype, neg_inf, shape):
    vocab = synth.serving_vocab(4096 if shape != "odd_vocab" else 4099, seed=9)
    fsa = FsaTensors.build(synth.EMAIL, vocab)
    tn = fsa.tok_next.numpy()
    rng = np.random.default_rng(1)
    B = 37
    st = rng.integers(-2, fsa.num_states, size=B).astype(np.int32)
    base = synth.logits(B, vocab.size, 3.0, dtype, seed=2)
    try:
        want = OD.apply_mask(base.clone(), tn, st, neg_inf)
    except RuntimeError:
        with pytest.raises(RuntimeError, match="overflow"):
            ops.apply_mask_(base.to(dev), fsa.to(dev), torch.from_numpy(st).to(dev), neg_inf)
        return
    fdev = fsa.to(dev)
    if shape in ("strided", "misaligned"):
        off = 8 if shape == "strided" else 1  # one element: not 16-byte aligned
        wide = torch.zeros(B, vocab.size + 9, dtype=dtype, device=dev)
        view = wide[:, off:off + vocab.size]
        view.copy_(base.to(dev))
        ops.apply_mask_(view, fdev, torch.from_numpy(st).to(dev), neg_inf)
        got = view.cpu()
        assert torch.equal(wide[:, :off].cpu(), torch.zeros(B, off, dtype=dtype))
        assert torch.equal(wide[:, off + vocab.size:].cpu(), torch.zeros(B, 9 - off, dtype=dtype))
    else:
        got = base.to(dev)
        ops.apply_mask_(got, fdev, torch.from_numpy(st).to(dev), neg_inf)  # allow-bit kernel
        got32 = base.to(dev)
        ops.dense_mask_(got32, fdev.tok_next, torch.from_numpy(st).to(dev), neg_inf=neg_inf)  # int32 table
        assert np.array_equal(bits_of(got32), bits_of(want))
    assert np.array_equal(bits_of(got), bits_of(want))
    bits = ops.compute_mask(fdev, torch.from_numpy(st).to(dev))
    assert np.array_equal(bits.cpu().numpy().view(np.uint32), OD.compute_mask_bits(tn, st))


def test_slots_and_pool_writeback(dev):
    fsa = FsaTensors.build("-?[0-9]+(\\.[0-9]+)?", TOY_VOCAB).to(dev)
    tn = fsa.tok_next.cpu().numpy()
    pool = torch.tensor([0, 1, 2, 3, -2, -1, 4, 0], dtype=torch.int32, device=dev)
    slots = torch.tensor([6, 0, 3, 4, 5], dtype=torch.int64, device=dev)
    lg = torch.randn(5, TOY_VOCAB.size, device=dev)
    want = OD.apply_mask(lg.cpu(), tn, pool.cpu().numpy()[slots.cpu().numpy()])
    ops.dense_mask_(lg, fsa.tok_next, pool, slots)
    assert torch.equal(lg.cpu(), want)
    toks = torch.tensor([5, 6, -1, 2, 0], dtype=torch.int64, device=dev)
    before = pool.cpu().numpy().copy()
    nxt = ops.dense_advance(fsa.tok_next, pool, toks, slots, write_back=True)
    exp = OD.advance(tn, before[slots.cpu().numpy()], toks.cpu().numpy())
    assert nxt.cpu().tolist() == exp.tolist()
    after = before.copy()
    after[slots.cpu().numpy()] = exp
    assert pool.cpu().numpy().tolist() == after.tolist()


def test_out_of_range_sets_error_flag(dev):
    fsa = FsaTensors.build("[01]+", TOY_VOCAB)
    batch = ConstraintBatch(fsa, capacity=2, device=dev)
    batch.add(0)
    batch.add(1)
    out = batch.commit([0, 1], torch.tensor([TOY_VOCAB.size + 5, 5], device=dev))
    assert out.cpu().tolist()[0] == -1
    with pytest.raises(IndexError):
        batch.check_errors()
    batch.check_errors()  # cleared
    with pytest.raises(IndexError):
        batch.commit([0], torch.tensor([TOY_VOCAB.size]))  # host ids are checked eagerly


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
def test_toy_patterns_all_states(dev, pattern):
    fsa = FsaTensors.build(pattern, TOY_VOCAB, dense=False)
    tn = oracle_table(fsa)
    S = fsa.num_states
    st = torch.arange(-2, S, dtype=torch.int32)
    lg = torch.randn(S + 2, TOY_VOCAB.size)
    want = OD.apply_mask(lg.clone(), tn, st.numpy())
    got = lg.to(dev)
    ops.apply_mask_(got, fsa.to(dev), st.to(dev))  # walked rows on the device
    assert torch.equal(got.cpu(), want)
    got2 = lg.to(dev)
    ops.apply_mask_(got2, fsa.to(dev).densify(), st.to(dev))
    assert torch.equal(got2.cpu(), want)


@pytest.mark.parametrize("S,M,seed", [(1, 1, 0), (5, 2, 1), (300, 7, 3), (5000, 5, 4), (20000, 3, 5)])
def test_device_reachability_matches_host(dev, S, M, seed):
    """The reachability kernel against the library's host reverse search on
    random tables with sinks and unreachable accepting states."""
    rng = np.random.default_rng(seed)
    trans = rng.integers(0, S, size=(S, M)).astype(np.int32)
    accept = (rng.random(S) < 0.05).astype(np.uint8)
    for s in rng.choice(S, size=max(1, S // 4), replace=False):
        trans[s] = s
    host = ops.build_reachability(torch.from_numpy(trans.reshape(-1)), torch.from_numpy(accept), M)
    got = ops.build_reachability(torch.from_numpy(trans.reshape(-1)).to(dev), torch.from_numpy(accept).to(dev), M)
    assert torch.equal(got.cpu(), host)
    assert 0 < int(host.sum()) < S or S == 1


def test_device_built_bundles_equal_host_built(dev, serving_vocab):
    """FsaTensors.build(..., device=cuda) builds the live set and the dense
    table with the device kernels: the same tables as the host build, for
    the email regex (dense) and the flat JSON-Schema DFA (above the auto
    limit: live set only)."""
    _log("case device-built bundles")
    host = FsaTensors.build(synth.EMAIL, serving_vocab)
    devb = FsaTensors.build(synth.EMAIL, serving_vocab, device=dev)
    assert devb.device.type == "cuda" and devb.tok_next is not None
    assert torch.equal(devb.live.cpu(), host.live) and torch.equal(devb.tok_next.cpu(), host.tok_next)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    h2 = FsaTensors.build(dfa, serving_vocab)
    d2 = FsaTensors.build(dfa, serving_vocab, device=dev)
    assert h2.tok_next is None and d2.tok_next is None
    assert torch.equal(d2.live.cpu(), h2.live) and torch.equal(d2.trans.cpu(), h2.trans)

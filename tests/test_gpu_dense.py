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


def test_email_serving_scale_churn(dev, serving_vocab):
    _log("case email V=151936 B=256 bf16 churn 24 steps")
    V = serving_vocab.size
    fsa_host = FsaTensors.build(synth.EMAIL, serving_vocab)
    fsa = fsa_host.to(dev)
    tn = fsa_host.tok_next.numpy()
    gpu_built = FsaTensors.build(synth.EMAIL, serving_vocab, dense=False).to(dev).densify()
    assert torch.equal(gpu_built.tok_next.cpu(), fsa_host.tok_next)
    sample_rows = [0, 1, fsa.num_states - 1]
    assert np.array_equal(tn[sample_rows], OD.build_token_transitions(
        fsa_host.trans.numpy(), fsa_host.accept.numpy(), fsa_host.live.numpy(), fsa_host.num_symbols,
        fsa_host.offsets.numpy(), fsa_host.symbols.numpy(), fsa_host.eos_id, rows=sample_rows))
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
    gen = torch.Generator().manual_seed(1)
    for step in range(24):
        ids = list(active)
        st = np.array([state[i] for i in ids], dtype=np.int32)
        lg = synth.logits(B, V, 3.0, torch.bfloat16, seed=1000 + step)
        want = OD.apply_mask(lg.clone(), tn, st)
        got = lg.to(dev)
        batch.apply_mask(ids, got)
        assert np.array_equal(bits_of(got), bits_of(want)), step
        toks = _sample(want, gen)
        nxt = batch.commit(ids, toks.to(dev))
        exp = OD.advance(tn, st, toks.numpy())
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


def test_flat_schema_dfa_b512(dev, serving_vocab):
    _log("case flat-schema DFA V=151936 B=512 bf16")
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    plain = FsaTensors.build(dfa, serving_vocab, dense=False)
    assert plain.num_states * plain.vocab_size > 32_000_000  # auto would not densify
    dense_dev = plain.to(dev).densify()
    rows = [0, 5, 100, plain.num_states - 1]
    part = ops.build_token_transitions(plain, rows=rows)
    assert np.array_equal(part.numpy(), oracle_table(plain)[rows] if plain.num_states < 64 else
                          OD.build_token_transitions(plain.trans.numpy(), plain.accept.numpy(),
                                                     plain.live.numpy(), plain.num_symbols,
                                                     plain.offsets.numpy(), plain.symbols.numpy(),
                                                     plain.eos_id, rows=rows))
    assert torch.equal(dense_dev.tok_next[rows].cpu(), part)
    tn_dev = dense_dev.tok_next
    starts = synth.random_walk_states(tn_dev.cpu(), plain.start, serving_vocab.eos_id, 512, 20, seed=4)
    tn = tn_dev.cpu().numpy()
    st = starts.numpy()
    lg = synth.logits(512, serving_vocab.size, 3.0, torch.bfloat16, seed=7)
    want = OD.apply_mask(lg.clone(), tn, st)
    got = lg.to(dev)
    ops.apply_mask_(got, dense_dev, starts.to(dev))
    assert np.array_equal(bits_of(got), bits_of(want))
    toks = _sample(want, torch.Generator().manual_seed(5))
    assert ops.advance_state(dense_dev, starts.to(dev), toks.to(dev)).cpu().tolist() == \
        OD.advance(tn, st, toks.numpy()).tolist()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("neg_inf", [float("-inf"), -1e4, 7.5, float("nan"), -1e9])
@pytest.mark.parametrize("shape", ["aligned", "odd_vocab", "strided"])
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
    if shape == "strided":
        wide = torch.zeros(B, vocab.size + 8, dtype=dtype, device=dev)
        view = wide[:, 8:]
        view.copy_(base.to(dev))
        ops.apply_mask_(view, fdev, torch.from_numpy(st).to(dev), neg_inf)
        got = view.cpu()
        assert torch.equal(wide[:, :8].cpu(), torch.zeros(B, 8, dtype=dtype))
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

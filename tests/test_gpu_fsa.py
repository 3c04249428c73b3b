"""Symbol-class FSA walking kernels (bundles without tok_next, the
reference's non-dense operators) on the device against the oracle: every
state of the toy grammars in every logits dtype with the transition table
in LDS and in global memory, the flat JSON-Schema DFA at serving scale
(826 states, V = 151,936: its table, 256 symbols merged into fewer
classes, is read through L2), ConstraintBatch with slots and churn, the
range flags, and MaskCache without a host round trip.  Bit-exact."""

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


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("table", [None, "global"])
def test_toy_every_state(dev, pattern, dtype, table, monkeypatch):
    _log(f"case fsa walk toy {pattern!r} {dtype} table={table}")
    if table:
        monkeypatch.setenv("BPD_FSA_TABLE", table)
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
    bits = ops.compute_mask(fd, torch.from_numpy(st).to(dev)).cpu().numpy().view(np.uint32)
    assert np.array_equal(bits, OD.compute_mask_bits(tn, st))
    for k in range(3):
        toks = np.array([(5 * i + 7 * k) % V for i in range(len(st))], dtype=np.int32)
        toks[::4] = f.eos_id
        toks[1::9] = -1  # indexes from the end, like the dense commit
        nxt = ops.advance_state(fd, torch.from_numpy(st).to(dev), torch.from_numpy(toks).to(dev))
        assert nxt.cpu().tolist() == OD.advance(tn, st, toks).tolist()


def test_flat_schema_serving_scale(dev):
    _log("case fsa walk flat-schema DFA V=151936 B=256 bf16")
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


def test_batch_churn_and_range_flags(dev):
    _log("case fsa walk ConstraintBatch churn")
    vocab = synth.serving_vocab(8192, seed=3)
    f = FsaTensors.build(synth.EMAIL, vocab, dense=False)
    tn = OD.build_token_transitions(f.trans.numpy(), f.accept.numpy(), f.live.numpy(), f.num_symbols,
                                    f.offsets.numpy(), f.symbols.numpy(), f.eos_id)
    batch = ConstraintBatch(f, capacity=48, device=dev)
    assert batch.fsa.tok_next is None
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

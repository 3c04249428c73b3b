"""torch.ops.bpdecode.*: the reference's seven schemas (bindings/torch_ops.cpp:
427-459) plus the two dense operators, registered by importing the package,
checked on CPU tensors against the operator layer and the oracles, with the
reference's dtype/shape errors."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bpdecode_amd.ops  # noqa: F401  (registers the operators)
from bpdecode_amd.grammar.device import build_pda_tensors
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.ops import FsaTensors
from oracle import dense as OD
from oracle import pda as OP
from tests._util import PDA_VOCAB, TOY_VOCAB, oracle_table

OPS = torch.ops.bpdecode

REFERENCE_SCHEMAS = {
    "build_reachability": "bpdecode::build_reachability(Tensor trans, Tensor accept, int num_symbols) -> Tensor",
    "apply_mask_": "bpdecode::apply_mask_(Tensor(a!) logits, Tensor trans, Tensor accept, Tensor live, "
                   "int num_symbols, int dead, Tensor offsets, Tensor symbols, int eos_id, Tensor states, "
                   "float neg_inf) -> Tensor(a!)",
    "compute_mask": "bpdecode::compute_mask(Tensor trans, Tensor accept, Tensor live, int num_symbols, "
                    "int dead, Tensor offsets, Tensor symbols, int eos_id, Tensor states) -> Tensor",
    "advance_state": "bpdecode::advance_state(Tensor trans, Tensor accept, Tensor live, int num_symbols, "
                     "int dead, Tensor offsets, Tensor symbols, int eos_id, Tensor states, "
                     "Tensor token_ids) -> Tensor",
    "pda_init": "bpdecode::pda_init(Tensor accept, Tensor live, Tensor edge_offsets, Tensor edge_kind, "
                "Tensor edge_lo, Tensor edge_hi, Tensor edge_dst, Tensor edge_callee, int root_start, "
                "int root_accept) -> Tensor",
    "pda_apply_mask_": "bpdecode::pda_apply_mask_(Tensor(a!) logits, Tensor accept, Tensor live, "
                       "Tensor edge_offsets, Tensor edge_kind, Tensor edge_lo, Tensor edge_hi, "
                       "Tensor edge_dst, Tensor edge_callee, int root_start, int root_accept, "
                       "Tensor tok_offsets, Tensor tok_bytes, int eos_id, Tensor configs, "
                       "float neg_inf) -> Tensor(a!)",
    "pda_advance_state": "bpdecode::pda_advance_state(Tensor(a!) configs, Tensor accept, Tensor live, "
                         "Tensor edge_offsets, Tensor edge_kind, Tensor edge_lo, Tensor edge_hi, "
                         "Tensor edge_dst, Tensor edge_callee, int root_start, int root_accept, "
                         "Tensor tok_offsets, Tensor tok_bytes, int eos_id, Tensor token_ids) -> Tensor",
}


def fsa_args(f: FsaTensors):
    return (f.trans, f.accept, f.live, f.num_symbols, f.dead, f.offsets, f.symbols, f.eos_id)


def pda_args(g):
    return (g.accept, g.live, g.edge_offsets, g.edge_kind, g.edge_lo, g.edge_hi, g.edge_dst,
            g.edge_callee, g.root_start, g.root_accept)


def test_reference_schemas_registered():
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(OPS, name).default._schema) == schema
    assert "dense_apply_mask_" in str(OPS.dense_apply_mask_.default._schema)
    assert "dense_advance_state" in str(OPS.dense_advance_state.default._schema)


@pytest.mark.parametrize("pattern", ["[01]+", "a+b*", "-?[0-9]+(\\.[0-9]+)?", "caf(e|é)"])
def test_fsa_ops_match_oracle(pattern):
    f = FsaTensors.build(pattern, TOY_VOCAB, dense=False)
    table = oracle_table(f)
    S, V = table.shape
    states = torch.tensor(list(range(S)) + [-1, -2], dtype=torch.int32)
    live = OPS.build_reachability(f.trans, f.accept, f.num_symbols)
    assert torch.equal(live, f.live)
    logits = torch.randn(len(states), V)
    want = OD.apply_mask(logits.clone(), table, states.numpy())
    out = OPS.apply_mask_(logits, *fsa_args(f), states, float("-inf"))
    assert out is logits and torch.equal(logits, want)
    bits = OPS.compute_mask(*fsa_args(f), states).numpy().view(np.uint32)
    assert np.array_equal(bits, OD.compute_mask_bits(table, states.numpy()))
    toks = torch.tensor([(3 * i) % V for i in range(len(states))], dtype=torch.int32)
    nxt = OPS.advance_state(*fsa_args(f), states, toks)
    assert np.array_equal(nxt.numpy(), OD.advance(table, states.numpy(), toks.numpy()))
    dense = FsaTensors.build(pattern, TOY_VOCAB, dense=True).tok_next
    lg = torch.randn(len(states), V)
    want = OD.apply_mask(lg.clone(), table, states.numpy())
    assert torch.equal(OPS.dense_apply_mask_(lg, dense, states, float("-inf")), want)
    assert np.array_equal(OPS.dense_advance_state(dense, states, toks).numpy(),
                          OD.advance(table, states.numpy(), toks.numpy()))


def test_fsa_op_errors_follow_reference():
    f = FsaTensors.build("[01]+", TOY_VOCAB, dense=False)
    st = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="float32"):
        OPS.apply_mask_(torch.zeros(2, TOY_VOCAB.size, dtype=torch.bfloat16), *fsa_args(f), st, -1.0)
    with pytest.raises(RuntimeError, match="int32"):
        OPS.apply_mask_(torch.zeros(2, TOY_VOCAB.size), *fsa_args(f), st.long(), -1.0)
    with pytest.raises(RuntimeError, match="one state per logits row"):
        OPS.apply_mask_(torch.zeros(3, TOY_VOCAB.size), *fsa_args(f), st, -1.0)
    with pytest.raises(RuntimeError, match="int32"):
        OPS.advance_state(*fsa_args(f), st, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(IndexError):
        OPS.advance_state(*fsa_args(f), st, torch.tensor([0, TOY_VOCAB.size], dtype=torch.int32))


def test_pda_ops_match_oracle():
    comp = CompiledGrammar.build(parse_gbnf('root ::= "(" root ")" | "x" | "[" "1"? "]"'))
    g = build_pda_tensors(comp, PDA_VOCAB)
    t = OP.Table(g)
    init = OPS.pda_init(*pda_args(g))
    assert np.array_equal(init.numpy(), OP.init(t))
    cfgs = torch.stack([init.clone() for _ in range(3)])
    tail = (g.tok_offsets, g.tok_bytes, g.eos_id)
    logits = torch.randn(3, PDA_VOCAB.size)
    want = logits.numpy().copy()
    OP.apply_mask(t, cfgs.numpy().copy(), want)
    out = OPS.pda_apply_mask_(logits, *pda_args(g), *tail, cfgs, float("-inf"))
    assert out is logits and np.array_equal(logits.numpy(), want)
    toks = torch.tensor([PDA_VOCAB.token_bytes.index(b) for b in (b"(", b"x", b"]")], dtype=torch.int32)
    mirror = cfgs.numpy().copy()
    ok_o = OP.advance(t, mirror, toks.numpy())
    ok = OPS.pda_advance_state(cfgs, *pda_args(g), *tail, toks)
    assert ok.dtype == torch.uint8 and ok.tolist() == ok_o.astype(np.uint8).tolist()
    assert np.array_equal(cfgs.numpy(), mirror)
    with pytest.raises(RuntimeError, match="configs must be"):
        OPS.pda_apply_mask_(torch.zeros(3, PDA_VOCAB.size), *pda_args(g), *tail, cfgs[:, :10].contiguous(), -1.0)
    with pytest.raises(RuntimeError, match="token_ids must be int32"):
        OPS.pda_advance_state(cfgs, *pda_args(g), *tail, toks.long())

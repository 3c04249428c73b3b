"""torch.ops.bpdecode.* on device tensors: the same results as on the host."""

from __future__ import annotations

import pytest
import torch

import bpdecode_amd.ops  # noqa: F401
from bpdecode_amd import synth
from bpdecode_amd.grammar.device import build_pda_tensors
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.ops import FsaTensors
from tests._util import PDA_VOCAB

pytestmark = pytest.mark.gpu
OPS = torch.ops.bpdecode


def test_fsa_ops_device_equal_host(dev):
    vocab = synth.ipv4_vocab(32_000, seed=0)
    f = FsaTensors.build(synth.IPV4, vocab, dense=False)
    fd = f.to(dev)
    args = lambda x: (x.trans, x.accept, x.live, x.num_symbols, x.dead, x.offsets, x.symbols, x.eos_id)  # noqa: E731
    st = torch.tensor([0, 1, 2, 3, -1, 5, -2, 7], dtype=torch.int32)
    lg = torch.randn(8, vocab.size)
    want = OPS.apply_mask_(lg.clone(), *args(f), st, float("-inf"))
    got = OPS.apply_mask_(lg.to(dev), *args(fd), st.to(dev), float("-inf"))
    assert torch.equal(got.cpu(), want)
    assert torch.equal(OPS.compute_mask(*args(fd), st.to(dev)).cpu(), OPS.compute_mask(*args(f), st))
    tk = torch.randint(0, vocab.size, (8,), dtype=torch.int32)
    assert torch.equal(OPS.advance_state(*args(fd), st.to(dev), tk.to(dev)).cpu(),
                       OPS.advance_state(*args(f), st, tk))
    tn = FsaTensors.build(synth.IPV4, vocab).tok_next
    lg2 = torch.randn(8, vocab.size)
    assert torch.equal(OPS.dense_apply_mask_(lg2.to(dev), tn.to(dev), st.to(dev), -1e4).cpu(),
                       OPS.dense_apply_mask_(lg2.clone(), tn, st, -1e4))
    assert torch.equal(OPS.dense_advance_state(tn.to(dev), st.to(dev), tk.to(dev)).cpu(),
                       OPS.dense_advance_state(tn, st, tk))


def test_pda_ops_device_equal_host(dev):
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, PDA_VOCAB, eps_reduce=True)
    gd = g.to(dev)
    pa = lambda x: (x.accept, x.live, x.edge_offsets, x.edge_kind, x.edge_lo, x.edge_hi,  # noqa: E731
                    x.edge_dst, x.edge_callee, x.root_start, x.root_accept)
    tail = lambda x: (x.tok_offsets, x.tok_bytes, x.eos_id)  # noqa: E731
    init = OPS.pda_init(*pa(gd))
    assert init.device.type == "cuda"
    assert torch.equal(init.cpu(), OPS.pda_init(*pa(g)))
    cfgs = torch.stack([init.cpu().clone() for _ in range(4)])
    lg = torch.randn(4, PDA_VOCAB.size)
    want = OPS.pda_apply_mask_(lg.clone(), *pa(g), *tail(g), cfgs, float("-inf"))
    got = OPS.pda_apply_mask_(lg.to(dev), *pa(gd), *tail(gd), cfgs.to(dev), float("-inf"))
    assert torch.equal(got.cpu(), want)
    toks = torch.tensor([PDA_VOCAB.token_bytes.index(b) for b in (b"{", b"[", b"tr", b"\"")],
                        dtype=torch.int32)
    cd = cfgs.to(dev)
    ok_d = OPS.pda_advance_state(cd, *pa(gd), *tail(gd), toks.to(dev))
    ok_h = OPS.pda_advance_state(cfgs, *pa(g), *tail(g), toks)
    assert torch.equal(ok_d.cpu(), ok_h) and torch.equal(cd.cpu(), cfgs)

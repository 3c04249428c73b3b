"""Empty batches on the device: every operator returns an empty result (or
leaves an empty logits tensor alone) without launching a kernel, as the
reference's ATen paths do for zero rows."""

from __future__ import annotations

import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import ConstraintBatch
from bpdecode_amd.grammar.device import build_pda_tensors, pda_compute_mask, pda_mask_, pda_step
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.ops import FsaTensors
from tests._util import PDA_VOCAB, TOY_VOCAB

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dense", [True, False])
def test_fsa_ops_zero_rows(dev, dense):
    print(f"case empty batch fsa dense={dense}", flush=True)
    f = FsaTensors.build("-?[0-9]+", TOY_VOCAB, dense=dense).to(dev)
    V = TOY_VOCAB.size
    st = torch.empty(0, dtype=torch.int32, device=dev)
    lg = torch.empty(0, V, device=dev)
    assert ops.apply_mask_(lg, f, st).shape == (0, V)
    assert ops.compute_mask(f, st).shape == (0, (V + 31) // 32)
    assert ops.advance_state(f, st, torch.empty(0, dtype=torch.int64, device=dev)).numel() == 0
    batch = ConstraintBatch(f, capacity=4, device=dev)
    batch.apply_mask([], lg)
    assert batch.commit([], torch.empty(0, dtype=torch.int64, device=dev)).numel() == 0


def test_soft_prior_zero_rows(dev):
    print("case empty batch soft prior", flush=True)
    f = FsaTensors.build("-?[0-9]+", TOY_VOCAB).densify().to(dev)
    lg = torch.empty(0, TOY_VOCAB.size, device=dev)
    ops.apply_soft_prior_(lg, f, torch.empty(0, dtype=torch.int32, device=dev), 3, 1.0)
    assert lg.shape == (0, TOY_VOCAB.size)


def test_pda_ops_zero_rows(dev):
    print("case empty batch pda", flush=True)
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF)), PDA_VOCAB).to(dev)
    cfg = torch.empty(0, 266, dtype=torch.int32, device=dev)
    assert pda_compute_mask(g, cfg).shape[0] == 0
    lg = torch.empty(0, PDA_VOCAB.size, device=dev)
    pda_mask_(lg, g, cfg)
    ok, status = pda_step(cfg, g, torch.empty(0, dtype=torch.int32, device=dev))
    assert ok.numel() == 0 and status.numel() == 0

"""Soft lookahead on the device against the float64 oracle (relative error
1e-5 with an absolute floor of 1e-5 near 0; -inf pattern exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import ConstraintBatch
from bpdecode_amd.ops import FsaTensors
from oracle import soft as OS
from tests._util import TOY_PATTERNS, TOY_VOCAB

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-5


def close(got: np.ndarray, want: np.ndarray) -> bool:
    inf_ok = np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    return inf_ok and bool(np.all(np.abs(got[fin] - want[fin]) <= RTOL * np.abs(want[fin]) + ATOL))


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_build_lookahead_toy(dev, pattern, k):
    fsa = FsaTensors.build(pattern, TOY_VOCAB).to(dev)
    la = ops.build_lookahead(fsa, k).cpu().numpy()
    want = OS.build_lookahead(fsa.tok_next.cpu().numpy(), fsa.live.cpu().numpy(),
                              fsa.accept.cpu().numpy(), fsa.eos_id, k)
    assert close(la, want)


def test_build_lookahead_email_serving(dev):
    vocab = synth.serving_vocab(151_936, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).to(dev)
    la = ops.build_lookahead(fsa, 4).cpu().numpy()
    want = OS.build_lookahead(fsa.tok_next.cpu().numpy(), fsa.live.cpu().numpy(),
                              fsa.accept.cpu().numpy(), fsa.eos_id, 4)
    assert close(la, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("alpha", [0.0, 1.0, -0.5, 2.0])
def test_apply_soft(dev, dtype, alpha):
    fsa = FsaTensors.build("a[012]+|b0", TOY_VOCAB).with_lookahead(3).to(dev)
    st = torch.tensor([0, 1, 2, -1, -2, 0], dtype=torch.int32)
    base = torch.randn(6, TOY_VOCAB.size).to(dtype)
    batch = ConstraintBatch(fsa, capacity=6, device=dev)
    for i in range(6):
        batch.add(i)
    batch._state[:6] = st.to(dev)
    got = base.to(dev)
    batch.apply_soft(list(range(6)), got, alpha)
    want = OS.apply_soft(base.float().numpy(), fsa.lookahead.cpu().numpy().astype(np.float64), st.numpy(), alpha)
    host = base.clone()
    ops.apply_soft_(host, fsa.to("cpu"), st, alpha)
    assert torch.equal(got.cpu().view(torch.uint8), host.view(torch.uint8))
    g = got.cpu().float().numpy().astype(np.float64)
    if dtype == torch.float32:
        assert close(g, want)
    else:
        assert np.array_equal(np.isneginf(g), np.isneginf(want))
        fin = np.isfinite(want)
        assert np.all(np.abs(g[fin] - want[fin]) <= 1e-2 * np.abs(want[fin]) + 1e-2)

"""The allocation-free prior lookahead (bpd_soft_prior_noalloc, static
device scratch) against the entry point with a caller workspace
(bpd_soft_prior), both through the C ABI: two calls in a row, the second on
a smaller input; a call needing more than the scratch holds is refused on
the host.  The bar is the lookahead's float tolerance (relative 1e-5 with an
absolute floor of 1e-5, the -inf pattern exact): its class sums are formed
with float atomics, whose order -- and so the last bit -- varies from run to
run of either entry point."""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from bpdecode_amd import _lib, synth
from bpdecode_amd._lib import lib, ptr
from bpdecode_amd.ops import FsaTensors

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _args(fd, sc, logits, states):
    B, V = logits.shape
    eos = fd.eos_id if fd.eos_id is not None and 0 <= fd.eos_id < V else -1
    return (ptr(logits), B, V, logits.stride(0), fd.num_states, ptr(fd.accept), ptr(fd.live), eos,
            ptr(states), None, C.byref(sc.c_struct()))


def _with_workspace(fd, sc, logits, states, k, alpha, dev):
    B, V = logits.shape
    need = int(lib().bpd_soft_prior_workspace_bytes(B, V, sc.num_classes, sc.num_pieces))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib().bpd_soft_prior(*_args(fd, sc, logits, states), k, alpha, ptr(ws), need, None,
                                    _lib.stream_of(dev)))


def _no_alloc(fd, sc, logits, states, k, alpha, dev):
    _lib.check(lib().bpd_soft_prior_noalloc(*_args(fd, sc, logits, states), k, alpha, None,
                                            _lib.stream_of(dev)))


def test_no_alloc_matches_workspace_entry_point(dev):
    vocab = synth.serving_vocab(151_936, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    fd = fsa.to(dev)
    sc = fd.ensure_soft_classes()
    for case, (B, k, alpha, seed) in enumerate([(128, 4, 1.0, 11), (37, 3, 0.5, 12)]):
        _log(f"case no-alloc prior lookahead call {case}: B={B} V={vocab.size} k={k}")
        states = synth.random_walk_states(fsa.tok_next, fsa.start, fsa.eos_id, B, 40, seed=seed)
        states = states.to(torch.int32).to(dev)
        src = synth.logits(B, vocab.size, std=3.0, dtype=torch.float32, seed=seed, device=dev)
        want = src.clone()
        _with_workspace(fd, sc, want, states, k, alpha, dev)
        got = src.clone()
        _no_alloc(fd, sc, got, states, k, alpha, dev)
        torch.cuda.synchronize()
        assert torch.equal(torch.isneginf(got), torch.isneginf(want)), case
        fin = torch.isfinite(want)
        assert torch.isfinite(got[fin]).all(), case
        diff = (got[fin].double() - want[fin].double()).abs()
        assert bool((diff <= 1e-5 * want[fin].double().abs() + 1e-5).all()), (case, float(diff.max()))
        assert torch.isfinite(got).any() and torch.isneginf(got).any()


def test_no_alloc_refuses_more_than_its_scratch(dev):
    vocab = synth.serving_vocab(151_936, seed=1)
    fd = FsaTensors.build(synth.EMAIL, vocab).densify().to(dev)
    sc = fd.ensure_soft_classes()
    B = 429  # 16,781,312 bytes of workspace at 126 classes: more than the 16 MiB scratch
    assert int(lib().bpd_soft_prior_workspace_bytes(B, vocab.size, sc.num_classes, sc.num_pieces)) > \
        _lib.SOFT_PRIOR_SCRATCH_BYTES
    logits = torch.zeros(B, vocab.size, device=dev)
    states = torch.zeros(B, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="scratch"):
        _no_alloc(fd, sc, logits, states, 4, 1.0, dev)
    assert torch.count_nonzero(logits) == 0

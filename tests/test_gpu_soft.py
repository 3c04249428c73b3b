"""Soft lookahead on the device against the float64 oracle (relative error
1e-5 with an absolute floor of 1e-5 near 0; -inf pattern exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from bpdecode_amd import ops, synth
from bpdecode_amd.batch import ConstraintBatch
from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
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


# ------------------------------------------------------- prior-weighted --
# The toy vocabulary with three more tokens: V = 20, a multiple of 4, so the
# vectorised kernels apply (V = 17 takes the scalar ones).
TOY_VOCAB20 = Vocabulary.from_tokens(list(TOY_VOCAB.token_bytes) + [b"d", b"e0", b"bb"],
                                     eos_id=TOY_VOCAB.eos_id)


@pytest.mark.parametrize("pattern", TOY_PATTERNS)
@pytest.mark.parametrize("k", [1, 2, 4])
@pytest.mark.parametrize("alpha", [0.0, 1.0, -0.5])
@pytest.mark.parametrize("vocab", ["v17", "v20"])
def test_prior_toy(dev, pattern, k, alpha, vocab):
    fsa = FsaTensors.build(pattern, TOY_VOCAB if vocab == "v17" else TOY_VOCAB20).densify()
    S, V = fsa.tok_next.shape
    st = torch.tensor(list(range(S)) + [-1, 0], dtype=torch.int32)
    g = torch.Generator().manual_seed(k * 13 + len(pattern))
    x = torch.randn(len(st), V, generator=g) * 3
    got = x.to(dev)
    ops.apply_soft_prior_(got, fsa.to(dev), st.to(dev), k, alpha)
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, st.numpy(), k, alpha)
    assert close(got.cpu().double().numpy(), want)


@pytest.mark.parametrize("vocab", ["v17", "v20"])
def test_prior_batch_slots_and_errors(dev, vocab):
    fsa = FsaTensors.build("a[012]+|b0", TOY_VOCAB if vocab == "v17" else TOY_VOCAB20).densify().to(dev)
    S, V = fsa.tok_next.shape
    batch = ConstraintBatch(fsa, capacity=8, device=dev)
    for i in range(6):
        batch.add(i)
    pool = torch.tensor([0, 1, 2, -1, 0, 2, -2, -2], dtype=torch.int32)
    batch._state[:] = pool.to(dev)
    ids = [4, 2, 0, 3, 1]
    x = torch.randn(5, V) * 3
    got = x.to(dev)
    batch.apply_soft_prior(ids, got, k=3, alpha=0.5)
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.cpu().numpy(), fsa.live.cpu().numpy(),
                              fsa.accept.cpu().numpy(), fsa.eos_id, pool[ids].numpy(), 3, 0.5)
    assert close(got.cpu().double().numpy(), want)
    batch.check_errors()
    batch._state[0] = S  # out-of-range state: -inf row and the device error flag
    got = x.to(dev)
    batch.apply_soft_prior([0], got[:1], k=3, alpha=0.5)
    assert torch.isneginf(got[0]).all()
    with pytest.raises(IndexError):
        batch.check_errors()


def test_prior_unaligned_vocab(dev):
    # V = 17 (not a multiple of 4) and a strided row view take the scalar kernels
    fsa = FsaTensors.build("[a-c]*", TOY_VOCAB).densify()
    S, V = fsa.tok_next.shape
    wide = torch.randn(4, V + 3, generator=torch.Generator().manual_seed(17)) * 3
    st = torch.tensor([0, 0, -1, 0], dtype=torch.int32)
    want = OS.prior_lookahead(wide[:, :V].double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, st.numpy(), 4, 1.0)
    w = wide.to(dev)
    ops.apply_soft_prior_(w[:, :V], fsa.to(dev), st.to(dev), 4, 1.0)
    assert close(w[:, :V].cpu().double().numpy(), want)
    assert torch.equal(w[:, V:].cpu(), wide[:, V:])


@pytest.fixture(scope="module")
def email_serving():
    """B=128, V=151,936, k=4 over the email DFA, logits N(0, 3),
    rows at random reachable states; the float64 oracle of every row,
    computed once with the rows split over host threads (numpy releases the
    interpreter lock in its array loops)."""
    from concurrent.futures import ThreadPoolExecutor

    vocab = synth.serving_vocab(151_936, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    tn = fsa.tok_next.numpy()
    st = synth.random_walk_states(fsa.tok_next, fsa.start, fsa.eos_id, 128, 40, seed=5).to(torch.int32)
    x = synth.logits(128, tn.shape[1], std=3.0, dtype=torch.float32, seed=11)
    xd = x.double().numpy()
    live, acc, stn = fsa.live.numpy(), fsa.accept.numpy(), st.numpy()
    with ThreadPoolExecutor(16) as ex:
        rows = list(ex.map(lambda b: OS.prior_lookahead(xd[b:b + 1], tn, live, acc, fsa.eos_id,
                                                         stn[b:b + 1], 4, 1.0), range(128)))
    return fsa, st, x, np.concatenate(rows)


@pytest.mark.parametrize("stats", ["list", "wave", "members", "classes"])
def test_prior_email_serving(dev, stats, monkeypatch, email_serving):
    """B=128, V=151,936, k=4 over the email DFA: every row against the
    float64 oracle and against the alpha-free identity (alpha = 0 leaves
    log_softmax on tokens whose k-1 lookahead is finite); class statistics
    with wave shifts over 8192-token chunks from the chunk member lists (and
    the member-list output pass) or from the class map, and over
    4096-token chunks from the member lists and from the class map."""
    monkeypatch.setenv("BPD_SOFT_STATS", stats)
    fsa, st, x, want = email_serving
    fd = fsa.to(dev)
    assert fd.ensure_soft_classes().chunk_cap in (256, 512, 1024)
    got = x.to(dev)
    ops.apply_soft_prior_(got, fd, st.to(dev), 4, 1.0)
    got = got.cpu().double().numpy()
    assert close(got, want)
    zero = x.to(dev)
    ops.apply_soft_prior_(zero, fd, st.to(dev), 4, 0.0)
    ls = torch.log_softmax(x.double(), dim=1).numpy()
    fin = np.isfinite(got)
    assert np.array_equal(np.isfinite(zero.cpu().numpy()), fin)
    z = zero.cpu().double().numpy()
    assert np.all(np.abs(z[fin] - ls[fin]) <= RTOL * np.abs(ls[fin]) + ATOL)


@pytest.mark.parametrize("pattern", ["a[012]+|b0", "[a-c]*"])
def test_prior_pieces_path(dev, pattern, monkeypatch):
    """The gather-over-class-pieces statistics (taken above 1024 token
    classes; forced here) give the same results."""
    monkeypatch.setenv("BPD_SOFT_PRIOR_PIECES", "1")
    fsa = FsaTensors.build(pattern, TOY_VOCAB).densify()
    S, V = fsa.tok_next.shape
    st = torch.tensor(list(range(S)) + [-1], dtype=torch.int32)
    x = torch.randn(len(st), V) * 3
    got = x.to(dev)
    ops.apply_soft_prior_(got, fsa.to(dev), st.to(dev), 4, 0.7)
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, st.numpy(), 4, 0.7)
    assert close(got.cpu().double().numpy(), want)


def test_prior_pieces_path_email(dev, monkeypatch):
    vocab = synth.serving_vocab(151_936, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    st = synth.random_walk_states(fsa.tok_next, fsa.start, fsa.eos_id, 16, 40, seed=9).to(torch.int32)
    x = synth.logits(16, 151_936, std=3.0, dtype=torch.float32, seed=12)
    fd = fsa.to(dev)
    a = x.to(dev)
    ops.apply_soft_prior_(a, fd, st.to(dev), 4, 1.0)
    monkeypatch.setenv("BPD_SOFT_PRIOR_PIECES", "1")
    b = x.to(dev)
    ops.apply_soft_prior_(b, fd, st.to(dev), 4, 1.0)
    a, b = a.cpu().double().numpy(), b.cpu().double().numpy()
    assert close(b, a)


@pytest.mark.parametrize("vocab", ["v17", "v20"])
def test_prior_wide_class_map_and_extreme_logits(dev, monkeypatch, vocab):
    """Every statistics path gives the oracle's results: wave shifts over the
    member lists (with the member-list output pass) and over the uint16
    class map (the -1e4 logits sit far below their wave's maximum, so those
    blocks take the exact per-class maximum), the 4096-token chunk member
    lists, the uint16 class map and the int32 one.  Rows mixing -inf, very negative
    and large logits keep every class sum exact."""
    fsa = FsaTensors.build("-?[0-9]+(\\.[0-9]+)?", TOY_VOCAB if vocab == "v17" else TOY_VOCAB20).densify()
    S, V = fsa.tok_next.shape
    st = torch.tensor(list(range(S)) * 2, dtype=torch.int32)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(len(st), V, generator=g) * 3
    x[1::2, ::3] = -1.0e4
    x[2::4, 1::5] = float("-inf")
    x[3::4, 2] = 60.0
    want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                              fsa.accept.numpy(), fsa.eos_id, st.numpy(), 4, 0.8)
    fd = fsa.to(dev)
    sc = fd.ensure_soft_classes()
    assert sc.token_class16 is not None
    a = x.to(dev)
    ops.apply_soft_prior_(a, fd, st.to(dev), 4, 0.8)
    assert close(a.cpu().double().numpy(), want)
    for stats in ("wave", "members", "classes"):
        monkeypatch.setenv("BPD_SOFT_STATS", stats)
        m = x.to(dev)
        ops.apply_soft_prior_(m, fd, st.to(dev), 4, 0.8)
        assert close(m.cpu().double().numpy(), want), stats
    monkeypatch.setenv("BPD_SOFT_STATS", "classes")
    sc.token_class16, sc._c = None, None
    b = x.to(dev)
    ops.apply_soft_prior_(b, fd, st.to(dev), 4, 0.8)
    assert close(b.cpu().double().numpy(), want)


@pytest.mark.parametrize("pattern", ["[a-c]*", "a[012]+|b0"])
@pytest.mark.parametrize("vocab", ["v17", "v20"])
def test_prior_error_stays_near_float32_rounding(dev, pattern, vocab):
    """Across seeded draws the device result stays at float32 rounding level
    of the float64 oracle at k = 4: within 2e-6 + 2e-7 * max|x| per row (the
    exponentials take x - max before scaling, so a large row maximum costs
    no precision beyond the rounding of the inputs themselves)."""
    fsa = FsaTensors.build(pattern, TOY_VOCAB if vocab == "v17" else TOY_VOCAB20).densify()
    S, V = fsa.tok_next.shape
    fd = fsa.to(dev)
    g = torch.Generator().manual_seed(23)
    worst = 0.0
    for _ in range(12):
        x = torch.randn(6, V, generator=g) * 3 + 20.0 * torch.rand(1, generator=g)
        st = torch.tensor([min(i, S - 1) for i in range(5)] + [-1], dtype=torch.int32)
        want = OS.prior_lookahead(x.double().numpy(), fsa.tok_next.numpy(), fsa.live.numpy(),
                                  fsa.accept.numpy(), fsa.eos_id, st.numpy(), 4, 1.0)
        got = x.to(dev)
        ops.apply_soft_prior_(got, fd, st.to(dev), 4, 1.0)
        got = got.cpu().double().numpy()
        assert np.array_equal(np.isneginf(got), np.isneginf(want))
        tol = 2e-6 + 2e-7 * x.abs().amax(dim=1, keepdim=True).double().numpy()
        fin = np.isfinite(want)
        err = np.zeros_like(want)
        err[fin] = np.abs(got[fin] - want[fin])
        worst = max(worst, float((err / tol).max()))
    assert worst <= 1.0, worst

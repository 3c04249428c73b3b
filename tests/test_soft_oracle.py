"""Pins the soft-lookahead oracle (oracle/soft.py) before anything is checked
against it.

* The reference's own known answers (test_soft.py:30-96) on its 12-token
  vocabulary: lookahead -inf exactly where the hard mask is, alpha = 0 is hard
  masking, more open continuations score higher, dead ends are -inf, the bias
  is scaled by alpha, k = 1 is flat.
* Brute-force path sums: Z_j(s) enumerated as explicit token sequences (every
  sequence of exactly j tokens whose walk stays live, plus every shorter one
  that ends in an accepting state and is then closed by EOS), uniformly
  weighted or weighted by the row prior, compared with the recurrences.
* Closed forms of the prior variant: with uniform logits and k = 2 it is the
  uniform table shifted by -log V; with k = 1 and alpha = 0 it is
  log_softmax under the hard mask.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
from oracle import dense as OD
from oracle import soft as OS
from tests._util import reachable

# test_soft.py:15-17
VOCAB = Vocabulary.from_tokens(
    ["a", "b", "c", "ab", "ba", "0", "1", "12", "-", ".", "ge", "<eos>"], eos_id=11
)
PATTERNS = ["[01]+", "a+b*", "(ab)+", "-?[0-9]+(\\.[0-9]+)?", "a[012]+|b0", "age"]


def tables(pattern: str):
    fsa = FsaTensors.build(pattern, VOCAB).densify()
    return fsa, fsa.tok_next.numpy(), fsa.live.numpy().astype(bool), fsa.accept.numpy().astype(bool)


def tok(text: str) -> int:
    return VOCAB.token_bytes.index(text.encode())


def hard_mask(tn: np.ndarray, states) -> np.ndarray:
    """0 where allowed, -inf where not, from the dense oracle's mask."""
    z = torch.zeros(len(states), tn.shape[1], dtype=torch.float32)
    return OD.apply_mask(z, tn, np.asarray(states), float("-inf")).numpy().astype(np.float64)


# ------------------------------------------------ reference known answers --
@pytest.mark.parametrize("pattern", PATTERNS[:4])
def test_lookahead_masks_exactly_like_hard_mask(pattern):
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start)
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 3)[states]
    assert np.array_equal(np.isneginf(la), np.isneginf(hard_mask(tn, states)))


@pytest.mark.parametrize("pattern", PATTERNS[:3])
def test_alpha_zero_is_hard_masking(pattern):
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start)
    base = np.random.default_rng(0).standard_normal((len(states), VOCAB.size)).astype(np.float32)
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 3)
    soft0 = OS.apply_soft(base, la, states, 0.0)
    hard = OD.apply_mask(torch.from_numpy(base.copy()), tn, np.asarray(states), float("-inf"))
    assert np.array_equal(soft0, hard.numpy().astype(np.float64))


def test_more_open_continuations_score_higher():
    fsa, tn, live, acc = tables("a[012]+|b0")
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 3)[fsa.start]
    a, b = la[tok("a")], la[tok("b")]
    assert math.isfinite(a) and math.isfinite(b) and a > b


def test_dead_end_token_becomes_neg_inf():
    fsa, tn, live, acc = tables("age")
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 3)[fsa.start]
    assert not np.isneginf(la[tok("a")])
    assert np.isneginf(la[tok("b")])


def test_apply_soft_adds_scaled_bias():
    fsa, tn, live, acc = tables("[012]+")
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 3)
    out = OS.apply_soft(np.zeros((1, VOCAB.size)), la, [fsa.start], 2.0)[0]
    fin = np.isfinite(la[fsa.start])
    assert np.allclose(out[fin], 2.0 * la[fsa.start][fin])
    assert np.isneginf(out[~fin]).all()


def test_k1_lookahead_is_flat_over_allowed():
    fsa, tn, live, acc = tables("[01]+")
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, 1)[fsa.start]
    assert np.all(la[np.isfinite(la)] == 0.0)


# ------------------------------------------------ brute-force path sums --
def path_sum(tn, live, acc, eos, s, j, weight) -> float:
    """Z_j(s) as an explicit sum over token sequences: weight(w) summed over
    every w of exactly j tokens whose walk from s visits live states only,
    plus weight(w) * weight((eos,)) over every shorter w whose live walk ends
    in an accepting state."""
    V = tn.shape[1]
    total = 0.0
    for m in range(j + 1):
        for w in itertools.product(range(V), repeat=m):
            cur, ok = s, bool(live[s])
            for t in w:
                cur = int(tn[cur, t])
                if cur < 0 or not live[cur]:
                    ok = False
                    break
            if not ok:
                continue
            if m == j:
                total += weight(w)
            elif acc[cur]:
                total += weight(w) * weight((eos,))
    return total


@pytest.mark.parametrize("pattern", ["[01]+", "a+b*", "a[012]+|b0", "age"])
@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_uniform_lookahead_is_path_count(pattern, k):
    fsa, tn, live, acc = tables(pattern)
    la = OS.build_lookahead(tn, live, acc, fsa.eos_id, k)
    for s in reachable(tn, fsa.start):
        for t in range(VOCAB.size):
            d = int(tn[s, t])
            if t == fsa.eos_id:
                assert la[s, t] == (0.0 if acc[s] else -np.inf)
                continue
            z = 0.0 if d < 0 else path_sum(tn, live, acc, fsa.eos_id, d, k - 1, lambda w: 1.0)
            want = math.log(z) if z > 0 else -np.inf
            assert la[s, t] == pytest.approx(want, rel=1e-12, abs=1e-12)


@pytest.mark.parametrize("pattern", ["[01]+", "a[012]+|b0", "-?[0-9]+(\\.[0-9]+)?"])
@pytest.mark.parametrize("k", [1, 2, 3])
def test_prior_lookahead_is_weighted_path_sum(pattern, k):
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start) + [-1]
    rng = np.random.default_rng(len(pattern) * 10 + k)
    logits = rng.normal(0.0, 3.0, size=(len(states), VOCAB.size))
    alpha = 0.75
    out = OS.prior_lookahead(logits, tn, live, acc, fsa.eos_id, states, k, alpha)
    for b, s in enumerate(states):
        pi = np.exp(logits[b] - logits[b].max())
        pi /= pi.sum()
        weight = lambda w: float(np.prod([pi[t] for t in w]))  # noqa: E731
        for t in range(VOCAB.size):
            lp = math.log(pi[t])
            if s < 0:
                want = -np.inf
            elif t == fsa.eos_id:
                want = lp if acc[s] else -np.inf
            else:
                d = int(tn[s, t])
                z = 0.0 if d < 0 else path_sum(tn, live, acc, fsa.eos_id, d, k - 1, weight)
                want = lp + alpha * math.log(z) if z > 0 else -np.inf
            assert out[b, t] == pytest.approx(want, rel=1e-9, abs=1e-9)


# ------------------------------------------------ prior closed forms --
@pytest.mark.parametrize("pattern", PATTERNS)
def test_prior_with_flat_logits_is_shifted_uniform_k2(pattern):
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start)
    V = VOCAB.size
    uni = OS.build_lookahead(tn, live, acc, fsa.eos_id, 2)[states]
    alpha = 1.5
    out = OS.prior_lookahead(np.zeros((len(states), V)), tn, live, acc, fsa.eos_id, states, 2, alpha)
    logv = math.log(V)
    want = np.where(np.isneginf(uni), -np.inf, -logv + alpha * (uni - logv))
    want[:, fsa.eos_id] = np.where(acc[states], -logv, -np.inf)
    assert np.array_equal(np.isneginf(out), np.isneginf(want))
    fin = np.isfinite(want)
    assert np.allclose(out[fin], want[fin], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pattern", PATTERNS)
def test_prior_k1_alpha0_is_masked_log_softmax(pattern):
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start) + [-1]
    logits = np.random.default_rng(7).normal(0.0, 3.0, size=(len(states), VOCAB.size))
    out = OS.prior_lookahead(logits, tn, live, acc, fsa.eos_id, states, 1, 0.0)
    ls = torch.log_softmax(torch.from_numpy(logits), dim=1).numpy()
    want = ls + hard_mask(tn, states)
    assert np.array_equal(np.isneginf(out), np.isneginf(want))
    fin = np.isfinite(want)
    assert np.allclose(out[fin], want[fin], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pattern", PATTERNS)
@pytest.mark.parametrize("k", [1, 2, 4])
def test_prior_torch_fp32_restatement_matches_float64(pattern, k):
    """The fp32 torch restatement timed as the CPU baseline computes the
    pinned float64 oracle's values to fp32 accuracy, with the same -inf
    pattern (rows at negative states included)."""
    fsa, tn, live, acc = tables(pattern)
    states = reachable(tn, fsa.start) + [-1]
    logits = np.random.default_rng(3 + k).normal(0.0, 3.0, size=(len(states), VOCAB.size))
    want = OS.prior_lookahead(logits, tn, live, acc, fsa.eos_id, states, k, 0.6)
    got = OS.prior_lookahead_torch(logits, tn, live, acc, fsa.eos_id, states, k, 0.6).double().numpy()
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    assert np.allclose(got[fin], want[fin], rtol=2e-6, atol=2e-6)
    part = OS.prior_lookahead_torch(logits, tn, live, acc, fsa.eos_id, states, k, 0.6, rows=[0])
    assert torch.equal(part[0], torch.from_numpy(got[0]).float()) and torch.isneginf(part[1:]).all()

"""Pins the CPU oracle before anything is checked against it.

* PDA restatement (oracle/pda_oracle.c) vs the reference's own pda_cpu.cpp
  compiled from its sources (oracle/_ref), on random trajectories: masks, ok
  flags and raw 266-word config-sets (stale words included).
* The reference's C++ known-answer tests re-expressed: the paren PdaTable of
  test_pda.cpp:20-44 / :55-186 and the "ab" FSA of test_mask.cpp:14-146.
* Dense restatement (oracle/dense.py) vs the reference's scalar step
  (mask_cpu.cpp:167-183 via oracle/_ref), vs ATen's masked_fill_ sequence of
  ops.py:271-276 (the reference's own arithmetic), and vs brute force.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from bpdecode_amd.fsa import fsa_from_dfa, token_symbols
from bpdecode_amd.grammar.device import build_pda_tensors
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.regex import compile_regex
from bpdecode_amd.tokenizer import Vocabulary
from oracle import dense as OD
from oracle import pda as OP
from oracle import ref as R
from tests.golden.cases import GRAMMARS, PATTERNS

need_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built (no reference checkout)")

PVOCAB = Vocabulary.from_tokens(
    ["(", ")", "x", "y", "{", "}", "a", "b", ":", "0", "1", ",", "<eos>", "((", "x)", "", "{a", ":0,", "\"", "[1"],
    eos_id=12,
)


class _G:
    """Hand-built table in the PdaTensors field layout."""

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)


def paren_table():
    # test_pda.cpp:20-44: root ::= "(" root ")" | "x"
    T = lambda xs, dt=torch.int32: torch.tensor(xs, dtype=dt)  # noqa: E731
    return _G(num_states=6, root_start=0, root_accept=4,
              accept=T([0, 0, 0, 0, 1, 0], torch.uint8), live=T([1] * 6, torch.uint8),
              edge_offsets=T([0, 2, 3, 4, 5, 5, 6]), edge_kind=T([0, 0, 1, 2, 1, 1]),
              edge_lo=T([0, 0, 40, 0, 41, 120]), edge_hi=T([0, 0, 40, 0, 41, 120]),
              edge_dst=T([1, 5, 2, 3, 4, 4]), edge_callee=T([-1, -1, -1, 0, -1, -1]),
              vocab_size=4, eos_id=3, tok_offsets=T([0, 1, 2, 3, 3]),
              tok_bytes=T([40, 41, 120], torch.uint8))


def feed(t, cfg, text: str) -> bool:
    return all(OP.advance_byte(t, cfg, b) for b in text.encode())


def complete(t, cfg) -> bool:
    return bool(OP.compute_mask(t, cfg[None])[0, 0] >> 3 & 1)  # eos = token 3


# ---------------------------------------------- PDA known answers (C++ tests)
def test_paren_known_answers():
    t = OP.Table(paren_table())
    c = OP.init(t)
    assert not complete(t, c)                                   # InitIsNotComplete
    x = c.copy(); assert feed(t, x, "x") and complete(t, x)      # AcceptsX
    assert not feed(t, c.copy(), "y")                            # RejectsY
    x = c.copy(); assert feed(t, x, "(") and not complete(t, x)  # RecursesOneLevel
    assert feed(t, x, "x") and not complete(t, x)
    assert feed(t, x, ")") and complete(t, x)
    x = c.copy(); assert feed(t, x, "((x))") and complete(t, x)  # RecursesTwoLevels
    x = c.copy(); assert feed(t, x, "((x)") and not complete(t, x)  # Unbalanced
    bits = int(OP.compute_mask(t, c[None])[0, 0])               # ComputeMaskMatchesTryToken
    assert [bits >> k & 1 for k in range(4)] == [1, 0, 1, 0]
    lg = np.ones((1, 4), np.float32)                            # ApplyMaskMatchesComputeMask
    OP.apply_mask(t, c[None].copy(), lg)
    assert [v == 1.0 for v in lg[0]] == [True, False, True, False]
    cfg = c[None].copy()                                         # AdvanceStateBatch...
    assert OP.advance(t, cfg, [0])[0] == 1 and not complete(t, cfg[0])
    before = cfg.copy()
    assert OP.advance(t, cfg, [1])[0] == 0 and np.array_equal(cfg, before)
    assert OP.advance(t, cfg, [2])[0] == 1
    assert OP.advance(t, cfg, [1])[0] == 1 and complete(t, cfg[0])
    assert OP.advance(t, cfg, [3])[0] == 1


@need_ref
def test_paren_raw_words_match_reference():
    t = OP.Table(paren_table())
    assert np.array_equal(OP.init(t), R.pda_init(t))
    for text in ["(", "((x", "x", "(((((x)))))", "y"]:
        a, b = OP.init(t), R.pda_init(t)
        for ch in text.encode():
            assert OP.advance_byte(t, a, ch) == R.pda_advance_byte(t, b, ch)
            assert np.array_equal(a, b)


# ------------------------------------------------- PDA vs the reference C++
@need_ref
@pytest.mark.parametrize("idx", range(len(GRAMMARS)))
@pytest.mark.parametrize("reduce", [False, True])
def test_pda_oracle_matches_reference(idx, reduce):
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[idx])), PVOCAB, eps_reduce=reduce)
    t = OP.Table(g)
    rng = np.random.default_rng(idx)
    B = 6
    a = np.repeat(OP.init(t)[None], B, 0)
    b = a.copy()
    assert np.array_equal(a[0], R.pda_init(t))
    for _ in range(25):
        ma, mb = OP.compute_mask(t, a), R.pda_compute_mask(t, b)
        assert np.array_equal(ma, mb)
        la = rng.standard_normal((B, t.vocab)).astype(np.float32)
        lb = la.copy()
        OP.apply_mask(t, a, la)
        R.pda_apply_mask(t, b, lb)
        assert np.array_equal(la, lb)
        # mostly allowed tokens, sometimes arbitrary ones (rejections)
        toks = []
        for r in range(B):
            allowed = [k for k in range(t.vocab) if ma[r, k >> 5] >> (k & 31) & 1]
            toks.append(int(rng.choice(allowed)) if allowed and rng.random() < 0.8 else int(rng.integers(t.vocab)))
        assert np.array_equal(OP.advance(t, a, toks), R.pda_advance(t, b, toks))
        assert np.array_equal(a, b)


@need_ref
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_reference_rows_over_threads_match_one_call(threads):
    """The parallel CPU baseline (the reference call over row slices on host
    threads) gives the single call's logits."""
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[-1])), PVOCAB, eps_reduce=True)
    t = OP.Table(g)
    rng = np.random.default_rng(threads)
    cfg = np.repeat(R.pda_init(t)[None], 7, 0)
    for r in range(7):
        for _ in range(r):
            ma = R.pda_compute_mask(t, cfg[r:r + 1])[0]
            allowed = [k for k in range(t.vocab) if ma[k >> 5] >> (k & 31) & 1 and k != t.eos]
            if allowed:
                R.pda_advance(t, cfg[r:r + 1], [int(rng.choice(allowed))])
    x = rng.standard_normal((7, t.vocab)).astype(np.float32)
    one = R.pda_apply_mask(t, cfg.copy(), x.copy())
    par = R.pda_apply_mask_threads(t, cfg.copy(), x.copy(), threads)
    assert np.array_equal(one, par)


# ------------------------------------------------------ dense known answers
def ab_fsa():
    # test_mask.cpp:14-39: "ab" over 2 classes; token 3 has an invalid class
    return dict(trans=[1, 3, 3, 2, 3, 3, 3, 3], accept=[0, 0, 1, 0], live=[1, 1, 1, 0], m=2, dead=3,
                off=[0, 1, 2, 4, 5, 5], sym=[0, 1, 0, 1, 255], eos=4)


def test_ab_fsa_known_answers():
    f = ab_fsa()
    # the oracle table builder treats class ids as table columns; the invalid
    # class of token 3 is modelled as an extra column leading to `dead`
    trans = np.array(f["trans"]).reshape(4, 2)
    trans3 = np.concatenate([trans, np.full((4, 1), 3)], axis=1).reshape(-1)
    sym = [0, 1, 0, 1, 2]
    tn = OD.build_token_transitions(trans3, f["accept"], f["live"], 3, f["off"], sym, f["eos"])
    assert tn[0].tolist() == [1, -1, 2, -1, -1]   # Step.WalksAndRejects, EOS off at start
    assert tn[1, 1] == 2 and tn[2, 4] == 2         # 'b' from s1; EOS at accept
    assert OD.advance(tn, [0, 1, 2], [0, 1, 4]).tolist() == [1, 2, 2]
    assert OD.advance(tn, [0], [1]).tolist() == [-1]
    bits = OD.compute_mask_bits(tn, [0, 2])
    assert bits[0, 0] & 1 and bits[0, 0] >> 2 & 1 and not bits[0, 0] >> 1 & 1 and not bits[0, 0] >> 4 & 1
    assert bits[1, 0] >> 4 & 1
    lg = torch.ones(2, 5)
    OD.apply_mask(lg, tn, [0, 2])
    assert lg[0].tolist() == [1.0, -np.inf, 1.0, -np.inf, -np.inf]
    assert lg[1, 4].item() == 1.0 and lg[1, 0].item() == -np.inf


@need_ref
def test_reference_reachability_and_steps_on_ab():
    f = ab_fsa()
    assert R.fsa_build_reachability(f["trans"], f["accept"], 2).tolist() == [1, 1, 1, 0]
    rf = R.Fsa(f["trans"], f["accept"], f["live"], 2, 3, f["off"], f["sym"], f["eos"])
    assert R.fsa_step_table(rf, [0])[0].tolist() == [1, -1, 2, -1, -1]


VOCAB = Vocabulary.from_tokens(
    ["a", "b", "c", "ab", "ba", "0", "1", "12", "-", ".", "aa", "", "caf", "\xc3", "\xe9", "é", "<eos>"], eos_id=16
)


def _dense_inputs(pattern):
    dfa = compile_regex(pattern)
    fsa = fsa_from_dfa(dfa)
    toks = token_symbols(dfa, VOCAB)
    tn = OD.build_token_transitions(fsa.trans, fsa.accept, fsa.live, fsa.num_symbols, toks.offsets,
                                    list(toks.symbols), toks.eos_id)
    return dfa, fsa, toks, tn


@need_ref
@pytest.mark.parametrize("pattern", PATTERNS)
def test_dense_table_matches_reference_step(pattern):
    dfa, fsa, toks, tn = _dense_inputs(pattern)
    rf = R.Fsa(fsa.trans, fsa.accept, fsa.live, fsa.num_symbols, fsa.dead, toks.offsets,
               list(toks.symbols), toks.eos_id)
    assert np.array_equal(tn, R.fsa_step_table(rf, range(fsa.num_states)))
    assert R.fsa_build_reachability(fsa.trans, fsa.accept, fsa.num_symbols).tolist() == list(fsa.live)
    states = list(range(fsa.num_states))
    logits = np.random.default_rng(0).standard_normal((len(states), VOCAB.size)).astype(np.float32)
    got = torch.from_numpy(logits.copy())
    OD.apply_mask(got, tn, states)
    assert np.array_equal(got.numpy(), R.fsa_apply_mask(rf, states, logits.copy()))
    assert np.array_equal(OD.compute_mask_bits(tn, states), R.fsa_compute_mask(rf, states))


@pytest.mark.parametrize("pattern", PATTERNS[:9])
def test_dense_table_is_brute_force_language_prefix(pattern):
    """tok_next[s, t] >= 0 iff (prefix reaching s) + token t is a prefix of a
    string the pattern accepts (Python's re over every string of length <= 6
    on the pattern's ASCII alphabet); EOS iff the prefix itself is accepted."""
    import re

    dfa, fsa, toks, tn = _dense_inputs(pattern)
    rx = re.compile(pattern)
    alphabet = "abcf012-."
    accepted, prefixes = set(), set()
    for n in range(7):
        for combo in itertools.product(alphabet, repeat=n):
            text = "".join(combo)
            if rx.fullmatch(text):
                accepted.add(text)
                prefixes.update(text[:k] for k in range(n + 1))
    reach = {}
    for n in range(3):
        for combo in itertools.product(alphabet, repeat=n):
            text = "".join(combo)
            st = dfa.start
            for byte in text.encode():
                st = dfa.step(st, byte)
            if st != dfa.dead:
                reach.setdefault(st, text)
    checked = 0
    for st, prefix in reach.items():
        assert (tn[st, VOCAB.eos_id] >= 0) == (prefix in accepted)
        for t in range(VOCAB.size):
            if t == VOCAB.eos_id:
                continue
            tb = VOCAB.token_bytes[t]
            if not tb.isascii():
                assert tn[st, t] == -1
                continue
            cont = prefix + tb.decode()
            if len(cont) <= 3:
                assert (tn[st, t] >= 0) == (cont in prefixes), (pattern, prefix, tb)
                checked += 1
    assert checked > 10


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("neg_inf", [float("-inf"), -1e4, -3.0e38, float("nan")])
def test_dense_oracle_matches_aten_sequence(dtype, neg_inf):
    """oracle.dense == the reference's ATen op sequence (ops.py:271-276)."""
    dfa, fsa, toks, tn = _dense_inputs("-?[0-9]+(\\.[0-9]+)?")
    rng = np.random.default_rng(1)
    states = rng.integers(-2, fsa.num_states, size=40)
    base = torch.from_numpy(rng.standard_normal((40, VOCAB.size)).astype(np.float32)).to(dtype)
    if dtype == torch.float16 and neg_inf == -3.0e38:
        with pytest.raises(RuntimeError):
            OD.apply_mask(base.clone(), tn, states, neg_inf)
        return
    want = base.clone()
    s = torch.from_numpy(states).long()
    rejected = torch.from_numpy(tn).index_select(0, s.clamp(min=0)) == -1
    rejected |= (s < 0).unsqueeze(1)
    want.masked_fill_(rejected, neg_inf)
    got = OD.apply_mask(base.clone(), tn, states, neg_inf)
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))
    toks_ = rng.integers(-VOCAB.size, VOCAB.size, size=40)
    nxt = torch.from_numpy(tn)[s.clamp(min=0), torch.from_numpy(toks_).long()]
    want_adv = torch.where(s < 0, torch.full_like(nxt, -1), nxt).to(torch.int32)
    assert OD.advance(tn, states, toks_).tolist() == want_adv.tolist()


def _random_dfa_table(rng, S, M):
    """Random transition table with absorbing sinks and an unreachable
    accepting cycle, so both live and dead states occur."""
    trans = rng.integers(0, S, size=(S, M)).astype(np.int32)
    accept = (rng.random(S) < 0.15).astype(np.uint8)
    for s in rng.choice(S, size=max(1, S // 5), replace=False):
        trans[s] = s  # absorbing
    return trans.reshape(-1), accept


@need_ref
@pytest.mark.parametrize("S,M,seed", [(1, 1, 0), (4, 2, 1), (37, 3, 2), (300, 7, 3), (2500, 4, 4)])
def test_host_reachability_matches_reference(S, M, seed):
    """The library's host reachability (reverse search) against the
    reference's own build_reachability compiled from mask_cpu.cpp, and the
    Python front-end's, on random tables."""
    from bpdecode_amd import ops
    from bpdecode_amd.fsa import build_reachability

    trans, accept = _random_dfa_table(np.random.default_rng(seed), S, M)
    want = R.fsa_build_reachability(trans, accept, M)
    got = ops.build_reachability(torch.from_numpy(trans), torch.from_numpy(accept), M)
    assert got.numpy().tolist() == want.tolist()
    assert build_reachability(S, M, trans.tolist(), accept.tolist()) == want.tolist()

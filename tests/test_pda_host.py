"""PDA path through the library's host entry points against the C oracle
(raw config words included), and the CFGConstraintBatch / processor
scenarios of the reference's test_pda_device.py and
test_grammar_device_batch.py against the C oracle, with complete strings
checked against an independent recursive matcher of the grammar."""

from __future__ import annotations

import itertools
import random

import numpy as np
import pytest
import torch

from bpdecode_amd import synth
from bpdecode_amd.grammar.device import (
    PDA_CONFIG_FLAT, CFGConstraintBatch, build_pda_tensors, pda_advance_state, pda_apply_mask_,
    _walk_order, pda_compute_mask, pda_mask_, pda_step,
)
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.hf import GrammarLogitsProcessor
from oracle import pda as OP
from tests._util import PDA_VOCAB as VOCAB
from tests._util import member
from tests.golden.cases import GRAMMARS


def tables(src, reduce):
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(src)), VOCAB, eps_reduce=reduce)
    return g, OP.Table(g)


@pytest.mark.parametrize("idx", range(len(GRAMMARS)))
@pytest.mark.parametrize("reduce", [False, True])
def test_host_matches_oracle_trajectories(idx, reduce):
    g, t = tables(GRAMMARS[idx], reduce)
    assert np.array_equal(g.init_config().numpy(), OP.init(t))
    rng = np.random.default_rng(idx + 10 * reduce)
    B, cap = 5, 8
    pool = g.init_batch(cap)
    broken = torch.zeros(cap, dtype=torch.bool)
    mirror = pool.numpy().copy()
    mirror_broken = np.zeros(cap, dtype=bool)
    for _ in range(20):
        slots = torch.from_numpy(rng.choice(cap, size=B, replace=False))
        sub = mirror[slots.numpy()]
        bits = pda_compute_mask(g, pool, slots).numpy().view(np.uint32)
        assert np.array_equal(bits, OP.compute_mask(t, sub))
        for dtype in (torch.float32, torch.bfloat16):
            lg = torch.randn(B, VOCAB.size).to(dtype)
            want = lg.float().numpy().copy()
            OP.apply_mask(t, sub, want)
            pda_mask_(lg, g, pool, slots, broken)
            dead = mirror_broken[slots.numpy()]
            want[dead] = -np.inf
            assert np.array_equal(torch.isneginf(lg).numpy(), np.isneginf(want))
        toks = []
        for r in range(B):
            allowed = [k for k in range(VOCAB.size) if bits[r, k >> 5] >> (k & 31) & 1]
            toks.append(int(rng.choice(allowed)) if allowed and rng.random() < 0.85
                        else int(rng.integers(VOCAB.size)))
        ok, status = pda_step(pool, g, torch.tensor(toks, dtype=torch.int32), slots, broken)
        sub_after = sub.copy()
        ok_o = OP.advance(t, sub_after, toks)
        mirror[slots.numpy()] = sub_after
        mirror_broken[slots.numpy()] |= ok_o == 0
        assert ok.numpy().tolist() == ok_o.tolist()
        assert status.tolist() == [-1 if mirror_broken[s] else 1 for s in slots.tolist()]
        assert np.array_equal(pool.numpy(), mirror)


def test_json_prefixes_match_oracle():
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    vocab = synth.serving_vocab(3000, seed=5)
    g = build_pda_tensors(comp, vocab, eps_reduce=True)
    t = OP.Table(g)
    rng = np.random.default_rng(7)
    rows = []
    for _ in range(6):
        c = g.init_config()
        assert g.feed(c, synth.json_prefix(rng, int(rng.integers(0, 9))))
        rows.append(c)
    cfgs = torch.stack(rows)
    assert np.array_equal(pda_compute_mask(g, cfgs).numpy().view(np.uint32), OP.compute_mask(t, cfgs.numpy()))


def test_feed_matches_oracle_bytes():
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, VOCAB, eps_reduce=True)
    t = OP.Table(g)
    rng = np.random.default_rng(11)
    for _ in range(20):
        data = synth.json_prefix(rng, int(rng.integers(0, 9)))
        c = g.init_config()
        o = OP.init(t)
        ok_o = all(OP.advance_byte(t, o, b) for b in data)
        assert g.feed(c, data) == ok_o
        if ok_o:
            assert np.array_equal(c.numpy(), o)


# ---------------------------------------------- reference scenarios -----
REF_GRAMMARS = GRAMMARS[:3]


def _allowed_ops(g, cfg):
    logits = torch.zeros(1, VOCAB.size)
    pda_apply_mask_(logits, g, cfg)
    return {i for i in range(VOCAB.size) if logits[0, i].item() == 0.0}


def _allowed_oracle(t, cfg: np.ndarray) -> set[int]:
    bits = OP.compute_mask(t, cfg.reshape(1, -1))[0]
    return {k for k in range(VOCAB.size) if bits[k >> 5] >> (k & 31) & 1}


def _text(toks) -> str:
    return b"".join(VOCAB.token_bytes[k] for k in toks).decode("latin-1")


@pytest.mark.parametrize("src", REF_GRAMMARS)
def test_random_walk_matches_oracle(src):
    """test_pda_device.py:62-87: a random walk through allowed tokens, the
    operators' allowed set equal to the C oracle's at every step and EOS
    allowed exactly when the text so far is in the language."""
    grammar = parse_gbnf(src)
    g = build_pda_tensors(CompiledGrammar.build(grammar), VOCAB)
    t = OP.Table(g)
    cfg = g.init_batch(1)
    mirror = OP.init(t).reshape(1, -1).copy()
    rng = random.Random(0)
    walked = []
    for _ in range(15):
        want = _allowed_oracle(t, mirror)
        assert _allowed_ops(g, cfg) == want
        assert (VOCAB.eos_id in want) == member(grammar, _text(walked))
        choices = sorted(want - {VOCAB.eos_id})
        if not choices:
            break
        tok = rng.choice(choices)
        assert bool(pda_advance_state(cfg, g, torch.tensor([tok], dtype=torch.int32)).item())
        assert OP.advance(t, mirror, [tok]).all()
        assert np.array_equal(cfg.numpy(), mirror)
        walked.append(tok)


@pytest.mark.parametrize("src", REF_GRAMMARS)
def test_exhaustive_short_strings_agree(src):
    """test_pda_device.py:90-120: every token string up to length 3 -- the
    operators' ok flags and config words equal the C oracle's, and a
    string they accept whole is complete exactly when the matcher says it is
    in the language."""
    grammar = parse_gbnf(src)
    g = build_pda_tensors(CompiledGrammar.build(grammar), VOCAB)
    t = OP.Table(g)
    alphabet = [i for i in range(13) if i != VOCAB.eos_id]
    tested = 0
    for n in range(4):
        for combo in itertools.product(alphabet, repeat=n):
            cfg = g.init_batch(1)
            mirror = OP.init(t).reshape(1, -1).copy()
            dead = False
            for tok in combo:
                ok_dev = bool(pda_advance_state(cfg, g, torch.tensor([tok], dtype=torch.int32)).item())
                ok_ref = bool(OP.advance(t, mirror, [tok])[0])
                assert ok_ref == ok_dev, (src, combo)
                assert np.array_equal(cfg.numpy(), mirror)
                if not ok_ref:
                    dead = True
                    break
            if not dead:
                assert member(grammar, _text(combo)) == (VOCAB.eos_id in _allowed_ops(g, cfg))
                tested += 1
    assert tested > 0


def test_reject_leaves_config_unchanged_and_flat_size():
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf('root ::= "x" | "y"')), VOCAB)
    cfg = g.init_batch(1)
    before = cfg.clone()
    assert not bool(pda_advance_state(cfg, g, torch.tensor([VOCAB.token_bytes.index(b"(")],
                                                              dtype=torch.int32)).item())
    assert torch.equal(cfg, before)
    assert g.init_config().shape == (PDA_CONFIG_FLAT,)
    with pytest.raises(IndexError):
        pda_advance_state(cfg, g, torch.tensor([VOCAB.size], dtype=torch.int32))


@pytest.mark.parametrize("src", REF_GRAMMARS[:2])
def test_batch_matches_oracle_random_walk(src):
    """test_grammar_device_batch.py:34-80: CFGConstraintBatch on CPU
    tensors, rows walking independently, against the C oracle per row."""
    grammar = parse_gbnf(src)
    g = build_pda_tensors(CompiledGrammar.build(grammar), VOCAB)
    t = OP.Table(g)
    n = 3
    batch = CFGConstraintBatch(g, capacity=n)
    mirror = np.repeat(OP.init(t)[None], n, axis=0)
    texts = [[] for _ in range(n)]
    for i in range(n):
        batch.add(i)
    rng = random.Random(0)
    for _ in range(12):
        logits = torch.zeros(n, VOCAB.size)
        batch.apply_mask(list(range(n)), logits)
        allowed = [_allowed_oracle(t, mirror[i]) for i in range(n)]
        for i in range(n):
            got = {k for k in range(VOCAB.size) if logits[i, k].item() == 0.0}
            assert got == allowed[i]
            assert batch.is_complete(i) == member(grammar, _text(texts[i]))
        toks = [rng.choice(sorted(allowed[i] - {VOCAB.eos_id}) or [VOCAB.eos_id]) for i in range(n)]
        batch.commit(list(range(n)), torch.tensor(toks, dtype=torch.int32))
        assert OP.advance(t, mirror, toks).all()
        for i in range(n):
            if toks[i] != VOCAB.eos_id:
                texts[i].append(toks[i])


def test_batch_lifecycle_and_broken_rows():
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf('root ::= "x"')), VOCAB)
    batch = CFGConstraintBatch(g, capacity=2)
    batch.add("a")
    batch.add("b")
    with pytest.raises(RuntimeError):
        batch.add("c")
    batch.evict("a")
    assert batch.add("c") in (0, 1)
    status = batch.commit(["c"], torch.tensor([VOCAB.token_bytes.index(b"y")], dtype=torch.int32))
    assert status.tolist() == [-1] and batch.is_broken("c")
    logits = torch.zeros(1, VOCAB.size)
    batch.apply_mask(["c"], logits)
    assert torch.isneginf(logits).all() and not batch.is_complete("c")
    batch.reset("c")
    logits = torch.zeros(1, VOCAB.size)
    batch.apply_mask(["c"], logits)
    assert logits[0, VOCAB.token_bytes.index(b"x")].item() == 0.0


def test_logits_processor_device_backend_matches_cpu_backend():
    """test_grammar_hf.py: both backends in generate()'s calling convention
    (bf16 and fp32 scores) against the C oracle, row by row."""
    src = 'root ::= "(" root ")" | "x" | "y"'
    lp_cpu = GrammarLogitsProcessor(src, VOCAB, backend="cpu")
    lp_dev = GrammarLogitsProcessor(src, VOCAB, device="cpu", backend="device")
    assert lp_cpu.backend == "cpu" and lp_dev.backend == "device"
    t = OP.Table(build_pda_tensors(CompiledGrammar.build(parse_gbnf(src)), VOCAB))
    mirror = np.repeat(OP.init(t)[None], 2, axis=0)
    input_ids = torch.zeros(2, 1, dtype=torch.long)
    rng = random.Random(1)
    for step in range(8):
        s_cpu = torch.zeros(2, VOCAB.size)
        s_dev = torch.zeros(2, VOCAB.size, dtype=torch.bfloat16)
        lp_cpu(input_ids, s_cpu)
        lp_dev(input_ids, s_dev)
        want = np.zeros((2, VOCAB.size), np.float32)
        OP.apply_mask(t, mirror, want)
        assert torch.equal(torch.isneginf(s_cpu), torch.from_numpy(np.isneginf(want)))
        assert torch.equal(torch.isneginf(s_cpu), torch.isneginf(s_dev))
        assert lp_cpu.is_complete(0) == lp_dev.is_complete(0)
        toks = [rng.choice((~torch.isneginf(s_cpu[r])).nonzero().flatten().tolist()) for r in range(2)]
        assert OP.advance(t, mirror, toks).all()
        input_ids = torch.cat([input_ids, torch.tensor(toks).unsqueeze(1)], dim=1)


def test_memo_walk_order_is_a_permutation_by_length_then_bytes():
    # tokens of every length class, duplicates, an empty token and tokens
    # longer than the 16 bytes the order looks at
    rng = random.Random(3)
    toks = [b"", b"b", b"a", b"ab", b"ab", b"aa", b"x" * 20 + b"b", b"x" * 20 + b"a"]
    toks += [bytes(rng.choice(b"ab\"[]{}") for _ in range(rng.randint(1, 24))) for _ in range(300)]
    off = torch.tensor([0] + list(itertools.accumulate(len(t) for t in toks)), dtype=torch.int32)
    tb = torch.tensor(list(b"".join(toks)), dtype=torch.uint8)
    order = _walk_order(off, tb, len(toks))
    assert order.dtype == torch.int32
    o = order.tolist()
    assert sorted(o) == list(range(len(toks)))
    keys = [(len(toks[t]), toks[t][:16]) for t in o]
    assert keys == sorted(keys)
    # an empty byte table (every token empty) still orders every id
    z = _walk_order(torch.zeros(4, dtype=torch.int32), torch.zeros(1, dtype=torch.uint8), 3)
    assert sorted(z.tolist()) == [0, 1, 2]

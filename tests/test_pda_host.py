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


def test_memo_walk_order_is_a_permutation_by_first_byte_length_then_bytes():
    # tokens of every length class, duplicates, empty tokens, an EOS token
    # with bytes, and tokens longer than the 16 bytes the order looks at
    rng = random.Random(3)
    toks = [b"", b"b", b"a", b"ab", b"ab", b"aa", b"x" * 20 + b"b", b"x" * 20 + b"a", b"</s>", b""]
    toks += [bytes(rng.choice(b"ab\"[]{}") for _ in range(rng.randint(1, 24))) for _ in range(300)]
    eos = 8
    off = torch.tensor([0] + list(itertools.accumulate(len(t) for t in toks)), dtype=torch.int32)
    tb = torch.tensor(list(b"".join(toks)), dtype=torch.uint8)
    order, runs = _walk_order(off, tb, len(toks), eos)
    assert order.dtype == torch.int32 and runs.dtype == torch.int32 and runs.numel() == 257
    o = order.tolist()
    assert sorted(o) == list(range(len(toks)))

    def group(t):
        return 256 if (t == eos or not toks[t]) else toks[t][0]

    keys = [(group(t), len(toks[t]), toks[t][1:16]) for t in o]
    assert keys == sorted(keys)
    # the runs: positions [runs[c], runs[c + 1]) hold exactly the tokens of
    # first byte c, [runs[256], V) the EOS token and the empty ones
    r = runs.tolist() + [len(toks)]
    for c in range(257):
        assert all(group(o[k]) == c for k in range(r[c], r[c + 1]))
    assert r == sorted(r)
    assert {o[k] for k in range(r[256], len(toks))} == {0, 8, 9}
    # an empty byte table (every token empty) still orders every id
    z, zr = _walk_order(torch.zeros(4, dtype=torch.int32), torch.zeros(1, dtype=torch.uint8), 3, -1)
    assert sorted(z.tolist()) == [0, 1, 2]
    assert zr.tolist() == [0] * 257


def test_token_pack_tag_follows_the_table_contents():
    """The tag under which the device mask keeps its packed token records:
    equal for equal tables, different when a byte, a boundary or the walk
    order changes, never 0."""
    from bpdecode_amd.grammar.device import _pack_tag

    off = torch.tensor([0, 1, 3, 3, 6], dtype=torch.int32)
    tb = torch.tensor(list(b"abcdef"), dtype=torch.uint8)
    order = torch.tensor([3, 0, 1, 2], dtype=torch.int32)
    tag = _pack_tag(off, tb, order, 4)
    assert tag != 0 and tag == _pack_tag(off.clone(), tb.clone(), order.clone(), 4)
    others = [
        _pack_tag(off, torch.tensor(list(b"abcdeg"), dtype=torch.uint8), order, 4),
        _pack_tag(torch.tensor([0, 2, 3, 3, 6], dtype=torch.int32), tb, order, 4),
        _pack_tag(off, tb, torch.tensor([3, 0, 2, 1], dtype=torch.int32), 4),
    ]
    assert len({tag, *others}) == 4


def _compose(key: np.ndarray, stack: np.ndarray, sat: int) -> np.ndarray:
    """The flat config-set of a frame list's key over a common stack."""
    from bpdecode_amd.grammar.frames import MAX_SUFFIX

    cfg = np.zeros(266, dtype=np.int32)
    n = int(key[0])
    cfg[0], cfg[1] = n, sat
    base = stack.size
    for i in range(n):
        ln = int(key[1 + i])
        cfg[2 + i] = base + ln
        row = cfg[10 + i * 32:10 + (i + 1) * 32]
        row[:base] = stack
        row[base:base + ln] = key[9 + i * MAX_SUFFIX:9 + i * MAX_SUFFIX + ln]
    return cfg


def _meaningful(cfg: np.ndarray) -> list:
    n = int(cfg[0])
    return [n, int(cfg[1])] + [tuple(cfg[10 + i * 32:10 + i * 32 + int(cfg[2 + i])]) for i in range(n)]


def _check_list(t, fl, order_np, cfg, l, base, vsize, what):
    fl = fl.host()
    """A set over list l at common-stack depth `base`: every token outside the
    list's seeds gets the oracle's verdict from the bitmap, and the oracle's
    step by each byte reaches the coded list over the same stack (saturation
    flag included) or empties the set."""
    want = np.unpackbits(OP.compute_mask(t, cfg[None].copy())[0].view(np.uint8), bitorder="little")
    have = np.unpackbits(fl["allowed"][l].view(np.uint8), bitorder="little")
    seeded = np.zeros(want.size, dtype=bool)
    seeded[order_np[fl["seeds"][fl["seed_off"][l]:fl["seed_off"][l + 1]]]] = True
    V = vsize
    assert not (have[:V].astype(bool) & seeded[:V]).any(), what
    off = ~seeded[:V]
    assert np.array_equal(have[:V][off], want[:V][off]), what
    assert not have[V:].any()
    stack = cfg[10:10 + base].copy()
    for byte in range(256):
        code = int(fl["trans"][l, byte])
        nxt = cfg.copy()
        ok = OP.advance_byte(t, nxt, byte)
        if code == -1:
            assert not ok, (what, byte)
        elif code >= 0:
            assert ok, (what, byte)
            sat = int(cfg[1]) | (1 if code & 0x10000 else 0)
            exp = _compose(fl["keys"][code & 0xFFFF], stack, sat)
            assert _meaningful(nxt) == _meaningful(exp), (what, byte)
            # the raw flag: the oracle's stepped set is the composed one in
            # every word exactly when the step's compaction dropped no config
            # (a dropped config leaves its depth word past the last)
            assert bool(code & 0x20000) == np.array_equal(nxt, exp), (what, byte)


def test_frame_lists_against_the_oracle():
    """Stack-relative frame lists against the C oracle: rows of real prefixes
    (string bodies, escapes, UTF-8 sequences, numbers, nested values) that
    the matcher finds, and every list composed over an empty and over a
    3-frame common stack: the bitmap gives the oracle's verdict of every
    token outside the seeds and the byte table the oracle's step."""
    from bpdecode_amd.grammar.frames import MAX_LISTS, frame_match, frame_lists
    from bpdecode_amd.tokenizer import Vocabulary

    base_v = synth.serving_vocab(6000, seed=4)
    extra = [b"\"", b"\\", b"\\n", b"\\\"", b"\xc3", b"\xa9", b"\xe2\x82", b"\xac\"", b"\xe9", b"ab\"",
             b"\" :", b"\\u", b"\x01", b"\x7f", b"", b"-1", b"12", b"\"}", b"\xc3\xa9x", b"[{", b"[[",
             b"{\"", b"\":[", b"],", b"},{"]
    vocab = Vocabulary.from_tokens(list(base_v.token_bytes[:-1]) + extra + [b"</s>"],
                                   eos_id=len(base_v.token_bytes) - 1 + len(extra))
    small = r"""
root   ::= string | "[" number "]"
string ::= "\"" ( [^"\\\x00-\x1F] | "\\" ["\\/bfnrt] )* "\""
number ::= "-"? [0-9]+ ( "." [0-9]+ )?
"""
    rng = np.random.default_rng(17)
    json_prefixes = [b"[\"ab", b"{\"k", b"[\"x\\", b"[\"\xc3", b"[\"\xe2\x82", b"{\"a\":[\"", b"[-",
                     b"{\"a\":-", b"[\"a\\u00", b"[[[\"deep", b"\"", b"[\"\\\\", b"{\"a\":\"b\",\"c", b"[",
                     b"[[", b"{\"a\":", b"{\"a\":[", b"[1,", b"{\"a\":{\"b\":["]
    json_prefixes += [synth.json_prefix(rng, int(rng.integers(0, 9))) for _ in range(80)]
    small_prefixes = [b"\"", b"\"ab", b"\"a\\", b"\"\xc3", b"\"\xe2\x82", b"\"x\\\\y", b"[-", b"[",
                      b"\"\xf0\x9f", b"\"\xf0\x9f\x98", b"\"a b c", b"\"\\n", b"\"\xed\x9f"]
    # the recursive JSON grammar saturates the 8 configs without the
    # epsilon reduction, so unreduced tables are covered by a small grammar
    for src, reduce, prefixes, need in ((synth.JSON_GBNF, True, json_prefixes, 60),
                                        (small, False, small_prefixes, 8),
                                        (small, True, small_prefixes, 8)):
        g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(src)), vocab, eps_reduce=reduce)
        t = OP.Table(g)
        order, _ = _walk_order(g.tok_offsets, g.tok_bytes, g.vocab_size, g.eos_id)
        order_np = order.numpy()
        fl = frame_lists(g, order_np)
        assert fl is not None and 0 < fl.num_lists <= MAX_LISTS
        hits = 0
        for p in prefixes:
            c = g.init_config()
            if not g.feed(c, p):
                continue
            cfg = c.numpy()
            l, base = frame_match(cfg, fl)
            if l < 0:
                continue
            hits += 1
            _check_list(t, fl, order_np, cfg, l, base, vocab.size, p)
        for l in range(fl.num_lists):
            for stack in (np.zeros(0, np.int32), np.array([0, 1, 2], np.int32) % g.num_states):
                cfg = _compose(fl.host()["keys"][l], stack, 0)
                assert frame_match(cfg, fl)[0] >= 0, l
                _check_list(t, fl, order_np, cfg, l, stack.size, vocab.size, (l, stack.size))
        assert hits >= need, (src[:20], reduce, hits)


def test_frame_lists_reject_bad_tables():
    """The enumeration's argument checks come back as errors (a negative
    count from the C ABI), never as a list count."""
    import dataclasses

    from bpdecode_amd import _lib
    from bpdecode_amd.grammar.frames import SLOTS, KEY_WORDS, frame_lists

    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[0])), VOCAB)
    order, _ = _walk_order(g.tok_offsets, g.tok_bytes, g.vocab_size, g.eos_id)
    assert frame_lists(g, order.numpy()) is not None
    dst = g.edge_dst.clone()
    dst[0] = g.num_states
    bad = dataclasses.replace(g, edge_dst=dst, _c={})
    with pytest.raises(RuntimeError, match="out of range"):
        frame_lists(bad, order.numpy())
    # the library's own check, past the Python validation
    bad._validate = lambda: None
    keys = np.zeros((4, KEY_WORDS), np.int32)
    trans = np.zeros((4, 256), np.int32)
    slots = np.zeros(SLOTS, np.uint32)
    ptr = lambda a: a.ctypes.data_as(_lib.C.c_void_p)  # noqa: E731
    lib = _lib.lib()
    assert lib.bpd_host_frame_lists(_lib.C.byref(bad.c_table()), 4, ptr(keys), ptr(trans),
                                    ptr(slots)) == -_lib.ERR_INVALID
    assert b"destination out of range" in lib.bpd_last_error()
    assert lib.bpd_host_frame_lists(None, 4, ptr(keys), ptr(trans), ptr(slots)) == -_lib.ERR_INVALID
    assert lib.bpd_host_frame_lists(_lib.C.byref(g.c_table()), 4, ptr(keys), ptr(trans), ptr(slots)) > 0


def test_feed_rejects_a_malformed_config_set():
    """bpd_pda_feed's argument checks come back as errors (negative codes),
    not as its 'every byte kept' result."""
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[0])), VOCAB)
    c = g.init_config()
    assert g.feed(c, b"((x")
    bad = c.clone()
    bad[0] = 99  # more configs than a set holds
    with pytest.raises(RuntimeError, match="malformed"):
        g.feed(bad, b"x")
    assert not g.feed(c, b"]")

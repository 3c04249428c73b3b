"""PDA step on the device (HIP kernels through the C ABI) against the C
oracle: masks, ok flags, status and raw 266-word config-sets, on the
reference's toy grammars (saturating flattening included) and on the
recursive JSON grammar at V = 151,936."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from bpdecode_amd import synth
from bpdecode_amd.grammar.device import (
    CFGConstraintBatch, build_pda_tensors, pda_compute_mask, pda_mask_, pda_step,
)
from bpdecode_amd.grammar.gbnf import parse_gbnf
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.tokenizer import Vocabulary
from oracle import pda as OP
from tests._util import PDA_VOCAB as VOCAB
from tests.golden.cases import GRAMMARS

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("idx", range(len(GRAMMARS)))
@pytest.mark.parametrize("reduce", [False, True])
def test_toy_trajectories_match_oracle(dev, idx, reduce):
    _log(f"case toy grammar {idx} reduce={reduce}")
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[idx])), VOCAB, eps_reduce=reduce)
    t = OP.Table(g)
    gd = g.to(dev)
    rng = np.random.default_rng(idx)
    cap, B = 12, 7
    pool = gd.init_batch(cap)
    broken = torch.zeros(cap, dtype=torch.bool, device=dev)
    mirror = pool.cpu().numpy().copy()
    mbroken = np.zeros(cap, dtype=bool)
    for step in range(20):
        sl = rng.choice(cap, size=B, replace=False)
        slots = torch.from_numpy(sl).to(dev)
        sub = mirror[sl]
        bits = pda_compute_mask(gd, pool, slots).cpu().numpy().view(np.uint32)
        assert np.array_equal(bits, OP.compute_mask(t, sub)), step
        for dtype in (torch.float32, torch.bfloat16, torch.float16):
            lg = torch.randn(B, VOCAB.size).to(dtype)
            want = lg.clone()
            ref = lg.float().numpy().copy()
            OP.apply_mask(t, sub, ref)
            ref[mbroken[sl]] = -np.inf
            want[torch.from_numpy(np.isneginf(ref))] = float("-inf")
            got = lg.to(dev)
            pda_mask_(got, gd, pool, slots, broken)
            assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8)), (step, dtype)
        toks = []
        for r in range(B):
            allowed = [k for k in range(VOCAB.size) if bits[r, k >> 5] >> (k & 31) & 1]
            toks.append(int(rng.choice(allowed)) if allowed and rng.random() < 0.85
                        else int(rng.integers(VOCAB.size)))
        ok, status = pda_step(pool, gd, torch.tensor(toks, dtype=torch.int32, device=dev), slots, broken)
        sub2 = sub.copy()
        ok_o = OP.advance(t, sub2, toks)
        mirror[sl] = sub2
        mbroken[sl] |= ok_o == 0
        assert ok.cpu().tolist() == ok_o.tolist(), step
        assert status.cpu().tolist() == [-1 if mbroken[s] else 1 for s in sl.tolist()]
        assert np.array_equal(pool.cpu().numpy(), mirror), step
        assert np.array_equal(broken.cpu().numpy(), mbroken)


@pytest.fixture(scope="module")
def json_case():
    vocab = synth.serving_vocab(151_936, seed=1)
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, vocab, eps_reduce=True)
    return vocab, g, OP.Table(g)


def _json_configs(g, n, seed):
    rng = np.random.default_rng(seed)
    rows = []
    while len(rows) < n:
        c = g.init_config()
        if g.feed(c, synth.json_prefix(rng, int(rng.integers(0, 9)))):
            rows.append(c)
    return torch.stack(rows)


def _frame_build_equal(g, dev):
    from bpdecode_amd.grammar.device import _walk_order
    from bpdecode_amd.grammar.frames import frame_lists

    order, _ = _walk_order(g.tok_offsets, g.tok_bytes, g.vocab_size, g.eos_id)
    host = frame_lists(g, order)
    on_dev = frame_lists(g.to(dev), order)
    assert (host is None) == (on_dev is None)
    if host is None:
        return 0
    assert on_dev.allowed.device.type == dev.type
    for n in ("keys", "slots", "trans", "allowed", "seed_off", "seeds"):
        assert torch.equal(getattr(host, n), getattr(on_dev, n).cpu()), n
    return host.num_lists


def test_frame_lists_device_build_equals_host(dev, json_case):
    """The frame lists' token classification on the device (count pass,
    prefix sums, fill pass) gives the host classifier's bitmaps, seed
    offsets and seeds word for word: recursive JSON at V=151,936 (as many
    lists as the cap allows), its unreduced tables, and the toy grammars."""
    vocab, g, _ = json_case
    _log("case frame lists json V=151936 reduced")
    from bpdecode_amd.grammar.frames import MAX_LISTS

    assert _frame_build_equal(g, dev) == MAX_LISTS
    _log("case frame lists json V=151936 unreduced")
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    assert _frame_build_equal(build_pda_tensors(comp, vocab, eps_reduce=False), dev) > 0
    for idx, src in enumerate(GRAMMARS):
        _log(f"case frame lists toy grammar {idx}")
        _frame_build_equal(build_pda_tensors(CompiledGrammar.build(parse_gbnf(src)), VOCAB), dev)


def test_json_full_vocab_masks_and_commits(dev, json_case):
    vocab, g, t = json_case
    _log("case json V=151936 B=12 mask+commit 4 steps")
    cfgs = _json_configs(g, 12, seed=3)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    mirror = cfgs.numpy().copy()
    gen = torch.Generator().manual_seed(0)
    for step in range(4):
        bits = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
        want = OP.compute_mask(t, mirror)
        assert np.array_equal(bits, want), step
        lg = synth.logits(12, vocab.size, 3.0, torch.float32, seed=step)
        got = lg.to(dev)
        pda_mask_(got, gd, pool)
        ref = lg.numpy().copy()
        OP.apply_mask(t, mirror, ref)
        assert np.array_equal(got.cpu().numpy(), ref), step
        probs = torch.softmax(torch.from_numpy(ref), dim=-1)
        toks = torch.multinomial(probs, 1, generator=gen).view(-1).to(torch.int32)
        ok, _ = pda_step(pool, gd, toks.to(dev))
        ok_o = OP.advance(t, mirror, toks.numpy())
        assert ok.cpu().tolist() == ok_o.tolist() and ok_o.all()
        assert np.array_equal(pool.cpu().numpy(), mirror), step


def test_json_batch_api_b64(dev, json_case):
    vocab, g, t = json_case
    _log("case json CFGConstraintBatch B=64 2 steps")
    cfgs = _json_configs(g, 64, seed=9)
    batch = CFGConstraintBatch(g, capacity=64, device=dev)
    for i in range(64):
        batch.add(i)
    batch._configs.copy_(cfgs.to(dev))
    mirror = cfgs.numpy().copy()
    ids = list(range(64))
    for step in range(2):
        lg = torch.zeros(64, vocab.size, device=dev)
        batch.apply_mask(ids, lg)
        ref = np.zeros((64, vocab.size), np.float32)
        OP.apply_mask(t, mirror, ref)
        assert np.array_equal(lg.cpu().numpy(), ref), step
        toks = [int(np.nonzero(ref[r] == 0)[0][step % max(1, np.count_nonzero(ref[r] == 0))])
                for r in range(64)]
        status = batch.commit(ids, torch.tensor(toks, device=dev))
        OP.advance(t, mirror, toks)
        assert status.cpu().tolist() == [1] * 64
        assert np.array_equal(batch._configs.cpu().numpy(), mirror)


@pytest.mark.parametrize("mode", ["row", "tile"])
@pytest.mark.parametrize("limit", ["1", "3", "12", "40"])
def test_json_memo_overflow_rows_match_oracle(dev, json_case, monkeypatch, limit, mode):
    """With the interned-set limit lowered, rows run out of sets: a row-wide
    walk that fills the pool starts again tile by tile, a tile that fills it
    restarts from an empty pool, and a row whose tile fills it twice is
    finished by the direct-walk kernel; masks stay identical."""
    vocab, g, t = json_case
    _log(f"case json V=151936 B=8 memo set limit {limit} mode {mode}")
    monkeypatch.setenv("BPD_PDA_MEMO_SETS", limit)
    monkeypatch.setenv("BPD_PDA_MEMO_MODE", mode)
    cfgs = _json_configs(g, 8, seed=21)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    bits = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
    assert np.array_equal(bits, OP.compute_mask(t, cfgs.numpy()))
    lg = synth.logits(8, vocab.size, 3.0, torch.bfloat16, seed=5)
    got = lg.to(dev)
    pda_mask_(got, gd, pool)
    ref = lg.float().numpy().copy()
    OP.apply_mask(t, cfgs.numpy().copy(), ref)
    assert np.array_equal(got.float().cpu().numpy(), ref)


@pytest.mark.parametrize("cap", ["16", "512"])
def test_json_full_queue_rows_match_oracle(dev, json_case, monkeypatch, cap):
    """With the queue buffers lowered to a few entries, rows that pause more
    tokens in one pass start again in tile mode; masks and commits stay the
    oracle's (the workspace is sized for the lowered buffers)."""
    vocab, g, t = json_case
    _log(f"case json V=151936 B=8 queue cap {cap}")
    monkeypatch.setenv("BPD_PDA_QUEUE_CAP", cap)
    cfgs = _json_configs(g, 8, seed=23)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    lg = synth.logits(8, vocab.size, 3.0, torch.float32, seed=6)
    got = lg.to(dev)
    pda_mask_(got, gd, pool)
    ref = lg.numpy().copy()
    OP.apply_mask(t, cfgs.numpy().copy(), ref)
    assert np.array_equal(got.cpu().numpy(), ref)
    cb = CFGConstraintBatch(gd, capacity=8, device=dev)
    for i in range(8):
        cb.add(i)
    cb._configs.copy_(pool)
    x = synth.logits(8, vocab.size, 3.0, torch.float32, seed=7).to(dev)
    cb.apply_mask(list(range(8)), x)
    toks = torch.argmax(x, dim=1).to(torch.int32)
    cb.commit(list(range(8)), toks)
    want = cfgs.numpy().copy()
    ok = OP.advance(t, want, toks.cpu().numpy())
    assert ok.all()
    assert np.array_equal(cb._configs.cpu().numpy(), want)


@pytest.mark.parametrize("cap", ["1", "3"])
def test_json_full_boundary_table_rows_match_oracle(dev, json_case, monkeypatch, cap):
    """With the boundary table lowered to one or three entries, rows whose
    list states meet more boundary bytes start again in tile mode; masks and
    the commits that read the kept tables stay the oracle's."""
    vocab, g, t = json_case
    _log(f"case json V=151936 B=16 boundary-table cap {cap}")
    monkeypatch.setenv("BPD_PDA_LT_CAP", cap)
    cfgs = _json_configs(g, 16, seed=29)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    bits = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
    assert np.array_equal(bits, OP.compute_mask(t, cfgs.numpy()))
    cb = CFGConstraintBatch(gd, capacity=16, device=dev)
    for i in range(16):
        cb.add(i)
    cb._configs.copy_(pool)
    x = synth.logits(16, vocab.size, 3.0, torch.float32, seed=8).to(dev)
    cb.apply_mask(list(range(16)), x)
    ref = synth.logits(16, vocab.size, 3.0, torch.float32, seed=8).numpy().copy()
    OP.apply_mask(t, cfgs.numpy().copy(), ref)
    assert np.array_equal(x.cpu().numpy(), ref)
    toks = torch.argmax(x, dim=1).to(torch.int32)
    cb.commit(list(range(16)), toks)
    want = cfgs.numpy().copy()
    ok = OP.advance(t, want, toks.cpu().numpy())
    assert ok.all()
    assert np.array_equal(cb._configs.cpu().numpy(), want)


def test_json_row_walk_equals_tile_walk(dev, json_case, monkeypatch):
    """The row-wide walk (default) and the tile-by-tile walk of the memoised
    kernel give the oracle's bits on 48 rows (string, number, after-value and
    nested contexts)."""
    vocab, g, t = json_case
    _log("case json V=151936 B=48 row vs tile walk")
    cfgs = _json_configs(g, 48, seed=61)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    want = OP.compute_mask(t, cfgs.numpy())
    monkeypatch.setenv("BPD_PDA_MEMO_MODE", "row")
    row = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
    monkeypatch.setenv("BPD_PDA_MEMO_MODE", "tile")
    tile = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
    assert np.array_equal(row, want)
    assert np.array_equal(tile, want)


def test_json_long_token_rows(dev, monkeypatch):
    """A token of 70,000 spaces (too long for the row walk's queue entries)
    sends the rows it pauses in to the tile walk; every row still matches the
    oracle, in both modes."""
    raw = [bytes([i]) for i in range(256)] + [b" " * 70_000, b" \"\"", b"1, ", b"</s>"]
    vocab = Vocabulary.from_tokens(raw, eos_id=len(raw) - 1)
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, vocab, eps_reduce=True)
    t = OP.Table(g)
    cfgs = _json_configs(g, 24, seed=71)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    want = OP.compute_mask(t, cfgs.numpy())
    for mode in ("row", "tile"):
        _log(f"case json long token mode {mode}")
        monkeypatch.setenv("BPD_PDA_MEMO_MODE", mode)
        got = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want), mode


def _masks_with_order(gd, pool, order):
    """Packed masks of the memoised kernel with the token walk order given
    explicitly (None: token id order)."""
    from bpdecode_amd._lib import TokenBytesC, check, lib, ptr

    B = pool.shape[0]
    V = gd.vocab_size
    need = int(lib().bpd_pda_workspace_bytes(B, V))
    ws = torch.empty(need, dtype=torch.uint8, device=pool.device)
    out = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=pool.device)
    o = None if order is None else order.to(torch.int32).to(pool.device)
    toks = TokenBytesC(V, gd.eos_id, ptr(gd.tok_offsets), ptr(gd.tok_bytes), ptr(o) if o is not None else None)
    stream = torch.cuda.current_stream(pool.device).cuda_stream
    check(lib().bpd_pda_compute_mask(gd.c_table(), toks, ptr(pool), None, B, ptr(out), ptr(ws), need, stream))
    return out.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("which", ["full", "small"])
def test_json_walk_orders_give_the_same_masks(dev, json_case, which):
    """Any permutation of the walk order gives the oracle's masks: the default
    order (by length, then bytes), token id order, a random permutation and
    the default reversed; the small vocabulary has empty tokens and the EOS
    token in the middle of the id range."""
    if which == "full":
        vocab, g, t = json_case
        cfgs = _json_configs(g, 32, seed=83)
    else:
        raw = [bytes([i]) for i in range(256)] + [b"", b"\"a", b"</s>", b"", b"1, ", b"[{\"", b"true]"]
        vocab = Vocabulary.from_tokens(raw, eos_id=258)
        g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF)), vocab, eps_reduce=True)
        t = OP.Table(g)
        cfgs = _json_configs(g, 32, seed=84)
    _log(f"case json walk orders {which} V={vocab.size} B=32")
    gd = g.to(dev)
    pool = cfgs.to(dev)
    want = OP.compute_mask(t, cfgs.numpy())
    default = gd.c_tokens()  # builds the default order
    from bpdecode_amd.grammar.device import _walk_order

    base, _ = _walk_order(gd.tok_offsets, gd.tok_bytes, gd.vocab_size, gd.eos_id)
    perm = torch.from_numpy(np.random.default_rng(9).permutation(gd.vocab_size))
    assert default is not None
    assert np.array_equal(pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32), want)
    for name, order in (("default", base), ("id", None), ("random", perm), ("reversed", base.flip(0))):
        got = _masks_with_order(gd, pool, order)
        assert np.array_equal(got, want), name


def test_json_bench_batch_every_row(dev, json_case):
    """The benchmark's batch (256 rows, prefixes of 0-200 bytes at depths
    0-8, the same seed): every row's mask and committed config-set against
    the oracle, one step."""
    vocab, g, t = json_case
    _log("case json V=151936 B=256 bench rows, mask + commit")
    rng = np.random.default_rng(5)
    rows = []
    while len(rows) < 256:
        d = int(rng.integers(0, 9))
        c = g.init_config()
        if g.feed(c, synth.json_prefix(rng, d)):
            rows.append(c)
    cfgs = torch.stack(rows)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    lg = synth.logits(256, vocab.size, 3.0, torch.float32, seed=11)
    got = lg.to(dev)
    pda_mask_(got, gd, pool)
    ref = lg.numpy().copy()
    OP.apply_mask(t, cfgs.numpy().copy(), ref)
    assert np.array_equal(got.cpu().numpy(), ref)
    toks = torch.multinomial(torch.softmax(torch.from_numpy(ref), dim=-1), 1,
                             generator=torch.Generator().manual_seed(12)).view(-1).to(torch.int32)
    ok, _ = pda_step(pool, gd, toks.to(dev))
    mirror = cfgs.numpy().copy()
    ok_o = OP.advance(t, mirror, toks.numpy())
    assert ok.cpu().tolist() == ok_o.tolist() and ok_o.all()
    assert np.array_equal(pool.cpu().numpy(), mirror)


def test_json_direct_walk_equals_memo(dev, json_case):
    """The C ABI without a workspace runs the direct per-token walk; with one,
    the memoised kernel: identical bits."""
    from bpdecode_amd import _lib
    from bpdecode_amd._lib import check, lib, ptr

    vocab, g, t = json_case
    _log("case json V=151936 B=16 direct vs memo")
    cfgs = _json_configs(g, 16, seed=33)
    gd = g.to(dev)
    pool = cfgs.to(dev)
    words = (vocab.size + 31) // 32
    direct = torch.empty((16, words), dtype=torch.int32, device=dev)
    check(lib().bpd_pda_compute_mask(gd.c_table(), gd.c_tokens(), ptr(pool), None, 16, ptr(direct),
                                     None, 0, _lib.stream_of(dev)))
    memo = pda_compute_mask(gd, pool)
    assert torch.equal(direct.cpu(), memo.cpu())


@pytest.mark.parametrize("mode", ["row", "tile"])
@pytest.mark.parametrize("limit", [None, "1", "12"])
def test_json_commit_paths_match_oracle(dev, json_case, monkeypatch, limit, mode):
    """Commit after the mask of the same config-sets (transition tables
    reused; with the set limit lowered they hold overflow entries), after a
    mask of other config-sets (stale tables) and with no mask at all: raw
    config words and ok flags as the oracle's."""
    vocab, g, t = json_case
    _log(f"case json commit paths limit={limit} mode {mode}")
    monkeypatch.setenv("BPD_PDA_MEMO_MODE", mode)
    if limit:
        monkeypatch.setenv("BPD_PDA_MEMO_SETS", limit)
    gd = g.to(dev)
    cfgs = _json_configs(g, 16, seed=41)
    other = _json_configs(g, 16, seed=42)
    rng = np.random.default_rng(3)
    for mode in ("fresh", "stale", "none"):
        pool = cfgs.to(dev)
        if mode == "fresh":
            pda_compute_mask(gd, pool)
        elif mode == "stale":
            pda_compute_mask(gd, other.to(dev))
        bits = OP.compute_mask(t, cfgs.numpy())
        allowed = [np.nonzero(np.unpackbits(bits[r].view(np.uint8), bitorder="little")[:vocab.size])[0]
                   for r in range(16)]
        # mostly allowed tokens, a few arbitrary ones (rejected paths)
        toks = [int(rng.choice(a)) if (len(a) and r % 4) else int(rng.integers(0, vocab.size))
                for r, a in enumerate(allowed)]
        mirror = cfgs.numpy().copy()
        ok_o = OP.advance(t, mirror, np.array(toks, dtype=np.int32))
        ok, _ = pda_step(pool, gd, torch.tensor(toks, dtype=torch.int32, device=dev))
        assert ok.cpu().numpy().astype(bool).tolist() == ok_o.astype(bool).tolist(), mode
        assert np.array_equal(pool.cpu().numpy(), mirror), mode


@pytest.mark.parametrize("eps_reduce", [False, True])
def test_grammar_logits_processor_on_device(dev, eps_reduce):
    """GrammarLogitsProcessor(device=cuda) -- the HF calling convention over
    the device PDA kernels, bf16 scores masked in place -- against the C
    oracle step after step on a recursive grammar, and equal to the host
    backend on fp32 scores."""
    import random

    from bpdecode_amd.hf import GrammarLogitsProcessor

    _log(f"case GrammarLogitsProcessor device eps_reduce={eps_reduce}")
    grammar = 'root ::= "(" root ")" | "[" "1"? "]" | "x" | "{a" ":0," root "}"'
    lp_cpu = GrammarLogitsProcessor(grammar, VOCAB, backend="cpu", eps_reduce=eps_reduce)
    lp_dev = GrammarLogitsProcessor(grammar, VOCAB, device=dev, eps_reduce=eps_reduce)
    assert lp_dev.backend == "device" and lp_cpu.backend == "cpu"
    t = OP.Table(build_pda_tensors(CompiledGrammar.build(parse_gbnf(grammar)), VOCAB, eps_reduce=eps_reduce))
    mirror = np.repeat(OP.init(t)[None], 3, axis=0)
    input_ids = torch.zeros(3, 1, dtype=torch.long)
    rng = random.Random(7)
    for step in range(10):
        s_cpu = torch.zeros(3, VOCAB.size)
        s_dev = torch.zeros(3, VOCAB.size, dtype=torch.bfloat16, device=dev)
        ptr0 = s_dev.data_ptr()
        lp_cpu(input_ids, s_cpu)
        assert lp_dev(input_ids.to(dev), s_dev).data_ptr() == ptr0
        want = np.zeros((3, VOCAB.size), np.float32)
        OP.apply_mask(t, mirror, want)
        assert torch.equal(torch.isneginf(s_dev.cpu()), torch.from_numpy(np.isneginf(want))), step
        assert torch.equal(torch.isneginf(s_cpu), torch.isneginf(s_dev.cpu())), step
        for r in range(3):
            assert lp_cpu.is_complete(r) == lp_dev.is_complete(r)
        toks = [rng.choice((~torch.isneginf(s_cpu[r])).nonzero().flatten().tolist()) for r in range(3)]
        assert OP.advance(t, mirror, toks).all()
        input_ids = torch.cat([input_ids, torch.tensor(toks).unsqueeze(1)], dim=1)


def _unpack_allowed(bits: np.ndarray, V: int, dev) -> torch.Tensor:
    """bool [B, V] on the device from packed LSB-first allow bits."""
    b = torch.from_numpy(np.ascontiguousarray(bits).view(np.int32)).to(dev)
    sh = torch.arange(32, device=dev, dtype=torch.int32)
    return ((b.unsqueeze(-1) >> sh) & 1).bool().reshape(b.shape[0], -1)[:, :V]


def _bench_rows(g, B):
    """The benchmark's starting rows: JSON prefixes of 0-200 bytes, nesting
    depth uniform over 0-8, seed 5."""
    rng = np.random.default_rng(5)
    rows = []
    while len(rows) < B:
        d = int(rng.integers(0, 9))
        c = g.init_config()
        if g.feed(c, synth.json_prefix(rng, d)):
            rows.append(c)
    return torch.stack(rows)


def _oracle_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


@pytest.mark.timeout(900)
def test_json_bench_trajectory_64_steps(dev, json_case):
    """The recursive-JSON workload in full: B = 256 rows from the bench's
    prefixes, V = 151,936, fp32 logits N(0, 3), 64 mask + commit steps with
    tokens sampled from the oracle's masked softmax; every row's mask and raw
    266-word config-set against the C oracle at every step."""
    vocab, g, t = json_case
    V, B = vocab.size, 256
    _log("case json V=151936 B=256 trajectory 64 steps")
    start = _bench_rows(g, B)
    batch = CFGConstraintBatch(g, capacity=B, device=dev)
    ids = list(range(B))
    for i in ids:
        batch.add(i)
    batch._configs.copy_(start.to(dev))
    mirror = start.numpy().copy()
    gen = torch.Generator(device=dev).manual_seed(7)
    threads = _oracle_threads()
    for step in range(64):
        lg = torch.randn((B, V), generator=gen, device=dev).mul_(3.0)
        got = lg.clone()
        batch.apply_mask(ids, got)
        allowed = _unpack_allowed(OP.compute_mask_threads(t, mirror, threads), V, dev)
        want = lg.masked_fill(~allowed, float("-inf"))
        assert torch.equal(got, want), step
        toks = torch.multinomial(torch.softmax(want, dim=-1), 1, generator=gen).view(-1)
        status = batch.commit(ids, toks)
        ok = OP.advance(t, mirror, toks.cpu().numpy())
        assert ok.all() and status.cpu().tolist() == [1] * B, step
        assert np.array_equal(batch._configs.cpu().numpy(), mirror), step
        if step % 16 == 0:
            _log(f"  step {step} ok")


def _longest_accepted(g, prefix: bytes):
    """The config-set after the longest head of ``prefix`` a PDA table
    accepts, and that head's length (feed leaves a set untouched when a
    byte would empty it)."""
    c = g.init_config()
    for i in range(len(prefix)):
        if not g.feed(c, prefix[i:i + 1]):
            return c, i
    return c, len(prefix)


@pytest.mark.timeout(900)
def test_json_reference_flattening_full_vocab(dev):
    """The reference's own flattening of the recursive JSON grammar (no
    epsilon reduction: it saturates the 8-config bound) at V = 151,936, from
    prefixes drawn as configured (nesting depth uniform over 0-8, 0-200
    bytes).  That flattening stops every prefix at its first opened
    container (its saturation drops the config that continues), so each row
    takes the config-set after the longest head of its prefix the flattening
    accepts: saturated sets at the point where the flattening stops (and the
    rows' later steps from there).  Masks and raw config words against the
    C oracle, 16 steps."""
    vocab = synth.serving_vocab(151_936, seed=1)
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, vocab)  # the default: the reference's flattening
    t = OP.Table(g)
    V, B = vocab.size, 64
    _log("case json reference flattening V=151936 B=64 16 steps")
    rng = np.random.default_rng(21)
    rows, cut = [], 0
    while len(rows) < B:
        prefix = synth.json_prefix(rng, int(rng.integers(0, 9)), max_len=200)
        c, used = _longest_accepted(g, prefix)
        cut += used < len(prefix)
        rows.append(c)
    assert cut > B // 2
    start = torch.stack(rows)
    gd = g.to(dev)
    pool = start.to(dev)
    mirror = start.numpy().copy()
    gen = torch.Generator(device=dev).manual_seed(22)
    threads = _oracle_threads()
    saturated = 0
    for step in range(16):
        saturated += int((mirror[:, 1] != 0).sum())
        bits = OP.compute_mask_threads(t, mirror, threads)
        got = pda_compute_mask(gd, pool).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, bits), step
        allowed = _unpack_allowed(bits, V, dev)
        lg = torch.randn((B, V), generator=gen, device=dev)
        want = lg.masked_fill(~allowed, float("-inf"))
        want[~allowed.any(dim=1)] = 0.0  # rows with nothing allowed sample anything (rejected)
        toks = torch.multinomial(torch.softmax(want, dim=-1), 1, generator=gen).view(-1).to(torch.int32)
        ok, _ = pda_step(pool, gd, toks)
        ok_o = OP.advance(t, mirror, toks.cpu().numpy())
        assert ok.cpu().numpy().tolist() == ok_o.tolist(), step
        assert np.array_equal(pool.cpu().numpy(), mirror), step
    assert saturated > 0, "no saturated config-set met"


def test_commit_after_smaller_mask_same_workspace(dev, json_case):
    """mask(16 rows), then mask(4 rows of the same config-sets) on the same
    workspace, then commit(16): the second launch overwrote parts of the
    first one's interned sets, so the commit must not reuse the 16-row
    tables it left.  Raw config words and ok flags against the oracle."""
    vocab, g, t = json_case
    _log("case json commit after a smaller mask")
    gd = g.to(dev)
    cfgs = _json_configs(g, 16, seed=51)
    pool = cfgs.to(dev)
    pda_compute_mask(gd, pool)
    pda_compute_mask(gd, pool[:4].clone())
    bits = OP.compute_mask(t, cfgs.numpy())
    rng = np.random.default_rng(52)
    toks = []
    for r in range(16):
        a = np.nonzero(np.unpackbits(bits[r].view(np.uint8), bitorder="little")[:vocab.size])[0]
        a = a[a != vocab.eos_id]
        toks.append(int(a[np.argmax([len(vocab.token_bytes[i]) for i in a])]) if len(a) else 0)
    mirror = cfgs.numpy().copy()
    ok_o = OP.advance(t, mirror, np.array(toks, dtype=np.int32))
    ok, _ = pda_step(pool, gd, torch.tensor(toks, dtype=torch.int32, device=dev))
    assert ok.cpu().numpy().tolist() == ok_o.tolist()
    assert np.array_equal(pool.cpu().numpy(), mirror)


def test_cfg_batch_commit_reads_int64_low_bits(dev, json_case):
    """CFGConstraintBatch.commit converts int64 ids with tokens.to(int32) as
    the reference does (device.py:278): 2**32 + t commits token t."""
    vocab, g, t = json_case
    cfgs = _json_configs(g, 4, seed=61)
    batch = CFGConstraintBatch(g, capacity=4, device=dev)
    for i in range(4):
        batch.add(i)
    batch._configs.copy_(cfgs.to(dev))
    bits = OP.compute_mask(t, cfgs.numpy())
    toks = [int(np.nonzero(np.unpackbits(bits[r].view(np.uint8), bitorder="little")[:vocab.size])[0][0])
            for r in range(4)]
    status = batch.commit(list(range(4)), torch.tensor([2**32 + k for k in toks], dtype=torch.int64, device=dev))
    mirror = cfgs.numpy().copy()
    ok_o = OP.advance(t, mirror, np.array(toks, dtype=np.int32))
    assert ok_o.all() and status.cpu().tolist() == [1, 1, 1, 1]
    assert np.array_equal(batch._configs.cpu().numpy(), mirror)


def _toy_rows(g, t, vocab, B, rng):
    """B config-sets reached by 0-5 random allowed tokens from the start."""
    rows = []
    for _ in range(B):
        c = g.init_config()
        for _ in range(int(rng.integers(0, 6))):
            bits = OP.compute_mask(t, c.numpy()[None])[0]
            allowed = [k for k in range(vocab.size) if bits[k >> 5] >> (k & 31) & 1 and k != vocab.eos_id]
            if not allowed or not g.feed(c, vocab.token_bytes[int(rng.choice(allowed))]):
                break
        rows.append(c)
    return torch.stack(rows)


@pytest.mark.parametrize("idx", range(len(GRAMMARS)))
def test_logits_views_of_every_alignment(dev, idx):
    """A 35-token vocabulary and logits rows inside wider buffers: aligned
    rows of four-column groups (stored whole) with a ragged last group,
    rows whose start or stride breaks the alignment (column by column), in
    every dtype; the oracle's masks, and columns outside the view untouched."""
    vocab = Vocabulary.from_tokens(list(VOCAB.token_bytes) + [b"xy", b"0,", b"}}"], eos_id=VOCAB.eos_id)
    g = build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[idx])), vocab, eps_reduce=True)
    t = OP.Table(g)
    B, V = 6, vocab.size
    cfgs = _toy_rows(g, t, vocab, B, np.random.default_rng(200 + idx))
    gd = g.to(dev)
    pool = cfgs.to(dev)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        for width, start in ((35, 0), (36, 0), (40, 1), (48, 4)):
            _log(f"case toy grammar {idx} logits {dtype} width {width} start {start}")
            base = torch.randn(B, width, generator=torch.Generator().manual_seed(width)).to(dtype)
            ref = base.float().numpy().copy()
            view = ref[:, start:start + V].copy()
            OP.apply_mask(t, cfgs.numpy().copy(), view)
            want = base.clone()
            want[:, start:start + V][torch.from_numpy(np.isneginf(view))] = float("-inf")
            got = base.to(dev)
            pda_mask_(got[:, start:start + V], gd, pool)
            assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8)), (dtype, width, start)


def test_json_token_records_across_row_counts(dev, json_case):
    """Masks at 16, 4, 16 and 16 rows on one workspace: the records packed
    at one row count are not taken at another (their place moves), and the
    last call reuses the records of the one before; each against the oracle."""
    vocab, g, t = json_case
    gd = g.to(dev)
    cfgs = _json_configs(g, 16, seed=91)
    for n in (16, 4, 16, 16):
        _log(f"case json token records B={n}")
        got = pda_compute_mask(gd, cfgs[:n].to(dev)).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, OP.compute_mask(t, cfgs[:n].numpy())), n


def test_token_records_of_two_vocabularies_one_workspace(dev):
    """Two vocabularies of the same size and different bytes, masked in turn
    through the C ABI on one workspace (header zeroed once): the content tags
    differ, so each call walks its own tables' records; against the oracle."""
    from bpdecode_amd._lib import check, lib, ptr

    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    base = [bytes([i]) for i in range(256)]
    cases = []
    for extra in ([b"", b"\"a", b"</s>", b"", b"1, ", b"[{\"", b"true]"],
                  [b"", b"{\"", b"</s>", b"", b"2]", b"\"k\":", b"null,"]):
        vocab = Vocabulary.from_tokens(base + extra, eos_id=258)
        g = build_pda_tensors(comp, vocab, eps_reduce=True)
        cfgs = _json_configs(g, 8, seed=93)
        cases.append((g.to(dev), cfgs.to(dev), OP.compute_mask(OP.Table(g), cfgs.numpy())))
    assert cases[0][0].c_tokens().pack_tag != cases[1][0].c_tokens().pack_tag
    V = cases[0][0].vocab_size
    need = int(lib().bpd_pda_workspace_bytes(8, V))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for i in (0, 1, 0, 0, 1):
        _log(f"case two vocabularies, tables {i}")
        gd, pool, want = cases[i]
        out = torch.empty((8, (V + 31) // 32), dtype=torch.int32, device=dev)
        check(lib().bpd_pda_compute_mask(gd.c_table(), gd.c_tokens(), ptr(pool), None, 8, ptr(out),
                                         ptr(ws), need, stream))
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want), i



def test_token_records_repacked_when_workspace_overwritten(dev, json_case):
    """Masks through the C ABI on one workspace that is overwritten between
    calls (0xAB in every byte, the pack stamp included): the first call packs
    the token records in a launch of its own; the next finds this workspace
    and key already packed by this process, so the mask checks the stamp
    itself, finds garbage and packs the records in every block before
    walking; the third takes them as they are.  Bits and fp32 logits at
    B=16, V=151,936 (the last four rows to finish leave their logits to the
    launch after the mask), each call against the oracle.  After each logits
    mask a commit on the same workspace (whose transition rows past the
    interned sets still hold the 0xAB fill after the overwrite) advances a
    copy of the config-sets by an allowed token per row (token 0 where none
    is), raw words and ok flags against the oracle."""
    from bpdecode_amd._lib import DTYPE_F32, check, index_code, lib, ptr

    vocab, g, t = json_case
    gd = g.to(dev)
    B, V = 16, g.vocab_size
    cfgs = _json_configs(g, B, seed=97)
    pool = cfgs.to(dev)
    want_bits = OP.compute_mask(t, cfgs.numpy())
    need = int(lib().bpd_pda_workspace_bytes(B, V))
    stream = torch.cuda.current_stream(dev).cuda_stream
    for mode in ("bits", "logits"):
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        for call in ("packs", "overwritten", "packed"):
            _log(f"case repack {mode} {call}")
            if call == "overwritten":
                ws.fill_(0xAB)
                torch.cuda.synchronize(dev)
            if mode == "bits":
                out = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device=dev)
                check(lib().bpd_pda_compute_mask(gd.c_table(), gd.c_tokens(), ptr(pool), None, B, ptr(out),
                                                 ptr(ws), need, stream))
                assert np.array_equal(out.cpu().numpy().view(np.uint32), want_bits), call
            else:
                lg = synth.logits(B, V, 3.0, torch.float32, seed=5)
                got = lg.to(dev)
                check(lib().bpd_pda_apply_mask(gd.c_table(), gd.c_tokens(), ptr(pool), None, None, B, ptr(got),
                                               DTYPE_F32, V, float("-inf"), ptr(ws), need, stream))
                ref = lg.numpy().copy()
                OP.apply_mask(t, cfgs.numpy(), ref)
                assert np.array_equal(got.cpu().numpy(), ref), call
                allowed = np.unpackbits(want_bits.view(np.uint8), axis=1, bitorder="little")[:, :V]
                pick = np.random.default_rng(13)
                toks = np.array([pick.choice(np.flatnonzero(r)) if r.any() else 0 for r in allowed], dtype=np.int32)
                adv = pool.clone()
                tk = torch.from_numpy(toks).to(dev)
                ok = torch.empty(B, dtype=torch.uint8, device=dev)
                status = torch.empty(B, dtype=torch.int32, device=dev)
                check(lib().bpd_pda_advance(gd.c_table(), gd.c_tokens(), ptr(adv), None, ptr(tk),
                                            index_code(torch.int32), B, ptr(ok), None, ptr(status), None,
                                            ptr(ws), need, stream))
                mirror = cfgs.numpy().copy()
                ok_o = OP.advance(t, mirror, toks)
                assert ok.cpu().numpy().tolist() == ok_o.tolist(), call
                assert np.array_equal(adv.cpu().numpy(), mirror), call

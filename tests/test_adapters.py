"""HF and vLLM adapters on top of the constraint step (the scenarios of the
reference's test_hf.py / test_vllm.py): no model is loaded, a fixed bias
vector stands in for the model and the generate() / vLLM calling conventions
are driven by hand. Each scenario runs on CPU tensors and, marked ``gpu``, on
the device. Ground truth is the oracle's tok_next table walked token by
token (tests._util.OracleWalk), and Python's re module for complete texts."""

from __future__ import annotations

import re

import pytest
import torch

from bpdecode_amd.hf import RegexLogitsProcessor as HFRegex
from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
from bpdecode_amd.vllm import BatchConstraintState, RegexLogitsProcessor, RegexLogitsProcessorFactory
from tests._util import OracleWalk

TOKENS = ["0", "1", "2", "3", "4", "5", "6", "7", "8", "9", ".", "-", " ", "x", "</s>"]
VOCAB = Vocabulary.from_tokens(TOKENS, eos_id=len(TOKENS) - 1)
DECIMAL = "-?[0-9]+(\\.[0-9]+)?"
DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


def _decode(ids):
    return "".join(TOKENS[i] for i in ids if i != VOCAB.eos_id)


def _hf_greedy(pattern, bias, device, max_new=12):
    lp = HFRegex(pattern, VOCAB, device=device)
    input_ids = torch.zeros(1, 1, dtype=torch.long, device=device)
    out = []
    for _ in range(max_new):
        scores = lp(input_ids, bias.clone().unsqueeze(0).to(device))
        nxt = int(scores[0].argmax())
        out.append(nxt)
        if nxt == VOCAB.eos_id:
            break
        input_ids = torch.cat([input_ids, torch.tensor([[nxt]], device=device)], dim=1)
    return out


def _walk(pattern):
    return OracleWalk(FsaTensors.build(pattern, VOCAB))


def _valid_prefix(pattern, ids):
    ref = _walk(pattern)
    for tok in ids:
        if tok == VOCAB.eos_id:
            return ref.is_complete()
        if tok not in ref.allowed():
            return False
        ref.advance(tok)
    return True


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("pattern", [DECIMAL, "[12][0-9][0-9]", "[0-9]+ [0-9]+"])
def test_hf_every_step_stays_a_valid_prefix(device, pattern):
    bias = torch.zeros(VOCAB.size)
    bias[TOKENS.index("x")] = 10.0
    ids = _hf_greedy(pattern, bias, device)
    assert TOKENS.index("x") not in ids
    assert _valid_prefix(pattern, ids)


@pytest.mark.parametrize("device", DEVICES)
def test_hf_eos_only_when_complete(device):
    pattern = "[12][0-9][0-9]"
    bias = torch.zeros(VOCAB.size)
    bias[VOCAB.eos_id] = 10.0
    ids = _hf_greedy(pattern, bias, device)
    assert ids[-1] == VOCAB.eos_id and re.fullmatch(pattern, _decode(ids))


@pytest.mark.parametrize("device", DEVICES)
def test_hf_tracks_reference_and_batches_rows(device):
    lp = HFRegex(DECIMAL, VOCAB, device=device)
    refs = [_walk(DECIMAL) for _ in range(2)]
    seqs = [[TOKENS.index(c) for c in "-4.2"], [TOKENS.index(c) for c in "17.05"]]
    input_ids = torch.zeros(2, 1, dtype=torch.long, device=device)
    for step in range(4):
        scores = lp(input_ids, torch.zeros(2, VOCAB.size, device=device)).cpu()
        for r in range(2):
            got = {i for i in range(VOCAB.size) if scores[r, i] == 0.0}
            assert got == refs[r].allowed()
            refs[r].advance(seqs[r][step])
        nxt = torch.tensor([[seqs[0][step]], [seqs[1][step]]], device=device)
        input_ids = torch.cat([input_ids, nxt], dim=1)


def _vllm_greedy(proc, bias, max_new=12):
    past = []
    for _ in range(max_new):
        nxt = int(proc(past, bias.clone()).argmax())
        if nxt == VOCAB.eos_id:
            break
        past.append(nxt)
    return past


@pytest.mark.parametrize("device", DEVICES)
def test_vllm_request_processor(device):
    bias = torch.zeros(VOCAB.size, device=device)
    bias[TOKENS.index("x")] = 9.0
    proc = RegexLogitsProcessor(DECIMAL, VOCAB, device=device)
    past = _vllm_greedy(proc, bias)
    assert TOKENS.index("x") not in past and _valid_prefix(DECIMAL, past)
    # tracks the reference token by token, and restarts when the history shrinks
    proc = RegexLogitsProcessorFactory(VOCAB, device=device).make(DECIMAL)
    ref = _walk(DECIMAL)
    past = []
    for tok in [TOKENS.index(c) for c in "-4.2"]:
        logits = proc(past, torch.zeros(VOCAB.size, device=device)).cpu()
        assert {i for i in range(VOCAB.size) if logits[i] == 0.0} == ref.allowed()
        ref.advance(tok)
        past.append(tok)
    fresh = proc([], torch.zeros(VOCAB.size, device=device)).cpu()
    assert {i for i in range(VOCAB.size) if fresh[i] == 0.0} == _walk(DECIMAL).allowed()


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("mask_cache", [True, False])
def test_vllm_batch_state_slot_events(device, mask_cache):
    st = BatchConstraintState(VOCAB, device=device, mask_cache=mask_cache, capacity=8)
    st.add(0, DECIMAL)
    st.add(2, DECIMAL)
    gen = {0: [TOKENS.index(c) for c in "-1"], 2: [TOKENS.index(c) for c in "3."]}
    for row, ids in gen.items():
        st.advance(row, ids)
    st.move(2, 5)
    st.advance(5, gen[2] + [TOKENS.index("7")])
    logits = torch.zeros(6, VOCAB.size, device=device)
    st.mask(logits)
    logits = logits.cpu()
    for row, text in ((0, "-1"), (5, "3.7")):
        ref = _walk(DECIMAL)
        for c in text:
            ref.advance(TOKENS.index(c))
        assert {i for i in range(VOCAB.size) if logits[row, i] == 0.0} == ref.allowed()
    for row in (1, 2, 3, 4):
        assert torch.all(logits[row] == 0.0)  # rows without a request are untouched
    assert st.is_complete(5) and st.is_complete(0)
    st.remove(0)
    with pytest.raises(KeyError):  # as the reference: the row no longer exists
        st.is_complete(0)


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float64])
def test_hf_scores_dtype(device, dtype):
    """bf16 / fp16 scores are masked in place in their own dtype; float64
    goes through the reference's float32 round trip (hf.py:106-113).  Either
    way the result equals that round trip."""
    lp = HFRegex(DECIMAL, VOCAB, device=device)
    ref = _walk(DECIMAL)
    input_ids = torch.zeros(2, 1, dtype=torch.long, device=device)
    g = torch.Generator().manual_seed(3)
    for step, tok in enumerate([TOKENS.index(c) for c in "-4.2"]):
        raw = (torch.randn(2, VOCAB.size + 3, generator=g) * 3).to(dtype)  # 3 padded columns
        want = raw.float()
        keep = torch.zeros(VOCAB.size + 3, dtype=torch.bool)
        keep[sorted(ref.allowed())] = True
        want[:, ~keep] = float("-inf")
        want = want.to(dtype)
        scores = raw.to(device)
        storage = scores.data_ptr()
        out = lp(input_ids, scores)
        assert out.data_ptr() == storage and out.dtype == dtype
        assert torch.equal(out.cpu().view(torch.uint8), want.view(torch.uint8)), step
        ref.advance(tok)
        input_ids = torch.cat([input_ids, torch.full((2, 1), tok, device=device)], dim=1)


@pytest.mark.parametrize("device", DEVICES)
def test_hf_regex_auto_density(device):
    """RegexLogitsProcessor follows the reference's density rule
    (ops.py:137-139): the 826-state JSON-Schema DFA over 50,000 tokens
    (41.3e6 entries) stays a symbol-class bundle, masked by the walking
    path; a small pattern is dense."""
    from bpdecode_amd import synth
    from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
    from bpdecode_amd.grammar.pda import CompiledGrammar
    from bpdecode_amd.grammar.regular import residual_dfa

    vocab = synth.serving_vocab(50_000, seed=2)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    lp = HFRegex(dfa, vocab, device=device)
    assert lp._fsa.tok_next is None and lp._fsa.num_states * vocab.size > 32_000_000
    assert HFRegex(DECIMAL, VOCAB, device=device)._fsa.tok_next is not None
    walk = OracleWalk(FsaTensors.build(dfa, vocab, dense=False))
    input_ids = torch.zeros(1, 1, dtype=torch.long, device=device)
    for tok in b'{ "name":':  # ids 0-255 are the single bytes
        scores = lp(input_ids, torch.zeros(1, vocab.size, device=device)).cpu()
        assert {int(i) for i in (scores[0] == 0).nonzero().flatten()} == walk.allowed()
        walk.advance(tok)
        input_ids = torch.cat([input_ids, torch.tensor([[tok]], device=device)], dim=1)


@pytest.mark.parametrize("device", DEVICES)
def test_vllm_batch_state_queued_rounds(device):
    """Ids queued by advance() are committed in rounds when the mask needs
    them (several per row, rows of different lengths); a rewound history
    replays from the start; a contiguous block of rows is masked where it
    lies."""
    st = BatchConstraintState(VOCAB, device=device, mask_cache=False, capacity=8)
    for row in range(3):
        st.add(row, DECIMAL)
    texts = {0: "-12.5", 1: "7", 2: "33.0"}
    for row, text in texts.items():
        st.advance(row, [TOKENS.index(c) for c in text[:2]])
    for row, text in texts.items():
        st.advance(row, [TOKENS.index(c) for c in text])
    st.advance(1, [TOKENS.index("4")])  # rewound and replaced: "4"
    texts[1] = "4"
    logits = torch.zeros(4, VOCAB.size, device=device)
    base = logits.data_ptr()
    st.mask(logits)
    assert logits.data_ptr() == base
    logits = logits.cpu()
    for row, text in texts.items():
        ref = _walk(DECIMAL)
        for c in text:
            ref.advance(TOKENS.index(c))
        assert {i for i in range(VOCAB.size) if logits[row, i] == 0.0} == ref.allowed(), row
        assert st.is_complete(row) == ref.is_complete()
    assert torch.all(logits[3] == 0.0)

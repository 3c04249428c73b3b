"""The host front-end reproduces the reference's numbering: DFA states of
compile_regex, the JSON-Schema residual DFA and the flattened PDA tables of
build_pda_tensors, against vectors written by tests/golden/make_golden.py from
the reference's own front-end.  Also the UTF-8 range lowering against the
Python codec."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from bpdecode_amd.fsa import fsa_from_dfa
from bpdecode_amd.grammar.device import build_pda_tensors
from bpdecode_amd.grammar.gbnf import GBNFSyntaxError, parse_gbnf
from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
from bpdecode_amd.grammar.pda import CompiledGrammar
from bpdecode_amd.grammar.regular import frame_is_regular, residual_dfa
from bpdecode_amd.regex import RegexSyntaxError, compile_regex
from bpdecode_amd.regex.utf8 import utf8_sequences
from bpdecode_amd.tokenizer import Vocabulary
from tests.golden.cases import GRAMMARS, PATTERNS, PDA_VOCAB, SCHEMAS

GOLD = np.load(Path(__file__).parent / "golden" / "frontend.npz")


def check_dfa(dfa, key):
    assert np.array_equal(np.array(dfa.symbols).reshape(-1, 2), GOLD[f"{key}/symbols"])
    assert np.array_equal(np.array(dfa.trans), GOLD[f"{key}/trans"])
    assert sorted(dfa.accept) == GOLD[f"{key}/accept"].tolist()
    assert [dfa.start, dfa.dead] == GOLD[f"{key}/start_dead"].tolist()
    assert list(fsa_from_dfa(dfa).live) == GOLD[f"{key}/live"].tolist()


def check_pda(g, key):
    assert [g.num_states, g.root_start, g.root_accept] == GOLD[f"{key}/meta"].tolist()
    for f in ("accept", "live", "edge_offsets", "edge_kind", "edge_lo", "edge_hi", "edge_dst", "edge_callee"):
        assert np.array_equal(getattr(g, f).numpy(), GOLD[f"{key}/{f}"]), f


@pytest.mark.parametrize("i", range(len(PATTERNS)))
def test_dfa_numbering(i):
    check_dfa(compile_regex(PATTERNS[i]), f"regex{i}")


VOCAB = Vocabulary.from_tokens(PDA_VOCAB[0], eos_id=PDA_VOCAB[1])


@pytest.mark.parametrize("i", range(len(GRAMMARS)))
def test_pda_tables(i):
    check_pda(build_pda_tensors(CompiledGrammar.build(parse_gbnf(GRAMMARS[i])), VOCAB), f"gbnf{i}")


@pytest.mark.parametrize("i", range(len(SCHEMAS)))
def test_schema_tables_and_residual(i):
    comp = CompiledGrammar.build(json_schema_to_grammar(SCHEMAS[i]))
    check_pda(build_pda_tensors(comp, VOCAB), f"schema{i}")
    start = comp.rules[comp.root].start
    if frame_is_regular(comp, comp.regular, comp.root, start):
        check_dfa(residual_dfa(comp, comp.root, start), f"residual{i}")
    else:
        assert f"residual{i}/trans" not in GOLD.files


@pytest.mark.parametrize("lo,hi", [(0, 0x7F), (0x80, 0x7FF), (0x7F0, 0x10FF), (0xD700, 0xE100),
                                   (0x10000, 0x10FFFF), (0x41, 0x41), (0, 0x10FFFF), (0xFFFF, 0x10000)])
def test_utf8_sequences_cover_exactly(lo, hi):
    seqs = utf8_sequences(lo, hi)
    step = max(1, (hi - lo) // 4000)
    for cp in list(range(lo, hi + 1, step)) + [hi]:
        if 0xD800 <= cp <= 0xDFFF:
            continue
        enc = chr(cp).encode()
        hits = [s for s in seqs if len(s) == len(enc) and all(a <= b <= c for (a, c), b in zip(s, enc))]
        assert len(hits) == 1, hex(cp)


def test_syntax_errors():
    for bad in ["(a", "a)", "*a", "a{2,1}", "[b-a]", "^a", "a{", "\\"]:
        with pytest.raises(RegexSyntaxError):
            compile_regex(bad)
    for bad in ['root ::= "a', "root ::= [a", "root = x", "root ::= (x"]:
        with pytest.raises((GBNFSyntaxError, KeyError)):
            parse_gbnf(bad)

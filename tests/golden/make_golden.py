"""Write tests/golden/frontend.npz: reference front-end outputs that no other
check pins -- DFA state numbering of compile_regex (regex/compile.py:194-255),
the JSON-Schema residual DFA (grammar/regular.py:184-199) and the flattened
PDA tables of build_pda_tensors (grammar/device.py:79-158).

Run in the development container only (it imports the reference checkout):

    PYTHONPATH=/root/reference/src python tests/golden/make_golden.py

Only data is written: integer arrays and table sizes.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from bpdecode.fsa import fsa_from_dfa  # noqa: E402  (reference)
from bpdecode.grammar.device import build_pda_tensors  # noqa: E402  (reference)
from bpdecode.grammar.gbnf import parse_gbnf  # noqa: E402  (reference)
from bpdecode.grammar.json_schema import json_schema_to_grammar  # noqa: E402  (reference)
from bpdecode.grammar.pda import CompiledGrammar  # noqa: E402  (reference)
from bpdecode.grammar.regular import frame_is_regular, residual_dfa  # noqa: E402  (reference)
from bpdecode.regex import compile_regex  # noqa: E402  (reference)
from bpdecode.tokenizer import Vocabulary  # noqa: E402  (reference)

from tests.golden.cases import GRAMMARS, PATTERNS, PDA_VOCAB, SCHEMAS  # noqa: E402


def dfa_arrays(dfa, key, out):
    out[f"{key}/symbols"] = np.array(dfa.symbols, dtype=np.int32).reshape(-1, 2)
    out[f"{key}/trans"] = np.array(dfa.trans, dtype=np.int32)
    out[f"{key}/accept"] = np.array(sorted(dfa.accept), dtype=np.int32)
    out[f"{key}/start_dead"] = np.array([dfa.start, dfa.dead], dtype=np.int32)
    out[f"{key}/live"] = np.array(fsa_from_dfa(dfa).live, dtype=np.uint8)


def pda_arrays(g, key, out):
    out[f"{key}/meta"] = np.array([g.num_states, g.root_start, g.root_accept], dtype=np.int32)
    for f in ("accept", "live", "edge_offsets", "edge_kind", "edge_lo", "edge_hi", "edge_dst",
              "edge_callee"):
        out[f"{key}/{f}"] = getattr(g, f).numpy()


def main() -> None:
    out: dict[str, np.ndarray] = {}
    for i, pat in enumerate(PATTERNS):
        dfa_arrays(compile_regex(pat), f"regex{i}", out)
    vocab = Vocabulary.from_tokens(PDA_VOCAB[0], eos_id=PDA_VOCAB[1])
    for i, src in enumerate(GRAMMARS):
        pda_arrays(build_pda_tensors(CompiledGrammar.build(parse_gbnf(src)), vocab), f"gbnf{i}", out)
    for i, schema in enumerate(SCHEMAS):
        comp = CompiledGrammar.build(json_schema_to_grammar(schema))
        pda_arrays(build_pda_tensors(comp, vocab), f"schema{i}", out)
        start = comp.rules[comp.root].start
        if frame_is_regular(comp, comp.regular, comp.root, start):
            dfa_arrays(residual_dfa(comp, comp.root, start), f"residual{i}", out)
    np.savez_compressed(HERE / "frontend.npz", **out)
    (HERE / "frontend_index.json").write_text(json.dumps(
        {"patterns": PATTERNS, "grammars": GRAMMARS, "schemas": SCHEMAS}, indent=1))
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()

"""Benchmark of the batched constraint step on one MI355X.

Default workload (serving scale, dense tok_next): the email regex
``[a-z0-9._]{1,32}@[a-z0-9-]{1,24}\\.(com|org|net|io)`` compiled to a byte DFA
over a seeded synthetic vocabulary of V = 151,936 tokens; B = 256 rows;
bf16 logits N(0, 3); continuous batching that evicts 10% of the rows and adds
as many fresh ones every step; tokens sampled from the masked softmax.

One step = ``ConstraintBatch.apply_mask`` + ``ConstraintBatch.commit``.  Each
step starts from cold caches: a 512 MB scratch buffer is read before it (no
dirty lines left behind), so logits and table rows come from HBM.  The two
calls are bracketed by HIP events on the stream they launch on, created with
hipEventDisableSystemFence (torch's timing events add a system-scope release
of several microseconds to each bracket); the slot list is staged and queued
slot writes applied just before the first bracket, so each bracket holds one
kernel.  Logits generation, the flush, sampling and churn sit outside the
brackets.

Roofline (dominant kernel = the dense mask): algorithmic bytes per launch
``D = B*V*2e + U*V*4`` (read + write of every logit, one int32 tok_next row per
distinct live state U of that step), divided by the kernel's event-timed
duration, against the 8 TB/s HBM3E peak.  The commit kernel adds 16 B per row.

CPU baseline: the oracle's numpy restatement of the reference dense path
timed on the host over a bounded replay of the first recorded steps.

Prints one JSON line.  ``--gpus N`` with N > 1 is refused: this build
measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


class HipEvents:
    """HIP events created with hipEventDisableSystemFence, recorded on a given
    stream: the bracket then holds no system-scope cache release, so it times
    the kernel between the markers (torch's timing events carry one)."""

    def __init__(self, n: int) -> None:
        import ctypes

        self._c = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.ev = []
        for _ in range(n):
            h = ctypes.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(ctypes.byref(h), ctypes.c_uint(HIP_EVENT_DISABLE_SYSTEM_FENCE))
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self.ev.append(h)

    def record(self, i: int, stream_handle: int) -> None:
        rc = self.hip.hipEventRecord(self.ev[i], self._c.c_void_p(stream_handle))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, i: int, j: int) -> float:
        ms = self._c.c_float()
        self.hip.hipEventSynchronize(self.ev[j])
        rc = self.hip.hipEventElapsedTime(self._c.byref(ms), self.ev[i], self.ev[j])
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baselines."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _profiled_traffic(name: str, kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprof counter
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration), or
    None when no summary for this kernel is present."""
    p = ROOT / "profiles" / name
    try:
        rec = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    return rec.get("traffic_bytes") if rec.get("kernel") == kernel else None


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--batch", type=int, default=256)
    p.add_argument("--vocab", type=int, default=151_936)
    p.add_argument("--churn", type=float, default=0.10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-steps", type=int, default=8, help="recorded steps replayed on the CPU")
    p.add_argument("--cpu-repeats", type=int, default=3)
    p.add_argument("--no-flush", action="store_true", help="keep caches warm between steps")
    p.add_argument("--workload", choices=["dense", "pda", "soft", "schema"], default="dense",
                   help="dense: email-regex tok_next step (the headline); pda: recursive-JSON PDA step; "
                        "soft: prior-weighted lookahead; schema: flat JSON-Schema DFA at B=512, dense "
                        "table and walking kernel side by side")
    p.add_argument("--schema-rows", type=int, default=512)
    p.add_argument("--schema-steps", type=int, default=64)
    p.add_argument("--pda-rows", type=int, default=256)
    p.add_argument("--pda-steps", type=int, default=64)
    p.add_argument("--pda-cpu-rows", type=int, default=4, help="rows of one step replayed on the CPU oracle")
    p.add_argument("--soft-rows", type=int, default=128)
    p.add_argument("--soft-k", type=int, default=4)
    p.add_argument("--soft-steps", type=int, default=64)
    p.add_argument("--soft-cpu-rows", type=int, default=2, help="rows replayed on the float64 oracle")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="instead: run a plain device copy of MB megabytes 20 times (PMC scale check)")
    return p.parse_args(argv)


def calibrate_copy(mb: int) -> None:
    import torch

    dev = torch.device("cuda:0")
    n = mb * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n * 4, "bytes_written": n * 4, "launches": 20}))


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the constraint "
              "step is row-parallel, so N GPUs each run it on their own B/N rows with no exchange, "
              "and the one-GPU figure is the per-GPU rate", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return 0
    if args.workload == "pda":
        return bench_pda(args)
    if args.workload == "soft":
        return bench_soft(args)
    if args.workload == "schema":
        return bench_schema(args)

    import numpy as np
    import torch

    from bpdecode_amd import synth
    from bpdecode_amd.batch import ConstraintBatch
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, V = args.batch, args.vocab
    t0 = time.perf_counter()
    vocab = synth.serving_vocab(V, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab, dense=False).to(dev).densify()
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    S = fsa.num_states
    e = 2  # bf16

    batch = ConstraintBatch(fsa, capacity=2 * B, device=dev)
    rng = np.random.default_rng(2)
    next_id = 0
    active: list[int] = []
    for _ in range(B):
        batch.add(next_id)
        active.append(next_id)
        next_id += 1

    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    logits = torch.empty((B, V), dtype=torch.bfloat16, device=dev)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    flush.zero_()
    flush64 = flush.view(torch.int64)
    stream = torch.cuda.current_stream(dev)

    n_total = args.warmup + args.steps
    kev = HipEvents(4 * n_total)
    sh = stream.cuda_stream
    distinct: list[int] = []
    host_api_s: list[float] = []
    recorded = []  # (logits bits, states, tokens, masked bits) of the first timed steps
    n_cpu = 0 if args.no_cpu else min(args.cpu_steps, args.steps)

    torch.cuda.synchronize()
    wall0 = None
    for k in range(n_total):
        if k == args.warmup:
            torch.cuda.synchronize()
            wall0 = time.perf_counter()
        ids = list(active)
        logits.copy_(torch.randn((B, V), generator=gen, device=dev).mul_(3.0))
        slots = batch._slots(ids)
        pool = batch._state  # applies queued slot writes before the timed region
        states_now = pool[slots].cpu().numpy()
        live = states_now[states_now >= 0]
        distinct.append(int(np.unique(live).size))
        keep = k >= args.warmup and len(recorded) < n_cpu
        if keep:
            rec_logits = logits.cpu()
        if not args.no_flush:
            flush64.sum()
        h0 = time.perf_counter()
        kev.record(4 * k, sh)
        batch.apply_mask(ids, logits)
        kev.record(4 * k + 1, sh)
        h1 = time.perf_counter()
        probs = torch.softmax(logits.float(), dim=-1)
        toks = torch.multinomial(probs, 1, generator=gen).view(-1)
        h2 = time.perf_counter()
        kev.record(4 * k + 2, sh)
        batch.commit(ids, toks)
        kev.record(4 * k + 3, sh)
        h3 = time.perf_counter()
        host_api_s.append((h1 - h0) + (h3 - h2))
        if keep:
            recorded.append((rec_logits, states_now.copy(), toks.cpu().numpy(), logits.cpu()))
        # continuous batching: evict 10% of the rows, add as many fresh ones
        n_churn = int(round(args.churn * B))
        for i in rng.choice(len(active), size=n_churn, replace=False).tolist():
            batch.evict(active[i])
            active[i] = next_id
            batch.add(next_id)
            next_id += 1
    torch.cuda.synchronize()
    wall1 = time.perf_counter()

    timed = range(args.warmup, n_total)
    mask_ms = [kev.elapsed_ms(4 * k, 4 * k + 1) for k in timed]
    commit_ms = [kev.elapsed_ms(4 * k + 2, 4 * k + 3) for k in timed]
    step_ms = [a + b for a, b in zip(mask_ms, commit_ms)]
    U = distinct[args.warmup:]
    d_bytes = [B * V * 2 * e + u * V * 4 for u in U]
    achieved_gbs = sum(d_bytes) / (sum(mask_ms) * 1e-3) / 1e9
    mean_step_ms = statistics.fmean(step_ms)

    out = {
        "metric": "µs/step apply_mask+commit & GB/s (% HBM roofline), B=256 V=151936 bf16",
        "value": round(mean_step_ms * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_step_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "dense tok_next apply_mask+commit, email-regex DFA, continuous batching 10% churn",
            "batch_rows": B,
            "vocab": V,
            "dfa_states": S,
            "logits": "bf16 N(0,3)",
            "cache_flush": "512 MB read before each step" if not args.no_flush else "none",
        },
        "median_us_per_step": round(statistics.median(step_ms) * 1e3, 3),
        "mask_us": round(statistics.fmean(mask_ms) * 1e3, 3),
        "commit_us": round(statistics.fmean(commit_ms) * 1e3, 3),
        "timing": "fence-free HIP events around ConstraintBatch.apply_mask and .commit on their stream",
        "row_vocab_entries_per_s": round(B * V / (mean_step_ms * 1e-3), 1),
        "distinct_live_states_mean": round(statistics.fmean(U), 2),
        "api_host_us_per_step": round(statistics.fmean(host_api_s[args.warmup:]) * 1e6, 2),
        "wall_ms_per_step_incl_setup_work": round((wall1 - wall0) * 1e3 / args.steps, 4),
        "setup_s": round(setup_s, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / PEAK_HBM_GBS, 4),
            "traffic": _profiled_traffic("dense_mask_bits_email_b256_v151936.traffic.json",
                                         "dense_mask_bits_kernel<2, 2>"),
            "kernel": "dense_mask_bits_kernel<2, 2>",
            "algorithmic_bytes_per_launch_mean": round(statistics.fmean(d_bytes), 1),
            "table_charged_as": "int32 tok_next rows (the kernel reads the packed allow-bit table)",
        },
    }

    if n_cpu:
        from oracle import dense as OD

        # the reference's CPU step is ATen: ops.py:271-276 (mask) and
        # ops.py:301-306 (commit), timed here op for op on CPU tensors with
        # torch's host threads (OMP_NUM_THREADS); the numpy oracle checks the
        # GPU's masks as well
        tn_host = fsa.tok_next.cpu()
        tn_np = tn_host.numpy()
        fill = OD.fill_bits(torch.bfloat16, float("-inf"))
        parity = True
        times = []
        for _ in range(args.cpu_repeats):
            for lg, st, tk, masked in recorded:
                x = lg.clone()
                st_t = torch.from_numpy(st.astype(np.int32))
                tk_t = torch.from_numpy(np.asarray(tk))
                c0 = time.perf_counter()
                s_ = st_t.long()
                broken = s_ < 0
                rejected = tn_host.index_select(0, s_.clamp_(min=0)) == -1
                rejected |= broken.unsqueeze(1)
                x.masked_fill_(rejected, float("-inf"))
                s2 = st_t.long()
                nxt = tn_host[s2.clamp_(min=0), tk_t.long()]
                nxt = torch.where(s2 < 0, torch.full_like(nxt, -1), nxt).to(torch.int32)
                times.append(time.perf_counter() - c0)
                parity &= bool(torch.equal(x.view(torch.int16), masked.view(torch.int16)))
                bits = lg.view(torch.int16).numpy().view(np.uint16).copy()
                OD.apply_mask_bits(bits, tn_np, st, fill)
                parity &= bool(np.array_equal(bits, masked.view(torch.int16).numpy().view(np.uint16)))
        out["cpu_baseline"] = {
            "value": round(statistics.fmean(times) * 1e6, 1),
            "unit": "us/step",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{len(recorded)} recorded steps of the same workload (B={B}, V={V}, bf16), "
                      f"replayed {args.cpu_repeats}x through the reference's ATen op sequence "
                      f"(ops.py:271-276 mask, ops.py:301-306 commit) on CPU tensors",
            "host_cpus": os.cpu_count(),
            "host_cpu_model": _cpu_model(),
        }
        out["parity_vs_oracle"] = parity
    print(json.dumps(out))
    return 0


def bench_schema(args) -> int:
    """Flat JSON-Schema document DFA (826 states) over the serving vocab,
    B rows at random reachable states, bf16 logits N(0, 3), no churn.  Each
    step masks and commits twice on identical inputs: through the dense
    allow-bit table (the timed headline of this workload) and through the
    symbol-class walking kernel (no [states, vocab] table); the two results
    are compared bit for bit every step."""
    import numpy as np
    import torch

    from bpdecode_amd import synth
    from bpdecode_amd.batch import ConstraintBatch
    from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
    from bpdecode_amd.grammar.pda import CompiledGrammar
    from bpdecode_amd.grammar.regular import residual_dfa
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, V = args.schema_rows, args.vocab
    vocab = synth.serving_vocab(V, seed=1)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    plain = FsaTensors.build(dfa, vocab, dense=False).to(dev)
    dense = plain.densify()
    dense.ensure_allow_bits()
    S = plain.num_states
    starts = synth.random_walk_states(dense.tok_next.cpu(), plain.start, vocab.eos_id, B, 12, seed=4)
    batches = [ConstraintBatch(dense, capacity=B, device=dev), ConstraintBatch(plain, capacity=B, device=dev)]
    for bt in batches:
        for i in range(B):
            bt.add(i)
        bt._state[:B] = starts.to(dev)
    ids = list(range(B))
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    logits = [torch.empty((B, V), dtype=torch.bfloat16, device=dev) for _ in range(2)]
    flush64 = torch.zeros(512 << 20, dtype=torch.uint8, device=dev).view(torch.int64)
    sh = torch.cuda.current_stream(dev).cuda_stream
    n_total = args.warmup + args.schema_steps
    kev = HipEvents(8 * n_total)
    distinct, parity = [], True
    for k in range(n_total):
        logits[0].copy_(torch.randn((B, V), generator=gen, device=dev).mul_(3.0))
        logits[1].copy_(logits[0])
        st = batches[0]._state[:B]
        distinct.append(int(torch.unique(st[st >= 0]).numel()))
        toks = None
        for p, bt in enumerate(batches):
            bt._slots(ids)
            bt._state  # queued slot writes land before the timed region
            if not args.no_flush:
                flush64.sum()
            kev.record(8 * k + 4 * p, sh)
            bt.apply_mask(ids, logits[p])
            kev.record(8 * k + 4 * p + 1, sh)
            if toks is None:
                toks = torch.multinomial(torch.softmax(logits[p].float(), dim=-1), 1, generator=gen).view(-1)
            kev.record(8 * k + 4 * p + 2, sh)
            bt.commit(ids, toks)
            kev.record(8 * k + 4 * p + 3, sh)
        parity &= bool(torch.equal(logits[0].view(torch.int16), logits[1].view(torch.int16)))
        parity &= bool(torch.equal(batches[0]._state[:B], batches[1]._state[:B]))
    torch.cuda.synchronize()
    timed = range(args.warmup, n_total)
    ms = {name: [kev.elapsed_ms(8 * k + a, 8 * k + a + 1) for k in timed]
          for name, a in (("mask", 0), ("commit", 2), ("walk_mask", 4), ("walk_commit", 6))}
    step_ms = [a + b for a, b in zip(ms["mask"], ms["commit"])]
    U = distinct[args.warmup:]
    d_bytes = [B * V * 2 * 2 + u * V * 4 for u in U]
    achieved = sum(d_bytes) / (sum(ms["mask"]) * 1e-3) / 1e9
    mean_ms = statistics.fmean(step_ms)
    out = {
        "metric": "µs/step apply_mask+commit, flat JSON-Schema DFA, B=512 V=151936 bf16",
        "value": round(mean_ms * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.schema_steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "dense tok_next apply_mask+commit, flat JSON-Schema document DFA",
                   "batch_rows": B, "vocab": V, "dfa_states": S, "symbol_classes": plain.num_symbols,
                   "logits": "bf16 N(0,3)", "cache_flush": "512 MB read before each mask and commit pair"},
        "mask_us": round(statistics.fmean(ms["mask"]) * 1e3, 3),
        "commit_us": round(statistics.fmean(ms["commit"]) * 1e3, 3),
        "walk_mask_us": round(statistics.fmean(ms["walk_mask"]) * 1e3, 3),
        "walk_commit_us": round(statistics.fmean(ms["walk_commit"]) * 1e3, 3),
        "distinct_live_states_mean": round(statistics.fmean(U), 2),
        "row_vocab_entries_per_s": round(B * V / (mean_ms * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "dense_mask_bits_kernel<2, 4>",
                     "algorithmic_bytes_per_launch_mean": round(statistics.fmean(d_bytes), 1)},
        "parity_dense_vs_walk_every_step": parity,
    }
    print(json.dumps(out))
    return 0


def bench_pda(args) -> int:
    """Recursive-JSON PDA step: B rows seeded with valid JSON prefixes of
    0-200 bytes (nesting depth uniform over 0-8) over the V = 151,936
    synthetic vocabulary, fp32 logits N(0, 3), mask + commit per step with the
    token sampled from the masked softmax."""
    import numpy as np
    import torch

    from bpdecode_amd import synth
    from bpdecode_amd.grammar.device import CFGConstraintBatch, build_pda_tensors
    from bpdecode_amd.grammar.gbnf import parse_gbnf
    from bpdecode_amd.grammar.pda import CompiledGrammar

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, V = args.pda_rows, args.vocab
    vocab = synth.serving_vocab(V, seed=1)
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, vocab, eps_reduce=True)
    rng = np.random.default_rng(5)
    rows = []
    depths = []
    while len(rows) < B:
        d = int(rng.integers(0, 9))
        c = g.init_config()
        if g.feed(c, synth.json_prefix(rng, d)):
            rows.append(c)
            depths.append(d)
    start = torch.stack(rows)
    batch = CFGConstraintBatch(g, capacity=B, device=dev)
    ids = list(range(B))
    for i in ids:
        batch.add(i)
    batch._configs.copy_(start.to(dev))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    n_total = args.warmup + args.pda_steps
    kev = HipEvents(4 * n_total)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    logits = torch.empty((B, V), dtype=torch.float32, device=dev)
    first = None
    torch.cuda.synchronize()
    wall0 = None
    for k in range(n_total):
        if k == args.warmup:
            torch.cuda.synchronize()
            wall0 = time.perf_counter()
        logits.copy_(torch.randn((B, V), generator=gen, device=dev).mul_(3.0))
        batch._slots(ids)
        if k == args.warmup:
            first = (batch._configs.cpu(), logits.cpu())
        kev.record(4 * k, sh)
        batch.apply_mask(ids, logits)
        kev.record(4 * k + 1, sh)
        if k == args.warmup:
            first = first + (logits.cpu(),)
        toks = torch.multinomial(torch.softmax(logits, dim=-1), 1, generator=gen).view(-1)
        kev.record(4 * k + 2, sh)
        status = batch.commit(ids, toks)
        kev.record(4 * k + 3, sh)
    torch.cuda.synchronize()
    wall1 = time.perf_counter()
    timed = range(args.warmup, n_total)
    mask_ms = [kev.elapsed_ms(4 * k, 4 * k + 1) for k in timed]
    commit_ms = [kev.elapsed_ms(4 * k + 2, 4 * k + 3) for k in timed]
    step_ms = statistics.fmean([a + b for a, b in zip(mask_ms, commit_ms)])
    broken = int(batch._broken.sum())
    sat = int((batch._configs[:, 1] != 0).sum())
    out = {
        "metric": "µs/step PDA apply_mask+commit, recursive-JSON grammar, B=256 V=151936 fp32",
        "value": round(step_ms * 1e3, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.pda_steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": False,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config-set PDA mask+commit, recursive JSON GBNF (epsilon-reduced tables)",
                   "batch_rows": B, "vocab": V, "pda_states": g.num_states,
                   "prefix_depths": "uniform 0-8", "logits": "fp32 N(0,3)"},
        "mask_us": round(statistics.fmean(mask_ms) * 1e3, 2),
        "commit_us": round(statistics.fmean(commit_ms) * 1e3, 2),
        "row_vocab_entries_per_s": round(B * V / (step_ms * 1e-3), 1),
        "broken_rows_at_end": broken,
        "saturated_rows_at_end": sat,
        "wall_ms_per_step_incl_setup_work": round((wall1 - wall0) * 1e3 / args.pda_steps, 3),
    }
    if not args.no_cpu and args.pda_cpu_rows:
        from oracle import pda as OP
        from oracle import ref as OR

        t = OP.Table(g)
        cfgs, raw, masked = first
        n = min(args.pda_cpu_rows, B)
        sub = cfgs[:n].numpy().copy()
        lg = raw[:n].numpy().copy()
        # the reference's own apply_mask_pda_batch (pda_cpu.cpp, compiled from
        # its sources into oracle/_ref) where that build is present, else the
        # C restatement
        use_ref = OR.available()
        c0 = time.perf_counter()
        if use_ref:
            OR.pda_apply_mask(t, sub, lg)
        else:
            OP.apply_mask(t, sub, lg)
        cpu_s = time.perf_counter() - c0
        out["cpu_baseline"] = {
            "value": round(cpu_s / n * B * 1e6, 1),
            "unit": "us/step",
            "cores": 1,
            "kind": "reference" if use_ref else "port",
            "sample": (f"mask of {n} rows of the first timed step through "
                       + ("the reference's pda_cpu.cpp apply_mask_pda_batch (oracle/_ref, one thread)"
                          if use_ref else "oracle/pda_oracle.c (C restatement of pda_cpu.cpp, one thread)")
                       + f", scaled to B={B}"),
            "host_cpus": os.cpu_count(),
            "host_cpu_model": _cpu_model(),
        }
        key = "parity_vs_reference_sampled_rows" if use_ref else "parity_vs_oracle_sampled_rows"
        out[key] = bool(np.array_equal(lg, masked[:n].numpy()))
        if use_ref:
            # the same reference call split over host threads by rows, on
            # two rows per thread
            threads = max(1, min(int(os.environ.get("OMP_NUM_THREADS", "16") or 16), os.cpu_count() or 1, 16))
            npar = min(2 * threads, B)
            subp = cfgs[:npar].numpy().copy()
            lgp = raw[:npar].numpy().copy()
            c0 = time.perf_counter()
            OR.pda_apply_mask_threads(t, subp, lgp, threads)
            par_s = time.perf_counter() - c0
            out["cpu_baseline_rows_parallel"] = {
                "value": round(par_s / npar * B * 1e6, 1),
                "unit": "us/step",
                "cores": threads,
                "kind": "reference",
                "sample": (f"mask of {npar} rows of the first timed step through the reference's "
                           f"apply_mask_pda_batch, rows split over {threads} host threads "
                           f"(oracle/_ref), scaled to B={B}"),
                "parity_vs_device": bool(np.array_equal(lgp, masked[:npar].numpy())),
            }
    print(json.dumps(out))
    return 0


def bench_soft(args) -> int:
    """Prior-weighted soft lookahead over the email DFA: B rows at random
    reachable states, fp32 logits N(0, 3), k-step lookahead with the row's
    softmax as the token prior; one step = one in-place rewrite of the
    [B, V] logits."""
    import numpy as np
    import torch

    from bpdecode_amd import ops, synth
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, V, K = args.soft_rows, args.vocab, args.soft_k
    vocab = synth.serving_vocab(V, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    S = fsa.num_states
    states = synth.random_walk_states(fsa.tok_next, fsa.start, fsa.eos_id, B, 40, seed=5).to(torch.int32)
    fd = fsa.to(dev)
    sc = fd.ensure_soft_classes()
    st = states.to(dev)
    src = synth.logits(B, V, std=3.0, dtype=torch.float32, seed=11, device=dev)
    work = torch.empty_like(src)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev) if not args.no_flush else None
    flush64 = flush.view(torch.int64) if flush is not None else None
    sh = torch.cuda.current_stream(dev).cuda_stream
    n_total = args.warmup + args.soft_steps
    kev = HipEvents(2 * n_total)
    for k in range(n_total):
        work.copy_(src)
        if flush64 is not None:
            flush64.sum()
        kev.record(2 * k, sh)
        ops.apply_soft_prior_(work, fd, st, K, 1.0)
        kev.record(2 * k + 1, sh)
    torch.cuda.synchronize()
    times = [kev.elapsed_ms(2 * k, 2 * k + 1) for k in range(args.warmup, n_total)]
    step_ms = statistics.fmean(times)
    U = int(torch.unique(states[states >= 0]).numel())
    members = int(sc.class_tok.numel())
    # algorithmic bytes of one step: the stats kernel reads the logits and
    # gathers the class members' logits; the output kernel reads the logits
    # and the token -> class map and writes the logits
    d_bytes = 3 * B * V * 4 + B * members * 4 + V * 4
    out = {
        "metric": "µs/step prior-weighted soft lookahead (k=4), email DFA, B=128 V=151936 fp32",
        "value": round(step_ms * 1e3, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.soft_steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": False,
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "soft lookahead with the row softmax as token prior, email DFA",
                   "batch_rows": B, "vocab": V, "k": K, "dfa_states": S,
                   "token_classes": sc.num_classes, "class_members": members,
                   "distinct_row_states": U, "logits": "fp32 N(0,3)"},
        "roofline": {"bound": "hbm", "achieved": round(d_bytes / (step_ms * 1e-3) / 1e9, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(d_bytes / (step_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": None, "scope": "whole step (3 kernels)",
                     "algorithmic_bytes": d_bytes},
        "row_vocab_entries_per_s": round(B * V / (step_ms * 1e-3), 1),
    }
    if not args.no_cpu and args.soft_cpu_rows:
        from oracle import soft as OS

        n = min(args.soft_cpu_rows, B)
        x = src[:n].double().cpu().numpy()
        tn = fsa.tok_next.numpy()
        c0 = time.perf_counter()
        want = OS.prior_lookahead(x, tn, fsa.live.numpy(), fsa.accept.numpy(), fsa.eos_id,
                                  states[:n].numpy(), K, 1.0)
        cpu_s = time.perf_counter() - c0
        got = work[:n].double().cpu().numpy()
        fin = np.isfinite(want)
        ok = np.array_equal(np.isneginf(got), np.isneginf(want)) and bool(
            np.all(np.abs(got[fin] - want[fin]) <= 1e-5 * np.abs(want[fin]) + 1e-5))
        out["cpu_baseline"] = {
            "value": round(cpu_s / n * B * 1e6, 1),
            "unit": "us/step",
            "cores": 1,
            "kind": "port",
            "sample": f"{n} rows through oracle/soft.py prior_lookahead (float64 numpy, dense "
                      f"[S, V] gathers per round), scaled to B={B}",
            "host_cpus": os.cpu_count(),
            "host_cpu_model": _cpu_model(),
        }
        out["parity_vs_oracle_sampled_rows"] = ok
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

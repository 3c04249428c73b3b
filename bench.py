"""Benchmark of the batched constraint step on one MI355X.

One JSON line.  The headline is the dense step at serving scale: the email
regex ``[a-z0-9._]{1,32}@[a-z0-9-]{1,24}\\.(com|org|net|io)`` compiled to a
byte DFA over a seeded synthetic vocabulary of V = 151,936 tokens; B = 256
rows; bf16 logits N(0, 3); continuous batching that evicts 10 % of the rows
and adds as many fresh ones every step; tokens sampled from the masked
softmax.  One step = ``ConstraintBatch.apply_mask`` + ``ConstraintBatch.commit``.
Nested objects carry the other workloads, each with its own roofline, CPU
baseline and parity flag: ``pda`` (recursive-JSON config-set PDA, B = 256,
fp32), ``soft`` (prior-weighted lookahead, k = 4, B = 128, fp32) and
``schema`` (flat JSON-Schema document DFA, B = 512, bf16, from random valid
partial documents of 0-80 bytes).

Timing.  Every step starts from cold caches: a 512 MB buffer is read before
it (no dirty lines left behind), so logits and tables come from HBM.  HIP
events created with hipEventDisableSystemFence are recorded on the stream the
kernels run on.  The dense step runs its trajectory three times with the same
logits, churn and tokens:

* record pass -- ``apply_mask`` and ``commit`` each in their own bracket, the
  sampling between them (``mask_us``, ``commit_us``, ``two_bracket_us``);
* kernel pass (``value``) -- the slot list and queued churn writes staged by
  ``ConstraintBatch.prepare`` before the bracket, then ``apply_mask`` and
  ``commit`` (with the token recorded for that step) in ONE bracket: the work
  of the constraint step and nothing else, without a second bracket's fixed
  cost (an empty kernel between two events measures 6.2 us against 3.8 us in
  the kernel trace);
* API pass -- the same single bracket with the slot/churn upload inside it
  (``api_us_per_step``), plus the host time of the two Python calls.

The passes must agree: the kernel and API passes commit the same states as
the record pass, step by step.

Roofline (HBM, 8 TB/s peak).  Dense step: ``D = B*V*2e + U*V*4 + 16*B`` (read
and write of every logit, one int32 tok_next row per distinct live state U of
the step, commit state/token/lookup/write), divided by the step time; the
mask kernel's own fraction (``D - 16*B`` over the record pass's mask bracket)
is reported beside it.  PDA: ``B*V*8 + B*1064*2 + sum(token bytes)``
(diagnostic; the walk is not bandwidth-bound).  Soft: ``B*V*4*2 + S*V*4``.

CPU baselines run on the host cores of the same box over bounded samples
(stated in each ``sample``).  ``--gpus N`` with N > 1 is refused: this build
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
METRIC = "µs/step apply_mask+commit & GB/s (% HBM roofline), B=256 V=151936 bf16"


class HipEvents:
    """HIP events created with hipEventDisableSystemFence, recorded on a given
    stream: the bracket then holds no system-scope cache release, so it times
    the kernels between the markers (torch's timing events carry one)."""

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

    def destroy(self) -> None:
        for h in self.ev:
            self.hip.hipEventDestroy(h)
        self.ev = []


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


def _roofline(d_bytes: float, seconds: float, **extra) -> dict:
    gbs = d_bytes / seconds / 1e9
    out = {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
           "frac": round(gbs / PEAK_HBM_GBS, 4)}
    out.update(extra)
    return out


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128, help="timed steps of the dense headline")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--batch", type=int, default=256)
    p.add_argument("--vocab", type=int, default=151_936)
    p.add_argument("--churn", type=float, default=0.10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--cpu-steps", type=int, default=8, help="recorded dense steps replayed on the CPU")
    p.add_argument("--cpu-repeats", type=int, default=3)
    p.add_argument("--no-flush", action="store_true", help="keep caches warm between steps")
    p.add_argument("--workload", choices=["all", "dense", "pda", "soft", "schema", "regex"], default="all",
                   help="all (default): the dense headline with pda, soft and schema nested; or one "
                        "workload alone")
    p.add_argument("--regex-steps", type=int, default=64)
    p.add_argument("--schema-rows", type=int, default=512)
    p.add_argument("--schema-steps", type=int, default=64)
    p.add_argument("--pda-rows", type=int, default=256)
    p.add_argument("--pda-steps", type=int, default=64)
    p.add_argument("--pda-cpu-rows", type=int, default=32,
                   help="rows of one step replayed on one CPU thread (all rows run over the host threads)")
    p.add_argument("--soft-rows", type=int, default=128)
    p.add_argument("--soft-k", type=int, default=4)
    p.add_argument("--soft-steps", type=int, default=64)
    p.add_argument("--soft-cpu-rows", type=int, default=8,
                   help="rows timed through the fp32 torch CPU restatement")
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
    import torch

    torch.cuda.set_device(0)
    if args.workload == "pda":
        out = bench_pda(args)
    elif args.workload == "soft":
        out = bench_soft(args)
    elif args.workload == "schema":
        out = bench_schema(args)
    elif args.workload == "regex":
        out = bench_regex(args)
    else:
        out = bench_dense(args)
        if args.workload == "all":
            for name, fn in (("pda", bench_pda), ("soft", bench_soft), ("schema", bench_schema),
                             ("regex_cpu", bench_regex)):
                print(f"[bench] {name}", file=sys.stderr, flush=True)
                out[name] = fn(args)
    print(json.dumps(out))
    return 0


# ------------------------------------------------------------------ dense --
class DenseRun:
    """One pass over a dense trajectory: a fresh batch at the same starting
    rows, the same logits (seeded device generator), the same churn (seeded
    host generator) and -- after the record pass -- the same tokens."""

    def __init__(self, fsa, B: int, V: int, dtype, churn: float, starts, seed: int) -> None:
        import numpy as np
        import torch

        from bpdecode_amd.batch import ConstraintBatch

        self.B, self.V, self.dtype, self.churn = B, V, dtype, churn
        self.dev = fsa.device
        self.batch = ConstraintBatch(fsa, capacity=2 * B, device=self.dev)
        self.active = []
        for i in range(B):
            self.batch.add(i)
            self.active.append(i)
        self.next_id = B
        if starts is not None:
            self.batch._state[:B] = starts.to(self.dev)
        self.rng = np.random.default_rng(seed)
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(seed + 1)
        self.logits = torch.empty((B, V), dtype=dtype, device=self.dev)

    def next_logits(self) -> None:
        import torch

        self.logits.copy_(torch.randn((self.B, self.V), generator=self.gen, device=self.dev).mul_(3.0))

    def states_now(self, ids):
        """The rows' states as the next launch will read them (pool plus
        queued writes), on the host; outside the timed region."""
        import numpy as np

        b = self.batch
        pool = b._pool.cpu().numpy()
        for q in (b._staged_pending, b._pending):
            for slot, v in q.items():
                pool[slot] = v
        return pool[np.array([b._slot_of[i] for i in ids], dtype=np.int64)]

    def churn_step(self) -> None:
        n = int(round(self.churn * self.B))
        for i in self.rng.choice(len(self.active), size=n, replace=False).tolist():
            self.batch.evict(self.active[i])
            self.active[i] = self.next_id
            self.batch.add(self.next_id)
            self.next_id += 1


def _line_bytes_per_state(fsa, e: int):
    """Per state (index S: a negative state), the bytes the memory side
    moves for one row's mask at 128-byte line granularity: a line whose
    elements are all rejected is written (128 B), a line mixing kept and
    rejected elements is read and written back (256 B: the partial write is
    merged below the caches), a line of kept elements is not touched."""
    import numpy as np

    bits = fsa.ensure_allow_bits().cpu().numpy().view(np.uint32)
    S, W = bits.shape
    V = fsa.vocab_size
    per = 128 // e  # elements per line
    allowed = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little")[:, :V]
    pad = (-V) % per
    if pad:
        allowed = np.concatenate([allowed, np.ones((S, pad), np.uint8)], axis=1)
    counts = allowed.reshape(S, -1, per).sum(axis=2, dtype=np.int32)
    full_rej = (counts == 0).sum(axis=1)
    mixed = ((counts > 0) & (counts < per)).sum(axis=1)
    out = full_rej * 128 + mixed * 256
    lines = -(-V // per)
    return np.concatenate([out, [lines * 128]]).astype(np.float64)


def _write_bytes_per_state(fsa, e: int, gran: int):
    """Per state (index S: a negative state), the bytes of one row's logits
    that lie in ``gran``-byte segments holding at least one rejected element
    -- what the mask kernel's stores dirty at that granularity, for
    comparison with the WRITE_SIZE counter."""
    import numpy as np

    bits = fsa.ensure_allow_bits().cpu().numpy().view(np.uint32)
    S, W = bits.shape
    V = fsa.vocab_size
    per = gran // e
    allowed = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little")[:, :V]
    pad = (-V) % per
    if pad:
        allowed = np.concatenate([allowed, np.ones((S, pad), np.uint8)], axis=1)
    dirty = (allowed.reshape(S, -1, per).sum(axis=2, dtype=np.int32) < per).sum(axis=1) * gran
    return np.concatenate([dirty, [-(-V // per) * gran]]).astype(np.float64)


def _dense_trajectory(args, fsa, B, V, dtype, churn, starts, seed, steps, warmup, record_cpu=0):
    """The three passes of the dense step over one trajectory.  Returns the
    timings (ms lists over the timed steps), the distinct live states per
    timed step, the host API times, the parity of the passes and the steps
    recorded for the CPU baseline."""
    import numpy as np
    import torch

    n_total = warmup + steps
    flush64 = None
    if not args.no_flush:
        flush64 = torch.zeros(512 << 20, dtype=torch.uint8, device=fsa.device).view(torch.int64)
    sh = torch.cuda.current_stream(fsa.device).cuda_stream
    tokens, distinct, recorded, nxt_ref, line_bytes = [], [], [], [], []
    esize = torch.tensor([], dtype=dtype).element_size()
    per_state = _line_bytes_per_state(fsa, esize)
    dirty_tab = {g: _write_bytes_per_state(fsa, esize, g) for g in (32, 64, 128)}
    dirty = {g: [] for g in dirty_tab}

    # record pass: two brackets, sampling between them
    run = DenseRun(fsa, B, V, dtype, churn, starts, seed)
    sgen = torch.Generator(device=fsa.device)
    sgen.manual_seed(seed + 2)
    ev = HipEvents(4 * n_total)
    for k in range(n_total):
        ids = list(run.active)
        run.next_logits()
        st = run.states_now(ids)
        live = st[st >= 0]
        distinct.append(int(np.unique(live).size))
        row_idx = np.where(st >= 0, st, len(per_state) - 1)
        line_bytes.append(float(per_state[row_idx].sum()))
        for g, tab in dirty_tab.items():
            dirty[g].append(float(tab[row_idx].sum()))
        keep = k >= warmup and len(recorded) < record_cpu
        if keep:
            raw = run.logits.cpu()
        run.batch.prepare(ids)
        if flush64 is not None:
            flush64.sum()
        ev.record(4 * k, sh)
        run.batch.apply_mask(ids, run.logits)
        ev.record(4 * k + 1, sh)
        toks = torch.multinomial(torch.softmax(run.logits.float(), dim=-1), 1, generator=sgen).view(-1)
        ev.record(4 * k + 2, sh)
        nxt = run.batch.commit(ids, toks)
        ev.record(4 * k + 3, sh)
        tokens.append(toks)
        nxt_ref.append(nxt)
        if keep:
            recorded.append((raw, st.copy(), toks.cpu().numpy(), run.logits.cpu()))
        run.churn_step()
    torch.cuda.synchronize()
    timed = range(warmup, n_total)
    mask_ms = [ev.elapsed_ms(4 * k, 4 * k + 1) for k in timed]
    commit_ms = [ev.elapsed_ms(4 * k + 2, 4 * k + 3) for k in timed]
    ev.destroy()
    pool_ref = run.batch._state.cpu()

    # kernel pass (staged upload) and API pass (upload inside the bracket)
    res = {"mask_ms": mask_ms, "commit_ms": commit_ms}
    parity = True
    for mode in ("kernel", "api"):
        run = DenseRun(fsa, B, V, dtype, churn, starts, seed)
        ev = HipEvents(2 * n_total)
        host_s = []
        agree = torch.ones((), dtype=torch.bool, device=fsa.device)
        for k in range(n_total):
            ids = list(run.active)
            run.next_logits()
            if mode == "kernel":
                run.batch.prepare(ids)
            if flush64 is not None:
                flush64.sum()
            ev.record(2 * k, sh)
            h0 = time.perf_counter()
            run.batch.apply_mask(ids, run.logits)
            nxt = run.batch.commit(ids, tokens[k])
            host_s.append(time.perf_counter() - h0)  # the two calls only, not the event records
            ev.record(2 * k + 1, sh)
            agree &= (nxt == nxt_ref[k]).all()
            run.churn_step()
            if mode == "api":
                # a serving loop waits for each step's tokens; without this the
                # host runs ~100 steps ahead, the hardware queue fills and the
                # launches inside the calls wait for the device
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        res[f"{mode}_ms"] = [ev.elapsed_ms(2 * k, 2 * k + 1) for k in timed]
        res[f"{mode}_host_s"] = host_s[warmup:]
        ev.destroy()
        parity &= bool(agree.item()) and torch.equal(run.batch._state.cpu(), pool_ref)
    res["distinct"] = distinct[warmup:]
    res["line_bytes"] = line_bytes[warmup:]
    res["dirty_bytes"] = {g: v[warmup:] for g, v in dirty.items()}
    res["passes_agree"] = parity
    res["recorded"] = recorded
    res["committed"] = torch.cat(nxt_ref).cpu()  # every step's committed states, in order
    return res


def bench_dense(args) -> dict:
    import numpy as np
    import torch

    from bpdecode_amd import synth
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    B, V = args.batch, args.vocab
    t0 = time.perf_counter()
    vocab = synth.serving_vocab(V, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab, dense=False).to(dev).densify()
    fsa.ensure_allow_bits()
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    S, e = fsa.num_states, 2
    n_cpu = 0 if args.no_cpu else min(args.cpu_steps, args.steps)
    r = _dense_trajectory(args, fsa, B, V, torch.bfloat16, args.churn, None, 2, args.steps,
                          args.warmup, record_cpu=n_cpu)
    U = r["distinct"]
    d_step = [B * V * 2 * e + u * V * 4 + 16 * B for u in U]
    d_mask = [B * V * 2 * e + u * V * 4 for u in U]
    t_step = statistics.fmean(r["kernel_ms"])
    t_mask = statistics.fmean(r["mask_ms"])
    two = [a + b for a, b in zip(r["mask_ms"], r["commit_ms"])]
    traffic = _profiled_traffic("dense_fill_email_b256_v151936.traffic.json", "dense_fill_kernel<2, true>")
    out = {
        "metric": METRIC,
        "value": round(t_step * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step, 5),
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
        "median_us_per_step": round(statistics.median(r["kernel_ms"]) * 1e3, 3),
        "timing": ("fence-free HIP events on the kernels' stream, one bracket per step around "
                   "ConstraintBatch.apply_mask + .commit (slot upload staged by prepare(); tokens "
                   "recorded from the masked softmax in the record pass)"),
        "mask_us": round(t_mask * 1e3, 3),
        "commit_us": round(statistics.fmean(r["commit_ms"]) * 1e3, 3),
        "two_bracket_us": round(statistics.fmean(two) * 1e3, 3),
        "api_us_per_step": round(statistics.fmean(r["api_ms"]) * 1e3, 3),
        "api_host_us_per_step": round(statistics.fmean(r["api_host_s"]) * 1e6, 2),
        "api_host_us_per_step_median": round(statistics.median(r["api_host_s"]) * 1e6, 2),
        "row_vocab_entries_per_s": round(B * V / (t_step * 1e-3), 1),
        "distinct_live_states_mean": round(statistics.fmean(U), 2),
        "setup_s": round(setup_s, 3),
        "passes_agree": r["passes_agree"],
        "roofline": _roofline(
            sum(d_step) / len(d_step), t_step * 1e-3,
            traffic=traffic,
            scope="apply_mask + commit step (one event bracket)",
            algorithmic_bytes_per_step_mean=round(statistics.fmean(d_step), 1),
            table_charged_as="int32 tok_next rows (the kernel reads the packed allow-bit table)",
            kernel="dense_fill_kernel<2, true>",
            mask_kernel=_roofline(sum(d_mask) / len(d_mask), t_mask * 1e-3,
                                  scope="mask launch alone (record pass bracket)",
                                  duration_us=round(t_mask * 1e3, 3)),
            two_bracket_frac=round(statistics.fmean(d_step) / (statistics.fmean(two) * 1e-3) / 1e9
                                   / PEAK_HBM_GBS, 4),
            memory_side=_memory_side(r, U, B, V, t_step),
        ),
    }
    if r["recorded"]:
        out["cpu_baseline"], out["parity_vs_oracle"] = _dense_cpu_baseline(args, fsa, r["recorded"], B, V)
    return out


def _memory_side(r, U, B, V, t_step_ms) -> dict:
    """The bytes the memory system moves for the step at 128-byte line
    granularity (see _line_bytes_per_state), plus the allow-bit rows read
    (V/8 per distinct state) and the commit's 16 B per row."""
    b = [lb + u * V / 8 + 16 * B for lb, u in zip(r["line_bytes"], U)]
    out = _roofline(statistics.fmean(b), t_step_ms * 1e-3)
    out["bytes_per_step_mean"] = round(statistics.fmean(b), 1)
    out["basis"] = ("per 128-byte line of logits: all rejected = one write, kept and rejected mixed "
                    "= read + write (merged below the caches), all kept = nothing; plus the allow-bit "
                    "rows and the commit")
    return out


def _dense_cpu_baseline(args, fsa, recorded, B, V):
    """The reference's CPU step is ATen: ops.py:271-276 (mask) and
    ops.py:301-306 (commit), timed here op for op on CPU tensors with torch's
    host threads; the numpy oracle checks the GPU's masks of the same steps."""
    import numpy as np
    import torch

    from oracle import dense as OD

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
    base = {
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
    return base, parity


# ------------------------------------------------------------------ regex --
def _aten_dense_step(tok_next, states, logits, tokens):
    """The reference's dense step as it is written in ATen (ops.py:271-276
    mask, ops.py:301-306 commit), on whatever device the tensors are on."""
    import torch

    s = states.long()
    rejected = tok_next.index_select(0, s.clamp(min=0)) == -1
    rejected |= (s < 0).unsqueeze(1)
    logits.masked_fill_(rejected, float("-inf"))
    nxt = tok_next[s.clamp(min=0), tokens.long()]
    return torch.where(s < 0, torch.full_like(nxt, -1), nxt).to(torch.int32)


def bench_regex(args) -> dict:
    """The regex dense-DFA path on the CPU: ([0-9]{1,3}\.){3}[0-9]{1,3} over
    a seeded V = 32,000 vocabulary, B = 8 rows from random valid prefixes,
    fp32 logits N(0, 1), 64 steps of apply_mask then commit with the token
    sampled from the masked softmax.  The value is the library's host path
    (ConstraintBatch on CPU tensors -> bpd_host_dense_*); the reference's
    ATen op sequence runs the same steps beside it (its CPU path), and the
    device path the same trajectory on the GPU."""
    import numpy as np
    import torch

    from bpdecode_amd import synth
    from bpdecode_amd.batch import ConstraintBatch
    from bpdecode_amd.ops import FsaTensors

    B, V, steps, warm = 8, 32_000, args.regex_steps, args.warmup
    vocab = synth.ipv4_vocab(V, seed=0)
    fsa = FsaTensors.build(synth.IPV4, vocab)
    starts = synth.random_walk_states(fsa.tok_next, fsa.start, vocab.eos_id, B, 3, seed=0)
    n_total = warm + steps
    logits = [synth.logits(B, V, 1.0, torch.float32, seed=300 + k) for k in range(n_total)]
    gen = torch.Generator().manual_seed(3)
    ids = list(range(B))

    # the library's host path, tokens sampled from its masks
    batch = ConstraintBatch(fsa, capacity=B)
    for i in ids:
        batch.add(i)
    batch._state[:B] = starts
    host_s, tokens, masks, committed = [], [], [], []
    for k in range(n_total):
        x = logits[k].clone()
        c0 = time.perf_counter()
        batch.apply_mask(ids, x)
        t_mask = time.perf_counter() - c0
        tok = torch.multinomial(torch.softmax(x, dim=-1), 1, generator=gen).view(-1)
        c0 = time.perf_counter()
        nxt = batch.commit(ids, tok)
        host_s.append(t_mask + time.perf_counter() - c0)
        tokens.append(tok)
        masks.append(x)
        committed.append(nxt.clone())

    # the reference's ATen sequence on the same inputs
    tn = fsa.tok_next
    st = starts.clone().to(torch.int32)
    aten_s, agree = [], True
    for k in range(n_total):
        x = logits[k].clone()
        c0 = time.perf_counter()
        nxt = _aten_dense_step(tn, st, x, tokens[k])
        aten_s.append(time.perf_counter() - c0)
        agree &= torch.equal(x, masks[k]) and torch.equal(nxt, committed[k])
        st = nxt

    dev_us = None
    if torch.cuda.is_available():
        dev_us, dev_agree = _regex_device(fsa, starts, logits, tokens, masks, committed, ids, warm)
        agree &= dev_agree
    host_us = statistics.fmean(host_s[warm:]) * 1e6
    aten_us = statistics.fmean(aten_s[warm:]) * 1e6
    return _regex_line(args, fsa, B, V, steps, host_s[warm:], host_us, aten_us, dev_us, agree)


def _regex_device(fsa, starts, logits, tokens, masks, committed, ids, warm):
    """The device path on the regex trajectory: (mean µs/step, agreement)."""
    import torch

    from bpdecode_amd.batch import ConstraintBatch

    B, n_total = len(ids), len(logits)
    dev = torch.device("cuda:0")
    dbatch = ConstraintBatch(fsa, capacity=B, device=dev)
    for i in ids:
        dbatch.add(i)
    dbatch._state[:B] = starts.to(dev)
    sh = torch.cuda.current_stream(dev).cuda_stream
    ev = HipEvents(2 * n_total)
    dev_logits = [x.to(dev) for x in logits]
    dev_tokens = [t.to(dev) for t in tokens]
    dev_next = []
    for k in range(n_total):
        dbatch.prepare(ids)
        ev.record(2 * k, sh)
        dbatch.apply_mask(ids, dev_logits[k])
        dev_next.append(dbatch.commit(ids, dev_tokens[k]))
        ev.record(2 * k + 1, sh)
    torch.cuda.synchronize()
    dev_ms = [ev.elapsed_ms(2 * k, 2 * k + 1) for k in range(warm, n_total)]
    ev.destroy()
    agree = all(torch.equal(dev_logits[k].cpu(), masks[k]) and torch.equal(dev_next[k].cpu(), committed[k])
                for k in range(n_total))
    return statistics.fmean(dev_ms) * 1e3, agree


def _regex_line(args, fsa, B, V, steps, host_s, host_us, aten_us, dev_us, agree) -> dict:
    import torch

    return {
        "metric": "µs/step apply_mask+commit on the CPU, IPv4 regex DFA, B=8 V=32000 fp32",
        "value": round(host_us, 2),
        "unit": "us/step",
        "steps": steps,
        "dtype": "fp32",
        "config": {"workload": "regex dense-DFA path on the CPU (library host entry points via "
                               "ConstraintBatch on CPU tensors)",
                   "batch_rows": B, "vocab": V, "dfa_states": fsa.num_states, "logits": "fp32 N(0,1)"},
        "median_us_per_step": round(statistics.median(host_s) * 1e6, 2),
        "us_per_token_per_sequence": round(host_us / B, 2),
        "cores": 1,
        "cpu_baseline": {
            "value": round(aten_us, 2),
            "unit": "us/step",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"the same {steps} steps through the reference's ATen op sequence "
                       "(ops.py:271-276 mask, ops.py:301-306 commit) on CPU tensors"),
            "us_per_token_per_sequence": round(aten_us / B, 2),
            "host_cpus": os.cpu_count(),
            "host_cpu_model": _cpu_model(),
        },
        "device_us_per_step": None if dev_us is None else round(dev_us, 3),
        "reference_published_cpu_us_per_token_per_sequence": {
            "value": 92, "hardware": "Apple M-series CPU, batch 8, V=151,643 (Qwen2.5 tokenizer)",
            "source": "bench/RESULTS.md:38-46 (ipv4)"},
        "parity_host_aten_device_every_step": bool(agree),
    }


# ----------------------------------------------------------------- schema --
def bench_schema(args) -> dict:
    """Flat JSON-Schema document DFA (826 states) over the serving vocab, B
    rows from random valid partial documents of 0-80 bytes, bf16 logits
    N(0, 3), no churn.  Three bundles of the same grammar on the same
    inputs: forced dense (the value: tok_next and its allow-bit table), the
    default ``auto`` bundle (S * V is above the density limit, so no
    tok_next: the allow-bit table built from trans, the fused walking
    commit) and the symbol-class walking kernels alone; all three commit the
    same states step for step."""
    import torch

    from bpdecode_amd import ops, synth
    from bpdecode_amd.batch import ConstraintBatch, build_bundle
    from bpdecode_amd.grammar.json_schema import json_schema_to_grammar
    from bpdecode_amd.grammar.pda import CompiledGrammar
    from bpdecode_amd.grammar.regular import residual_dfa
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    B, V = args.schema_rows, args.vocab
    steps = min(args.schema_steps, args.steps)
    vocab = synth.serving_vocab(V, seed=1)
    comp = CompiledGrammar.build(json_schema_to_grammar(synth.FLAT_SCHEMA))
    dfa = residual_dfa(comp, comp.root, comp.rules[comp.root].start)
    plain = FsaTensors.build(dfa, vocab, dense=False).to(dev)
    dense = plain.densify()
    dense.ensure_allow_bits()
    starts = synth.random_byte_walk_states(dense.tok_next, plain.start, B, 80, seed=4)
    r = _dense_trajectory(args, dense, B, V, torch.bfloat16, 0.0, starts, 6, steps, args.warmup)
    U = r["distinct"]
    d_step = [B * V * 2 * 2 + u * V * 4 + 16 * B for u in U]
    t_step = statistics.fmean(r["kernel_ms"])

    # the default auto bundle: no tok_next, allow bits built from trans
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    auto = build_bundle(dfa, vocab, dev)
    auto.ensure_allow_bits()
    torch.cuda.synchronize()
    auto_setup_s = time.perf_counter() - t0
    assert auto.tok_next is None
    ra = _dense_trajectory(args, auto, B, V, torch.bfloat16, 0.0, starts, 6, steps, args.warmup)
    t_auto = statistics.fmean(ra["kernel_ms"])
    auto_agree = bool(torch.equal(ra["committed"], r["committed"])) and ra["passes_agree"]

    # the walking kernels alone (no allow-bit table) on the same logits and tokens
    sh = torch.cuda.current_stream(dev).cuda_stream
    limit, ops.ALLOW_BITS_LIMIT = ops.ALLOW_BITS_LIMIT, 0
    try:
        walk = ConstraintBatch(plain, capacity=B, device=dev)
    finally:
        ops.ALLOW_BITS_LIMIT = limit
    assert not walk._fast
    ref = ConstraintBatch(dense, capacity=B, device=dev)
    for bt in (walk, ref):
        for i in range(B):
            bt.add(i)
        bt._state[:B] = starts.to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    ids = list(range(B))
    n_total = args.warmup + steps
    ev = HipEvents(2 * n_total)
    flush64 = torch.zeros(512 << 20, dtype=torch.uint8, device=dev).view(torch.int64)
    lw = torch.empty((B, V), dtype=torch.bfloat16, device=dev)
    ld = torch.empty_like(lw)
    agree = True
    for k in range(n_total):
        lw.copy_(torch.randn((B, V), generator=gen, device=dev).mul_(3.0))
        ld.copy_(lw)
        ref.apply_mask(ids, ld)
        toks = torch.multinomial(torch.softmax(ld.float(), dim=-1), 1, generator=gen).view(-1)
        n_ref = ref.commit(ids, toks)
        walk.prepare(ids)
        if not args.no_flush:
            flush64.sum()
        ev.record(2 * k, sh)
        walk.apply_mask(ids, lw)
        n_walk = walk.commit(ids, toks)
        ev.record(2 * k + 1, sh)
        agree &= bool(torch.equal(lw.view(torch.int16), ld.view(torch.int16))) and bool(torch.equal(n_ref, n_walk))
    torch.cuda.synchronize()
    walk_ms = [ev.elapsed_ms(2 * k, 2 * k + 1) for k in range(args.warmup, n_total)]
    ev.destroy()
    side = _memory_side(r, U, B, V, t_step)
    side["written_bytes_per_mask_by_granularity"] = {
        f"{g}B": round(statistics.fmean(v), 1) for g, v in r["dirty_bytes"].items()}
    traffic = _profiled_traffic("dense_fill_schema_b512_v151936.traffic.json", "dense_fill_kernel<2, true>")
    roof = _roofline(side["bytes_per_step_mean"], t_step * 1e-3, traffic=traffic,
                     scope="apply_mask + commit step (one event bracket)",
                     bytes_basis=side["basis"],
                     written_bytes_per_mask_by_granularity=side["written_bytes_per_mask_by_granularity"],
                     algorithmic_bytes_per_step_mean=side["bytes_per_step_mean"],
                     kernel="dense_fill_kernel<2, true>",
                     mask_kernel=_roofline(statistics.fmean(r["line_bytes"]) + statistics.fmean(U) * V / 8,
                                           statistics.fmean(r["mask_ms"]) * 1e-3,
                                           scope="mask launch alone (record pass bracket)",
                                           duration_us=round(statistics.fmean(r["mask_ms"]) * 1e3, 3)),
                     survey_formula={"bytes_per_step_mean": round(statistics.fmean(d_step), 1),
                                     "formula": "B*V*2e + U*V*4 + 16*B",
                                     "frac": round(statistics.fmean(d_step) / (t_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                                     "note": ("charges a read of every logit besides its write; the "
                                              "mask kernel reads no logit (FETCH_SIZE: the allow-bit "
                                              "rows and states) and writes the segments holding "
                                              "rejected ones, so this figure exceeds the peak and is "
                                              "not a measure of this kernel")})
    return {
        "metric": "µs/step apply_mask+commit, flat JSON-Schema DFA, B=512 V=151936 bf16",
        "value": round(t_step * 1e3, 3),
        "unit": "us/step",
        "steps": steps,
        "dtype": "bf16",
        "config": {"workload": "dense tok_next apply_mask+commit, flat JSON-Schema document DFA, "
                               "starting rows = random valid partial documents of 0-80 bytes",
                   "batch_rows": B, "vocab": V, "dfa_states": plain.num_states,
                   "symbol_classes": plain.num_symbols, "logits": "bf16 N(0,3)",
                   "bundle": "forced dense (tok_next + allow-bit table)"},
        "mask_us": round(statistics.fmean(r["mask_ms"]) * 1e3, 3),
        "commit_us": round(statistics.fmean(r["commit_ms"]) * 1e3, 3),
        "api_us_per_step": round(statistics.fmean(r["api_ms"]) * 1e3, 3),
        "auto_bundle": {
            "bundle": "GrammarCache default (dense='auto'): no tok_next; allow-bit table built "
                      "from trans on the device, dense fill mask, fused walking commit",
            "us_per_step": round(t_auto * 1e3, 3),
            "mask_us": round(statistics.fmean(ra["mask_ms"]) * 1e3, 3),
            "commit_us": round(statistics.fmean(ra["commit_ms"]) * 1e3, 3),
            "api_us_per_step": round(statistics.fmean(ra["api_ms"]) * 1e3, 3),
            "setup_s": round(auto_setup_s, 4),
            "table_bytes": int(auto.allow_bits.numel() * 4),
            "same_states_as_dense_every_step": auto_agree,
        },
        "walking_kernel_us_per_step": round(statistics.fmean(walk_ms) * 1e3, 3),
        "distinct_live_states_mean": round(statistics.fmean(U), 2),
        "row_vocab_entries_per_s": round(B * V / (t_step * 1e-3), 1),
        "roofline": roof,
        "passes_agree": r["passes_agree"],
        "parity_dense_vs_walking_kernel_every_step": agree,
    }


# -------------------------------------------------------------------- pda --
def bench_pda(args) -> dict:
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
    B, V = args.pda_rows, args.vocab
    steps = min(args.pda_steps, args.steps)
    vocab = synth.serving_vocab(V, seed=1)
    comp = CompiledGrammar.build(parse_gbnf(synth.JSON_GBNF))
    g = build_pda_tensors(comp, vocab, eps_reduce=True)
    rng = np.random.default_rng(5)
    rows = []
    while len(rows) < B:
        d = int(rng.integers(0, 9))
        c = g.init_config()
        if g.feed(c, synth.json_prefix(rng, d)):
            rows.append(c)
    start = torch.stack(rows)
    batch = CFGConstraintBatch(g, capacity=B, device=dev)
    ids = list(range(B))
    for i in ids:
        batch.add(i)
    batch._configs.copy_(start.to(dev))
    sh = torch.cuda.current_stream(dev).cuda_stream
    n_total = args.warmup + steps
    kev = HipEvents(4 * n_total)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    logits = torch.empty((B, V), dtype=torch.float32, device=dev)
    flush64 = None if args.no_flush else torch.zeros(512 << 20, dtype=torch.uint8, device=dev).view(torch.int64)
    first = None
    for k in range(n_total):
        logits.copy_(torch.randn((B, V), generator=gen, device=dev).mul_(3.0))
        batch._slots(ids)
        if k == args.warmup:
            first = (batch._configs.cpu(), logits.cpu())
        if flush64 is not None:
            flush64.sum()
        kev.record(4 * k, sh)
        batch.apply_mask(ids, logits)
        kev.record(4 * k + 1, sh)
        if k == args.warmup:
            first = first + (logits.cpu(),)
        toks = torch.multinomial(torch.softmax(logits, dim=-1), 1, generator=gen).view(-1)
        kev.record(4 * k + 2, sh)
        batch.commit(ids, toks)
        kev.record(4 * k + 3, sh)
        if k == args.warmup:
            first = first + (toks.cpu(), batch._configs.cpu())
    torch.cuda.synchronize()
    timed = range(args.warmup, n_total)
    mask_ms = [kev.elapsed_ms(4 * k, 4 * k + 1) for k in timed]
    commit_ms = [kev.elapsed_ms(4 * k + 2, 4 * k + 3) for k in timed]
    kev.destroy()
    step_ms = statistics.fmean([a + b for a, b in zip(mask_ms, commit_ms)])
    tok_bytes = int(g.tok_bytes.numel())
    d_bytes = B * V * 8 + B * 1064 * 2 + tok_bytes
    out = {
        "metric": "µs/step PDA apply_mask+commit, recursive-JSON grammar, B=256 V=151936 fp32",
        "value": round(step_ms * 1e3, 2),
        "unit": "us/step",
        "steps": steps,
        "dtype": "fp32",
        "config": {"workload": "config-set PDA mask+commit, recursive JSON GBNF (epsilon-reduced tables)",
                   "batch_rows": B, "vocab": V, "pda_states": g.num_states,
                   "prefix_depths": "uniform 0-8", "logits": "fp32 N(0,3)"},
        "mask_us": round(statistics.fmean(mask_ms) * 1e3, 2),
        "commit_us": round(statistics.fmean(commit_ms) * 1e3, 2),
        "row_vocab_entries_per_s": round(B * V / (step_ms * 1e-3), 1),
        "broken_rows_at_end": int(batch._broken.sum()),
        "saturated_rows_at_end": int((batch._configs[:, 1] != 0).sum()),
        "roofline": _roofline(d_bytes, step_ms * 1e-3, traffic=None,
                              scope="mask + commit step; diagnostic only (the walk is bound by its "
                                    "instructions, not by HBM)",
                              algorithmic_bytes=d_bytes, kernel="pda_memo_mask_kernel"),
    }
    if not args.no_cpu:
        out.update(_pda_cpu_baseline(args, g, first, B))
    return out


def _pda_cpu_baseline(args, g, first, B) -> dict:
    """The reference's own CPU step -- apply_mask_pda_batch and
    advance_state_pda_batch of pda_cpu.cpp, compiled from its sources into
    oracle/_ref -- on the first timed step's config-sets, logits and tokens:
    every row of the batch over the host threads (no scaling), and a fixed
    sample of rows on one thread (the reference runs one), scaled to B.
    Without that build, the C restatement (oracle/pda_oracle.c) stands in."""
    import numpy as np

    from oracle import pda as OP
    from oracle import ref as OR

    t = OP.Table(g)
    cfgs, raw, masked, toks, after = first
    use_ref = OR.available()
    kind = "reference" if use_ref else "port"
    src = ("the reference's pda_cpu.cpp (oracle/_ref)" if use_ref
           else "oracle/pda_oracle.c (C restatement of pda_cpu.cpp)")
    threads = max(1, min(int(os.environ.get("OMP_NUM_THREADS", "16") or 16), os.cpu_count() or 1, 16))
    tk = toks.numpy().astype(np.int32)
    res = {}
    # every row, rows split over the host threads; then the commit of every row
    lg = raw.numpy().copy()
    sub = cfgs.numpy().copy()
    c0 = time.perf_counter()
    if use_ref:
        OR.pda_apply_mask_threads(t, sub, lg, threads)
    else:
        OP.apply_mask(t, sub, lg)
    mask_s = time.perf_counter() - c0
    c0 = time.perf_counter()
    ok = OR.pda_advance(t, sub, tk) if use_ref else OP.advance(t, sub, tk)
    commit_s = time.perf_counter() - c0
    res["cpu_baseline"] = {
        "value": round((mask_s + commit_s) * 1e6, 1),
        "unit": "us/step",
        "cores": threads if use_ref else 1,
        "kind": kind,
        "sample": (f"one whole step (all {B} rows, no scaling) of the first timed step through {src}: "
                   f"apply_mask_pda_batch with the rows split over {threads if use_ref else 1} host "
                   "threads, then advance_state_pda_batch on one thread"),
        "mask_us": round(mask_s * 1e6, 1),
        "commit_us": round(commit_s * 1e6, 1),
        "host_cpus": os.cpu_count(),
        "host_cpu_model": _cpu_model(),
    }
    res["parity_cpu_vs_device"] = {
        "masks_all_rows": bool(np.array_equal(lg, masked.numpy())),
        "committed_configs_all_rows": bool(np.array_equal(sub, after.numpy())),
        "all_tokens_accepted": bool(ok.all()),
    }
    # a fixed sample of rows on one thread, mask + commit, scaled to B
    n = min(args.pda_cpu_rows, B)
    lg1 = raw[:n].numpy().copy()
    sub1 = cfgs[:n].numpy().copy()
    c0 = time.perf_counter()
    if use_ref:
        OR.pda_apply_mask(t, sub1, lg1)
        OR.pda_advance(t, sub1, tk[:n])
    else:
        OP.apply_mask(t, sub1, lg1)
        OP.advance(t, sub1, tk[:n])
    one_s = time.perf_counter() - c0
    res["cpu_baseline_single_thread"] = {
        "value": round(one_s / n * B * 1e6, 1),
        "unit": "us/step",
        "cores": 1,
        "kind": kind,
        "sample": (f"rows 0-{n - 1} of the first timed step (mask + commit) through {src} on one "
                   f"thread, scaled to B={B}"),
        "parity_vs_device": bool(np.array_equal(lg1, masked[:n].numpy())
                                 and np.array_equal(sub1, after[:n].numpy())),
    }
    return res


# ------------------------------------------------------------------- soft --
def bench_soft(args) -> dict:
    """Prior-weighted soft lookahead over the email DFA: B rows at random
    reachable states, fp32 logits N(0, 3), k-step lookahead with the row's
    softmax as the token prior; one step = one in-place rewrite of the
    [B, V] logits."""
    import numpy as np
    import torch

    from bpdecode_amd import ops, synth
    from bpdecode_amd.ops import FsaTensors

    dev = torch.device("cuda:0")
    B, V, K = args.soft_rows, args.vocab, args.soft_k
    steps = min(args.soft_steps, args.steps)
    vocab = synth.serving_vocab(V, seed=1)
    fsa = FsaTensors.build(synth.EMAIL, vocab).densify()
    S = fsa.num_states
    states = synth.random_walk_states(fsa.tok_next, fsa.start, fsa.eos_id, B, 40, seed=5).to(torch.int32)
    fd = fsa.to(dev)
    sc = fd.ensure_soft_classes()
    st = states.to(dev)
    src = synth.logits(B, V, std=3.0, dtype=torch.float32, seed=11, device=dev)
    work = torch.empty_like(src)
    flush64 = None if args.no_flush else torch.zeros(512 << 20, dtype=torch.uint8, device=dev).view(torch.int64)
    sh = torch.cuda.current_stream(dev).cuda_stream
    n_total = args.warmup + steps
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
    kev.destroy()
    step_ms = statistics.fmean(times)
    d_bytes = B * V * 4 * 2 + S * V * 4
    out = {
        "metric": "µs/step prior-weighted soft lookahead (k=4), email DFA, B=128 V=151936 fp32",
        "value": round(step_ms * 1e3, 2),
        "unit": "us/step",
        "steps": steps,
        "dtype": "fp32",
        "config": {"workload": "soft lookahead with the row softmax as token prior, email DFA",
                   "batch_rows": B, "vocab": V, "k": K, "dfa_states": S,
                   "token_classes": sc.num_classes, "class_members": int(sc.class_tok.numel()),
                   "distinct_row_states": int(torch.unique(states[states >= 0]).numel()),
                   "logits": "fp32 N(0,3)"},
        "roofline": _roofline(d_bytes, step_ms * 1e-3, traffic=None,
                              scope="whole step (statistics, rounds and output kernels)",
                              algorithmic_bytes=d_bytes, bytes_formula="B*V*4*2 + S*V*4"),
        "row_vocab_entries_per_s": round(B * V / (step_ms * 1e-3), 1),
    }
    if not args.no_cpu and args.soft_cpu_rows:
        from oracle import soft as OS

        torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
        n = min(args.soft_cpu_rows, B)
        x = src.cpu()
        tn, live, acc = fsa.tok_next, fsa.live, fsa.accept
        OS.prior_lookahead_torch(x, tn, live, acc, fsa.eos_id, states, K, 1.0, rows=[0])  # warm-up
        c0 = time.perf_counter()
        part = OS.prior_lookahead_torch(x, tn, live, acc, fsa.eos_id, states, K, 1.0, rows=range(n))
        cpu_s = time.perf_counter() - c0
        got = work.cpu()
        rel = ((got[:n] - part[:n]).abs() / part[:n].abs().clamp(min=1.0))[torch.isfinite(part[:n])]
        out["cpu_baseline"] = {
            "value": round(cpu_s / n * B * 1e6, 1),
            "unit": "us/step",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"{n} rows through the fp32 torch restatement of the reference's lookahead "
                       f"(ops.py:200-259: [S, V] gathers of logZ through tok_next, logsumexp, "
                       f"logaddexp) with the row's log-softmax as prior, on CPU tensors with "
                       f"{torch.get_num_threads()} threads; a row costs the same at any state, "
                       f"scaled to B={B}"),
            "max_rel_diff_vs_device": float(rel.max()) if rel.numel() else 0.0,
            "host_cpus": os.cpu_count(),
            "host_cpu_model": _cpu_model(),
        }
        out["parity_vs_oracle_all_rows"] = _soft_parity_all_rows(
            src.double().cpu().numpy(), got.double().numpy(), fsa, states.numpy(), K)
    return out


def _soft_parity_all_rows(x, got, fsa, states, K) -> dict:
    """Every row of the step against the float64 oracle (oracle/soft.py),
    rows split over host threads (numpy releases the interpreter lock in
    its array loops): relative 1e-5 with an absolute floor of 1e-5, -inf
    pattern exact."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle import soft as OS

    tn, live, acc = fsa.tok_next.numpy(), fsa.live.numpy(), fsa.accept.numpy()
    threads = max(1, min(16, os.cpu_count() or 1, x.shape[0]))
    c0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as ex:
        want = np.concatenate(list(ex.map(
            lambda b: OS.prior_lookahead(x[b:b + 1], tn, live, acc, fsa.eos_id, states[b:b + 1], K, 1.0),
            range(x.shape[0]))))
    fin = np.isfinite(want)
    err = np.abs(got[fin] - want[fin])
    return {
        "rows": int(x.shape[0]),
        "ok": bool(np.array_equal(np.isneginf(got), np.isneginf(want))
                   and np.all(err <= 1e-5 * np.abs(want[fin]) + 1e-5)),
        "max_abs_err": float(err.max()) if err.size else 0.0,
        "max_rel_err": float((err / np.maximum(np.abs(want[fin]), 1.0)).max()) if err.size else 0.0,
        "oracle": f"oracle/soft.py prior_lookahead (float64 numpy) over {threads} host threads",
        "oracle_s": round(time.perf_counter() - c0, 2),
    }

if __name__ == "__main__":
    raise SystemExit(main())

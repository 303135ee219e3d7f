"""Decode-tail benchmark: LM-head + sample tokens/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-batches] [--only NAME]

Headline workload (one "step" = one decode-tail pass for one batch): B=1 stochastic sampling on
the affine-int4 tied LM head, V = 262144, D = 2816, group 64 (BF16 scale + bias): final RMSNorm ->
head -> softcap 30 -> repetition penalty 1.1 over a 256-token history that grows with every
sampled token (appended on the device) -> top-p 0.95 -> top-k 64 -> temperature 0.8 ->
Philox4x32-10 draw with (seed, counter = step). Fresh N(0,1) hidden state every step. All inputs
are resident in HBM before the timed region.

The JSON line also carries one object per other configuration ("lines"): greedy B=1, B=32 mixed
per-row parameters with presence/frequency over 1024-id Zipf histories, B=64 constrained decode
(5 % ban bitmask, 300-entry logit bias, repetition 1.15 over 2048 ids, top-k 40 / top-p 0.9 /
T 0.7) and B=256 full-vocabulary top-p 0.9 on bf16 hidden states; and ("widened") the int4 matvec
at the reference's projection shapes and the embedding lookup.

Timing. The K timed steps run with nothing but the step's own kernels on the stream, bracketed by
torch.cuda.synchronize(). The head kernel's duration is measured afterwards, in a separate pass
of the same workload in which every head launch carries HIP start/stop events stamped by its own
dispatch, on the stream it runs on (the events add launch gaps, so they stay out of the timed
steps). roofline.achieved = algorithmic bytes (B <= 64) or flops (B = 256) per head launch / the
head's mean duration. Algorithmic bytes = 415,236,096 (nibbles + BF16 scales + BF16 biases) +
B*D*(4 fp32 | 2 bf16) + the side inputs (history 4 B/id, ban 32,768 B/row, bias 8 B/entry) +
4 B/token; flops = 2*V*D*B.
cpu_baseline: the oracle's C restatement of the reference CPU path (src/cpu_reference.cpp
RMSNorm/matvec/softcap + src/sampling.cpp penalty/sampler) for config-2 steps, timed inside C
(CLOCK_MONOTONIC per step, median) at 1 thread and at the host's nproc threads (capped at the 16
CPUs one GPU's job may use). parity: those CPU steps' tokens against the GPU line's first steps,
which ran on identical inputs ({"steps", "equal", "near_ties", "first_mismatch"}).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for sub in ("turbo-winfare_amd", "oracle"):
    sys.path.insert(0, str(ROOT / sub))

V, D = 262144, 2816
SEED = 20260801
WEIGHT_BYTES = V * D // 2 + 2 * (V * (D // 64) * 2)  # 415,236,096
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16 / fp16
METRIC = "LM-head+sample tokens/sec at B=1/32/256; % HBM roofline (B=1), % MFMA (B=256)"
TRAFFIC_FILE = ROOT / "profiles" / "head_traffic.json"
CPU_THREADS_CAP = 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--timing-steps", type=int, default=64,
                    help="steps of the separate pass that times the head kernel")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batches", action="store_true")
    ap.add_argument("--only", choices=["b1", "greedy", "b32", "b64", "b256", "widened", "cpu"], default=None,
                    help="run one workload only (profiling); prints its own JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="copy a buffer of the table's size 5 times (a plain copy kernel of known "
                         "size, to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def head_kernel_name(B: int, meta: bool) -> str:
    """The head kernel the library launches for a batch of B rows over this head's shape (group
    count divisible by 4, every scale below 1/16); meta: some row has modifiers or a ban mask."""
    if B <= 2:
        return f"k_head_digits_fused<{B}>"
    nb = 1 if B <= 32 else 2 if B <= 64 else 4
    wv, pf, occ = {1: (4, 4, 3), 2: (16, 2, 1), 4: (4, 4, 2)}[nb]
    return f"k_head_mfma<{nb}, {wv}, {pf}, {occ}, true, {'true' if meta else 'false'}>"


class Workload:
    """One configuration: device-resident inputs for every step it will run, and step(s)."""

    name = ""
    B = 1
    describe = ""

    def side_bytes(self) -> int:
        return 0

    def hidden_bytes(self) -> int:
        return self.B * D * 4

    def algorithmic_bytes(self) -> int:
        return WEIGHT_BYTES + self.hidden_bytes() + self.side_bytes() + 4 * self.B

    def flops(self) -> float:
        return 2.0 * V * D * self.B


class SampledB1(Workload):
    """Config 2: B=1 sampled decode with the token appended to the history on the device."""
    name, B = "b1", 1
    describe = ("B=1 sampled decode: T 0.8, top-k 64, top-p 0.95, repetition 1.1 over a 256-token "
                "history (+1 per step), Philox(seed, counter=step)")

    def __init__(self, T, torch, head, total_steps):
        import synth
        self.T, self.torch, self.head = T, torch, head
        self.hidden = torch.from_numpy(synth.hidden_states(total_steps, D, SEED + 1)).cuda()
        self.hist_cap = 256 + total_steps
        self.hist = torch.zeros((1, self.hist_cap), dtype=torch.int32, device="cuda")
        self.hist[0, :256] = torch.from_numpy(synth.uniform_ids(256, V, SEED).astype(np.int32))
        self.hlen = torch.tensor([256], dtype=torch.int32, device="cuda")
        self.tokens = torch.zeros(total_steps, dtype=torch.int32, device="cuda")
        self.row = T.row_default(temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.1,
                                 seed=SEED, counter=0)
        # kept alive with the struct: it holds raw device pointers
        self.inp, self._keep = head.make_inputs(1, [self.row], hidden=self.hidden,
                                                flags=T.TURBO_STEP_APPEND_HISTORY,
                                                history=self.hist, history_len=self.hlen)
        self.base_hidden = self.hidden.data_ptr()
        self.base_tok = self.tokens.data_ptr()

    def side_bytes(self):
        return 4 * 256

    def step(self, s):
        self._keep[0].counter = s
        self.inp.hidden = self.base_hidden + s * D * 4
        self.head.step(self.inp, self.base_tok + 4 * s)


class GreedyB1(Workload):
    """Config 1: B=1 greedy (RMSNorm -> head -> softcap -> argmax), fresh hidden state per step."""
    name, B = "greedy", 1
    describe = "B=1 greedy: RMSNorm -> head -> softcap 30 -> argmax (ties to the lowest id)"

    def __init__(self, T, torch, head, total_steps):
        import synth
        self.head = head
        self.hidden = torch.from_numpy(synth.hidden_states(total_steps, D, SEED + 5)).cuda()
        self.tokens = torch.zeros(total_steps, dtype=torch.int32, device="cuda")
        self.inp, self._keep = head.make_inputs(1, [T.row_default()], hidden=self.hidden)
        self.base_hidden = self.hidden.data_ptr()
        self.base_tok = self.tokens.data_ptr()

    def step(self, s):
        self.inp.hidden = self.base_hidden + s * D * 4
        self.head.step(self.inp, self.base_tok + 4 * s)


class Batched(Workload):
    """Configs 3, 5 and 4 (B = 32, 64, 256): one batch of rows, the counter advanced per step."""

    def __init__(self, T, torch, head, B):
        import synth
        self.head, self.B, self.name = head, B, f"b{B}"
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        keep = []
        if B == 32:
            x = dev(synth.hidden_states(B, D, SEED + 2))
            pu = synth.uniform(SEED, synth.S_PARAMS, 2 * B)
            ks = [0, 20, 40, 100]
            rows = [T.row_default(temperature=float(0.3 + 1.2 * pu[b]), top_k=ks[b % 4],
                                  top_p=float(0.8 + 0.2 * pu[B + b]), presence_penalty=0.5,
                                  frequency_penalty=0.3, seed=1000 + b, counter=0,
                                  flags=T.TURBO_ROW_FULL_VOCAB if ks[b % 4] == 0 else 0) for b in range(B)]
            hists = dev(np.stack([synth.zipf_ids(1024, V, 1.1, SEED + 10 + b) for b in range(B)]).astype(np.int32))
            hl = torch.full((B,), 1024, dtype=torch.int32, device="cuda")
            keep += [x, hists, hl]
            self.inp, self.rows = head.make_inputs(B, rows, hidden=x, history=hists, history_len=hl)
            self._side = B * 1024 * 4
            self.describe = ("B=32 mixed per-row T/top-k/top-p, presence 0.5 + frequency 0.3 over 1024 "
                             "Zipf(1.1) ids per row")
        elif B == 64:
            x = dev(synth.hidden_states(B, D, SEED + 4))
            rows = [T.row_default(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.15,
                                  seed=500 + b, counter=0) for b in range(B)]
            hists = dev(np.stack([synth.uniform_ids(2048, V, SEED + 20 + b) for b in range(B)]).astype(np.int32))
            bans = dev(np.stack([synth.ban_mask(V, 0.05, SEED, b) for b in range(B)]).view(np.int32))
            bl = [synth.bias_list(300, V, -5.0, 5.0, SEED, b) for b in range(B)]
            bids = dev(np.stack([a for a, _ in bl]).astype(np.int32))
            bvals = dev(np.stack([v for _, v in bl]))
            hl = torch.full((B,), 2048, dtype=torch.int32, device="cuda")
            bc = torch.full((B,), 300, dtype=torch.int32, device="cuda")
            keep += [x, hists, bans, bids, bvals, hl, bc]
            self.inp, self.rows = head.make_inputs(B, rows, hidden=x, history=hists, history_len=hl, ban=bans,
                                                   bias_ids=bids, bias_values=bvals, bias_count=bc)
            self._side = B * (2048 * 4 + V // 8 + 300 * 8)
            self.describe = ("B=64 constrained: 5 % banned ids, 300-entry logit bias in [-5, 5], repetition "
                             "1.15 over 2048 ids, top-k 40, top-p 0.9, T 0.7")
        else:
            xb = synth.f32_to_bf16(synth.hidden_states(B, D, SEED + 3))
            x = dev(xb.view(np.int16))
            rows = [T.row_default(temperature=1.0, top_p=0.9, top_k=0, seed=77 + b, counter=0,
                                  flags=T.TURBO_ROW_FULL_VOCAB) for b in range(B)]
            keep += [x]
            self.inp, self.rows = head.make_inputs(B, rows, hidden=x, dtype=T.TURBO_HIDDEN_BF16,
                                                   flags=T.TURBO_STEP_NORMED)
            self._side = 0
            self.describe = "B=256 bf16 hidden (normed), full-vocabulary top-p 0.9, T=1.0"
        self._keep = keep  # the inputs hold raw device pointers
        self.tok = torch.zeros(B, dtype=torch.int32, device="cuda")

    def hidden_bytes(self):
        return self.B * D * (2 if self.B == 256 else 4)

    def side_bytes(self):
        return self._side

    def step(self, s):
        for r in self.rows:
            r.counter = s
        self.head.step(self.inp, self.tok)


def time_loop(torch, fn, first, count):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(first, first + count):
        fn(s)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def measure(torch, head, wl, warmup, steps, tsteps, first=0):
    """Throughput over `steps` untimed-kernel steps, then the head's mean duration over a
    separate pass of `tsteps` steps with dispatch events on every head launch."""
    head.enable_head_timing(False)
    time_loop(torch, wl.step, first, warmup)
    el = time_loop(torch, wl.step, first + warmup, steps)
    head.enable_head_timing(True, every=1)
    head.head_kernel_time(reset=True)
    time_loop(torch, wl.step, first + warmup + steps, tsteps)
    kms, n = head.head_kernel_time(reset=True)
    head.enable_head_timing(False)
    kavg = kms / max(n, 1)
    out = {"workload": wl.describe, "batch": wl.B, "tokens_per_s": wl.B * steps / el,
           "ms_per_step": 1e3 * el / steps, "steps": steps, "warmup": warmup}
    nbytes, flops = wl.algorithmic_bytes(), wl.flops()
    gbs = nbytes / (kavg * 1e-3) / 1e9
    tfl = flops / (kavg * 1e-3) / 1e12
    bound = "mfma" if wl.B == 256 else "hbm"
    out["roofline"] = {
        "bound": bound,
        "achieved": tfl if bound == "mfma" else gbs,
        "peak": MFMA_PEAK_TFLOPS if bound == "mfma" else HBM_PEAK_GBS,
        "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
        "frac": (tfl / MFMA_PEAK_TFLOPS) if bound == "mfma" else (gbs / HBM_PEAK_GBS),
        "traffic": None,
        "kernel": head_kernel_name(wl.B, wl.B in (32, 64)), "kernel_avg_us": 1e3 * kavg, "timed_launches": n,
        "algorithmic_bytes_per_launch": nbytes, "algorithmic_flops_per_launch": flops,
        "hbm_GBs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS, "TFLOPs": tfl, "mfma_frac": tfl / MFMA_PEAK_TFLOPS,
    }
    # the whole step against the same roofline (everything the step does, per step)
    out["step_frac"] = ((flops / (1e-3 * out["ms_per_step"]) / 1e12 / MFMA_PEAK_TFLOPS) if bound == "mfma"
                        else (nbytes / (1e-3 * out["ms_per_step"]) / 1e9 / HBM_PEAK_GBS))
    return out


def widened_lines(T, torch):
    """Rows beyond the decode tail that share its kernels: the int4 matvec at the reference's
    projection shapes (B = 1; digit GEMV, split over the groups of each 64-row tile) and the
    embedding lookup on the tied table. Kernel times come from the head's dispatch events on
    every call of a second loop (the events themselves lengthen a short kernel's measured
    span); call times are wall clock per call of a loop without them (preparation and head
    kernels, host launch cost included)."""
    import synth
    out = {"matvec_b1": {}, "embed": {}}
    for rows, k in [(704, 2816), (2816, 704), (2112, 2816), (2816, 2112), (4096, 2816)]:
        W, S, B, _ = synth.make_head(rows, k, rows + k)
        h = T.LMHead(W, S, B, None, vocab=rows, hidden=k, softcap=0.0)
        x = torch.from_numpy(synth.hidden_states(1, k, 3)).cuda()
        o = torch.empty((1, rows), dtype=torch.float32, device="cuda")
        for _ in range(20):
            h.matvec(x, 1, o)
        n = 200
        el = time_loop(torch, lambda s: h.matvec(x, 1, o), 0, n)
        h.enable_head_timing(True, every=1)
        h.head_kernel_time(reset=True)
        time_loop(torch, lambda s: h.matvec(x, 1, o), 0, n)
        kms, cnt = h.head_kernel_time(reset=True)
        kus = 1e3 * kms / max(cnt, 1)
        byts = rows * k // 2 + rows * (k // 64) * 4 + k * 4 + rows * 4
        out["matvec_b1"][f"{rows}x{k}"] = {"kernel_us": kus, "call_us": 1e6 * el / n,
                                           "kernel_GBs": byts / (kus * 1e-6) / 1e9,
                                           "algorithmic_bytes": byts}
        h.close()
    # the 8 routed experts of one token: gate + up (16 x 704 x 2816, one input row) in one grouped
    # launch, then the 8 down matrices (2816 x 704) in another; against one call per matrix
    out["experts_grouped"] = {}
    for name, shape, n in (("gate_up_16x704x2816", (704, 2816), 16), ("down_8x2816x704", (2816, 704), 8)):
        rows, k = shape
        mats, heads = [], []
        for i in range(n):
            W, S, B, _ = synth.make_head(rows, k, 3000 + i)
            m = T.Int4Matrix(rows, k)
            m.load_weights(W, S, B)
            mats.append(m)
        xs = [torch.from_numpy(synth.hidden_states(1, k, 80 + i)[0]).cuda() for i in range(n)]
        outs = [torch.empty(rows, dtype=torch.float32, device="cuda") for _ in range(n)]
        for _ in range(20):
            T.matvec_grouped(mats, xs, outs)
        reps = 200
        el = time_loop(torch, lambda s: T.matvec_grouped(mats, xs, outs), 0, reps)
        byts = n * (rows * k // 2 + rows * (k // 64) * 4 + k * 4 + rows * 4)
        out["experts_grouped"][name] = {"call_us": 1e6 * el / reps, "matrices": n, "algorithmic_bytes": byts,
                                        "GBs": byts / (el / reps) / 1e9}
        for m in mats:
            m.close()
    W, S, B, g = synth.make_head(V, D, SEED)
    h = T.LMHead(W, S, B, g, vocab=V, hidden=D)
    for ntok in (1, 256):
        ids = torch.from_numpy((np.arange(ntok, dtype=np.int64) * 1021 % V).astype(np.int32)).cuda()
        e = torch.empty((ntok, D), dtype=torch.float32, device="cuda")
        for _ in range(20):
            h.embed(ids, ntok, e)
        n = 500
        el = time_loop(torch, lambda s: h.embed(ids, ntok, e), 0, n)
        byts = ntok * (D // 2 + (D // 64) * 4 + D * 4)
        out["embed"][f"{ntok}_tokens"] = {"call_us": 1e6 * el / n, "algorithmic_bytes": byts}
    h.close()
    return out


def host_nproc() -> int:
    """What `nproc` prints: the CPUs this process may run on."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(W, S, B, g, one_steps=5, many_steps=16):
    """Config-2 decode steps of the oracle's C restatement, timed inside C (no Python between
    the clock reads): the median step at 1 thread (the reference CPU path is single-threaded,
    README.md:223-225) and at the host's nproc threads, row-parallel over the vocabulary with
    per-row arithmetic unchanged (bit-identical tokens)."""
    import orc_py as O
    import synth
    nproc = host_nproc()
    threads = max(1, min(nproc, CPU_THREADS_CAP))
    p = O.params(0.8, 0.95, 64, 1.1)
    hist = synth.uniform_ids(256, V, SEED)

    def run(nthreads, n):
        x = synth.hidden_states(n + 1, D, SEED + 1)  # step 0 warms the caches and is dropped
        toks, secs = O.time_decode_steps(W, S, B, g, x, p, SEED, hist, threads=nthreads)
        return toks, float(np.median(secs[1:]))

    toks1, med1 = run(1, one_steps)
    toksn, medn = run(threads, many_steps)
    assert np.array_equal(toks1, toksn[:toks1.size]), "thread count changed the CPU tokens"
    return toksn, {"value": 1.0 / medn, "unit": "tokens/s", "cores": threads, "kind": "port",
            "nproc": nproc, "single_thread_value": 1.0 / med1,
            "median_step_ms": 1e3 * medn, "single_thread_median_step_ms": 1e3 * med1,
            "sample": (f"config-2 decode steps (B=1, V=262144) of oracle/orc.c -O2 -ffp-contract=off "
                       f"(RMSNorm, int4 matvec, softcap, repetition penalty, sample_token), timed per step "
                       f"inside C: median of {many_steps} steps at {threads} threads (nproc {nproc}, capped "
                       f"at {CPU_THREADS_CAP}) and of {one_steps} steps at 1 thread, each after one warm-up step")}


def token_parity(gpu_toks, cpu_toks, W, S, B, g):
    """The CPU baseline's config-2 tokens against the GPU line's on the same inputs (hidden row s,
    Philox counter s, the same 256-id history growing by each step's token): the reference's
    token-for-token gate (CONTRIBUTING.md:38-47). Up to the first difference both histories are
    equal; a difference is reported with the oracle's CDF margin at that step (a near tie when
    the margin is below 1e-3 of r), and the comparison stops there because the histories then
    diverge."""
    import orc_py as O
    import synth
    n = min(len(gpu_toks), len(cpu_toks))
    diff = np.nonzero(np.asarray(gpu_toks[:n], np.uint32) != np.asarray(cpu_toks[:n], np.uint32))[0]
    out = {"steps": n, "equal": n if diff.size == 0 else int(diff[0]), "near_ties": 0, "first_mismatch": None,
           "kind": "oracle/orc.c decode steps vs the GPU line's first steps, identical inputs"}
    if diff.size:
        k = int(diff[0])
        hist = np.concatenate([synth.uniform_ids(256, V, SEED), np.asarray(cpu_toks[:k], np.uint32)])
        x = synth.hidden_states(1, D, SEED + 1, k)[0]
        p = O.params(0.8, 0.95, 64, 1.1)
        l = O.apply_modifiers(O.head_logits(W, S, B, g, x, threads=CPU_THREADS_CAP), p, 30.0, history=hist)
        info = O.sample(l, p, O.philox_uniform(SEED, k))
        margin = min(info.acc_at - info.r, info.r - info.acc_prev) / max(info.r, 1e-300)
        out["first_mismatch"] = {"step": k, "gpu": int(gpu_toks[k]), "cpu": int(cpu_toks[k]), "cdf_margin_rel": margin}
        out["near_ties"] = 1 if margin <= 1e-3 else 0
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}): the head would shard by vocabulary "
              f"rows across GPUs, which is not implemented", file=sys.stderr)
        sys.exit(2)
    import torch
    if a.copy_calibration:
        src = torch.ones(WEIGHT_BYTES // 4, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": WEIGHT_BYTES, "copies": 5}), flush=True)
        return
    import synth
    import turbo_decode_tail as T

    assert torch.cuda.is_available(), "bench needs a GPU"
    if a.only == "widened":
        print(json.dumps({"only": a.only, **widened_lines(T, torch)}), flush=True)
        return
    log("generating the synthetic head")
    W, S, B, g = synth.make_head(V, D, SEED)
    if a.only == "cpu":
        print(json.dumps({"only": a.only, **cpu_baseline(W, S, B, g)[1]}), flush=True)
        return
    head = T.LMHead(W, S, B, g, vocab=V, hidden=D)
    tsteps = max(1, a.timing_steps)
    total = a.warmup + a.steps + tsteps
    lines = {}
    gpu_toks = None
    if a.only in (None, "b1"):
        log(f"B=1 sampled: warmup {a.warmup}, timed {a.steps}, head-timing pass {tsteps}")
        b1 = SampledB1(T, torch, head, total)
        main_line = measure(torch, head, b1, a.warmup, a.steps, tsteps)
        gpu_toks = b1.tokens.cpu().numpy().astype(np.uint32)  # every step's token, step 0 first
    if a.only in (None, "greedy"):
        log("B=1 greedy")
        lines["greedy_b1"] = measure(torch, head, GreedyB1(T, torch, head, total), a.warmup, a.steps, tsteps)
    batched = [] if a.no_batches else [32, 64, 256]
    if a.only in ("b32", "b64", "b256"):
        batched = [int(a.only[1:])]
    elif a.only is not None:
        batched = []
    for Bn in batched:
        log(f"B={Bn}")
        # at least 64 timed steps per batched line, whatever --steps is: the first steps of a
        # workload carry one-time costs that a handful of steps would not amortise
        st = max(a.steps // 4, 64) if Bn == 256 else max(a.steps // 2, 64)
        lines[f"b{Bn}"] = measure(torch, head, Batched(T, torch, head, Bn), max(a.warmup, 3), st,
                                  min(tsteps, 32))
    head.close()
    if a.only is not None:
        res = main_line if a.only == "b1" else next(iter(lines.values()))
        print(json.dumps({"only": a.only, **res}), flush=True)
        return

    # HBM bytes per head launch from the committed counter summary (FETCH_SIZE + WRITE_SIZE, each
    # calibrated on a copy kernel); workloads without a counter pass keep null
    measured = {}
    if TRAFFIC_FILE.exists():
        try:
            measured = {k: v.get("hbm_bytes_per_launch")
                        for k, v in json.loads(TRAFFIC_FILE.read_text()).get("workloads", {}).items()}
        except Exception:
            measured = {}
    traffic = measured.get("b1")
    for name, ln in lines.items():
        ln["roofline"]["traffic"] = measured.get({"greedy_b1": "greedy"}.get(name, name))
    roof = dict(main_line["roofline"])
    roof["traffic"] = traffic
    line = {
        "metric": METRIC,
        "value": main_line["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": main_line["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x int4-digit dot (i32) + fp32 epilogue, fp64 sampler",
        "data": "synthetic (seeded counter-based generator; random int4 head of the Gemma 4 shape)",
        "config": {"workload": SampledB1.describe, "vocab": V, "hidden": D, "group": 64, "batch": 1,
                   "softcap": 30.0},
        "roofline": roof,
        "step_frac": main_line["step_frac"],
        "lines": lines,
    }
    if not a.no_batches:
        log("matvec shapes and embedding lookup")
        line["widened"] = widened_lines(T, torch)
    if not a.no_cpu:
        log("cpu baseline")
        cpu_toks, line["cpu_baseline"] = cpu_baseline(W, S, B, g)
        line["parity"] = token_parity(gpu_toks, cpu_toks, W, S, B, g)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

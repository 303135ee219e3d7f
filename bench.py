"""Decode-tail benchmark: LM-head + sample tokens/s on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-batches]

Workload (one "step" = one decode-tail pass for one batch): B=1 stochastic sampling on the
affine-int4 tied LM head, V = 262144, D = 2816, group 64 (BF16 scale + bias): final RMSNorm ->
head -> softcap 30 -> repetition penalty 1.1 over a 256-token history that grows with every
sampled token (appended on the device) -> top-p 0.95 -> top-k 64 -> temperature 0.8 ->
Philox4x32-10 draw with (seed, counter = step). Fresh N(0,1) hidden state every step. All inputs
are resident in HBM before the timed region.

The JSON line also reports the same head at B = 32 (mixed per-row parameters with
presence/frequency penalties over 1024-id Zipf histories) and B = 256 (full-vocabulary top-p
0.9 on bf16 hidden states), each with its head kernel's roofline, and ("widened") the int4
matvec at the reference's projection shapes and the embedding lookup.

roofline: the dominant kernel is the head (int4 GEMV at B <= 2, MFMA at B > 2). Its average
duration is measured during the timed region with HIP start/stop events of the kernel's own
dispatch on the stream it runs on, on every 16th step (events add launch gaps).
Algorithmic bytes per launch = 415,236,096 (nibbles + BF16 scales + BF16 biases) + B*D*4
(activations); algorithmic flops = 2*V*D*B.
cpu_baseline: the oracle's C restatement of the reference CPU path (src/cpu_reference.cpp
RMSNorm/matvec/softcap + src/sampling.cpp penalty/sampler), timed on this host for a bounded
number of steps.
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
TRAFFIC_FILE = ROOT / "profiles" / "head_b1_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batches", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--only", choices=["b1", "b32", "b256", "widened"], default=None,
                    help="run one workload only (profiling); prints its own JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="copy a buffer of the table's size 5 times (a plain copy kernel of known "
                         "size, to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Config2:
    """B=1 sampled decode with on-device history append."""

    def __init__(self, T, torch, head, total_steps):
        import synth
        self.T, self.torch, self.head = T, torch, head
        hid = synth.hidden_states(total_steps, D, SEED + 1)
        self.hidden = torch.from_numpy(hid).cuda()
        self.hist_cap = 256 + total_steps
        self.hist = torch.zeros((1, self.hist_cap), dtype=torch.int32, device="cuda")
        self.hist[0, :256] = torch.from_numpy(synth.uniform_ids(256, V, SEED).astype(np.int32))
        self.hlen = torch.tensor([256], dtype=torch.int32, device="cuda")
        self.tokens = torch.zeros(total_steps, dtype=torch.int32, device="cuda")
        self.row = T.row_default(temperature=0.8, top_k=64, top_p=0.95, repetition_penalty=1.1,
                                 seed=SEED, counter=0)
        self.inp, self._keep = head.make_inputs(1, [self.row], hidden=self.hidden,
                                                flags=T.TURBO_STEP_APPEND_HISTORY,
                                                history=self.hist, history_len=self.hlen)
        self.base_hidden = self.hidden.data_ptr()
        self.base_tok = self.tokens.data_ptr()

    def step(self, s):
        self._keep[0].counter = s
        self.inp.hidden = self.base_hidden + s * D * 4
        self.head.step(self.inp, self.base_tok + 4 * s)


def time_loop(torch, fn, first, count):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(first, first + count):
        fn(s)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def batched_line(T, torch, head, B, warm, steps):
    import synth
    if B == 32:
        x = torch.from_numpy(synth.hidden_states(B, D, SEED + 2)).cuda()
        pu = synth.uniform(SEED, synth.S_PARAMS, 2 * B)
        ks = [0, 20, 40, 100]
        rows = [T.row_default(temperature=float(0.3 + 1.2 * pu[b]), top_k=ks[b % 4],
                              top_p=float(0.8 + 0.2 * pu[B + b]), presence_penalty=0.5,
                              frequency_penalty=0.3, seed=1000 + b, counter=0,
                              flags=T.TURBO_ROW_FULL_VOCAB if ks[b % 4] == 0 else 0) for b in range(B)]
        hists = np.stack([synth.zipf_ids(1024, V, 1.1, SEED + 10 + b) for b in range(B)])
        hl = torch.full((B,), 1024, dtype=torch.int32, device="cuda")
        inp, keep = head.make_inputs(B, rows, hidden=x, history=torch.from_numpy(hists.astype(np.int32)).cuda(),
                                     history_len=hl)
        workload = "B=32 mixed per-row T/top-k/top-p, presence 0.5 + frequency 0.3 over 1024 Zipf(1.1) ids"
    else:
        xb = synth.f32_to_bf16(synth.hidden_states(B, D, SEED + 3))
        x = torch.from_numpy(xb.view(np.int16)).cuda()
        rows = [T.row_default(temperature=1.0, top_p=0.9, top_k=0, seed=77 + b, counter=0,
                              flags=T.TURBO_ROW_FULL_VOCAB) for b in range(B)]
        inp, keep = head.make_inputs(B, rows, hidden=x, dtype=T.TURBO_HIDDEN_BF16, flags=T.TURBO_STEP_NORMED)
        workload = "B=256 bf16 hidden, full-vocabulary top-p 0.9, T=1.0"
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")

    def fn(s):
        for r in keep:
            r.counter = s
        head.step(inp, tok)

    time_loop(torch, fn, 0, warm)
    head.head_kernel_time(reset=True)
    el = time_loop(torch, fn, warm, steps)
    kms, n = head.head_kernel_time(reset=True)
    kavg = kms / max(n, 1)
    step_ms = 1e3 * el / steps
    bytes_ = WEIGHT_BYTES + B * D * (4 if B == 32 else 2)
    flops = 2.0 * V * D * B
    out = {"workload": workload, "tokens_per_s": B * steps / el, "ms_per_step": step_ms,
           "head_kernel_us": 1e3 * kavg,
           "head_hbm_GBs": bytes_ / (kavg * 1e-3) / 1e9,
           "head_hbm_frac": bytes_ / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "head_TFLOPs": flops / (kavg * 1e-3) / 1e12,
           "head_mfma_frac": flops / (kavg * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS}
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
        # call time without the dispatch timer (its periodic read-back synchronises the stream)
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


def cpu_baseline(W, S, B, g, nsteps):
    """Oracle restatement of the reference CPU path for config-2 steps on this host."""
    import orc_py as O
    import synth
    threads = min(16, os.cpu_count() or 1)
    hist = list(synth.uniform_ids(256, V, SEED))
    p = O.params(0.8, 0.95, 64, 1.1)

    def run(nthreads, n):
        t0 = time.perf_counter()
        for s in range(n):
            x = synth.hidden_states(1, D, SEED + 1, s)[0]
            l = O.head_logits(W, S, B, g, x, threads=nthreads)
            l = O.apply_modifiers(l, p, 30.0, history=np.array(hist, np.uint32))
            info = O.sample(l, p, O.philox_uniform(SEED, s))
            hist.append(info.token)
        return n / (time.perf_counter() - t0)

    run(threads, 1)  # warm caches
    one = run(1, max(1, nsteps // 2))
    many = run(threads, nsteps * 2)
    return {"value": many, "unit": "tokens/s", "cores": threads, "kind": "port",
            "single_thread_value": one,
            "sample": (f"config-2 decode steps on the host: {nsteps * 2} steps at {threads} threads "
                       f"(row-parallel matvec), {max(1, nsteps // 2)} steps at 1 thread; oracle/orc.c "
                       "-O2 -ffp-contract=off (RMSNorm, int4 matvec, softcap, repetition penalty, "
                       "sample_token)")}


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}); the sharded design is in DESIGN.md",
              file=sys.stderr)
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
    head = T.LMHead(W, S, B, g, vocab=V, hidden=D)
    # Events around a launch add a few microseconds of gap, so the head kernel is timed on every
    # 16th step of the timed region (its average duration; the step rate is not perturbed).
    # Short runs (counter passes) time every launch so that at least one is timed.
    head.enable_head_timing(True, every=16 if a.steps >= 64 else 1)
    if a.only in ("b32", "b256"):
        B = 32 if a.only == "b32" else 256
        res = batched_line(T, torch, head, B, a.warmup, a.steps)
        head.close()
        print(json.dumps({"only": a.only, **res}), flush=True)
        return
    total = a.warmup + a.steps
    c2 = Config2(T, torch, head, total)
    log(f"warmup {a.warmup} steps")
    time_loop(torch, c2.step, 0, a.warmup)
    head.head_kernel_time(reset=True)
    log(f"timing {a.steps} steps")
    el = time_loop(torch, c2.step, a.warmup, a.steps)
    kms, n = head.head_kernel_time(reset=True)
    kavg_ms = kms / max(n, 1)
    bytes_per_launch = WEIGHT_BYTES + 1 * D * 4
    achieved = bytes_per_launch / (kavg_ms * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    line = {
        "metric": METRIC,
        "value": a.steps / el,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": 1e3 * el / a.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x int4-digit dot (i32) + fp32 epilogue, fp64 sampler",
        "data": "synthetic (seeded counter-based generator; random int4 head of the Gemma 4 shape)",
        "config": {"workload": "B=1 sampled decode: T 0.8, top-k 64, top-p 0.95, repetition 1.1 over a "
                               "256-token history (+1 per step), Philox(seed, counter=step)",
                   "vocab": V, "hidden": D, "group": 64, "batch": 1, "softcap": 30.0},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "k_head_digits_fused<1>", "kernel_avg_us": 1e3 * kavg_ms,
                     "algorithmic_bytes_per_launch": bytes_per_launch},
    }
    if not a.no_batches and a.only is None:
        log("batched lines")
        line["batches"] = {"B32": batched_line(T, torch, head, 32, 10, 96),
                           "B256": batched_line(T, torch, head, 256, 5, 64)}
    head.close()
    if not a.no_batches and a.only is None:
        log("matvec shapes and embedding lookup")
        line["widened"] = widened_lines(T, torch)
    if not a.no_cpu and a.only is None:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(W, S, B, g, a.cpu_steps)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

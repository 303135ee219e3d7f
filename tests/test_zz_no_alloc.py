"""turbo_sample_logits_noalloc (no handle, static device scratch) against turbo_sample_logits on a
handle (its own allocated scratch): the same logits, rows and side inputs must give the same
tokens, reports and modified logits, bit for bit. Two calls in a row, the second with a smaller
vocabulary and batch, so that the static array's contents after the first call (the history
counts, their bitmap and the full-vocabulary sums it leaves at zero, and everything else it
overwrites) cannot leak into the second. The inputs exercise every stage: greedy, shortlist and
full-vocabulary rows; history penalties (repetition, presence, frequency) with repeated ids;
logit bias with duplicate ids; banned ids."""
import numpy as np
import pytest

import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

D = 64  # the handle only needs a head of the vocabulary's size; its weights are not used


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def case(V, Bn, seed):
    base = (synth.normal(seed, 81, Bn * V).reshape(Bn, V) * 3).astype(np.float32)
    cfgs = [(0.0, 1.0, 0, 0, 1.0), (0.8, 0.95, 64, 0, 1.1), (1.0, 0.9, 0, 1, 1.2), (0.7, 0.9, 40, 0, 1.15)]
    rows = [T.row_default(temperature=t, top_p=p, top_k=k, repetition_penalty=rp, presence_penalty=0.3 * (b % 2),
                          frequency_penalty=0.1 * (b % 2), seed=seed + b, counter=7 + b,
                          flags=T.TURBO_ROW_FULL_VOCAB if f else 0)
            for b, (t, p, k, f, rp) in enumerate(cfgs[:Bn])]
    nh, nb = 700, 300
    hists = np.stack([synth.zipf_ids(nh, V, 1.1, seed + 10 + b) for b in range(Bn)]).astype(np.uint32)
    bl = [synth.bias_list(nb, V, -4.0, 4.0, seed + 3, b) for b in range(Bn)]
    bids = np.stack([a for a, _ in bl]).astype(np.uint32)
    bids[:, 1::2] = bids[:, 0::2]  # duplicates summed in list order
    bvals = np.stack([v for _, v in bl])
    bans = np.stack([synth.ban_mask(V, 0.05, seed, b) for b in range(Bn)])
    hl = np.array([nh, nh - 50, 0, 17][:Bn], np.int32)
    bc = np.array([nb, 0, 120, nb][:Bn], np.int32)
    return base, rows, dict(history=hists, history_len=hl, ban=bans, bias_ids=bids, bias_values=bvals, bias_count=bc)


def run(sample, base, rows, side):
    Bn = len(rows)
    lt = dev(base)
    kw = dict(history=dev(side["history"].view(np.int32)), history_len=dev(side["history_len"]),
              ban=dev(side["ban"].view(np.int32)), bias_ids=dev(side["bias_ids"].view(np.int32)),
              bias_values=dev(side["bias_values"]), bias_count=dev(side["bias_count"]))
    inp, keep = T.LMHead.make_inputs(Bn, rows, **kw)
    tok = torch.zeros(Bn, dtype=torch.int32, device="cuda")
    rep = torch.zeros((Bn, 56 // 4), dtype=torch.int32, device="cuda")
    sample(lt, inp, tok, rep)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), lt.cpu().numpy(), rep.cpu().numpy()


def test_noalloc_matches_handle_sampler_on_two_calls():
    assert torch.cuda.is_available()
    for V, Bn, seed in ((T.TURBO_NOALLOC_MAX_VOCAB, T.TURBO_NOALLOC_MAX_BATCH, 11), (50021, 3, 12)):
        W, S, B, _ = synth.make_head(V, D, seed)
        h = T.LMHead(W, S, B, None, vocab=V, hidden=D, softcap=30.0)
        try:
            base, rows, side = case(V, Bn, seed)
            t0, l0, r0 = run(lambda lt, inp, tok, rep: h.sample_logits(lt, inp, tok, rep), base, rows, side)
            t1, l1, r1 = run(lambda lt, inp, tok, rep: T.sample_logits_noalloc(lt, V, inp, tok, rep, softcap=30.0),
                             base, rows, side)
        finally:
            h.close()
        print(f"V={V} B={Bn}: tokens {t1.tolist()} paths {r1.view(np.uint32)[:, 5].tolist()}")
        assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32)), V
        assert np.array_equal(t0, t1), (V, t0, t1)
        assert np.array_equal(r0, r1), V
        assert not np.array_equal(l1, base)  # the modifiers ran


def test_noalloc_rejects_inputs_past_its_scratch():
    lt = torch.zeros((1, 16), dtype=torch.float32, device="cuda")
    tok = torch.zeros(8, dtype=torch.int32, device="cuda")
    inp, keep = T.LMHead.make_inputs(1, [T.row_default()])
    with pytest.raises(T.TurboError, match="vocab must be in"):
        T.sample_logits_noalloc(lt, T.TURBO_NOALLOC_MAX_VOCAB + 64, inp, tok)
    rows = [T.row_default() for _ in range(T.TURBO_NOALLOC_MAX_BATCH + 1)]
    inp, keep = T.LMHead.make_inputs(len(rows), rows)
    with pytest.raises(T.TurboError, match="batch must be in"):
        T.sample_logits_noalloc(lt, 16, inp, tok)


def test_noalloc_allocates_nothing():
    """Once the library has run, an eager call leaves the device's free memory unchanged (no
    hipMalloc behind it; every buffer is caller-provided or the static array)."""
    V, Bn, seed = 70001, 4, 14
    base, rows, side = case(V, Bn, seed)
    kw = dict(history=dev(side["history"].view(np.int32)), history_len=dev(side["history_len"]),
              ban=dev(side["ban"].view(np.int32)), bias_ids=dev(side["bias_ids"].view(np.int32)),
              bias_values=dev(side["bias_values"]), bias_count=dev(side["bias_count"]))
    inp, keep = T.LMHead.make_inputs(Bn, rows, **kw)
    lt = dev(base)
    tok = torch.zeros(Bn, dtype=torch.int32, device="cuda")
    T.sample_logits_noalloc(lt, V, inp, tok, softcap=30.0)  # the static array is set up by now
    torch.cuda.synchronize()
    lt.copy_(dev(base))
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        T.sample_logits_noalloc(lt, V, inp, tok, softcap=30.0)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)


CAPTURE_CHILD = r"""
import sys
sys.path[:0] = {paths!r}
import numpy as np, torch
import turbo_decode_tail as T
import test_zz_no_alloc as Z
V, Bn, seed = 50021, 4, 15
base, rows, side = Z.case(V, Bn, seed)
kw = dict(history=Z.dev(side["history"].view(np.int32)), history_len=Z.dev(side["history_len"]),
          ban=Z.dev(side["ban"].view(np.int32)), bias_ids=Z.dev(side["bias_ids"].view(np.int32)),
          bias_values=Z.dev(side["bias_values"]), bias_count=Z.dev(side["bias_count"]))
inp, keep = T.LMHead.make_inputs(Bn, rows, **kw)
lt = Z.dev(base)
tok = torch.zeros(Bn, dtype=torch.int32, device="cuda")
rep = torch.zeros((Bn, 14), dtype=torch.int32, device="cuda")
torch.cuda.synchronize()
# the process's FIRST call of the entry point is the captured one: the array's address lookup
# and its clear (a fill kernel, recorded as a graph node) happen under capture
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    T.sample_logits_noalloc(lt, V, inp, tok, rep, softcap=30.0, stream=torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()
# the eager result of the handle sampler on the same inputs
W, S, B, _ = Z.synth.make_head(V, Z.D, seed)
h = T.LMHead(W, S, B, None, vocab=V, hidden=Z.D, softcap=30.0)
t0, l0, r0 = Z.run(lambda lt_, i, t, r: h.sample_logits(lt_, i, t, r), base, rows, side)
h.close()
bad = 0
for replay in range(3):
    lt.copy_(Z.dev(base))           # eager work between replays
    tok.zero_(); rep.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    same = (np.array_equal(tok.cpu().numpy(), t0) and np.array_equal(rep.cpu().numpy(), r0)
            and np.array_equal(lt.cpu().numpy().view(np.uint32), l0.view(np.uint32)))
    print(f"replay {{replay}}: {{'equal' if same else 'DIFFERENT'}} tokens {{tok.cpu().numpy().tolist()}}", flush=True)
    bad += 0 if same else 1
# an eager call after the captured ones (the array is cleared again outside capture)
t1, l1, r1 = Z.run(lambda lt_, i, t, r: T.sample_logits_noalloc(lt_, V, i, t, r, softcap=30.0), base, rows, side)
same = np.array_equal(t1, t0) and np.array_equal(r1, r0) and np.array_equal(l1.view(np.uint32), l0.view(np.uint32))
print(f"eager after replays: {{'equal' if same else 'DIFFERENT'}}", flush=True)
bad += 0 if same else 1
sys.exit(1 if bad else 0)
"""


def test_noalloc_first_call_under_graph_capture():
    """The use the entry point exists for: a call recorded into a HIP graph (torch's global capture
    mode, under which any hipMalloc fails) and replayed. Run in a fresh process so that the
    recorded call is the process's first, taking the array's set-up path under capture; every
    replay and a later eager call must equal the handle sampler's eager result bit for bit."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    paths = [str(root / "turbo-winfare_amd"), str(root / "oracle"), str(root / "tests")]
    code = CAPTURE_CHILD.format(paths=paths)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ))
    print(r.stdout)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    assert r.stdout.count("equal") >= 4 and "DIFFERENT" not in r.stdout

"""GPU parity of each kernel-level entry point against the oracle, at sizes the oracle finishes in
seconds. Mirrors the reference's tests/test_gpu_kernels.cpp sections for this path."""
import numpy as np
import pytest

import orc_py as O
import parity_util as U
import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

V_SMALL, D = 16384, 2816


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def small_head():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    W, S, B, g = synth.make_head(V_SMALL, D, 101)
    h = T.LMHead(W, S, B, g, vocab=V_SMALL, hidden=D)
    yield h, (W, S, B, g)
    h.close()


def test_rms_norm_matches_oracle(small_head):
    h, (W, S, B, g) = small_head
    x = synth.hidden_states(3, D, 5)
    out = torch.empty((3, D), dtype=torch.float32, device="cuda")
    h.rms_norm(dev(x), 3, out)
    h.sync()
    got = out.cpu().numpy()
    for b in range(3):
        want = O.rms_norm(x[b], g, 1e-6)
        # same operation sequence (double sum, float 1/sqrt, x*inv*w); the double sum's order
        # differs, so allow one ulp
        assert np.max(np.abs(got[b] - want) / np.maximum(np.abs(want), 1e-30)) <= 2.0**-23


@pytest.mark.parametrize("batch", [1, 2])
def test_logits_digit_path(small_head, batch):
    """GemvInt4 + Softcap at B <= 2: the reference's own tolerance (allclose 1e-5 + 1e-4 |want|)."""
    h, (W, S, B, g) = small_head
    x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, D, 6)])
    out = torch.empty((batch, V_SMALL), dtype=torch.float32, device="cuda")
    h.logits(dev(x), batch, out)
    h.sync()
    got = out.cpu().numpy()
    for b in range(batch):
        want = O.softcap(O.matvec(W, S, B, x[b], U.THREADS), 30.0)
        err = np.abs(got[b] - want)
        assert np.all(err <= 1e-5 + 1e-4 * np.abs(want)), float(np.max(err))
        raw = torch.empty((1, V_SMALL), dtype=torch.float32, device="cuda")
        h.logits(dev(x[b:b + 1]), 1, raw, softcap=False)
        h.sync()
        want_raw = O.matvec(W, S, B, x[b], U.THREADS)
        assert np.all(np.abs(raw.cpu().numpy()[0] - want_raw) <= 1e-5 + 1e-4 * np.abs(want_raw))


@pytest.mark.parametrize("batch", [3, 32, 64, 100, 256])
def test_logits_mfma_path(small_head, batch):
    """Batched head: fp16-dequantised weights, fp32 accumulation, 2e-3 relative (RMS floor)."""
    h, (W, S, B, g) = small_head
    x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, D, 7)])
    out = torch.empty((batch, V_SMALL), dtype=torch.float32, device="cuda")
    h.logits(dev(x), batch, out)
    h.sync()
    got = out.cpu().numpy()
    rows = sorted({0, 1, batch // 2, batch - 1})
    for b in rows:
        want = O.softcap(O.matvec(W, S, B, x[b], U.THREADS), 30.0)
        e = U.logit_err(got[b], want)
        assert e <= U.LOGIT_RTOL, (b, e)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("batch", [3, 64, 256])
def test_logits_mfma_large_activations(small_head, batch, dtype):
    """Normalised rows scaled far past the normalised range (largest |x| 1e4 and 6e4; at 6e4 even
    the unscaled fp16 value is within 10 % of the fp16 maximum and 16 x would be infinite): the
    step prep stores such a row times a power of two and the epilogue multiplies its accumulators
    back, so its logits stay finite and within the tolerance of the oracle's fp32 ones. Rows
    within range are bit-identical to the same rows in a batch without the large ones."""
    h, (W, S, B, g) = small_head
    base = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, D, 12)])
    big = {0: 1.0e4, batch - 1: 6.0e4}
    if batch >= 64:
        big[batch // 2] = 2.5e3  # just past the 2^11 limit
    x = base.copy()
    for b, top in big.items():
        x[b] = (base[b] * (top / np.abs(base[b]).max())).astype(np.float32)

    def run(rows):
        if dtype == "bf16":
            xin, hd = synth.f32_to_bf16(rows), T.TURBO_HIDDEN_BF16
        else:
            xin, hd = rows, T.TURBO_HIDDEN_F32
        out = torch.empty((batch, V_SMALL), dtype=torch.float32, device="cuda")
        h.logits(dev(xin.view(np.int16) if dtype == "bf16" else xin), batch, out, dtype=hd, softcap=False)
        h.sync()
        return out.cpu().numpy()

    got, ref = run(x), run(base)
    for b, top in big.items():
        xb = synth.bf16_to_f32(synth.f32_to_bf16(x[b])) if dtype == "bf16" else x[b]
        want = O.matvec(W, S, B, xb, U.THREADS)
        assert np.all(np.isfinite(got[b])), (b, int((~np.isfinite(got[b])).sum()))
        e = U.logit_err(got[b], want)
        assert e <= U.LOGIT_RTOL, (b, top, e)
    keep = [b for b in range(batch) if b not in big]
    assert np.array_equal(got[keep].view(np.uint32), ref[keep].view(np.uint32))


def test_step_normed_large_activations(small_head):
    """The same through turbo_lmhead_step with TURBO_STEP_NORMED (the caller's rows are not
    normalised again): softcapped logits of rows reaching |x| = 3e4 against the oracle, and greedy
    tokens that are the oracle's (or inside the stated near-tie margin)."""
    h, (W, S, B, g) = small_head
    Bn = 4
    x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(Bn, D, 13)])
    x[1] *= 3.0e4 / np.abs(x[1]).max()
    x[3] *= 5.0e3 / np.abs(x[3]).max()
    x = x.astype(np.float32)
    rows = [T.row_default() for _ in range(Bn)]
    xd = dev(x)  # kept alive: the inputs hold its raw device pointer
    inp, keep = h.make_inputs(Bn, rows, hidden=xd, flags=T.TURBO_STEP_NORMED)
    tok = torch.zeros(Bn, dtype=torch.int32, device="cuda")
    lg = torch.empty((Bn, V_SMALL), dtype=torch.float32, device="cuda")
    h.step(inp, tok, lg)
    h.sync()
    got, toks = lg.cpu().numpy(), tok.cpu().numpy()
    for b in range(Bn):
        raw = O.matvec(W, S, B, x[b], U.THREADS)
        want = O.softcap(raw, 30.0)
        # the tolerance is set on the raw logits (their RMS is ~1e4 for the large rows) and carries
        # through the softcap, whose slope is at most 1
        scale = np.maximum(np.abs(raw), np.sqrt(np.mean(raw.astype(np.float64) ** 2)))
        err = np.abs(got[b].astype(np.float64) - want) / scale
        assert np.all(np.isfinite(got[b])) and float(err.max()) <= U.LOGIT_RTOL, (b, float(err.max()))
        assert U.draw_check(want, O.params(0.0), 0.0, int(toks[b]), mode="margin") in ("exact", "within")


@pytest.mark.parametrize("vocab", [4099, 4100])
@pytest.mark.parametrize("batch", [5, 40, 100])
def test_mfma_history_modifiers_partial_tiles(vocab, batch):
    """Repetition, presence and frequency penalties in the matrix-core epilogue at 32, 64 and 128
    columns per workgroup, where the history counts are read and cleared as 16-byte runs on full
    tiles and one id at a time on a partial last tile (4100 ids: 4 in the last tile) or when rows
    are not 16-byte aligned (4099 ids). The step's final logits must equal the oracle's modifiers
    applied to the head's raw logits bit for bit, twice in a row with different histories (the
    first step's counts must all be cleared)."""
    W, S, B, g = synth.make_head(vocab, D, 107)
    h = T.LMHead(W, S, B, g, vocab=vocab, hidden=D)
    try:
        x = synth.hidden_states(batch, D, 14)
        xd = dev(x)
        rows = [T.row_default(temperature=0.8, top_k=40, top_p=0.9, repetition_penalty=1.3, presence_penalty=0.4,
                              frequency_penalty=0.2, seed=60 + b, counter=1) for b in range(batch)]
        xn = torch.empty((batch, D), dtype=torch.float32, device="cuda")
        h.rms_norm(xd, batch, xn)
        raw = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
        h.logits(xn, batch, raw)
        h.sync()
        raw = raw.cpu().numpy()
        for call in range(2):
            n = 300
            hists = np.stack([synth.zipf_ids(n, vocab, 1.1, 900 + 31 * call + b) for b in range(batch)]).astype(np.uint32)
            hists[:, :6] = [vocab - 1, vocab - 2, vocab - 4, vocab - 1, vocab + 3, 0]  # the last tile, repeats, ignored ids
            hd = dev(hists.view(np.int32))
            hl = torch.full((batch,), n, dtype=torch.int32, device="cuda")
            inp, keep = h.make_inputs(batch, rows, hidden=xd, history=hd, history_len=hl)
            tok = torch.zeros(batch, dtype=torch.int32, device="cuda")
            got = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
            h.step(inp, tok, got)
            h.sync()
            got = got.cpu().numpy()
            for b in sorted({0, batch // 2, batch - 1}):
                want = O.apply_modifiers(raw[b], O.params(0.8, 0.9, 40, 1.3, 0.4, 0.2), 30.0, history=hists[b])
                bad = np.nonzero(got[b].view(np.uint32) != want.view(np.uint32))[0]
                assert bad.size == 0, (call, b, [(int(i), float(got[b, i]), float(want[i])) for i in bad[:6]])
    finally:
        h.close()


@pytest.mark.parametrize("batch", [1, 2, 5, 40, 100])
def test_step_all_modifiers_partial_last_tile(batch):
    """The whole step with every modifier (logit bias with duplicate ids, repetition, presence,
    frequency and a ban mask) on a vocabulary whose last 64-id tile holds 3 ids (4099), through
    each head kernel: the folded digit kernel (1 and 2 rows) and the matrix-core kernels at 32, 64
    and 128 columns. Bias, history and ban hit the last tile's ids. The final logits must equal
    the oracle's modifiers on the head's raw logits bit for bit, and the tokens must pass the
    interval check on those logits. Rows past the vocabulary stay -inf-free: the returned logits
    hold exactly vocab ids per row."""
    vocab = 4099
    W, S, B, g = synth.make_head(vocab, D, 109)
    h = T.LMHead(W, S, B, g, vocab=vocab, hidden=D)
    try:
        x = synth.hidden_states(batch, D, 15)
        xd = dev(x)
        cfgs = [(0.9, 0.9, 40), (0.7, 0.95, 0), (1.2, 0.8, 100)]
        rows = [T.row_default(temperature=cfgs[b % 3][0], top_p=cfgs[b % 3][1], top_k=cfgs[b % 3][2] or 64,
                              repetition_penalty=1.25, presence_penalty=0.3, frequency_penalty=0.15,
                              seed=70 + b, counter=2) for b in range(batch)]
        nh, nbias = 400, 120
        hists = np.stack([synth.zipf_ids(nh, vocab, 1.1, 950 + b) for b in range(batch)]).astype(np.uint32)
        hists[:, :4] = [vocab - 1, vocab - 3, vocab - 1, vocab + 9]
        bl = [synth.bias_list(nbias, vocab, -3.0, 3.0, 960, b) for b in range(batch)]
        bids = np.stack([a for a, _ in bl]).astype(np.uint32)
        bids[:, :3] = [vocab - 2, vocab - 2, vocab - 1]      # the last tile, a duplicate
        bvals = np.stack([v for _, v in bl])
        bans = np.stack([synth.ban_mask(vocab, 0.05, 970, b) for b in range(batch)])
        bans[:, -1] |= np.uint32(1 << ((vocab - 3) % 32))    # a banned id in the last tile
        kw = dict(history=dev(hists.view(np.int32)), history_len=torch.full((batch,), nh, dtype=torch.int32, device="cuda"),
                  ban=dev(bans.view(np.int32)), bias_ids=dev(bids.view(np.int32)), bias_values=dev(bvals),
                  bias_count=torch.full((batch,), nbias, dtype=torch.int32, device="cuda"))
        inp, keep = h.make_inputs(batch, rows, hidden=xd, **kw)
        tok = torch.zeros(batch, dtype=torch.int32, device="cuda")
        got = torch.full((batch, vocab + 1), 7.0, dtype=torch.float32, device="cuda")
        h.step(inp, tok, got)
        xn = torch.empty((batch, D), dtype=torch.float32, device="cuda")
        h.rms_norm(xd, batch, xn)
        raw = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
        h.logits(xn, batch, raw)
        h.sync()
        got, raw, toks = got.cpu().numpy(), raw.cpu().numpy(), tok.cpu().numpy()
        flat = got.reshape(-1)[:batch * vocab].reshape(batch, vocab)  # the step writes [batch][vocab]
        assert np.all(got.reshape(-1)[batch * vocab:] == 7.0)          # nothing past it
        ps, us, finals = [], [], []
        for b in range(batch):
            p = O.params(rows[b].temperature, rows[b].top_p, rows[b].top_k, 1.25, 0.3, 0.15)
            want = O.apply_modifiers(raw[b], p, 30.0, history=hists[b], bias_ids=bids[b], bias_values=bvals[b],
                                     ban=bans[b])
            bad = np.nonzero(flat[b].view(np.uint32) != want.view(np.uint32))[0]
            assert bad.size == 0, (b, [(int(i), float(flat[b, i]), float(want[i])) for i in bad[:6]])
            assert np.isneginf(flat[b, vocab - 3])
            ps.append(p)
            us.append(T.row_uniform(rows[b]))
            finals.append(want)
        U.check_tokens(ps, toks.astype(np.uint32), finals, us, label=f"all modifiers B={batch}")
    finally:
        h.close()


@pytest.mark.parametrize("batch", [1, 2, 4])
def test_step_injected_uniforms(small_head, batch):
    """Caller-supplied uniforms (TurboStepInputs.uniforms) replace each row's generator: the
    edge values 0 (the top survivor) and 1 - 2^-24 (the last one) and two inner values, on
    shortlist and full-vocabulary rows, through the folded digit head (1, 2 rows) and the
    matrix-core head (4 rows). The report carries the uniform used, and every token is the oracle
    sampler's on the GPU's logits with that uniform (interval-checked)."""
    h, (W, S, B, g) = small_head
    cfgs = [(0.8, 0.95, 64, 0), (1.0, 0.9, 0, 1), (0.7, 1.0, 40, 0), (1.3, 0.5, 0, 1)]
    us_all = np.array([0.0, 1.0 - 2.0 ** -24, 0.5, 0.123456], np.float32)
    x = synth.hidden_states(batch, D, 16)
    xd = dev(x)
    for shift in range(4):
        rows = [T.row_default(temperature=cfgs[(b + shift) % 4][0], top_p=cfgs[(b + shift) % 4][1],
                              top_k=cfgs[(b + shift) % 4][2], seed=5, counter=9,
                              flags=T.TURBO_ROW_FULL_VOCAB if cfgs[(b + shift) % 4][3] else 0)
                for b in range(batch)]
        us = np.roll(us_all, shift)[:batch].copy()
        ud = dev(us)
        inp, keep = h.make_inputs(batch, rows, hidden=xd, uniforms=ud)
        tok = torch.zeros(batch, dtype=torch.int32, device="cuda")
        lg = torch.empty((batch, V_SMALL), dtype=torch.float32, device="cuda")
        rep = torch.zeros((batch, 56 // 4), dtype=torch.int32, device="cuda")
        h.step(inp, tok, lg, rep)
        h.sync()
        got = rep.cpu().numpy()
        assert np.array_equal(got[:, 1].view(np.float32), us), (shift, got[:, 1].view(np.float32), us)
        ps = [O.params(r.temperature, r.top_p, r.top_k, 1.0, 0.0, 0.0, r.flags) for r in rows]
        c = U.check_tokens(ps, tok.cpu().numpy().astype(np.uint32), lg.cpu().numpy(), [float(u) for u in us],
                           within_frac=1.0, label=f"injected uniforms B={batch} shift {shift}")
        assert c["exact"] == batch


@pytest.mark.parametrize("batch", [1, 4])
def test_step_on_caller_stream_and_head_timing(batch):
    """turbo_lmhead_set_stream: steps enqueued on a caller's stream run after the work already on
    it (here a hidden-state copy queued behind a chain of matrix products) and give the null
    stream's tokens, logits and reports bit for bit. turbo_lmhead_enable_head_timing counts every
    N-th head launch: 3 of 3 at N = 1, launches 0, 3 and 6 of 7 at N = 3, none when off."""
    W, S, B, g = synth.make_head(V_SMALL, D, 101)
    h = T.LMHead(W, S, B, g, vocab=V_SMALL, hidden=D)
    try:
        rows = [T.row_default(temperature=0.8, top_p=0.95, top_k=64, seed=3 + b, counter=1) for b in range(batch)]
        x = synth.hidden_states(batch, D, 21)
        xd = dev(x)

        def outputs():
            return (torch.zeros(batch, dtype=torch.int32, device="cuda"),
                    torch.empty((batch, V_SMALL), dtype=torch.float32, device="cuda"),
                    torch.zeros((batch, 56 // 4), dtype=torch.int32, device="cuda"))

        tok0, lg0, rep0 = outputs()
        inp0, keep0 = h.make_inputs(batch, rows, hidden=xd)
        h.step(inp0, tok0, lg0, rep0)
        h.sync()

        s = torch.cuda.Stream()
        xs = torch.zeros_like(xd)
        tok1, lg1, rep1 = outputs()
        torch.cuda.synchronize()
        h.set_stream(s.cuda_stream)
        h.enable_head_timing(True, every=1)
        with torch.cuda.stream(s):
            m = torch.full((2048, 2048), 1.0 / 2048, device="cuda")
            for _ in range(8):
                m = m @ m
            xs.copy_(xd)
        inp1, keep1 = h.make_inputs(batch, rows, hidden=xs)
        for _ in range(3):
            h.step(inp1, tok1, lg1, rep1)
        h.sync()
        ms, n = h.head_kernel_time(reset=True)
        assert n == 3 and ms > 0.0, (ms, n)
        assert np.array_equal(tok1.cpu().numpy(), tok0.cpu().numpy())
        assert np.array_equal(lg1.cpu().numpy().view(np.uint32), lg0.cpu().numpy().view(np.uint32))
        assert np.array_equal(rep1.cpu().numpy(), rep0.cpu().numpy())

        h.enable_head_timing(True, every=3)
        for _ in range(7):
            h.step(inp1, tok1, lg1, rep1)
        ms, n = h.head_kernel_time(reset=True)
        assert n == 3 and ms > 0.0, (ms, n)
        h.enable_head_timing(False)
        for _ in range(2):
            h.step(inp1, tok1, lg1, rep1)
        ms, n = h.head_kernel_time(reset=True)
        assert n == 0 and ms == 0.0, (ms, n)
        h.set_stream(None)  # waits for s
        assert np.array_equal(tok1.cpu().numpy(), tok0.cpu().numpy())
    finally:
        h.close()


@pytest.mark.parametrize("vocab,batch", [(300, 40), (4099, 48), (1100, 33)])
def test_logits_mfma_partial_workgroups(vocab, batch):
    """64-column heads run 16 tiles per workgroup: vocabularies of 5, 65 and 18 tiles leave the
    only or the last workgroup partly past the table, and batches of 33 - 48 rows a partial
    column block (columns past the batch read zeros and store nothing)."""
    W, S, B, g = synth.make_head(vocab, D, 105)
    h = T.LMHead(W, S, B, g, vocab=vocab, hidden=D)
    try:
        x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, D, 11)])
        out = torch.full((batch + 1, vocab), 7.0, dtype=torch.float32, device="cuda")
        h.logits(dev(x), batch, out)
        h.sync()
        got = out.cpu().numpy()
        for b in sorted({0, 31, 32, batch - 1}):
            want = O.softcap(O.matvec(W, S, B, x[b], U.THREADS), 30.0)
            assert U.logit_err(got[b], want) <= U.LOGIT_RTOL, b
        assert np.all(got[batch] == 7.0)  # the row past the batch is untouched
    finally:
        h.close()


def test_logits_mfma_bf16_input(small_head):
    h, (W, S, B, g) = small_head
    xb = synth.f32_to_bf16(synth.hidden_states(8, D, 8))
    out = torch.empty((8, V_SMALL), dtype=torch.float32, device="cuda")
    h.logits(dev(xb.view(np.int16)), 8, out, dtype=T.TURBO_HIDDEN_BF16)
    h.sync()
    got = out.cpu().numpy()
    for b in (0, 7):
        want = O.softcap(O.matvec(W, S, B, synth.bf16_to_f32(xb[b]), U.THREADS), 30.0)
        assert U.logit_err(got[b], want) <= U.LOGIT_RTOL


def test_greedy_matches_full_gemv_argmax():
    """LMHeadGreedy + ArgmaxReduce (tests/test_gpu_kernels.cpp:743-802): 4096 x 2816, x ~ U(-1.5,1.5)."""
    W, S, B, g = synth.make_head(4096, D, 12345)
    h = T.LMHead(W, S, B, None, vocab=4096, hidden=D)
    try:
        for seed in range(4):
            x = (synth.uniform(seed, 70, D) * 3.0 - 1.5).astype(np.float32)
            tok = torch.zeros(1, dtype=torch.int32, device="cuda")
            h.greedy(dev(x[None]), 1, tok)
            h.sync()
            want = O.softcap(O.matvec(W, S, B, x), 30.0)
            if U.greedy_near_tie(want):
                continue
            assert int(tok.item()) == int(np.argmax(want))
    finally:
        h.close()


def test_greedy_ties_go_to_lowest_row():
    """Rows 5, 77 and 1000 are identical and hold the maximum: the lowest index must win."""
    V = 2048
    W, S, B, _ = synth.make_head(V, D, 3)
    x = synth.hidden_states(1, D, 9)[0]
    q = np.where(x > 0, 15, 0).astype(np.uint8)
    row = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    for r in (1000, 77, 5):
        W[r] = row
        S[r] = synth.f32_to_bf16(np.full(D // 64, 0.01, np.float32))
        B[r] = 0
    want = O.softcap(O.matvec(W, S, B, x), 30.0)
    assert want[5] == want[77] == want[1000] == want.max()
    h = T.LMHead(W, S, B, None, vocab=V, hidden=D)
    try:
        tok = torch.zeros(1, dtype=torch.int32, device="cuda")
        h.greedy(dev(x[None]), 1, tok)
        h.sync()
        assert int(tok.item()) == 5
    finally:
        h.close()


def test_softcap_kernel():
    z = (synth.uniform(1, 71, 4096) * 400 - 200).astype(np.float32)  # U(-200, 200) as :389-411
    t = torch.from_numpy(z).cuda()
    T.softcap(t, z.size, 30.0)
    torch.cuda.synchronize()
    want = O.softcap(z, 30.0)
    got = t.cpu().numpy()
    assert np.all(np.abs(got - want) <= 1e-5 + 1e-4 * np.abs(want))
    assert np.all(got[np.abs(z) > 300] == np.sign(z[np.abs(z) > 300]) * 30.0)


def test_repetition_penalty_kernel():
    V = 262144
    for (n, p) in [(256, 1.1), (2048, 1.15), (5000, 0.8), (0, 2.0)]:
        l = (synth.normal(n, 72, V) * 10).astype(np.float32)
        hist = synth.zipf_ids(max(n, 1), V + 100, 1.1, n)[:n]  # duplicates and out-of-range ids
        t = torch.from_numpy(l).cuda()
        T.apply_repetition_penalty(t, V, torch.from_numpy(hist.astype(np.int32)).cuda() if n else None,
                                   n, p, 30.0)
        torch.cuda.synchronize()
        want = l.copy()
        O.orc().orc_apply_repetition_penalty(want, V, hist.ctypes.data if n else None, n, p, 30.0)
        assert np.array_equal(t.cpu().numpy(), want)


@pytest.mark.parametrize("batch", [3, 64])
def test_logits_mfma_path_large_scales(batch):
    """The batched head's fp16 dequant has two forms: nibbles as fp16 denormals times s * 2^20
    (every |s| < 1/16) and nibbles through the mantissa of 1024.0 (any scale). A head whose group
    scales reach past 1/16 (the synthetic scales times 16, so the largest are ~0.3) takes the
    second form on every batched kernel, with the same tolerance."""
    Vh = 8192
    W, S, B, g = synth.make_head(Vh, D, 103)
    S = synth.f32_to_bf16(synth.bf16_to_f32(S) * 16.0)
    B = synth.f32_to_bf16(synth.bf16_to_f32(B) * 16.0)  # the same q - 8 centring
    assert float(synth.bf16_to_f32(S).max()) > 1.0 / 16
    h = T.LMHead(W, S, B, g, vocab=Vh, hidden=D)
    try:
        x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, D, 8)])
        out = torch.empty((batch, Vh), dtype=torch.float32, device="cuda")
        h.logits(dev(x), batch, out)
        h.sync()
        got = out.cpu().numpy()
        for b in sorted({0, batch // 2, batch - 1}):
            want = O.softcap(O.matvec(W, S, B, x[b], U.THREADS), 30.0)
            assert U.logit_err(got[b], want) <= U.LOGIT_RTOL, b
    finally:
        h.close()


@pytest.mark.parametrize("hidden", [2944, 2880])
@pytest.mark.parametrize("batch", [3, 64, 130])
def test_logits_mfma_path_other_group_counts(hidden, batch):
    """The batched head prefetches four 64-element groups ahead when the group count allows it,
    else two (hidden 2944: 46 groups), else one (hidden 2880: 45 groups). A vocabulary of 4099
    rows leaves a partial last tile and rows that are not 16-byte aligned (element stores), and
    130 rows a partial second column block."""
    Vh = 4099
    W, S, B, g = synth.make_head(Vh, hidden, 104)
    h = T.LMHead(W, S, B, g, vocab=Vh, hidden=hidden)
    try:
        x = np.stack([O.rms_norm(r, g, 1e-6) for r in synth.hidden_states(batch, hidden, 9)])
        out = torch.empty((batch, Vh), dtype=torch.float32, device="cuda")
        h.logits(dev(x), batch, out)
        h.sync()
        got = out.cpu().numpy()
        for b in sorted({0, batch // 2, batch - 1}):
            want = O.softcap(O.matvec(W, S, B, x[b], U.THREADS), 30.0)
            assert U.logit_err(got[b], want) <= U.LOGIT_RTOL, b
    finally:
        h.close()

"""turbo_int4_matvec at the projection shapes the reference dispatches GemvInt4 for
(src/runner.cpp:431-442, :621-646, :671-678): routed-expert gate/up (704 x 2816) and down
(2816 x 704), shared-expert gate/up (2112 x 2816) and down (2816 x 2112), and the q projection
(4096 x 2816). Small batches run the digit-plane GEMV and meet the reference's allclose
(1e-5 + 1e-4 |want|); batched calls run the fp16-dequant MFMA path and meet 2e-3 relative to
the row RMS. The oracle is the pinned matvec restatement (src/cpu_reference.cpp:55-84)."""
import numpy as np
import pytest

import orc_py as O
import parity_util as U
import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SHAPES = [(704, 2816), (2816, 704), (2112, 2816), (2816, 2112), (4096, 2816)]


@pytest.mark.parametrize("rows,in_dim", SHAPES)
def test_matvec_projection_shapes(rows, in_dim):
    W, S, B, _ = synth.make_head(rows, in_dim, rows + in_dim)
    h = T.LMHead(W, S, B, None, vocab=rows, hidden=in_dim, softcap=0.0)
    try:
        for batch in (1, 2, 8):
            x = synth.hidden_states(batch, in_dim, 40 + batch)
            out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
            h.matvec(torch.from_numpy(x).cuda(), batch, out)
            h.sync()
            got = out.cpu().numpy()
            for b in range(batch):
                want = O.matvec(W, S, B, x[b], U.THREADS)
                if batch <= 2:
                    assert np.all(np.abs(got[b] - want) <= 1e-5 + 1e-4 * np.abs(want)), (batch, b)
                else:
                    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
                    err = np.abs(got[b] - want) / np.maximum(np.abs(want), rms)
                    assert float(err.max()) <= 2e-3, (batch, b, float(err.max()))
    finally:
        h.close()


@pytest.mark.parametrize("rows,in_dim", SHAPES)
@pytest.mark.parametrize("bf16", [False, True])
def test_folded_matvec_matches_prepared(rows, in_dim, bf16):
    """One or two 16-byte-aligned rows run the split kernel with the digit planes computed in
    each workgroup (no preparation kernel); a row at a 4-byte offset takes the preparation
    kernel. Both must give bit-identical outputs, for fp32 and bf16 input."""
    W, S, B, _ = synth.make_head(rows, in_dim, rows + in_dim + 1)
    h = T.LMHead(W, S, B, None, vocab=rows, hidden=in_dim, softcap=0.0)
    try:
        for batch in (1, 2):
            x = synth.hidden_states(batch, in_dim, 60 + batch)
            if bf16:
                xs = torch.from_numpy(synth.f32_to_bf16(x).view(np.int16)).cuda()
                dt = T.TURBO_HIDDEN_BF16
                pad = 8  # 16 bytes of bf16: the unaligned copy starts 2 elements (4 bytes) in
            else:
                xs = torch.from_numpy(x).cuda()
                dt = T.TURBO_HIDDEN_F32
                pad = 4
            flat = xs.reshape(-1)
            buf = torch.zeros(flat.numel() + pad, dtype=flat.dtype, device="cuda")
            off = 2 if bf16 else 1
            buf[off:off + flat.numel()] = flat
            un = buf[off:off + flat.numel()]
            assert xs.data_ptr() % 16 == 0 and un.data_ptr() % 16 == 4
            o1 = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
            o2 = torch.full_like(o1, float("nan"))
            h.matvec(xs, batch, o1, dtype=dt)
            h.matvec(un, batch, o2, dtype=dt)
            h.sync()
            a, b = o1.cpu().numpy(), o2.cpu().numpy()
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (batch, bf16)
            # the greedy entry folds the same way; its select reads the rows the head stored
            t1 = torch.full((batch,), -1, dtype=torch.int32, device="cuda")
            t2 = torch.full_like(t1, -1)
            h.greedy(xs, batch, t1, dtype=dt)
            h.greedy(un, batch, t2, dtype=dt)
            h.sync()
            want = [int(np.argmax(a[r])) for r in range(batch)]  # no softcap on this head
            assert t1.cpu().tolist() == want and t2.cpu().tolist() == want, (batch, bf16)
    finally:
        h.close()


def test_folded_logits_big_head_matches_prepared():
    """turbo_lmhead_logits on a head with many tiles folds the digit planes into the 16-tile
    workgroup kernel; the same rows at an unaligned address take the preparation kernel."""
    V, D = 262144, 2816
    W, S, B, g = synth.make_head(V, D, 91)
    h = T.LMHead(W, S, B, g, vocab=V, hidden=D, softcap=30.0)
    try:
        for batch in (1, 2):
            x = torch.from_numpy(synth.hidden_states(batch, D, 92 + batch)).cuda()
            flat = x.reshape(-1)
            buf = torch.zeros(flat.numel() + 4, dtype=torch.float32, device="cuda")
            buf[1:1 + flat.numel()] = flat
            un = buf[1:1 + flat.numel()]
            l1 = torch.full((batch, V), float("nan"), dtype=torch.float32, device="cuda")
            l2 = torch.full_like(l1, float("nan"))
            h.logits(x, batch, l1)
            h.logits(un, batch, l2)
            h.sync()
            a, b = l1.cpu().numpy(), l2.cpu().numpy()
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), batch
            t1 = torch.full((batch,), -1, dtype=torch.int32, device="cuda")
            t2 = torch.full_like(t1, -1)
            h.greedy(x, batch, t1)
            h.greedy(un, batch, t2)
            h.sync()
            want = [int(np.argmax(a[r])) for r in range(batch)]  # argmax of the softcapped logits
            assert t1.cpu().tolist() == want and t2.cpu().tolist() == want, batch
    finally:
        h.close()


def test_grouped_matvec_matches_head_calls():
    """turbo_int4_matvec_grouped: the 8 routed experts' gate and up matrices (16 x 704 x 2816)
    with one input row, then their 8 down matrices (2816 x 704) each with its own row, in one
    launch each, from matrix handles that hold only the tables. Every output must equal the
    same matrix's turbo_int4_matvec through a head bit for bit, and the oracle to the reference's
    tolerance. One matrix is loaded from device memory (the slot-refill path), the rest from host
    arrays; a second load replaces a matrix's contents."""
    rng_mats = []
    for e in range(8):
        for kind, (rows, k) in (("gate", (704, 2816)), ("up", (704, 2816))):
            rng_mats.append((rows, k, 1000 + 2 * e + (kind == "up")))
    downs = [(2816, 704, 2000 + e) for e in range(8)]
    for group, shared_x in ((rng_mats, True), (downs, False)):
        mats, tables = [], []
        for i, (rows, k, seed) in enumerate(group):
            W, S, B, _ = synth.make_head(rows, k, seed)
            m = T.Int4Matrix(rows, k)
            if i == 0:
                m.load_weights(torch.from_numpy(W).cuda(), torch.from_numpy(S.view(np.int16)).cuda(),
                               torch.from_numpy(B.view(np.int16)).cuda(), on_device=True)
            else:
                m.load_weights(W, S, B)
            mats.append(m)
            tables.append((W, S, B))
        k = group[0][1]
        xs_np = [synth.hidden_states(1, k, 70 + (0 if shared_x else i))[0] for i in range(len(group))]
        xs = [torch.from_numpy(x).cuda() for x in xs_np]
        outs = [torch.full((r,), float("nan"), dtype=torch.float32, device="cuda") for r, _, _ in group]
        T.matvec_grouped(mats, xs, outs)
        torch.cuda.synchronize()
        for i, (rows, kk, seed) in enumerate(group):
            W, S, B = tables[i]
            got = outs[i].cpu().numpy()
            want = O.matvec(W, S, B, xs_np[i], U.THREADS)
            assert np.all(np.abs(got - want) <= 1e-5 + 1e-4 * np.abs(want)), i
            h = T.LMHead(W, S, B, None, vocab=rows, hidden=kk, softcap=0.0)
            try:
                ref = torch.empty((1, rows), dtype=torch.float32, device="cuda")
                h.matvec(xs[i].view(1, kk), 1, ref)
                h.sync()
                assert np.array_equal(got.view(np.uint32), ref.cpu().numpy()[0].view(np.uint32)), i
            finally:
                h.close()
        # reload one matrix with another table: the next call uses the new contents
        W2, S2, B2, _ = synth.make_head(group[1][0], group[1][1], 999)
        mats[1].load_weights(W2, S2, B2)
        T.matvec_grouped(mats[:2], xs[:2], outs[:2])
        torch.cuda.synchronize()
        want = O.matvec(W2, S2, B2, xs_np[1], U.THREADS)
        assert np.all(np.abs(outs[1].cpu().numpy() - want) <= 1e-5 + 1e-4 * np.abs(want))
        for m in mats:
            m.close()


def test_grouped_matvec_rejects_bad_calls():
    m = T.Int4Matrix(64, 128)
    try:
        x = torch.zeros(128, dtype=torch.float32, device="cuda")
        o = torch.zeros(64, dtype=torch.float32, device="cuda")
        with pytest.raises(T.TurboError, match="count must be in"):
            T.matvec_grouped([m] * 33, [x] * 33, [o] * 33)
        with pytest.raises(T.TurboError, match="16-byte aligned"):
            T.matvec_grouped([m], [x.data_ptr() + 4], [o])
        T.matvec_grouped([], [], [])  # nothing to do
    finally:
        m.close()
    with pytest.raises(T.TurboError, match="in_dim must be"):
        T.Int4Matrix(64, 100)

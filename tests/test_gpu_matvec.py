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

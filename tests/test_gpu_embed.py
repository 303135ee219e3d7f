"""turbo_lmhead_embed on the GPU against the oracle's embedding row (src/cpu_reference.cpp:108-124,
:323-329), bit-exact: the lookup reads the head's tiled copy of the tied table, so this also
checks the tiling round trip row by row."""
import numpy as np
import pytest

import orc_py as O
import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("V,D", [(8192, 2816), (704, 2816), (4096, 704)])
def test_embed_rows_bit_exact(V, D):
    W, S, B, g = synth.make_head(V, D, 21)
    h = T.LMHead(W, S, B, g, vocab=V, hidden=D)
    try:
        rng = np.random.default_rng(5)
        ids = np.concatenate([[0, 1, 63, 64, V - 1, V - 1], rng.integers(0, V, 26)]).astype(np.uint32)
        tok = torch.from_numpy(ids.view(np.int32)).cuda()
        out = torch.empty((ids.size, D), dtype=torch.float32, device="cuda")
        h.embed(tok, ids.size, out)
        h.sync()
        got = out.cpu().numpy()
        for i, t in enumerate(ids):
            want = O.embed(W, S, B, int(t))
            assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), (i, int(t))
        # an id past the vocabulary gives a NaN row; a zero-length call is a no-op
        bad = torch.tensor([V, 3], dtype=torch.int32, device="cuda")
        out2 = torch.zeros((2, D), dtype=torch.float32, device="cuda")
        h.embed(bad, 2, out2)
        h.embed(bad, 0, out2)
        h.sync()
        o2 = out2.cpu().numpy()
        assert np.isnan(o2[0]).all()
        assert np.array_equal(o2[1], O.embed(W, S, B, 3))
    finally:
        h.close()

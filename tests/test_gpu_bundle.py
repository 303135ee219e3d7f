"""turbo_lmhead_create_from_bundle on the GPU: a head read from a resident.bin (the tied table
and the final norm at their 16 KB-aligned regions) computes exactly what the same tensors
handed over as arrays compute, on both head paths."""
import numpy as np
import pytest

import bundle_util as BU
import synth
import turbo_decode_tail as T

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_bundle_head_matches_array_head(tmp_path):
    V, D = 4096, 2816
    W, S, B, g = synth.make_head(V, D, 11)
    p = tmp_path / "resident.bin"
    BU.write_resident(p, BU.head_tensors(W, S, B, g))
    ha = T.LMHead(W, S, B, g, vocab=V, hidden=D, softcap=30.0, eps=1e-6)
    hb = T.LMHead.from_bundle(p, softcap=30.0, eps=1e-6)
    try:
        assert (hb.vocab, hb.hidden) == (V, D)
        for batch in (1, 4):  # digit-plane GEMV, then the MFMA path
            x = torch.from_numpy(synth.hidden_states(batch, D, 11, batch)).cuda()
            la = torch.empty((batch, V), dtype=torch.float32, device="cuda")
            lb = torch.empty_like(la)
            n = torch.empty((batch, D), dtype=torch.float32, device="cuda")
            ha.rms_norm(x, batch, n)
            ha.logits(n, batch, la)
            hb.logits(n, batch, lb)
            ha.sync()
            hb.sync()
            assert torch.equal(la, lb), batch
            ta = torch.zeros(batch, dtype=torch.int32, device="cuda")
            tb = torch.zeros_like(ta)
            ha.greedy(n, batch, ta)
            hb.greedy(n, batch, tb)
            ha.sync()
            hb.sync()
            assert torch.equal(ta, tb), batch
    finally:
        ha.close()
        hb.close()


def test_bundle_without_norm_is_rejected(tmp_path):
    V, D = 256, 128
    W, S, B, g = synth.make_head(V, D, 3)
    p = tmp_path / "resident.bin"
    BU.write_resident(p, BU.head_tensors(W, S, B, g, extra=False)[:1])  # the table only
    with pytest.raises(T.TurboError, match="no tensor 'model.norm.weight'"):
        T.LMHead.from_bundle(p)

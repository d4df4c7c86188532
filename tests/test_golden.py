"""Golden fixture tests (tests/golden/wlq_small.npz, written by make_golden.py):
the oracle reproduces the frozen vectors bit for bit (CPU), and the HIP path
matches them (GPU: dequant bit-exact, products within the layer tolerance)."""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import wlq_oracle as O

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "wlq_small.npz")
TAGS = ("b4g128", "b3row")


def _load(tag):
    z = np.load(FIX, allow_pickle=False)
    d = {k[len(tag) + 1:]: z[k] for k in z.files if k.startswith(tag + "_")}
    N, K, bits, gs, wpr = (int(v) for v in d["meta"])
    return d, N, K, bits, gs, wpr


@pytest.mark.parametrize("tag", TAGS)
def test_oracle_reproduces_golden(tag):
    d, N, K, bits, gs, wpr = _load(tag)
    assert wpr == O.words_per_row(K, bits)
    W0 = O.dequant(d["q"], d["lut"], N, K, bits, d["offsets"], d["cols"], d["vals"], group_size=gs)
    assert np.array_equal(W0.view(np.uint16), d["W0"].view(np.uint16))
    for m in ("1", "16"):
        y = O.apply(d["x" + m], W0, d["A"], d["B"], d["gamma"], 1.0)
        assert np.array_equal(y.view(np.uint16), d["y" + m].view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("tag", TAGS)
def test_hip_matches_golden(vw, tag):
    import torch

    from gpu_helpers import DEV, check_close

    d, N, K, bits, gs, wpr = _load(tag)
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).to(DEV) for k, v in d.items() if k != "meta"}
    cols = torch.from_numpy(d["cols"].view(np.int16)).to(DEV).view(torch.uint16)
    W = torch.empty((N, K), dtype=torch.float16, device=DEV)
    vw._C.dequant_w0(t["q"], t["lut"], W, N, K, bits, wpr, t["offsets"], cols, t["vals"], gs)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy().view(np.uint16), d["W0"].view(np.uint16))
    for m in ("1", "16"):
        x = t["x" + m]
        M = x.shape[0]
        out = torch.empty((M, N), dtype=torch.float16, device=DEV)
        torch.ops.wlq_fastShot.gemm(x, t["q"], t["lut"], out, N, K, bits, wpr, t["offsets"], cols, t["vals"], None,
                                    t["B"], t["gamma"], 1.0, gs, t["A"])
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), d["y" + m], what=f"golden {tag} M={M}")

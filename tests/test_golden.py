"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the
oracle): the oracle must reproduce them bit for bit (CPU), and the device path must match them
(GPU: the Q8_0 GEMV and the 4-layer engine through the C ABI)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

NAMES = list(G.MAKERS)


def load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    want = load(name)
    got = G.MAKERS[name]()
    assert set(got) == set(want)
    for k in want:
        a, b = np.asarray(got[k]), want[k]
        assert a.shape == b.shape and a.dtype == b.dtype, k
        assert a.tobytes() == b.tobytes(), f"{name}.{k} differs"


@pytest.mark.gpu
def test_gpu_gemv_matches_golden(dev):
    import torch
    import oxe_amd as A
    g = load("config1_slice")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    isum = torch.empty(g["isum"].shape, dtype=torch.int32, device=dev)
    y = A.gemv_q8_0(t(g["wq"]), t(g["wd"].view(np.int16)), t(g["xq"]), t(g["xd"].view(np.int16)), isum=isum)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), g["y"].view(np.uint32))
    assert np.array_equal(isum.cpu().numpy(), g["isum"])


@pytest.mark.gpu
def test_gpu_engine_matches_golden(dev):
    import oracle as O
    import oxe_amd as A
    g = load("engine_small")
    e = A.Engine(O.desc_small(), seed=3, n_ctx=256)
    x = None
    for t in g["prompt"]:
        x = e.step(int(t))
    for i in range(len(g["ids"])):
        assert x == int(g["ids"][i]), i
        assert G.fnv64(e.logits(0)) == int(g["logits_fnv"][i]), i
        assert G.fnv64(e.hidden(0)) == int(g["hidden_fnv"][i]), i
        x = e.step(x)
    e.close()

"""K-quant kernels on the GPU against the oracle (oracle/kquants.cpp, pinned in test_kquants.py):
the q8_K quantizer byte for byte, and the Q3_K / Q4_K / Q5_K / Q6_K lane GEMVs (oxe_vl_gemv) bit
for bit for 1..4 lanes, ragged row counts and every chunking of k the kernel takes."""
import numpy as np
import pytest

import kquant_blocks as KB
import oracle as O

pytestmark = pytest.mark.gpu


def test_quantize_q8_K_matches_oracle(dev):
    import oxe_amd as A
    import torch
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 1024)).astype(np.float32)
    x[0, :256] = 0.0                                   # zero block
    x[1, 10], x[1, 200] = 4.0, -4.0                    # |max| tie: the first wins
    x[2, :256] = rng.standard_normal(256).astype(np.float32) * 1e-30   # tiny values
    x[3] *= 1e4
    x[4, 256:512] = np.round(x[4, 256:512] * 4) / 4   # quarter steps: halves after scaling are common
    x[5, 512] = -127.0                                 # unit scale: codes = round-half-even(x)
    x[5, 513:768] = (np.arange(255) - 127) * 0.5
    got = A.quantize_q8_K(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert np.array_equal(got, O.quantize_q8_K(x))


CASES = [   # (type, k, nr, nl)
    (4, 2048, 300, 2), (4, 256, 5, 1), (4, 768, 33, 3), (4, 4096, 64, 4), (4, 512, 7, 2),
    (5, 2048, 300, 2), (5, 256, 9, 4), (5, 1280, 17, 1), (5, 512, 128, 3),
    (6, 2048, 300, 2), (6, 512, 7, 1), (6, 2560, 19, 4), (6, 4096, 40, 3),
    (3, 2048, 300, 2), (3, 512, 11, 4), (3, 1536, 23, 1), (3, 4096, 8, 3),
]


@pytest.mark.parametrize("ty,k,nr,nl", CASES)
def test_vl_gemv_matches_oracle(dev, ty, k, nr, nl):
    import oxe_amd as A
    import torch
    print(f"vl_gemv type {ty} k {k} nr {nr} nl {nl}", flush=True)
    w = KB.random_blocks(ty, nr, k, seed=1000 * ty + k + nr)
    x = np.random.default_rng(nr + k).standard_normal((nl, k)).astype(np.float32)
    yd = A.quantize_q8_K(torch.from_numpy(x).to(dev))
    y = yd.cpu().numpy()
    assert np.array_equal(y, O.quantize_q8_K(x))
    got = A.vl_gemv(ty, torch.from_numpy(w).to(dev), k, yd)
    assert got is not None
    want = O.vl_gemv(ty, w, k, y)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_vl_gemv_not_handled(dev):
    import oxe_amd as A
    import torch
    w = torch.zeros((4, 3 * 210), dtype=torch.uint8, device=dev)
    y = torch.zeros((1, 3 * 292), dtype=torch.uint8, device=dev)
    s = torch.full((1, 4), 7.0, device=dev)
    assert A.vl_gemv(6, w, 768, y, s) is None          # Q6_K with an odd block count
    assert A.vl_gemv(2, w, 768, y, s) is None          # Q2_K: no kernel
    y5 = torch.zeros((5, 3 * 292), dtype=torch.uint8, device=dev)
    assert A.vl_gemv(4, torch.zeros((4, 3 * 144), dtype=torch.uint8, device=dev), 768, y5) is None   # 5 lanes
    torch.cuda.synchronize()
    assert bool((s == 7.0).all())                       # nothing written

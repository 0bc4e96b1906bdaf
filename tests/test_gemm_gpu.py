"""The prefill Q8_0 GEMM (int8 matrix cores for the block dots, fp32 chain over blocks in order)
through the C ABI against the oracle's GEMV: ggml_gemm_q8_0_4x8_q8_0 equals the GEMV per (row,
token) bit for bit (docs/lab-notes/M3-PREFILL.md:70-71), so the oracle runs the GEMV with one lane
per token. Bar: fp32 outputs bit-exact, including ragged row and token counts."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("k,nr,nt", [(2048, 256, 64), (2048, 1000, 37), (512, 2048, 100), (4096, 130, 5),
                                     (2048, 40, 1), (2048, 4096, 200),
                                     # one and three 128-byte stages (the double-buffered loop's odd ends)
                                     (128, 64, 3), (384, 200, 70)])
def test_gemm_bitexact_vs_oracle(dev, k, nr, nt):
    import oxe_amd as A
    wq, wd = O.synth_q8(11, 3, O.T["OUTPUT"], nr, k)
    x = (O.synth_normal(11, 7 * 64 + nt, nt * k).reshape(nt, k) * 3.0).astype(np.float32)
    xq, xd = O.quantize_q8_0(x)
    y_ref = O.gemv_q8_0(wq, wd, xq, xd)
    y = A.gemm_q8_0(_t(wq, dev), _t(wd.view(np.int16), dev), _t(xq, dev), _t(xd.view(np.int16), dev))
    got = y.cpu().numpy()
    assert got.shape == (nt, nr)
    bad = np.nonzero(got.view(np.uint32) != y_ref.view(np.uint32))
    assert bad[0].size == 0, f"{bad[0].size} outputs differ, first (token, row) {bad[0][0]}, {bad[1][0]}"


def test_gemm_equals_gemv_large(dev):
    """2048 tokens (the prefill batch of BASELINE config 5) against the device GEMV, 2 lanes at a
    time (the GEMV itself is checked bit for bit against the oracle in test_gemv_gpu.py)."""
    import oxe_amd as A
    import torch
    k, nr, nt = 2048, 1024, 2048
    wq, wd = O.synth_q8(5, 9, O.T["OUTPUT"], nr, k)
    x = torch.randn(nt, k, device=dev) * 2.0
    xq, xd = A.quantize_q8_0(x)
    w_q, w_d = _t(wq, dev), _t(wd.view(np.int16), dev)
    y = A.gemm_q8_0(w_q, w_d, xq, xd)
    ref = torch.empty_like(y)
    for t0 in range(0, nt, 2):
        ref[t0:t0 + 2] = A.gemv_q8_0(w_q, w_d, xq[t0:t0 + 2].contiguous(), xd[t0:t0 + 2].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))


def test_gemm_rejects_bad_shapes(dev):
    import oxe_amd as A
    import torch
    wq = torch.zeros((64, 300), dtype=torch.int8, device=dev)   # k not a multiple of 128
    wd = torch.zeros((64, 300 // 32), dtype=torch.int16, device=dev)
    with pytest.raises(RuntimeError):
        A.gemm_q8_0(wq, wd, torch.zeros((4, 300), dtype=torch.int8, device=dev),
                    torch.zeros((4, 300 // 32), dtype=torch.int16, device=dev))
    # codes not 16-byte aligned (the kernel's 16-byte global-to-LDS loads): refused, nothing launched
    k = 256
    buf = torch.zeros(64 * k + 16, dtype=torch.int8, device=dev)
    wq = buf[1:1 + 64 * k].view(64, k)
    wd = torch.zeros((64, k // 32), dtype=torch.int16, device=dev)
    with pytest.raises(RuntimeError):
        A.gemm_q8_0(wq, wd, torch.zeros((4, k), dtype=torch.int8, device=dev),
                    torch.zeros((4, k // 32), dtype=torch.int16, device=dev))

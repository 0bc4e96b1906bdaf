"""Config 1 parity on the GPU: the Q8_0 activation quantizer and the 1-4 lane Q8_0 GEMV through the
C ABI against the oracle (oracle/ops.cpp: quantize_row_q8_0 NEON order, ggml_gemv_q8_0_4x8_q8_0
NEON order). Bar: int32 block sums and fp32 outputs bit-exact."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_quantize_matches_oracle(dev):
    import oxe_amd as A
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((3, 2048)) * rng.choice([1e-3, 1.0, 50.0], size=(3, 1))).astype(np.float32)
    # edge blocks: all zero, exact .5 steps after scaling, a single large value, tiny subnormal scales
    x[0, :32] = 0.0
    x[1, 32:64] = np.arange(32, dtype=np.float32) - 15.5
    x[2, 64:96] = 0.0
    x[2, 70] = 127.0
    x[2, 96:128] = np.float32(1e-30)
    q_ref, d_ref = O.quantize_q8_0(x)
    q, d = A.quantize_q8_0(_t(x, dev))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(d.cpu().numpy().view(np.uint16), d_ref)


# the tuned shapes (k 512, 2048, 4096) and the any-k kernel (k a multiple of 32: the reference GEMV's
# contract, crates/kernels-sys/src/lib.rs:75, 113)
@pytest.mark.parametrize("k,nr,nl", [(2048, 4096, 2), (2048, 4096, 1), (4096, 2048, 2), (512, 2048, 2), (2048, 40, 2),
                                     (32, 7, 2), (96, 130, 1), (1024, 257, 2), (3200, 64, 2), (8192, 33, 1),
                                     (2048, 4096, 3), (2048, 4096, 4), (4096, 520, 4), (512, 300, 3), (1024, 65, 4),
                                     (32768, 9, 4)])
def test_gemv_bitexact(dev, k, nr, nl):
    import oxe_amd as A
    import torch
    wq, wd = O.synth_q8(7, 61, O.T["OUTPUT"], nr, k)
    x = O.synth_normal(7, 61 * 64 + 41, nl * k).reshape(nl, k)
    xq, xd = O.quantize_q8_0(x)
    y_ref, isum_ref = O.gemv_q8_0(wq, wd, xq, xd, want_isum=True)
    isum = torch.empty((nl, nr, k // 32), dtype=torch.int32, device=dev)
    y = A.gemv_q8_0(_t(wq, dev), _t(wd.view(np.int16), dev), _t(xq, dev), _t(xd.view(np.int16), dev), isum=isum)
    torch.cuda.synchronize()
    assert np.array_equal(isum.cpu().numpy(), isum_ref)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_ref.view(np.uint32))


def test_gemv_lanes_equal_per_lane_calls(dev):
    """3 and 4 lanes in one weight pass == one call per lane, bit for bit (the reference's
    vl_gemv_bitwise invariant, crates/kernels-sys/src/lib.rs:640-646)."""
    import oxe_amd as A
    import torch
    k, nr = 2048, 777
    wq, wd = O.synth_q8(5, 3, O.T["OUTPUT"], nr, k)
    x = O.synth_normal(5, 77, 4 * k).reshape(4, k)
    xq, xd = O.quantize_q8_0(x)
    W = (_t(wq, dev), _t(wd.view(np.int16), dev))
    for nl in (3, 4):
        y = A.gemv_q8_0(*W, _t(xq[:nl], dev), _t(xd[:nl].view(np.int16), dev)).cpu().numpy()
        for l in range(nl):
            y1 = A.gemv_q8_0(*W, _t(xq[l:l + 1], dev), _t(xd[l:l + 1].view(np.int16), dev)).cpu().numpy()
            assert np.array_equal(y[l].view(np.uint32), y1[0].view(np.uint32)), (nl, l)
            assert np.array_equal(y[l].view(np.uint32), O.gemv_q8_0(wq, wd, xq[l:l + 1], xd[l:l + 1])[0].view(np.uint32))


def test_gemv_not_handled_writes_nothing(dev):
    """oxe_vl_gemv's convention (crates/kernels-sys/csrc/oxe_vl.inc:78-107): 1 done; 0 when there is
    no kernel for the call, with nothing written."""
    import oxe_amd as A
    import torch
    y = torch.full((5, 8), 7.0, device=dev)
    z = torch.zeros(4 * 65536, dtype=torch.int8, device=dev)
    for k, nr, nl in ((48, 8, 2), (0, 8, 2), (64, 0, 2), (64, 8, 5), (64, 8, 0), (-32, 8, 1), (65536, 8, 4)):
        rc = A.lib().oxe_hip_gemv_q8_0(k, nr, nl, A._p(z), A._p(z), A._p(z), A._p(z), A._p(y), None, A._stream())
        assert rc == 0, (k, nr, nl)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    rc = A.lib().oxe_hip_gemv_q8_0(64, 8, 4, A._p(z), A._p(z), A._p(z), A._p(z), A._p(y), None, A._stream())
    torch.cuda.synchronize()
    assert rc == 1 and bool((y[:4] == 0.0).all()) and bool((y[4] == 7.0).all())


def test_config1_gemv(dev):
    """BASELINE config 1 exactly: W [4096 x 2048], 2 lanes, seed 0."""
    import oxe_amd as A
    import torch
    wq, wd, x, xq_ref, xd_ref = O.config1_inputs(0)
    xq, xd = A.quantize_q8_0(_t(x, dev))
    assert np.array_equal(xq.cpu().numpy(), xq_ref) and np.array_equal(xd.cpu().numpy().view(np.uint16), xd_ref)
    y_ref, isum_ref = O.gemv_q8_0(wq, wd, xq_ref, xd_ref, want_isum=True)
    isum = torch.empty((2, 4096, 64), dtype=torch.int32, device=dev)
    y = A.gemv_q8_0(_t(wq, dev), _t(wd.view(np.int16), dev), xq, xd, isum=isum)
    torch.cuda.synchronize()
    assert np.array_equal(isum.cpu().numpy(), isum_ref)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_ref.view(np.uint32))

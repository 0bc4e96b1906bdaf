"""Device scalar functions against the host, over float bit patterns, bit for bit (NaNs of either
sign match): expf and log1pf against this host's C library over all 2^32 inputs (the reference
calls them in its gates, oxe_ops.cpp:80-89); ggml_v_expf, sigmoid, softplus and ggml_v_silu
against the oracle on every 16th pattern."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


@pytest.mark.parametrize("fn,stride", [(0, 1), (1, 1), (2, 16), (3, 16), (4, 16), (5, 16)],
                         ids=["expf", "log1pf", "v_expf", "sigmoid", "softplus", "v_silu"])
def test_device_scalar_functions_match_host(dev, fn, stride):
    import torch
    import oxe_amd as A
    total = (1 << 32) // stride
    y = torch.empty(CHUNK, dtype=torch.float32, device=dev)
    ref = np.empty(CHUNK, np.float32)
    bad = 0
    for c0 in range(0, total, CHUNK):
        n = min(CHUNK, total - c0)
        start = c0 * stride
        A.eval_unary(fn, start, n, stride, y)
        O.lib().oxo_eval_unary(fn, start, n, stride, O.ptr(ref, O.C.c_float))
        got = y[:n].cpu().numpy()
        r = ref[:n]
        diff = got.view(np.uint32) != r.view(np.uint32)
        if diff.any():
            diff &= ~(np.isnan(got) & np.isnan(r))
            bad += int(diff.sum())
    assert bad == 0

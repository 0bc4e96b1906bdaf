"""The allocation-free GGUF loader (oxe_engine_load_gguf_noalloc: uploads staged through the
library's static 16 MiB device array) against the allocating one (oxe_engine_load_gguf), through the
C ABI: two engines started from different synthetic weights load the same file, one through each
entry point, and must then decode bit for bit alike (prefill logits and hidden rows, a step, MTP
steps). Two calls in a row, the second with a smaller file (vocabulary 1024 instead of 4096), so the
array's leftover contents from the first call must not matter."""
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"


def test_noalloc_loader_equals_allocating_loader():
    import oxe_amd as A
    for call, vocab in enumerate((4096, 1024)):
        d = O.desc_small(n_vocab=vocab)
        path = os.path.join(scratch_dir(), f"oxe_test_noalloc_{os.getpid()}_{call}.gguf")
        try:
            print(f"call {call}: writing a vocab-{vocab} model", flush=True)
            W.write_synth_model(path, O, d, 40 + call)
            f = A.Gguf(path)
            ref = A.Engine(d, seed=7, n_ctx=256)
            ref.load_gguf(f)
            got = A.Engine(d, seed=8, n_ctx=256)
            got.load_gguf_noalloc(f)
            f.close()
            print(f"call {call}: loaded; decoding", flush=True)
            toks = [int(v) % vocab for v in O.bench_prompt(9)]
            assert got.prefill(toks) == ref.prefill(toks)
            assert np.array_equal(bits(got.logits(0)), bits(ref.logits(0)))
            assert np.array_equal(bits(got.hidden(0)), bits(ref.hidden(0)))
            x = ref.step(5)
            assert got.step(5) == x
            assert np.array_equal(bits(got.logits(0)), bits(ref.logits(0)))
            for _ in range(3):
                a, b = got.mtp_step(x), ref.mtp_step(x)
                assert a == b
                x = b[-1]
            assert np.array_equal(bits(got.hidden(0)), bits(ref.hidden(0)))
            got.close()
            ref.close()
        finally:
            if os.path.exists(path):
                os.remove(path)

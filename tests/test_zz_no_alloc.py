"""The allocation-free GGUF loader (oxe_engine_load_gguf_noalloc: uploads staged through the
library's static 16 MiB device array) against the allocating one (oxe_engine_load_gguf), through the
C ABI: two engines started from different synthetic weights load the same file, one through each
entry point, and must then decode bit for bit alike (prefill logits and hidden rows, a step, MTP
steps). Two calls in a row, the second with a smaller file (vocabulary 1024 instead of 4096), so the
array's leftover contents from the first call must not matter. The allocation-free call must leave
the device's free memory where it was, and two such calls overlapping from two threads on one GPU
(each engine on its own stream) must both load correctly: the per-device staging lock serialises
them."""
import os
import threading

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"


def device_free_bytes():
    import torch
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(0)[0]


def same_decode(got, ref, vocab):
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
            free0 = device_free_bytes()
            got.load_gguf_noalloc(f)
            free1 = device_free_bytes()
            f.close()
            print(f"call {call}: loaded (device free bytes {free0} -> {free1}); decoding", flush=True)
            # the allocating loader takes a 256 MiB staging buffer per call; this one allocates nothing
            assert free1 >= free0, f"device free memory fell by {free0 - free1} bytes"
            same_decode(got, ref, vocab)
            got.close()
            ref.close()
        finally:
            if os.path.exists(path):
                os.remove(path)


def test_noalloc_loader_overlapping_calls():
    import oxe_amd as A
    d = O.desc_small(n_vocab=4096)
    path = os.path.join(scratch_dir(), f"oxe_test_noalloc_{os.getpid()}_mt.gguf")
    try:
        print("writing a vocab-4096 model", flush=True)
        W.write_synth_model(path, O, d, 42)
        f = A.Gguf(path)
        refs = [A.Engine(d, seed=7, n_ctx=256) for _ in range(2)]
        for r in refs:
            r.load_gguf(f)
        engines = [A.Engine(d, seed=8 + i, n_ctx=256) for i in range(2)]
        errors = []

        def load(e):
            try:
                e.load_gguf_noalloc(f)
            except Exception as ex:  # reported below, in the test's thread
                errors.append(ex)

        threads = [threading.Thread(target=load, args=(e,)) for e in engines]
        for th in threads:
            th.start()
        for th in threads:
            th.join(timeout=100)
        assert not any(th.is_alive() for th in threads), "a load did not finish"
        assert not errors, errors
        f.close()
        print("both loaded; decoding", flush=True)
        for e, r in zip(engines, refs):
            same_decode(e, r, 4096)
            e.close()
            r.close()
    finally:
        if os.path.exists(path):
            os.remove(path)

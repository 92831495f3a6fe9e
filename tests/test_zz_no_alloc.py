"""ivh_set_input_f32_noalloc (the allocation-free f32 input conversion) against
ivh_set_input_f32 through the C ABI: bit-identical graph inputs on two calls in a row, the
second with a smaller batch, on inputs larger than the 2^21-float staging array (so every
image passes through it in more than one chunk)."""
import ctypes as C
import os

import numpy as np
import pytest

import infvino_amd as ia
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _inputs(n, batch, seed):
    g = np.load(os.path.join(HERE, "golden", "half_trunc.npz"))
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 30, n * batch).astype(np.float32)
    x[: g["x"].size] = g["x"]  # special values (denormal / overflow / NaN boundaries) first
    return x


def test_set_input_f32_noalloc_matches(tmp_path):
    # [1, 3, 1024, 1024]: 3 Mi floats per image, two chunks of the staging array each
    n = 3 * 1024 * 1024
    path = tmp_path / "io.plan"
    path.write_text(f"input x 1 3 1024 1024\ntensor y 1 3 1024 1024\nnode ew_unary x y op=2 n={n}\noutput y\n")
    m = ia.PlanModel(str(path), 0, 3)
    L = ia.lib()
    for batch, seed in ((3, 1), (1, 2)):
        x = _inputs(n, batch, seed)
        assert L.ivh_set_input_f32(m._h, x.ctypes.data_as(C.c_void_p), batch) == 0
        want = m.readTensor("x", batch)
        assert L.ivh_set_input_f16(m._h, np.zeros(n * batch, np.uint16).ctypes.data_as(C.c_void_p), batch) == 0
        rc = L.ivh_set_input_f32_noalloc(m._h, x.ctypes.data_as(C.c_void_p), batch)
        assert rc == 0, L.ivh_last_error()
        got = m.readTensor("x", batch)
        assert np.array_equal(got, want), f"batch {batch}"
        assert np.array_equal(got, O.f2h_trunc(x)), f"batch {batch} vs the reference truncation"
    # a batch above the model's maximum is rejected like ivh_set_input_f32's
    big = np.zeros(n * 4, np.float32)
    assert L.ivh_set_input_f32_noalloc(m._h, big.ctypes.data_as(C.c_void_p), 4) != 0
    m.close()


def test_set_input_f32_noalloc_two_models_threads(tmp_path):
    """Two models on one GPU converting in alternation from two threads (ctypes releases the
    GIL, so the calls overlap): the per-device lock keeps each model's input bit-identical to
    the reference truncation of its own data."""
    import threading
    n = 3 * 1024 * 1024
    path = tmp_path / "io.plan"
    path.write_text(f"input x 1 3 1024 1024\ntensor y 1 3 1024 1024\nnode ew_unary x y op=2 n={n}\noutput y\n")
    L = ia.lib()
    models = [ia.PlanModel(str(path), 0, 2) for _ in range(2)]
    data = [_inputs(n, 2, 10 + k) for k in range(2)]
    want = [O.f2h_trunc(d) for d in data]
    errors = []

    def worker(k):
        try:
            for it in range(6):
                rc = L.ivh_set_input_f32_noalloc(models[k]._h, data[k].ctypes.data_as(C.c_void_p), 2)
                if rc != 0:
                    errors.append((k, it, L.ivh_last_error()))
                    return
                if not np.array_equal(models[k].readTensor("x", 2), want[k]):
                    errors.append((k, it, "mismatch"))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((k, -1, repr(e)))

    ts = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    for m in models:
        m.close()
    assert not any(t.is_alive() for t in ts)
    assert not errors, errors

"""mxh_gemm_q_f16_noalloc: the exact-weight prefill GEMM with its staging in
a static device scratch array instead of an allocation (GPU).

Its results must be identical to mxh_gemm_q_f16's (the same kernels over the
same staged values), on two calls in a row with the second one smaller, and
requests beyond the scratch must be refused before any launch.
"""
from __future__ import annotations

import numpy as np
import pytest

import mxhip
import mxo

pytestmark = pytest.mark.gpu


def call(fn, t, a, m, w, n, k, out):
    mxhip.check(fn(t, a.ptr, m, w.ptr, n, k, out.ptr, 0), fn.__name__)
    mxhip.synchronize()
    return out.download(np.float32, m * n).reshape(m, n)


@pytest.mark.parametrize("name", ["Q4_K", "Q8_0"])
def test_noalloc_matches_allocating_entry_twice(mxh, name):
    t = {"Q4_K": mxo.Q4_K, "Q8_0": mxo.Q8_0}[name]
    lib = mxhip.lib
    rng = np.random.default_rng(31)
    # first call: 300 x 4096 activations (4.9 MB of staging), second: 40 x 1024
    for m, n, k in ((300, 520, 4096), (40, 200, 1024)):
        w = mxo.quantize(t, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        a = rng.standard_normal((m, k), dtype=np.float32)
        dw, da = mxhip.DeviceBuffer.from_array(w), mxhip.DeviceBuffer.from_array(a)
        o1, o2 = mxhip.DeviceBuffer(4 * m * n), mxhip.DeviceBuffer(4 * m * n)
        want = call(lib.mxh_gemm_q_f16, t, da, m, dw, n, k, o1)
        got = call(lib.mxh_gemm_q_f16_noalloc, t, da, m, dw, n, k, o2)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{m}x{n}x{k}"
        # and within the exact-weight bar of the float64 product
        wd = mxo.dequant(t, w, n, k).astype(np.float64)
        ref = a.astype(np.float64) @ wd.T
        assert np.all(np.abs(got - ref) <= 2.0 ** -19 * (np.abs(a).astype(np.float64) @ np.abs(wd).T))
        for b in (dw, da, o1, o2):
            b.close()


def test_noalloc_rejects_requests_beyond_the_scratch(mxh):
    lib = mxhip.lib
    dw, da, out = mxhip.DeviceBuffer(1 << 20), mxhip.DeviceBuffer(1 << 20), mxhip.DeviceBuffer(1 << 20)
    # 1024 x 4096 activations need about 16.8 MB of staging, above the 12 MiB scratch
    assert lib.mxh_gemm_q_f16_noalloc(mxo.Q8_0, da.ptr, 1024, dw.ptr, 16, 4096, out.ptr, 0) == -1
    assert b"scratch" in lib.mxh_last_error()
    for b in (dw, da, out):
        b.close()

"""GPU test of the allocation-free entry point llmi_hip_matmul_mfma_noalloc_dev
(the bf16-MFMA product with its activation copy in a fixed per-GPU array).
Its output must equal llmi_hip_matmul_mfma_dev's -- the same kernels -- bit
for bit, on consecutive calls whose inputs shrink (the array keeps the last
call's contents), at the array's size limit, and it must reject a product
beyond that limit.  Both entry points are called through the C ABI."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 33554432  # LLMI_MFMA_NOALLOC_SCRATCH_BYTES (include/llmi_hip.h)


def scratch_need(rows, n_in, out):
    """The header's formula: the bf16 copy of x rounded up to 256 bytes, plus
    fp32 partials when K is split (more than 24 K-steps of 64 on fewer than
    256 output tiles of 128 x 256, into as many chunks of at least 8 steps as
    256 // tiles allows)."""
    ldx = -(-n_in // 64) * 64
    need = -(-(2 * rows * ldx) // 256) * 256
    nk = -(-n_in // 64)
    tiles = -(-rows // 128) * -(-out // 256)
    if nk > 24 and tiles < 256:
        k = min(256 // tiles, nk // 8)
        if k >= 2:
            need += 4 * rows * out * -(-nk // -(-nk // k))
    return need


def product(fn, w, x, rows, bias):
    """y = fn(w, x) through the C ABI on device copies of x and bias; y starts
    as NaN, so every element must be written."""
    lib = H.init()
    xd = H.DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
    bd = None if bias is None else H.DeviceBuffer.from_array(np.ascontiguousarray(bias, dtype=np.float32))
    yd = H.DeviceBuffer.from_array(np.full(rows * w.out, np.nan, np.float32))
    H.check(getattr(lib, fn)(w.h, xd.ptr, rows, None if bd is None else bd.ptr, yd.ptr, None))
    H.synchronize()
    y = yd.download(np.float32)
    for b in (xd, bd, yd):
        if b is not None:
            b.free()
    return y


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("out,n_in,calls", [(896, 896, (512, 77)), (4864, 896, (300, 64)), (896, 4864, (512, 1)),
                                            (200, 100, (130, 3))])
def test_noalloc_equals_the_allocating_entry_point(qt, out, n_in, calls):
    orc = O.oracle()
    data, scales = orc.quantize(synth.normal(out + n_in, out * n_in, 0.0, 0.02), out, n_in, qt)
    w = H.Weight.upload(data, scales, out, n_in, qt)
    bias = synth.normal(out, out, 0.0, 0.5)
    for k, rows in enumerate(calls):  # the second call is smaller than the first
        x = synth.normal(1000 * k + rows, rows * n_in, 0.0, 1.0)
        b = bias if k == 0 else None
        want = product("llmi_hip_matmul_mfma_dev", w, x, rows, b)
        got = product("llmi_hip_matmul_mfma_noalloc_dev", w, x, rows, b)
        assert not np.isnan(got).any(), (out, n_in, rows)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (out, n_in, rows)
    w.free()


def test_noalloc_limit():
    """The largest product that fits the array (here with K split, so x's copy
    and the partials share it) is accepted and exact; one row more is
    rejected before anything runs."""
    orc = O.oracle()
    out, n_in = 128, 4864  # ldx = 4864, 76 K-steps: split into 9 chunks
    data, scales = orc.quantize(synth.normal(9, out * n_in, 0.0, 0.02), out, n_in, O.Q8_0)
    w = H.Weight.upload(data, scales, out, n_in, O.Q8_0)
    rows = 1
    while scratch_need(rows + 1, n_in, out) <= SCRATCH_BYTES:
        rows += 1
    assert scratch_need(rows, n_in, out) > 2 * rows * n_in  # the partials are part of it
    x = synth.normal(10, rows * n_in, 0.0, 1.0)
    want = product("llmi_hip_matmul_mfma_dev", w, x, rows, None)
    got = product("llmi_hip_matmul_mfma_noalloc_dev", w, x, rows, None)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    x2 = synth.normal(11, (rows + 1) * n_in, 0.0, 1.0)
    with pytest.raises(H.HipError, match="exceeds"):
        product("llmi_hip_matmul_mfma_noalloc_dev", w, x2, rows + 1, None)
    # Still usable after the rejected call, on a small product.
    x3 = synth.normal(12, 5 * n_in, 0.0, 1.0)
    assert np.array_equal(product("llmi_hip_matmul_mfma_noalloc_dev", w, x3, 5, None).view(np.uint32),
                          product("llmi_hip_matmul_mfma_dev", w, x3, 5, None).view(np.uint32))
    w.free()

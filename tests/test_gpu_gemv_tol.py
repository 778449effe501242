"""GPU checks of the tolerance-mode Q4_0 product (llmi_hip_matmul_tol_dev,
llmi_hip_tol_group_*): quant::matmul (src/model/quant.cpp:119-153) summed
on the matrix cores in another order.  The bar is the path's fp32-accumulate
tolerance, written here as

    max_o |y_o - ref_o| <= 1e-4 * max_o |ref_o|          (the contract)
    |y_o - ref_o| <= 1e-5 * (sum_b |scale_ob| sum_i |x_i c_i| + |bias_o|)

with ref the oracle's bit-exact restatement of the reference.  The second,
tighter bound is relative to the magnitude of the terms of each output, so
outputs that cancel to near zero are held to it as well."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu

TOL_CONTRACT = 1e-4
TOL_TERMS = 1e-5


def deq_abs(o, data, scales, out, n_in):
    """|W| after dequantization, row by row from the oracle (float64)."""
    return np.abs(np.stack([o.dequantize_row(data, scales, out, n_in, O.Q4_0, r) for r in range(out)]).astype(np.float64))


def check(y, ref, mag):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(y - ref)
    assert np.all(np.isfinite(y))
    assert err.max() <= TOL_CONTRACT * max(np.abs(ref).max(), 1e-30), (err.max(), np.abs(ref).max())
    assert np.all(err <= TOL_TERMS * mag + 1e-30), float((err / np.maximum(mag, 1e-30)).max())


def case(out, n_in, rows, seed, scale=1.0):
    w = synth.normal(seed, out * n_in, 0.0, 0.02)
    x = (synth.normal(seed + 1, rows * n_in, 0.0, 1.0) * scale).astype(np.float32)
    bias = synth.normal(seed + 2, out, 0.0, 1.0)
    return w, x, bias


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("out,n_in", [(1, 1), (63, 33), (65, 100), (200, 576), (130, 1536), (96, 4864), (64, 8192)])
def test_single_product_within_tolerance(out, n_in, rows):
    o = O.oracle()
    w, x, bias = case(out, n_in, rows, 1000 + out + n_in + rows)
    dev = H.Weight.quantize(w, out, n_in, O.Q4_0)
    data, scales = dev.download()
    mag_w = deq_abs(o, data, scales, out, n_in)
    for b in (None, bias):
        y = dev.matmul_tol(x, rows, b)
        ref = o.matmul(x, rows, n_in, data, scales, O.Q4_0, out, b)
        mag = (np.abs(x.reshape(rows, n_in).astype(np.float64)) @ mag_w.T)
        if b is not None:
            mag = mag + np.abs(b.astype(np.float64))
        check(y, ref, mag.reshape(-1))
    dev.free()


@pytest.mark.parametrize("scale", [1e-30, 1e-3, 1e3, 1e30])
def test_activation_magnitudes(scale):
    """bf16 keeps fp32's exponent range: tiny and huge activations keep the
    same relative accuracy; zeros contribute nothing."""
    o = O.oracle()
    out, n_in, rows = 128, 576, 2
    w, x, _ = case(out, n_in, rows, 77, scale)
    x[::7] = 0.0
    dev = H.Weight.quantize(w, out, n_in, O.Q4_0)
    data, scales = dev.download()
    y = dev.matmul_tol(x, rows)
    ref = o.matmul(x, rows, n_in, data, scales, O.Q4_0, out, None)
    mag = (np.abs(x.reshape(rows, n_in).astype(np.float64)) @ deq_abs(o, data, scales, out, n_in).T).reshape(-1)
    check(y, ref, mag)
    dev.free()


def test_group_matches_reference():
    """A group of products with shared and distinct inputs, batches 1..8,
    long and short rows and a bias, launched as one tolerance-mode group."""
    o = O.oracle()
    specs = [(576, 576, 1, 0), (192, 576, 1, 0), (1536, 576, 1, 1), (576, 1536, 1, 2), (300, 100, 3, 3),
             (64, 4864, 8, 4), (1000, 576, 8, 5)]
    xs = {}
    items, checks, bufs = [], [], []
    for i, (out, n_in, rows, xk) in enumerate(specs):
        w, _, bias = case(out, n_in, rows, 500 + i)
        if xk not in xs:
            xv = synth.normal(900 + xk, rows * n_in, 0.0, 1.0)
            xs[xk] = (xv, H.DeviceBuffer.from_array(xv))
        xv, xb = xs[xk]
        dev = H.Weight.quantize(w, out, n_in, O.Q4_0)
        yb = H.DeviceBuffer(rows * out * 4)
        bb = H.DeviceBuffer.from_array(bias) if i % 2 else None
        items.append((dev, xb.ptr, yb.ptr, rows, None if bb is None else bb.ptr))
        checks.append((dev, xv, rows, n_in, out, yb, bias if i % 2 else None))
        bufs += [yb] + ([bb] if bb is not None else [])
    g = H.TolGroup(items)
    for _ in range(2):  # launches repeat: the split activations are rewritten each time
        g.launch()
        H.synchronize()
        for dev, xv, rows, n_in, out, yb, bias in checks:
            data, scales = dev.download()
            ref = o.matmul(xv, rows, n_in, data, scales, O.Q4_0, out, bias)
            mag = np.abs(xv.reshape(rows, n_in).astype(np.float64)) @ deq_abs(o, data, scales, out, n_in).T
            if bias is not None:
                mag = mag + np.abs(bias.astype(np.float64))
            check(yb.download(np.float32, rows * out), ref, mag.reshape(-1))
    g.free()
    for dev, *_ in checks:
        dev.free()
    for b in bufs + [xb for _, xb in xs.values()]:
        b.free()


def test_rejects_what_it_does_not_cover():
    w = synth.normal(1, 64 * 64, 0.0, 0.02)
    q8 = H.Weight.quantize(w, 64, 64, O.Q8_0)
    x = synth.normal(2, 9 * 64, 0.0, 1.0)
    with pytest.raises(H.HipError, match="Q4_0"):
        q8.matmul_tol(x[:64], 1)
    q4 = H.Weight.quantize(w, 64, 64, O.Q4_0)
    with pytest.raises(H.HipError, match="1..8"):
        q4.matmul_tol(x, 9)
    q8.free()
    q4.free()


@pytest.mark.parametrize("rows", [1, 8])
def test_qwen_lm_head_shape(rows):
    """The 151936 x 896 lm_head (2374 tiles): every output within the
    contract of the exact kernel's (= the reference's) output, and a sample
    of 1500 rows within the per-output bound."""
    o = O.oracle()
    out, n_in = 151936, 896
    buf = H.DeviceBuffer(out * n_in * 4)
    H.synth_normal_dev(buf, out * n_in, 4242, 0.0, 0.02)
    w = H.Weight.quantize_dev(buf.ptr, out, n_in, O.Q4_0)
    buf.free()
    x = synth.normal(4243, rows * n_in, 0.0, 1.0)
    exact = w.matmul(x, rows).astype(np.float64)
    tol = w.matmul_tol(x, rows).astype(np.float64)
    assert np.abs(tol - exact).max() <= TOL_CONTRACT * np.abs(exact).max()
    data, scales = w.download()
    sample = np.random.default_rng(1).choice(out, 1500, replace=False)
    wabs = np.abs(np.stack([o.dequantize_row(data, scales, out, n_in, O.Q4_0, int(r)) for r in sample]).astype(np.float64))
    mag = np.abs(x.reshape(rows, n_in).astype(np.float64)) @ wabs.T
    err = np.abs(tol.reshape(rows, out)[:, sample] - exact.reshape(rows, out)[:, sample])
    assert np.all(err <= TOL_TERMS * mag), float((err / mag).max())
    w.free()

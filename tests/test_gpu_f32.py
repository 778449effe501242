"""GPU parity of fp32 weights (Type::F32): kernels::matmul
(src/model/kernels.cpp:97-113, y = dot(x_r, w_o) + bias with the AVX2
kernels::dot arithmetic) and Weight::row, bit for bit against the oracle's
dot -- itself pinned to the compiled reference's golden dot vectors -- over
tails of every length, and the reference's own known-answer tests
(tests/transformer_test.cpp:30-72)."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def want_matmul(x, rows, n_in, w, out, bias):
    orc = O.oracle()
    y = np.empty(rows * out, np.float32)
    for o in range(out):
        add = np.float32(bias[o]) if bias is not None else np.float32(0.0)
        for r in range(rows):
            y[r * out + o] = np.float32(orc.dot(x[r * n_in:(r + 1) * n_in], w[o * n_in:(o + 1) * n_in])) + add
    return y


def test_matmul_with_bias_known_answer():
    # transformer_test.cpp:30-44
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)
    w = H.Weight.quantize(np.array([1, 0, -1, 0.5, 0.5, 0.5], np.float32), 2, 3, H.F32)
    y = w.matmul(x, 2, np.array([10, -1], np.float32))
    assert list(y) == [1 - 3 + 10.0, 3 - 1.0, 4 - 6 + 10.0, 7.5 - 1]
    assert w.matmul(x, 2)[0] == -2.0
    w.free()


@pytest.mark.parametrize("n_in", list(range(1, 41)) + [300, 896])
def test_matmul_matches_oracle_dot_every_tail(n_in):
    out, rows = 37, 3
    x = synth.normal(n_in, rows * n_in, 0.0, 1.0)
    w = synth.normal(n_in + 1, out * n_in, 0.0, 0.5)
    bias = synth.normal(n_in + 2, out, 0.0, 0.5)
    dev = H.Weight.quantize(w, out, n_in, H.F32)
    got = dev.matmul(x, rows, bias)
    assert np.array_equal(bits(got), bits(want_matmul(x, rows, n_in, w, out, bias))), n_in
    for r in (0, out - 1):
        assert np.array_equal(bits(dev.dequantize_row(r)), bits(w[r * n_in:(r + 1) * n_in]))
    dev.free()


def test_matmul_above_the_threading_threshold():
    # transformer_test.cpp:46-72: rows 3, in 300, out 4000, each y = dot + bias.
    rows, n_in, out = 3, 300, 4000
    x = synth.normal(1, rows * n_in, 0.0, 0.6)
    w = synth.normal(2, out * n_in, 0.0, 0.6)
    bias = synth.normal(3, out, 0.0, 0.6)
    dev = H.Weight.quantize(w, out, n_in, H.F32)
    got = dev.matmul(x, rows, bias)
    assert np.array_equal(bits(got), bits(want_matmul(x, rows, n_in, w, out, bias)))
    dev.free()

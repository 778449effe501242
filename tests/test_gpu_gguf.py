"""GPU parity of llmi_hip_weight_from_gguf (gguf::to_quantized, gguf.cpp:577-640,
plus the upload): the device-converted weight downloads to the oracle's
to_quantized output bit for bit, and products through it match the oracle's
quant::matmul on that output bit for bit."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth
from test_oracle_gguf import GGUF_Q4_0, GGUF_Q8_0, random_blocks

pytestmark = pytest.mark.gpu


def qtype_of(gtype):
    return H.Q8_0 if gtype == GGUF_Q8_0 else H.Q4_0


def test_reference_known_answers_on_device():
    # gguf_test.cpp:389-416 and :418-453.
    w = H.Weight.from_gguf(np.array([0x00, 0x3C] + list(range(32)), np.uint8), 1, 32, GGUF_Q8_0)
    assert list(w.dequantize_row(0)) == [float(i) for i in range(32)]
    w.free()
    w = H.Weight.from_gguf(np.array([0x00, 0x40, 0x91] + [0x88] * 15, np.uint8), 1, 32, GGUF_Q4_0)
    row = w.dequantize_row(0)
    assert row[0] == -14.0 and row[16] == 2.0 and np.count_nonzero(row) == 2
    w.free()


@pytest.mark.parametrize("gtype", [GGUF_Q8_0, GGUF_Q4_0])
@pytest.mark.parametrize("out,n_in", [(2048, 1024), (896, 896), (65, 64), (1, 32), (4864, 896)])
def test_device_conversion_matches_oracle(gtype, out, n_in):
    """All 65536 fp16 scale patterns (cycled), random codes, tile-ragged rows."""
    nb = out * n_in // 32
    raw = random_blocks(nb, gtype, out + n_in, scales_u16=np.arange(nb, dtype=np.uint32) % 65536)
    want_d, want_s = O.oracle().gguf_to_quantized(raw, out, n_in, gtype)
    w = H.Weight.from_gguf(raw, out, n_in, gtype)
    got_d, got_s = w.download()
    assert np.array_equal(got_d, want_d)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))
    w.free()


@pytest.mark.parametrize("gtype", [GGUF_Q8_0, GGUF_Q4_0])
def test_products_through_converted_weight_match_oracle(gtype):
    """Finite scales of a realistic magnitude (a GGUF file's): the GEMV and the
    exact multi-row path on the converted weight equal the oracle's matmul on
    to_quantized's output."""
    out, n_in = 896, 896
    nb = out * n_in // 32
    scales = np.abs(synth.normal(11, nb, 0.0, 0.002)).astype(np.float16).view(np.uint16)
    raw = random_blocks(nb, gtype, 12, scales_u16=scales)
    data, sc = O.oracle().gguf_to_quantized(raw, out, n_in, gtype)
    w = H.Weight.from_gguf(raw, out, n_in, gtype)
    for rows in (1, 8, 20):
        x = synth.normal(13 + rows, rows * n_in, 0.0, 1.0)
        want = O.oracle().matmul(x, rows, n_in, data, sc, qtype_of(gtype), out, None)
        got = w.matmul(x, rows)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rows
    w.free()


def test_rejects_what_to_quantized_rejects():
    raw = random_blocks(4, GGUF_Q8_0, 1)
    for args in ((raw, 2, 64, 0),                              # F32 tensor type
                 (raw, 2, 64, GGUF_Q4_0),                      # byte count of another type
                 (raw[:-1], 2, 64, GGUF_Q8_0),                 # one byte short
                 (random_blocks(1, GGUF_Q8_0, 2), 1, 16, GGUF_Q8_0),  # in % 32 != 0
                 (np.zeros(0, np.uint8), 0, 32, GGUF_Q8_0)):   # empty shape
        with pytest.raises(H.HipError):
            H.Weight.from_gguf(*args)

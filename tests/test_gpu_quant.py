"""GPU parity of the block quantizer, the device layout and the row
dequantizer: bit-exact against the compiled reference's golden fixtures and
the oracle."""

import hashlib

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_device_generator_matches_host_generator():
    n = 1 << 20
    buf = H.DeviceBuffer(n * 4)
    for seed, mean, std, off in ((1, 0.0, 0.02, 0), (12345, 1.0, 0.3, 777), (2**63 + 5, 0.0, 1.0, 2**33)):
        H.synth_normal_dev(buf, n, seed, mean, std, off)
        got = buf.download(np.float32)
        want = synth.normal(seed, n, mean, std, offset=off)
        assert np.array_equal(bits(got), bits(want)), seed


def test_quantize_matches_reference_small_and_edges(golden):
    rec, arrays = golden
    g = arrays["quant_small"]
    for c in rec["quant_small"]:
        k, qt, out, n_in = c["key"], c["type"], c["out"], c["n_in"]
        w = synth.normal(c["w_seed"], out * n_in, 0.0, c["w_std"])
        data, scales = H.quantize(w, out, n_in, qt)
        assert np.array_equal(data, g[k + "_data"]), k
        assert np.array_equal(bits(scales), bits(g[k + "_scales"])), k
    for qt in (O.Q8_0, O.Q4_0):
        data, scales = H.quantize(g["edge_w"], 6, 64, qt)
        assert np.array_equal(data, g[f"edge_t{qt}_data"])
        assert np.array_equal(bits(scales), bits(g[f"edge_t{qt}_scales"]))


def test_quantize_matches_reference_at_baseline_shapes(golden):
    rec, _ = golden
    done = set()
    for c in rec["shapes"]:
        key = (c["w_seed"], c["out"], c["n_in"], c["type"])
        if key in done:
            continue
        done.add(key)
        out, n_in, qt = c["out"], c["n_in"], c["type"]
        buf = H.DeviceBuffer(out * n_in * 4)
        H.synth_normal_dev(buf, out * n_in, c["w_seed"], 0.0, c["w_std"])
        # Planar output through the device quantizer.
        lib = H.init()
        data_d = H.DeviceBuffer(out * H.row_bytes(n_in, qt))
        sc_d = H.DeviceBuffer(out * H.nblocks(n_in) * 4)
        H.check(lib.llmi_hip_quantize_dev(buf.ptr, out, n_in, qt, data_d.ptr, sc_d.ptr, None))
        H.synchronize()
        assert sha(data_d.download(np.uint8)) == c["data_sha256"], c["name"]
        assert sha(sc_d.download(np.float32)) == c["scales_sha256"], c["name"]
        # Straight into the tiled device layout, then back to planar.
        w = H.Weight.quantize_dev(buf.ptr, out, n_in, qt)
        data, scales = w.download()
        assert sha(data) == c["data_sha256"], c["name"]
        assert sha(scales) == c["scales_sha256"], c["name"]
        assert w.byte_size == c["byte_size"]
        w.free()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("out,n_in", [(1, 1), (3, 7), (65, 33), (130, 100), (64, 4864), (7, 31)])
def test_upload_download_round_trip_and_dequantize(qt, out, n_in):
    orc = O.oracle()
    w = synth.normal(out * 1000 + n_in, out * n_in, 0.0, 0.3)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    d2, s2 = dev.download()
    assert np.array_equal(d2, data)
    assert np.array_equal(bits(s2), bits(scales))
    for r in sorted({0, out // 2, out - 1}):
        want = orc.dequantize_row(data, scales, out, n_in, qt, r)
        assert np.array_equal(bits(dev.dequantize_row(r)), bits(want)), r
    dq = H.Weight.quantize(w, out, n_in, qt)
    d3, s3 = dq.download()
    assert np.array_equal(d3, data)
    assert np.array_equal(bits(s3), bits(scales))


def test_dequantize_rows_gather():
    orc = O.oracle()
    out, n_in, qt = 300, 576, O.Q8_0
    w = synth.normal(99, out * n_in, 0.0, 0.02)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    ids = np.array([0, 299, 64, 63, 5, 5], dtype=np.int32)
    ids_d = H.DeviceBuffer.from_array(ids)
    dst = H.DeviceBuffer(ids.size * n_in * 4)
    H.check(H.init().llmi_hip_dequantize_rows_dev(dev.h, ids_d.ptr, ids.size, dst.ptr, None))
    H.synchronize()
    got = dst.download(np.float32).reshape(ids.size, n_in)
    for t, r in enumerate(ids):
        assert np.array_equal(bits(got[t]), bits(orc.dequantize_row(data, scales, out, n_in, qt, int(r))))


def test_bad_arguments_are_errors_not_faults():
    lib = H.init()
    w = np.zeros(64, np.float32)
    data = np.zeros(64, np.uint8)
    scales = np.zeros(2, np.float32)
    rc = lib.llmi_hip_quantize(w.ctypes.data, 1, 64, 7, data.ctypes.data, scales.ctypes.data)
    assert rc == 1
    dev = H.Weight.upload(np.zeros(32, np.uint8), np.ones(1, np.float32), 1, 32, O.Q8_0)
    y = np.zeros(32, np.float32)
    x = np.zeros(32, np.float32)
    assert lib.llmi_hip_matmul(dev.h, x.ctypes.data, 1, 31, 1, None, y.ctypes.data) == 1  # in mismatch
    assert lib.llmi_hip_dequantize_row(dev.h, 1, y.ctypes.data) == 1  # row out of range

"""CPU tests of the oracle (oracle/oracle.cpp): it must reproduce the
compiled reference bit for bit (golden fixtures from tests/golden/
gen_golden.py) and pass the reference's own known-answer tests."""

import hashlib

import numpy as np
import pytest

import oracle as O
import synth

Q8, Q4 = O.Q8_0, O.Q4_0


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def orc():
    return O.oracle()


# ------------------------------------------------------------ golden vectors
def test_quantize_matmul_dequantize_match_reference_small(orc, golden):
    rec, arrays = golden
    g = arrays["quant_small"]
    for c in rec["quant_small"]:
        k, qt, out, n_in, rows = c["key"], c["type"], c["out"], c["n_in"], c["rows"]
        w = synth.normal(c["w_seed"], out * n_in, 0.0, c["w_std"])
        x = synth.normal(c["x_seed"], rows * n_in, 0.0, 1.0)
        bias = synth.normal(c["bias_seed"], out, 0.0, 1.0)
        data, scales = orc.quantize(w, out, n_in, qt)
        assert np.array_equal(data, g[k + "_data"]), k
        assert np.array_equal(bits(scales), bits(g[k + "_scales"])), k
        assert np.array_equal(bits(orc.matmul(x, rows, n_in, data, scales, qt, out, bias)), bits(g[k + "_y"])), k
        assert np.array_equal(bits(orc.matmul(x, rows, n_in, data, scales, qt, out, None)), bits(g[k + "_ynb"])), k
        for r in range(out):
            assert np.array_equal(bits(orc.dequantize_row(data, scales, out, n_in, qt, r)), bits(g[k + "_deq"][r]))


def test_edge_blocks_match_reference(orc, golden):
    _, arrays = golden
    g = arrays["quant_small"]
    for qt in (Q8, Q4):
        data, scales = orc.quantize(g["edge_w"], 6, 64, qt)
        assert np.array_equal(data, g[f"edge_t{qt}_data"])
        assert np.array_equal(bits(scales), bits(g[f"edge_t{qt}_scales"]))


_W_CACHE = {}


def _weights(seed, n):
    if (seed, n) not in _W_CACHE:
        _W_CACHE.clear()
        _W_CACHE[(seed, n)] = synth.normal(seed, n, 0.0, 0.02)
    return _W_CACHE[(seed, n)]


def test_baseline_shapes_match_reference(orc, golden):
    """C1, every C2 shape at batch 1 and 8, and the Qwen2.5 shapes."""
    rec, arrays = golden
    g = arrays["shapes"]
    for c in sorted(rec["shapes"], key=lambda c: (c["w_seed"], c["out"] * c["n_in"])):
        out, n_in, qt = c["out"], c["n_in"], c["type"]
        w = _weights(c["w_seed"], out * n_in)
        data, scales = orc.quantize(w, out, n_in, qt)
        assert sha(data) == c["data_sha256"], c["name"]
        assert sha(scales) == c["scales_sha256"], c["name"]
        assert data.size + 4 * scales.size == c["byte_size"]
        for b, yrec in c["y"].items():
            x = synth.normal(c["x_seed"], int(b) * n_in, 0.0, 1.0)
            y = orc.matmul(x, int(b), n_in, data, scales, qt, out, None)
            assert sha(y) == yrec["sha256"], (c["name"], b)
            key = f"{c['name']}_t{qt}_b{b}_y"
            if key in g:
                assert np.array_equal(bits(y), bits(g[key]))


def test_glue_kernels_match_reference(orc, golden):
    _, arrays = golden
    g = arrays["kernels"]
    for n, want in zip(g["dot_n"], g["dot_out"]):
        got = orc.dot(g["dot_a"][:n], g["dot_b"][:n])
        assert bits(np.float32(got)) == bits(want), n
    assert np.array_equal(bits(orc.rmsnorm(g["rms_x"][:576], g["rms_w"][:576], 1e-5)), bits(g["rms_576"]))
    assert np.array_equal(bits(orc.rmsnorm(g["rms_x"], g["rms_w"], 1e-6)), bits(g["rms_896"]))
    for key in [k[:-4] for k in g if k.startswith("rope_") and k.endswith("_inv")]:
        for p, want in zip(g[key + "_pos"], g[key + "_out"]):
            assert np.array_equal(bits(orc.rope(g[key + "_v"], int(p), g[key + "_inv"])), bits(want)), (key, p)
    assert np.array_equal(bits(orc.softmax(g["softmax_in"])), bits(g["softmax_out"]))
    got = np.array([orc.silu(v) for v in g["silu_in"]], dtype=np.float32)
    assert np.array_equal(bits(got), bits(g["silu_out"]))


def test_tiny_models_match_reference(orc, golden):
    """Every arch x tie x {F32, Q8_0, Q4_0} of the reference's 2-layer test
    model: prefill logits (all positions), per-step logits, greedy ids."""
    rec, arrays = golden
    g = arrays["tiny_models"]
    for c in rec["tiny_models"]:
        tensors = synth.make_tensors(c["cfg"], c["seed"], c["convention"])
        m = orc.model(c["cfg"], tensors, c["type"])
        assert m.new_cache(len(g["prompt"]) + len(g["steps"]))
        pre = m.forward_cached(g["prompt"], all_positions=True)
        assert np.array_equal(bits(pre), bits(g[c["key"] + "_prefill"])), c["key"]
        for i, s in enumerate(g["steps"]):
            assert np.array_equal(bits(m.forward_cached([s])), bits(g[c["key"] + "_steps"][i])), (c["key"], i)
        ids, _ = m.generate_greedy(np.array([1, 2, 3], np.int32), 12)
        assert np.array_equal(ids, g[c["key"] + "_greedy"]), c["key"]


# -------------------------------------------- the reference's own KATs
def test_q4_extreme_value_round_trips_exactly(orc):
    """tests/quant_test.cpp:85-99 with its literal blocks."""
    for w in ([0.9, -0.3, 0.1, 0.4, -0.5, 0.2, -0.1, 0.05], [-0.9, 0.3, 0.1, 0.4, -0.5, 0.2, -0.1, 0.05]):
        w = np.array(w, dtype=np.float32)
        data, scales = orc.quantize(w, 1, 8, Q4)
        row = orc.dequantize_row(data, scales, 1, 8, Q4, 0)
        assert row[0] == w[0]
        assert (data[0] & 0x0F) == 0  # the extreme sits on code -8


def test_all_zero_block_round_trips_to_zero(orc):
    """tests/quant_test.cpp:101-112."""
    w = np.zeros(40, dtype=np.float32)
    for qt in (Q8, Q4):
        data, scales = orc.quantize(w, 1, 40, qt)
        assert np.all(scales == 1.0)
        assert np.all(orc.dequantize_row(data, scales, 1, 40, qt, 0) == 0.0)
        if qt == Q4:
            assert np.all(data[:20] == 0x88)


@pytest.mark.parametrize("qt,bound", [(Q8, 254.0), (Q4, 8.0)])
def test_round_trip_error_bounds(orc, qt, bound):
    """tests/quant_test.cpp:27-83: |deq - w| <= amax/254 (Q8_0), amax/8 (Q4_0)."""
    for n_in in (1, 7, 31, 32, 33, 100):
        out = 3
        w = synth.normal(77 + n_in, out * n_in, 0.0, 0.3)
        data, scales = orc.quantize(w, out, n_in, qt)
        for r in range(out):
            row = orc.dequantize_row(data, scales, out, n_in, qt, r)
            for b0 in range(0, n_in, 32):
                blk = w[r * n_in + b0: r * n_in + min(n_in, b0 + 32)]
                tol = np.abs(blk).max() / bound + 1e-6
                assert np.all(np.abs(row[b0:b0 + blk.size] - blk) <= tol)


def test_byte_ratios(orc):
    """tests/quant_test.cpp:114-127: 3.55x (Q8_0) and 6.4x (Q4_0)."""
    out, n_in = 100, 3200
    w = synth.normal(3, out * n_in, 0.0, 0.3)
    for qt, ratio, tol in ((Q8, 3.55, 0.05), (Q4, 6.4, 0.1)):
        data, scales = orc.quantize(w, out, n_in, qt)
        assert abs(out * n_in * 4 / (data.size + 4 * scales.size) - ratio) <= tol


@pytest.mark.parametrize("cfg,qt,want", [
    (synth.SMOLLM2_135M, Q8, 151_289_856), (synth.SMOLLM2_135M, Q4, 84_049_920),
    (synth.QWEN25_05B, Q8, 555_706_368), (synth.QWEN25_05B, Q4, 308_725_760)])
def test_weight_bytes_equal_published(cfg, qt, want):
    """docs/evidence/m5-speed-and-memory.txt:8-16: Transformer::weight_bytes
    = sum over quantized matrices of out*row_bytes + 4*out*ceil(in/32)."""
    total = 0
    for name, shape, kind in synth.tensor_specs(cfg):
        if kind == "matrix":
            out, n_in = shape
            total += out * O.row_bytes(n_in, qt) + 4 * out * O.nblocks(n_in)
    assert total == want


def test_q8_codes_in_order_dequantize(orc):
    """tests/gguf_test.cpp:389-417: Q8_0 codes 0..31 at scale 1.0."""
    data = np.arange(32, dtype=np.uint8)
    row = orc.dequantize_row(data, np.ones(1, np.float32), 1, 32, Q8, 0)
    assert np.array_equal(row, np.arange(32, dtype=np.float32))


def test_q4_engine_layout_pairs_adjacent_elements(orc):
    """The engine's Q4_0 pairs adjacent elements in a byte (quant.cpp:87-96),
    unlike GGUF's j / j+16 (gguf_test.cpp:419-453): byte 0x91 at scale 2 is
    element 0 = (1-8)*2 = -14 and element 1 = (9-8)*2 = 2."""
    data = np.full(16, 0x88, dtype=np.uint8)
    data[0] = 0x91
    row = orc.dequantize_row(data, np.array([2.0], np.float32), 1, 32, Q4, 0)
    assert row[0] == -14.0 and row[1] == 2.0
    assert np.all(row[2:] == 0.0)


def test_matmul_matches_fp64_brute_force(orc):
    """quant_test.cpp:131-183's check, tightened: y vs an fp64 dot product of
    the dequantized rows, relative to max|y| <= 1e-5."""
    rows, n_in, out = 3, 300, 4000
    x = synth.normal(6, rows * n_in, 0.0, 1.0)
    bias = synth.normal(8, out, 0.0, 1.0)
    w = synth.normal(7, out * n_in, 0.0, 0.3)
    for qt in (Q8, Q4):
        data, scales = orc.quantize(w, out, n_in, qt)
        y = orc.matmul(x, rows, n_in, data, scales, qt, out, bias).reshape(rows, out)
        deq = np.stack([orc.dequantize_row(data, scales, out, n_in, qt, o) for o in range(out)]).astype(np.float64)
        want = x.reshape(rows, n_in).astype(np.float64) @ deq.T + bias.astype(np.float64)
        assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 1e-5
        # Threaded and serial runs are the same computation.
        y1 = orc.matmul(x, rows, n_in, data, scales, qt, out, bias, threads=1).reshape(rows, out)
        assert np.array_equal(bits(y), bits(y1))


def test_rope_relative_position_and_softmax_properties(orc):
    """transformer_test.cpp:88-141 (RoPE at position 0 is the identity,
    scores depend on relative position only; softmax is normalised and
    stable)."""
    d = 16
    inv = np.array([np.float32(1.0) / np.power(np.float32(10000.0), np.float32(2 * i) / np.float32(d))
                    for i in range(d // 2)], dtype=np.float32)
    q = synth.normal(2, d, 0.0, 0.5)
    k = synth.normal(3, d, 0.0, 0.5)
    assert np.array_equal(orc.rope(q, 0, inv), q)
    score = lambda m, n: orc.dot(orc.rope(q, m, inv), orc.rope(k, n, inv))  # noqa: E731
    assert abs(score(5, 2) - score(13, 10)) < 1e-4
    s = orc.softmax(np.array([1000, 1001, 999], np.float32))
    assert abs(s.sum() - 1.0) < 1e-6 and abs(s[1] / s[0] - np.e) < 1e-4
    assert orc.softmax(np.array([-5.0], np.float32))[0] == 1.0
    assert orc.argmax(np.array([1, 3, 2, 3], np.float32)) == 1


def test_cached_prefill_equals_one_token_at_a_time(orc):
    """transformer_test.cpp:322-381: the KV cache reproduces the same logits
    whether the prompt is prefilled at once or fed token by token; and the
    model is causal (transformer_test.cpp:201-218)."""
    for arch in (0, 1):
        cfg = synth.tiny(arch, True)
        for qt in (O.F32, Q8, Q4):
            m = orc.model(cfg, synth.make_tensors(cfg, 11, "tiny"), qt)
            ids = np.array([2, 17, 4, 9, 21, 0, 13], np.int32)
            assert m.new_cache(len(ids))
            allpos = m.forward_cached(ids, all_positions=True).reshape(len(ids), -1)
            assert m.new_cache(len(ids))
            for t, tok in enumerate(ids):
                assert np.array_equal(bits(m.forward_cached([tok])), bits(allpos[t])), (arch, qt, t)
            other = ids.copy()
            other[4] = 1
            assert m.new_cache(len(ids))
            alt = m.forward_cached(other, all_positions=True).reshape(len(ids), -1)
            assert np.array_equal(bits(alt[:4]), bits(allpos[:4]))
            assert not np.array_equal(alt[4:], allpos[4:])


def test_forward_rejects_bad_input(orc):
    """transformer_test.cpp:242-250, 400-411: empty input, out-of-range ids,
    full cache."""
    cfg = synth.tiny(0, True)
    m = orc.model(cfg, synth.make_tensors(cfg, 6, "tiny"), Q8)
    assert m.new_cache(3)
    assert m.forward_cached([]) is None
    assert m.forward_cached([32]) is None
    assert m.forward_cached([-1]) is None
    assert m.forward_cached([1, 2, 3]) is not None
    assert m.forward_cached([4]) is None  # cache is full
    assert not m.new_cache(0)

"""GPU parity of the quantized matmul (decode GEMV, small batches and the
exact multi-row path): bit-exact against the compiled reference's golden
outputs and the oracle."""

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


def test_small_cases_match_reference(golden):
    rec, arrays = golden
    g = arrays["quant_small"]
    for c in rec["quant_small"]:
        k, qt, out, n_in, rows = c["key"], c["type"], c["out"], c["n_in"], c["rows"]
        x = synth.normal(c["x_seed"], rows * n_in, 0.0, 1.0)
        bias = synth.normal(c["bias_seed"], out, 0.0, 1.0)
        dev = H.Weight.upload(g[k + "_data"], g[k + "_scales"], out, n_in, qt)
        assert np.array_equal(bits(dev.matmul(x, rows, bias)), bits(g[k + "_y"])), k
        assert np.array_equal(bits(dev.matmul(x, rows, None)), bits(g[k + "_ynb"])), k
        for r in range(rows):  # batch-1 kernel on each row
            y1 = dev.matmul(x[r * n_in:(r + 1) * n_in], 1, bias)
            assert np.array_equal(bits(y1), bits(g[k + "_y"][r * out:(r + 1) * out])), (k, r)


def test_baseline_shapes_match_reference(golden):
    """C1 (Q8_0 1536x576 b1), every C2 SmolLM2 shape in Q4_0 at b1 and b8,
    and the Qwen2.5-0.5B shapes (incl. the 151936x896 lm_head)."""
    rec, _ = golden
    for c in rec["shapes"]:
        out, n_in, qt = c["out"], c["n_in"], c["type"]
        buf = H.DeviceBuffer(out * n_in * 4)
        H.synth_normal_dev(buf, out * n_in, c["w_seed"], 0.0, c["w_std"])
        w = H.Weight.quantize_dev(buf.ptr, out, n_in, qt)
        buf.free()
        for b, yrec in c["y"].items():
            x = synth.normal(c["x_seed"], int(b) * n_in, 0.0, 1.0)
            y = w.matmul(x, int(b))
            assert sha(y) == yrec["sha256"], (c["name"], qt, b, float(np.max(np.abs(y))), yrec["max_abs"])
        w.free()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 7, 8, 9, 17, 64])
@pytest.mark.parametrize("out,n_in", [(1, 1), (63, 33), (65, 100), (200, 576), (130, 4864), (96, 8192),
                                      (40, 20000)])
def test_batches_and_ragged_shapes_match_oracle(qt, rows, out, n_in):
    """Batch 1-8 GEMVs and, above 8 rows, the multi-row products on ragged
    shapes."""
    orc = O.oracle()
    w = synth.normal(out * 7 + n_in, out * n_in, 0.0, 0.02)
    x = synth.normal(rows * 13 + n_in, rows * n_in, 0.0, 1.0)
    bias = synth.normal(5, out, 0.0, 0.5)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    for b in (bias, None):
        got = dev.matmul(x, rows, b)
        want = orc.matmul(x, rows, n_in, data, scales, qt, out, b)
        assert np.array_equal(bits(got), bits(want)), (rows, out, n_in, b is None)


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("out,n_in,rows", [(40000, 100, 100), (40000, 100, 64), (4000, 200, 64), (200, 576, 64),
                                           (130, 4864, 33)])
def test_multi_row_launch_shapes_match_oracle(qt, out, n_in, rows):
    """Each multi-row launch shape with a partial final block: the per-tile
    product (64-row chunks giving >= 1024 workgroups) and the split-block
    product at 4 rows x 4 wavefronts, 4 x 8 and 2 x 8."""
    orc = O.oracle()
    w = synth.normal(out + 3 * n_in, out * n_in, 0.0, 0.02)
    x = synth.normal(rows + 7 * n_in, rows * n_in, 0.0, 1.0)
    bias = synth.normal(9, out, 0.0, 0.5)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    got = dev.matmul(x, rows, bias)
    want = orc.matmul(x, rows, n_in, data, scales, qt, out, bias)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("out,n_in", [(1, 1536), (15, 1537), (17, 1550), (64, 4864), (100, 4870), (576, 1536),
                                      (896, 4864), (2000, 3000), (33, 15000)])
def test_long_row_products_match_oracle(qt, out, n_in):
    """Batch-1 products on long rows (48 to 469 blocks: the 16-row tiles
    with many lane groups, or the 64-row tiles with the blocks spread over
    up to 16 wavefronts): ragged rows and partial final blocks, with and
    without bias, three calls in a row on different activations."""
    orc = O.oracle()
    w = synth.normal(out * 3 + n_in, out * n_in, 0.0, 0.02)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    bias = synth.normal(out + 1, out, 0.0, 0.5)
    for call in range(3):
        x = synth.normal(call * 101 + n_in, n_in, 0.0, 1.0)
        b = bias if call != 1 else None
        got = dev.matmul(x, 1, b)
        want = orc.matmul(x, 1, n_in, data, scales, qt, out, b)
        assert np.array_equal(bits(got), bits(want)), (out, n_in, call)
    dev.free()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("out,rows", [(40, 1), (8200, 1), (8200, 3)])
def test_block_chain_round_boundaries_match_oracle(qt, out, rows):
    """Rows of 3 to 65 blocks around the block chains' rounds (4 and 8
    blocks on the 64-row tiles, 16 and 32 pairs on the 16-row tiles, whose
    look-ahead reads past the last block; up to 33 blocks on the 64-row
    tiles, where the rounds are shorter): 40 outputs take the 16-row tiles,
    8200 (129 tiles, the last one partial) the 64-row tiles, 3 input rows
    the multi-row chains."""
    orc = O.oracle()
    wide = (3, 4, 5, 7, 8, 9, 12, 15, 16, 17, 24, 33)
    narrow = (3, 4, 5, 7, 8, 9, 15, 16, 17, 24, 31, 32, 33, 40, 47, 48, 63, 64, 65)
    for nblk in narrow if out < 64 else wide:
        n_in = 32 * nblk - (5 if nblk % 2 else 0)  # odd block counts end on a partial block
        w = synth.normal(nblk * 11 + out, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, qt)
        dev = H.Weight.upload(data, scales, out, n_in, qt)
        x = synth.normal(nblk + 3 * rows, rows * n_in, 0.0, 1.0)
        got = dev.matmul(x, rows, None)
        want = orc.matmul(x, rows, n_in, data, scales, qt, out, None)
        dev.free()
        assert np.array_equal(bits(got), bits(want)), (nblk, n_in)


def test_long_row_products_in_one_group_match_oracle():
    """A grouped launch holding long-row products next to short-row and
    multi-row ones: every output equals the oracle's, on two launches of the
    group."""
    orc = O.oracle()
    specs = [(896, 4864, 1, O.Q4_0), (576, 1536, 1, O.Q8_0), (4864, 896, 1, O.Q4_0), (100, 2000, 1, O.Q4_0),
             (300, 4864, 4, O.Q8_0), (65, 33, 1, O.Q8_0)]
    keep, items = [], []
    for i, (out, n_in, rows, qt) in enumerate(specs):
        w = synth.normal(60 + i, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, qt)
        dev = H.Weight.upload(data, scales, out, n_in, qt)
        xd = H.DeviceBuffer(rows * n_in * 4)
        yd = H.DeviceBuffer(rows * out * 4)
        keep.append((dev, xd, yd, rows, n_in, out, data, scales, qt))
        items.append((dev, xd.ptr, yd.ptr, rows))
    g = H.Group(items)
    for rep in range(2):
        for i, (dev, xd, yd, rows, n_in, out, data, scales, qt) in enumerate(keep):
            xd.upload(synth.normal(700 + 10 * rep + i, rows * n_in, 0.0, 1.0))
            yd.upload(np.full(rows * out, np.nan, np.float32))
        g.launch()
        H.synchronize()
        for i, (dev, xd, yd, rows, n_in, out, data, scales, qt) in enumerate(keep):
            x = synth.normal(700 + 10 * rep + i, rows * n_in, 0.0, 1.0)
            want = orc.matmul(x, rows, n_in, data, scales, qt, out, None)
            assert np.array_equal(bits(yd.download(np.float32)), bits(want)), (rep, specs[i])
    g.free()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q4_0])
def test_extreme_activations_match_oracle(qt):
    """Subnormal, zero, negative-zero and very large activations: the f16
    code operands of the Q4_0 fused multiply-adds and the Q8_0 conversions
    give the oracle's fp32 results bit for bit in every kernel shape."""
    orc = O.oracle()
    rng = np.random.default_rng(11)
    for out, n_in, rows in ((200, 576, 1), (4000, 96, 1), (200, 576, 3), (130, 100, 9), (65, 33, 1),
                             (130, 4864, 1)):
        w = synth.normal(out + n_in, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, qt)
        dev = H.Weight.upload(data, scales, out, n_in, qt)
        x = synth.normal(rows + n_in, rows * n_in, 0.0, 1.0)
        kind = rng.integers(0, 6, x.size)
        sub = (rng.uniform(-1, 1, x.size) * 2.0 ** -127).astype(np.float32)  # subnormal
        x = np.where(kind == 0, sub, x)
        x = np.where(kind == 1, np.float32(0.0), x)
        x = np.where(kind == 2, np.float32(-0.0), x)
        x = np.where(kind == 3, x * np.float32(1e30), x).astype(np.float32)
        assert np.count_nonzero(np.abs(x[kind == 0]) < 2.0 ** -126) > 0
        got = dev.matmul(x, rows, None)
        want = orc.matmul(x, rows, n_in, data, scales, qt, out, None)
        assert np.array_equal(bits(got), bits(want)), (out, n_in, rows)


@pytest.mark.parametrize("case", ["tiny", "edges", "one_bad_block", "huge"])
def test_q4_batch1_extreme_magnitudes(case):
    """Batch-1 Q4_0 products (f16 code operands of v_fma_mix_f32) on
    activations of extreme magnitude: all near 2^-100 (block sums that cancel
    down to a few units of 2^-123), values on both sides of 2^-100 and 2^101,
    one tiny value among ordinary ones, and values near 2^120 (sums that
    overflow).  The oracle's bits in the single-product kernels and in
    grouped launches (both tile sizes)."""
    orc = O.oracle()
    rng = np.random.default_rng({"tiny": 1, "edges": 2, "one_bad_block": 3, "huge": 4}[case])
    lo, hi_ok = np.float32(2.0 ** -100), np.nextafter(np.float32(2.0 ** 101), np.float32(0))
    shapes = ((200, 576), (4000, 96), (1536, 576), (65, 33))
    for out, n_in in shapes:
        w = synth.normal(out + n_in, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, O.Q4_0)
        dev = H.Weight.upload(data, scales, out, n_in, O.Q4_0)
        sign = np.where(rng.random(n_in) < 0.5, -1.0, 1.0).astype(np.float32)
        if case == "tiny":  # every |x| a little above 2^-100: sums cancel towards the 2^-123 grid
            x = (sign * lo * (1 + rng.integers(0, 4, n_in))).astype(np.float32)
        elif case == "edges":
            pick = rng.integers(0, 5, n_in)
            vals = np.array([lo, np.nextafter(lo, np.float32(0)), hi_ok, np.float32(2.0 ** 101), 0.0], np.float32)
            x = (sign * vals[pick]).astype(np.float32)
        elif case == "one_bad_block":  # ordinary values, one below the range
            x = synth.normal(n_in, n_in, 0.0, 1.0)
            x[rng.integers(0, n_in)] = np.float32(1e-35)
        else:
            x = (synth.normal(n_in, n_in, 0.0, 1.0) * np.float32(2.0 ** 120)).astype(np.float32)
        want = orc.matmul(x, 1, n_in, data, scales, O.Q4_0, out, None)
        got = dev.matmul(x, 1, None)
        assert np.array_equal(bits(got), bits(want)), (case, out, n_in)
        for spread in (False, True):  # grouped: alone (16-row tiles) or beside a big product (64-row tiles)
            xd, yd = H.DeviceBuffer.from_array(x), H.DeviceBuffer(out * 4)
            items = [(dev, xd.ptr, yd.ptr, 1, None)]
            extra = []
            if spread:
                big = H.Weight.quantize(synth.normal(5, 70000 * 96, 0.0, 0.02), 70000, 96, H.Q4_0)
                bx, by = H.DeviceBuffer.from_array(synth.normal(6, 96, 0.0, 1.0)), H.DeviceBuffer(70000 * 4)
                items.append((big, bx.ptr, by.ptr, 1, None))
                extra = [big, bx, by]
            g = H.Group(items)
            g.launch()
            H.synchronize()
            assert np.array_equal(bits(yd.download(np.float32)), bits(want)), (case, out, n_in, spread)
            g.free()
            for e in extra + [xd, yd]:
                e.free()
        dev.free()


def test_device_pointer_entry_point_and_determinism():
    orc = O.oracle()
    out, n_in, qt = 4864, 896, O.Q4_0
    w = synth.normal(1, out * n_in, 0.0, 0.02)
    data, scales = orc.quantize(w, out, n_in, qt)
    dev = H.Weight.upload(data, scales, out, n_in, qt)
    x = synth.normal(2, n_in, 0.0, 1.0)
    xd = H.DeviceBuffer.from_array(x)
    yd = H.DeviceBuffer(out * 4)
    first = None
    for _ in range(3):
        dev.matmul_dev(xd.ptr, 1, None, yd.ptr)
        H.synchronize()
        y = yd.download(np.float32)
        if first is None:
            first = y
        assert np.array_equal(bits(y), bits(first))
    assert np.array_equal(bits(first), bits(orc.matmul(x, 1, n_in, data, scales, qt, out, None)))


def test_graph_replays_match_eager_launches():
    """A captured sequence of matmuls, replayed several times with other
    eager work and synchronisations in between, gives the eager result on
    every replay."""
    orc = O.oracle()
    shapes = [(576, 576, O.Q4_0), (1536, 576, O.Q8_0), (576, 1536, O.Q4_0), (49152, 576, O.Q4_0)]
    weights, xs, ys, want = [], [], [], []
    for i, (out, n_in, qt) in enumerate(shapes):
        w = synth.normal(50 + i, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, qt)
        weights.append(H.Weight.upload(data, scales, out, n_in, qt))
        x = synth.normal(60 + i, n_in, 0.0, 1.0)
        xs.append(H.DeviceBuffer.from_array(x))
        ys.append(H.DeviceBuffer(out * 4))
        want.append(orc.matmul(x, 1, n_in, data, scales, qt, out, None))

    def record():
        for w, x, y in zip(weights, xs, ys):
            w.matmul_dev(x.ptr, 1, None, y.ptr)

    g = H.Graph(record)
    other = weights[1]
    for rep in range(4):
        for y in ys:
            y.upload(np.zeros(y.nbytes // 4, np.float32))
        g.launch()
        other.matmul_dev(xs[1].ptr, 1, None, ys[1].ptr)  # eager work between replays
        H.synchronize()
        for i, y in enumerate(ys):
            assert np.array_equal(bits(y.download(np.float32)), bits(want[i])), (rep, i)


def _group_case(specs, seed):
    """Weights, device inputs/outputs and oracle outputs for a group."""
    orc = O.oracle()
    items, want, keep = [], [], []
    for i, (out, n_in, qt, rows, with_bias) in enumerate(specs):
        w = synth.normal(seed + 31 * i, out * n_in, 0.0, 0.02)
        data, scales = orc.quantize(w, out, n_in, qt)
        dev = H.Weight.upload(data, scales, out, n_in, qt)
        x = synth.normal(seed + 31 * i + 1, rows * n_in, 0.0, 1.0)
        bias = synth.normal(seed + 31 * i + 2, out, 0.0, 0.5) if with_bias else None
        xd, yd = H.DeviceBuffer.from_array(x), H.DeviceBuffer(rows * out * 4)
        bd = H.DeviceBuffer.from_array(bias) if with_bias else None
        keep += [dev, xd, yd, bd]
        items.append((dev, xd.ptr, yd.ptr, rows, bd.ptr if bd is not None else None))
        want.append(orc.matmul(x, rows, n_in, data, scales, qt, out, bias))
    return items, want, keep


GROUP_SMALL = [(576, 576, O.Q8_0, 1, True), (192, 576, O.Q4_0, 1, False), (63, 33, O.Q4_0, 3, True),
               (130, 4864, O.Q8_0, 8, False), (1, 1, O.Q4_0, 2, True), (96, 8192, O.Q8_0, 1, False),
               (65, 100, O.Q4_0, 5, False), (1536, 576, O.Q4_0, 1, False)]


@pytest.mark.parametrize("big", [False, True])
def test_grouped_launch_matches_oracle(big):
    """llmi_hip_group: every product of one launch bit-identical to the
    oracle, in the few-tiles regime (16-row tiles at batch 1) and, with a
    70000-row matrix in the list, the many-tiles regime (64-row tiles)."""
    specs = GROUP_SMALL + ([(70000, 96, O.Q8_0, 1, True), (2000, 600, O.Q4_0, 7, False)] if big else [])
    items, want, keep = _group_case(specs, 700 + big)
    g = H.Group(items)
    for rep in range(2):
        for i in range(len(items)):
            keep[4 * i + 2].upload(np.full(keep[4 * i + 2].nbytes // 4, np.nan, np.float32))
        g.launch()
        H.synchronize()
        for i, it in enumerate(items):
            got = keep[4 * i + 2].download(np.float32)
            assert np.array_equal(bits(got), bits(want[i])), (rep, specs[i])
    g.free()


def test_grouped_launch_in_a_graph():
    items, want, keep = _group_case(GROUP_SMALL[:4], 900)
    g = H.Group(items)
    graph = H.Graph(lambda: g.launch())
    for rep in range(3):
        for i in range(len(items)):
            keep[4 * i + 2].upload(np.zeros(keep[4 * i + 2].nbytes // 4, np.float32))
        graph.launch()
        H.synchronize()
        for i in range(len(items)):
            assert np.array_equal(bits(keep[4 * i + 2].download(np.float32)), bits(want[i])), (rep, i)
    g.free()


def test_grouped_launch_rejects_bad_input():
    items, _, keep = _group_case([(64, 64, O.Q4_0, 1, False)], 5)
    dev, xp, yp = items[0][:3]
    with pytest.raises(H.HipError, match="1..8"):
        H.Group([(dev, xp, yp, 9)])
    with pytest.raises(H.HipError, match="null"):
        H.Group([(dev, None, yp, 1)])
    H.Group([]).launch()  # an empty group is a no-op

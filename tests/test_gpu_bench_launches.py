"""The launches bench.py times, checked at their own composition: the
211-product grouped launch of configs[1] (30 SmolLM2-135M layers x
{q, k, v, o, gate, up, down} + the 49152x576 lm_head, Q4_0) at batch 1 and
batch 8, and the same 211 products as one tolerance-mode group, built as
bench.WeightSet builds them (same seeds) with the bench's activations.
Each product writes its own output here (the bench shares an output
buffer among products of one shape, which only its timing tolerates).

Exact outputs must equal the oracle's quant::matmul (src/model/quant.cpp:
119-153) bit for bit; tolerance-mode outputs must stay within
1e-4 * max|y_ref| per product (the path's fp32-accumulate contract)."""

import numpy as np
import pytest

import bench
import llmi_hip as H
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def step_set():
    """One copy of the bench's weight set (copy 0, seed0 = 1) and the
    oracle's outputs at batch 1 and 8 on the bench's activations."""
    shapes = bench.step_shapes()
    assert len(shapes) == 211
    wset = bench.WeightSet(shapes, H.Q4_0, 1, 1)
    orc = O.oracle()
    packed = [w.download() for w in wset.copies[0]]
    per_batch = {}
    for batch in (1, 8):
        xs, _, keep = bench.activations(shapes, batch, 77)
        want = []
        for (_, out, n_in), (data, scales), x in zip(shapes, packed, xs):
            xh = x.download(np.float32, batch * n_in)
            want.append(orc.matmul(xh, batch, n_in, data, scales, H.Q4_0, out, None))
        per_batch[batch] = (xs, keep, want)
    yield shapes, wset, per_batch
    for _, keep, _ in per_batch.values():
        for xb, yb in keep.values():
            xb.free()
            yb.free()
    wset.free()


def _run(kind, shapes, ws, xs, batch):
    ys = [H.DeviceBuffer(batch * out * 4) for _, out, _ in shapes]
    g = kind([(w, x.ptr, y.ptr, batch) for w, x, y in zip(ws, xs, ys)])
    outs = []
    for _rep in range(2):  # launched twice: the second launch must not depend on the first's leftovers
        for y, (_, out, _) in zip(ys, shapes):
            y.upload(np.full(batch * out, np.nan, np.float32))
        g.launch()
        H.synchronize()
        outs.append([y.download(np.float32, batch * out) for y, (_, out, _) in zip(ys, shapes)])
    g.free()
    for y in ys:
        y.free()
    return outs


@pytest.mark.parametrize("batch", [1, 8])
def test_bench_exact_group_matches_oracle(step_set, batch):
    shapes, wset, per_batch = step_set
    xs, _, want = per_batch[batch]
    for rep, outs in enumerate(_run(H.Group, shapes, wset.copies[0], xs, batch)):
        for i, (got, ref) in enumerate(zip(outs, want)):
            assert np.array_equal(bits(got), bits(ref)), (batch, rep, i, shapes[i])


@pytest.mark.parametrize("batch", [1, 8])
def test_bench_tolerance_group_within_contract(step_set, batch):
    shapes, wset, per_batch = step_set
    xs, _, want = per_batch[batch]
    worst = 0.0
    for outs in _run(H.TolGroup, shapes, wset.copies[0], xs, batch):
        for i, (got, ref) in enumerate(zip(outs, want)):
            ref64 = ref.astype(np.float64)
            err = float(np.abs(got.astype(np.float64) - ref64).max() / max(np.abs(ref64).max(), 1e-30))
            assert err <= TOL, (batch, i, shapes[i], err)
            worst = max(worst, err)
    print(f"tolerance group, batch {batch}: worst relative error {worst:.3e}")

"""GPU parity of token sampling (src/model/sampling.cpp:11-77) through the
C ABI: llmi_hip_sampling_probabilities bit for bit against the oracle's
sampling_probabilities, and llmi_hip_sample's index equal to the oracle's
sample() for the same draw -- itself pinned to the compiled reference's
sample() sequences -- over vocabulary sizes up to Qwen2.5's, masked (-inf)
and tied logits, every filter, draws placed exactly on a running sum (where
the parallel sums' bound cannot decide and the sequential pass must), and
the reference's own sampling tests (tests/sampling_test.cpp)."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu

CONFIGS = [(1.0, 0, 1.0), (0.7, 40, 0.9), (1.3, 0, 0.5), (0.8, 1, 1.0), (1.0, 0, 0.0), (2.0, 5000, 0.95),
           (0.05, 0, 0.99), (1.0, 3, 0.3), (100.0, 0, 1.0)]


def logits_case(kind: str, n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, n).astype(np.float32)
    if kind == "masked":
        x[rng.random(n) < 0.9] = -np.inf
        x[n // 2] = 1.0
    elif kind == "ties":
        x = rng.integers(-3, 4, n).astype(np.float32)
    elif kind == "peaked":
        x[rng.integers(0, n)] = 40.0
    return x


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(autouse=True)
def _sequential_off():
    H.init()
    H.sampling_set_exact_only(False)
    yield
    H.sampling_set_exact_only(False)


def test_reference_known_answers_on_device():
    # sampling_test.cpp:15-110.
    cfg0 = H.Sampling(0.0)
    assert all(H.sample(np.array([1, 5, 3, 5, 2], np.float32), cfg0, t) == 1 for t in (0.0, 0.3, 0.99))
    p = H.sampling_probabilities(np.array([1, 2, 3, 4], np.float32), H.Sampling(1.0))
    e = np.exp(np.arange(1, 5, dtype=np.float64))
    assert abs(p.astype(np.float64).sum() - 1) < 1e-6 and np.allclose(p, e / e.sum(), atol=1e-5)
    hot = H.sampling_probabilities(np.array([0, 1, 2], np.float32), H.Sampling(100.0))
    cold = H.sampling_probabilities(np.array([0, 1, 2], np.float32), H.Sampling(0.01))
    assert abs(hot[0] - hot[2]) < 0.05 and cold[2] > 0.99
    p = H.sampling_probabilities(np.array([5, 1, 4, 2, 3], np.float32), H.Sampling(1.0, top_k=2))
    assert p[0] > 0 and p[2] > 0 and p[1] == p[3] == p[4] == 0
    p = H.sampling_probabilities(np.array([10, 0, 0, 0, 0], np.float32), H.Sampling(1.0, top_p=0.5))
    assert abs(p[0] - 1) < 1e-5 and np.all(p[1:] == 0)
    p = H.sampling_probabilities(np.array([1, 1, 1, 1], np.float32), H.Sampling(1.0, top_p=0.0))
    assert np.count_nonzero(p) == 1 and p[0] == 1.0
    draws = O.oracle().draw_uniform(7, 200)
    lg = np.array([5, 1, 4, 2, 3], np.float32)
    assert {H.sample(lg, H.Sampling(1.0, top_k=2), t) for t in draws} <= {0, 2}


@pytest.mark.parametrize("kind", ["normal", "masked", "ties", "peaked"])
@pytest.mark.parametrize("n", [1, 5, 1000, 49152])
def test_probabilities_and_draws_match_oracle(kind, n):
    o = O.oracle()
    for c, (temp, top_k, top_p) in enumerate(CONFIGS):
        lg = logits_case(kind, n, 100 * n + c)
        cfg = H.Sampling(temp, top_k, top_p)
        want = o.sampling_probabilities(lg, temp, top_k, top_p)
        got = H.sampling_probabilities(lg, cfg)
        assert np.array_equal(bits(got), bits(want)), (temp, top_k, top_p)
        for t in o.draw_uniform(1000 + c, 12):
            assert H.sample(lg, cfg, t) == o.sample_target(lg, temp, top_k, top_p, t), (temp, top_k, top_p, t)


@pytest.mark.parametrize("kind", ["normal", "masked", "ties"])
@pytest.mark.parametrize("n", [70, 4100, 8193, 151936])
def test_top_k_around_the_selection_limit(kind, n):
    """top_k up to 64 takes the per-slice selection, 65 and above the full
    sort; ties and zero probabilities straddle the k-th entry, and slices
    hold fewer entries than k when n is small."""
    o = O.oracle()
    for k in (2, 63, 64, 65):
        lg = logits_case(kind, n, 7 * n + k)
        want = o.sampling_probabilities(lg, 1.0, k, 1.0)
        assert np.array_equal(bits(H.sampling_probabilities(lg, H.Sampling(1.0, k, 1.0))), bits(want)), k
        assert np.count_nonzero(want) <= k
        for t in o.draw_uniform(k, 4):
            assert H.sample(lg, H.Sampling(1.0, k, 0.9), t) == o.sample_target(lg, 1.0, k, 0.9, t), (k, t)


@pytest.mark.parametrize("cfg", [(1.0, 0, 1.0), (0.8, 40, 0.9), (0.6, 0, 0.95), (1.0, 1000, 1.0)])
def test_qwen_vocabulary(cfg):
    """151936 entries (Qwen2.5's vocabulary), device-resident logits."""
    o = O.oracle()
    lg = logits_case("normal", 151936, 5)
    c = H.Sampling(*cfg)
    assert np.array_equal(bits(H.sampling_probabilities(lg, c)), bits(o.sampling_probabilities(lg, *cfg)))
    buf = H.DeviceBuffer(lg.nbytes)
    buf.upload(lg)
    for t in o.draw_uniform(9, 6):
        assert H.sample_dev(buf, lg.size, c, t) == o.sample_target(lg, *cfg, t)
    buf.free()


def running_sums(f: np.ndarray) -> np.ndarray:
    """sample()'s running sum in index order (sequential double additions)."""
    return np.cumsum(f.astype(np.float64))


@pytest.mark.parametrize("cfg", [(1.0, 0, 1.0), (0.9, 50, 0.8)])
def test_draws_on_a_running_sum_take_the_sequential_pass(cfg):
    """target equal to the reference's running sum at j (or one ulp either
    side): the parallel bound cannot separate j from its neighbours, so the
    device must take the sequential passes -- and still return the
    reference's index."""
    o = O.oracle()
    lg = logits_case("normal", 20000, 11)
    f = o.sampling_probabilities(lg, *cfg)
    run = running_sums(f)
    nz = np.flatnonzero(f)
    c = H.Sampling(*cfg)
    seen = 0
    for j in nz[[0, 1, len(nz) // 3, len(nz) // 2, -2]]:
        for t in (run[j], np.nextafter(run[j], 0.0), np.nextafter(run[j], 2.0)):
            got = H.sample(lg, c, t)
            assert got == o.sample_target(lg, *cfg, t), (j, t)
            seen |= H.sampling_last_paths()
    # The draw's running sum and/or the renormalisation sum went sequential
    # (with top_k <= 64 they always do, over the select's ranked values).
    assert seen & (4 | 8 | 16)


@pytest.mark.parametrize("kind", ["normal", "ties", "masked"])
@pytest.mark.parametrize("n", [1000, 49152, 151936])
def test_top_p_sweep_over_the_ranking(kind, n):
    """top_p alone (and with a top_k above the selection limit) ranks the
    whole vocabulary with the radix sort: kept prefixes from one entry to
    nearly all of them, cut inside groups of tied logits, must be the
    reference's (descending p, ties in index order)."""
    o = O.oracle()
    lg = logits_case(kind, n, 11 * n + len(kind))
    for top_p in (0.001, 0.05, 0.2, 0.45, 0.6, 0.8, 0.9, 0.97, 0.995, 0.99999):
        for temp, top_k in ((1.0, 0), (0.5, 0), (1.0, 700)):
            want = o.sampling_probabilities(lg, temp, top_k, top_p)
            got = H.sampling_probabilities(lg, H.Sampling(temp, top_k, top_p))
            assert np.array_equal(bits(got), bits(want)), (top_p, temp, top_k)


@pytest.mark.parametrize("kind", ["ties", "normal"])
def test_ranking_past_a_thousand_tiles_of_1024(kind):
    """5,000,000 logits: the ranking sort's tiles grow past 1024 elements
    (at most 4096 tiles), so each workgroup of its passes walks several
    rounds of 256; top-p cuts inside groups of tied logits."""
    o = O.oracle()
    lg = logits_case(kind, 5_000_000, 17)
    for cfg in ((1.0, 0, 0.3), (0.8, 2000, 0.99)):
        want = o.sampling_probabilities(lg, *cfg)
        got = H.sampling_probabilities(lg, H.Sampling(*cfg))
        assert np.array_equal(bits(got), bits(want)), cfg


def test_top_p_on_a_running_sum():
    """Probabilities that are exact binary fractions put top_p exactly on a
    ranked running sum (keep = 2 for top_p 0.5 over four equal logits)."""
    lg = np.zeros(4, np.float32)
    o = O.oracle()
    for top_p, keep in ((0.5, 2), (0.75, 3), (0.25, 1), (1.0 - 2**-24, 4)):
        p = H.sampling_probabilities(lg, H.Sampling(1.0, 0, top_p))
        assert np.count_nonzero(p) == keep, top_p
        assert np.array_equal(bits(p), bits(o.sampling_probabilities(lg, 1.0, 0, top_p)))
        assert H.sampling_last_paths() & 2 or keep == 4


@pytest.mark.parametrize("n", [16, 5000])
def test_select_path_on_exact_boundaries(n):
    """top_k <= 64 takes the select path, whose top-p cumulative,
    renormalisation sum and draw run sequentially over the ranked values.
    Equal logits make every one of them a binary fraction: top_p and the
    draw's targets land exactly on running sums (and one ulp either side)."""
    o = O.oracle()
    lg = np.zeros(n, np.float32)
    lg[n // 2:] = -1.0  # a second level: the kept come from the first half, ties by index
    for top_k, top_p in ((8, 1.0), (8, 0.0), (8, 2.0**-20), (40, 1.0), (64, 1.0)):
        cfg = (1.0, top_k, top_p)
        p = H.sampling_probabilities(lg, H.Sampling(*cfg))
        assert np.array_equal(bits(p), bits(o.sampling_probabilities(lg, *cfg))), cfg
        run = running_sums(p)
        nz = np.flatnonzero(p)
        for j in sorted({nz[0], nz[min(1, len(nz) - 1)], nz[-2 if len(nz) > 1 else 0], nz[-1]}):
            for t in (run[j], np.nextafter(run[j], 0.0), np.nextafter(run[j], 2.0), 0.0):
                assert H.sample(lg, H.Sampling(*cfg), t) == o.sample_target(lg, *cfg, t), (cfg, j, t)
        assert bool(H.sampling_last_paths() & 16) == (top_k < n)


@pytest.mark.parametrize("n", [5, 3000])
def test_sequential_passes_agree(n):
    """With every sum forced onto its sequential pass the results are the same."""
    o = O.oracle()
    for c, (temp, top_k, top_p) in enumerate(CONFIGS[:6]):
        lg = logits_case("normal", n, 7 + c)
        cfg = H.Sampling(temp, top_k, top_p)
        ts = o.draw_uniform(50 + c, 5)
        fast = [H.sample(lg, cfg, t) for t in ts]
        H.sampling_set_exact_only(True)
        slow = [H.sample(lg, cfg, t) for t in ts]
        H.sampling_set_exact_only(False)
        assert fast == slow == [o.sample_target(lg, temp, top_k, top_p, t) for t in ts]


def test_edge_inputs():
    o = O.oracle()
    one = np.array([3.0], np.float32)
    assert H.sample(one, H.Sampling(1.0), 0.7) == 0
    assert list(H.sampling_probabilities(one, H.Sampling(0.5))) == [1.0]
    neg = np.full(6, -np.inf, np.float32)  # every entry masked: the reference falls back to argmax (0)
    assert H.sample(neg, H.Sampling(1.0), 0.4) == 0
    p = H.sampling_probabilities(neg, H.Sampling(1.0, top_k=2))
    assert np.all(np.isnan(p[:2])) and np.all(p[2:] == 0)
    assert np.array_equal(np.isnan(p), np.isnan(o.sampling_probabilities(neg, 1.0, 2)))
    tiny_t = np.array([1.0, 2.0, 3e38], np.float32)
    for bad, cfg in ((np.array([1.0, np.nan], np.float32), H.Sampling(1.0)),
                     (np.array([1.0, np.inf], np.float32), H.Sampling(1.0)),
                     (tiny_t, H.Sampling(1e-3))):  # 3e38 / 1e-3 overflows to +inf
        with pytest.raises(H.HipError):
            H.sample(bad, cfg, 0.5)
    with pytest.raises(H.HipError):
        H.sample(np.zeros(0, np.float32), H.Sampling(1.0), 0.5)
    # target 0 picks index 0 (0 >= 0), even when that entry is filtered out.
    lg = np.array([0.0, 5.0, 1.0], np.float32)
    assert H.sample(lg, H.Sampling(1.0, top_k=1), 0.0) == o.sample_target(lg, 1.0, 1, 1.0, 0.0) == 0


def toy_cfg():
    return dict(arch=1, vocab_size=512, hidden_size=128, intermediate_size=256, num_layers=2, num_heads=2,
                num_kv_heads=1, max_position_embeddings=256, rms_norm_eps=1e-6, rope_theta=10000.0,
                tie_word_embeddings=1, qkv_bias=1)


@pytest.mark.parametrize("qt", [H.Q8_0, H.Q4_0])
def test_model_steps_sample_like_the_reference_loop(qt):
    """forward_sample / generate_sampled against the oracle's model running
    the server loop (server.cpp:109-195): forward_cached, sample(), repeat."""
    cfg = toy_cfg()
    tensors = synth.make_tensors(cfg, 60 + qt, "bench")
    cpu = O.reference() or O.oracle()
    cm = O.CpuModel(cpu, cfg, tensors, qt)
    prompt = synth.uniform_ids(61, 12, cfg["vocab_size"])
    sc = (0.9, 40, 0.95)
    steps = 24
    targets = O.oracle().draw_uniform(62, steps)
    assert cm.new_cache(64)
    want = []
    logits = cm.forward_cached(prompt)
    for s in range(steps):
        nxt = O.oracle().sample_target(logits, *sc, targets[s])
        want.append(nxt)
        logits = cm.forward_cached([nxt])
    cm.close()
    gm = H.Model(cfg, tensors, qt)
    c = gm.new_cache(64)
    got = [gm.forward_sample(c, prompt, H.Sampling(*sc), targets[0])]
    for s in range(1, steps):
        got.append(gm.forward_sample(c, [got[-1]], H.Sampling(*sc), targets[s]))
    c.free()
    assert got == want
    ids = gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets)
    assert list(ids) == want
    assert gm.last_redraws() == 0  # every step ran queued on the device
    stop = want[5]
    ids = gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets, stop_ids=[stop])
    assert list(ids) == want[: want.index(stop) + 1]
    gm.free()


@pytest.mark.parametrize("crafted", [(0, 37), (6, 37)])
@pytest.mark.parametrize("sc", [(1.0, 0, 1.0), (0.9, 100, 0.8), (0.9, 50, 0.8)])
def test_generate_sampled_redraws_an_undecided_queued_step(sc, crafted):
    """generate_sampled queues its steps on the device in windows of 32.  A
    draw whose target sits on the reference's running sum (the bounds cannot
    decide it on the device) sends the run back to that step: the cache is
    rolled back (to the prompt for step 0), the step's logits recomputed and
    the draw settled exactly, and queueing resumes after it.  The ids must
    still be the reference loop's, with at least one crafted step redrawn
    (a bound may happen to decide one; 37 lies in the second window) --
    except with top_k <= 64, whose draw is exact on the device: none."""
    cfg = toy_cfg()
    tensors = synth.make_tensors(cfg, 70, "bench")
    cpu = O.reference() or O.oracle()
    o = O.oracle()
    cm = O.CpuModel(cpu, cfg, tensors, H.Q4_0)
    prompt = synth.uniform_ids(71, 9, cfg["vocab_size"])
    steps = 45
    targets = o.draw_uniform(72, steps).astype(np.float64)
    assert cm.new_cache(64)
    want = []
    logits = cm.forward_cached(prompt)
    for s in range(steps):
        if s in crafted:
            f = o.sampling_probabilities(logits, *sc)
            nz = np.flatnonzero(f)
            targets[s] = running_sums(f)[nz[len(nz) // 2]]
        want.append(o.sample_target(logits, *sc, targets[s]))
        logits = cm.forward_cached([want[-1]])
    cm.close()
    gm = H.Model(cfg, tensors, H.Q4_0)
    ids = gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets)
    assert list(ids) == want
    if sc[1] == 50:
        assert gm.last_redraws() == 0
    else:
        assert 1 <= gm.last_redraws() <= len(crafted)
    for stop in (want[crafted[0]], want[40]):  # a stop drawn at a crafted step, and after one
        ids = gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets, stop_ids=[stop])
        assert list(ids) == want[: want.index(stop) + 1]
    gm.free()


@pytest.mark.parametrize("steps", [1, 31, 32, 33, 64])
def test_generate_sampled_at_window_boundaries(steps):
    """generate_sampled queues 32 steps per host read-back: runs of one step,
    a window less one, exactly one and two windows, and one step past a
    window give the reference loop's ids, as does a stop id drawn at the last
    step; temperature 0 redraws nothing."""
    cfg = toy_cfg()
    tensors = synth.make_tensors(cfg, 80, "bench")
    cpu = O.reference() or O.oracle()
    o = O.oracle()
    cm = O.CpuModel(cpu, cfg, tensors, H.Q8_0)
    prompt = synth.uniform_ids(81, 7, cfg["vocab_size"])
    sc = (1.1, 0, 1.0)
    targets = o.draw_uniform(82, steps)
    assert cm.new_cache(96)
    want = []
    logits = cm.forward_cached(prompt)
    for s in range(steps):
        want.append(o.sample_target(logits, *sc, targets[s]))
        logits = cm.forward_cached([want[-1]])
    cm.close()
    gm = H.Model(cfg, tensors, H.Q8_0)
    assert list(gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets)) == want
    stop = want[-1]
    assert list(gm.generate_sampled(prompt, steps, H.Sampling(*sc), targets, stop_ids=[stop])) == \
        want[: want.index(stop) + 1]
    greedy = gm.generate_greedy(prompt, steps)
    assert list(gm.generate_sampled(prompt, steps, H.Sampling(0.0), [])) == list(greedy)
    assert gm.last_redraws() == 0
    gm.free()


def test_shutdown_releases_and_reinit_works():
    """llmi_hip_shutdown frees the library's sampling and GEMM workspaces;
    a later llmi_hip_init starts clean and sampling still gives the oracle's
    index."""
    lib = H.init()
    lg = logits_case("normal", 5000, 21)
    want = O.oracle().sample_target(lg, 0.9, 20, 0.9, 0.37)
    assert H.sample(lg, H.Sampling(0.9, 20, 0.9), 0.37) == want
    H.check(lib.llmi_hip_shutdown())
    H.check(lib.llmi_hip_init(0))
    assert H.sample(lg, H.Sampling(0.9, 20, 0.9), 0.37) == want

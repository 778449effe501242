"""The oracle's restatement of sampling (src/model/sampling.cpp:11-77) pinned
four ways: the reference's own sampling tests (tests/sampling_test.cpp), the
compiled reference (probabilities bit for bit; ids and drawn numbers of whole
sample() sequences on one seeded generator), a plain double-precision softmax
and the ranking invariants of top-k / top-p, and -- for the random numbers --
the C++ standard's known answer for mt19937_64 plus the closed form of
uniform_real_distribution<double>(0, 1) in libstdc++ (one 64-bit output x
gives double(x) / 2^64)."""

import numpy as np
import pytest

import oracle as O


def impls():
    out = [("oracle", O.oracle())]
    ref = O.reference()
    if ref is not None:
        out.append(("reference", ref))
    return out


# -- sampling_test.cpp, on both implementations ---------------------------------
@pytest.mark.parametrize("name,cpu", impls())
def test_reference_known_answers(name, cpu):
    # TemperatureZeroIsGreedy: first maximum.
    assert list(cpu.sampling_probabilities([1, 5, 3, 5, 2], 0.0)) == [0, 1, 0, 0, 0]
    # ProbabilitiesSumToOneAndFollowSoftmax.
    p = cpu.sampling_probabilities([1, 2, 3, 4], 1.0)
    assert abs(p.astype(np.float64).sum() - 1.0) < 1e-6 and np.all(np.diff(p) > 0)
    e = np.exp(np.arange(1, 5, dtype=np.float64))
    assert np.allclose(p, e / e.sum(), atol=1e-5)
    # TemperatureFlattensOrSharpensTheDistribution.
    hot, cold = cpu.sampling_probabilities([0, 1, 2], 100.0), cpu.sampling_probabilities([0, 1, 2], 0.01)
    assert abs(hot[0] - hot[2]) < 0.05 and cold[2] > 0.99
    # TopKKeepsOnlyTheKHighest.
    p = cpu.sampling_probabilities([5, 1, 4, 2, 3], 1.0, top_k=2)
    assert p[0] > 0 and p[2] > 0 and p[1] == p[3] == p[4] == 0
    # TopPKeepsTheSmallestSufficientNucleus.
    p = cpu.sampling_probabilities([10, 0, 0, 0, 0], 1.0, top_p=0.5)
    assert abs(p[0] - 1.0) < 1e-5 and np.all(p[1:] == 0)
    # TopPAlwaysKeepsAtLeastOneToken.
    p = cpu.sampling_probabilities([1, 1, 1, 1], 1.0, top_p=0.0)
    assert np.count_nonzero(p) == 1 and p[0] == 1.0


def test_draws_stay_in_the_filtered_set_and_repeat_with_the_seed():
    # DrawsStayWithinTheFilteredSet / SameSeedReproducesTheSameDraws.
    o = O.oracle()
    lg = np.array([5, 1, 4, 2, 3], np.float32)
    t = o.draw_uniform(7, 200)
    assert set(o.sample_target(lg, 1.0, 2, 1.0, x) for x in t) <= {0, 2}
    assert np.array_equal(o.draw_uniform(42, 20), o.draw_uniform(42, 20))
    assert not np.array_equal(o.draw_uniform(1, 50), o.draw_uniform(2, 50))


# -- the compiled reference --------------------------------------------------------
CONFIGS = [(1.0, 0, 1.0), (0.7, 40, 0.9), (1.3, 0, 0.5), (0.8, 1, 1.0), (1.0, 0, 0.0), (0.0, 0, 1.0),
           (2.0, 5000, 0.95), (0.05, 0, 0.99), (1.0, 3, 0.3), (100.0, 0, 1.0)]


def logits_case(kind: str, n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, n).astype(np.float32)
    if kind == "masked":  # a grammar mask: most entries -inf (constraint.cpp:62-69)
        x[rng.random(n) < 0.9] = -np.inf
        x[n // 2] = 1.0
    elif kind == "ties":  # few distinct values: ranking ties resolved by index
        x = rng.integers(-3, 4, n).astype(np.float32)
    elif kind == "peaked":
        x[rng.integers(0, n)] = 40.0
    return x


@pytest.mark.skipif(O.reference() is None, reason="oracle/_ref was not built (no reference sources)")
@pytest.mark.parametrize("kind", ["normal", "masked", "ties", "peaked"])
@pytest.mark.parametrize("n", [1, 5, 1000, 49152])
def test_oracle_matches_compiled_reference(kind, n):
    o, r = O.oracle(), O.reference()
    for c, (temp, top_k, top_p) in enumerate(CONFIGS):
        lg = logits_case(kind, n, 100 * n + c)
        a = o.sampling_probabilities(lg, temp, top_k, top_p)
        b = r.sampling_probabilities(lg, temp, top_k, top_p)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (temp, top_k, top_p)
        seed = 1000 + c
        ids, drawn = r.sample_sequence(lg, temp, top_k, top_p, seed, 40)
        if temp > 0:
            assert np.array_equal(drawn, o.draw_uniform(seed, 40))
        got = [o.sample_target(lg, temp, top_k, top_p, t) for t in drawn]
        assert list(ids) == got, (temp, top_k, top_p)


@pytest.mark.skipif(O.reference() is None, reason="oracle/_ref was not built (no reference sources)")
def test_oracle_matches_reference_at_the_qwen_vocabulary():
    o, r = O.oracle(), O.reference()
    lg = logits_case("normal", 151936, 5)
    for temp, top_k, top_p in [(1.0, 0, 1.0), (0.8, 40, 0.9), (0.6, 0, 0.95)]:
        a = o.sampling_probabilities(lg, temp, top_k, top_p)
        b = r.sampling_probabilities(lg, temp, top_k, top_p)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        ids, drawn = r.sample_sequence(lg, temp, top_k, top_p, 9, 8)
        assert list(ids) == [o.sample_target(lg, temp, top_k, top_p, t) for t in drawn]


# -- mathematics -------------------------------------------------------------------
def test_unfiltered_probabilities_are_a_double_softmax():
    lg = logits_case("normal", 2000, 3)
    for temp in (0.5, 1.0, 3.0):
        p = O.oracle().sampling_probabilities(lg, temp)
        z = lg.astype(np.float64) / temp
        e = np.exp(z - z.max())
        assert np.allclose(p, e / e.sum(), rtol=2e-6, atol=1e-12)


def test_filters_keep_the_right_ranks():
    """top-k keeps exactly the k most probable entries; top-p keeps the
    shortest most-probable prefix whose probability reaches top_p."""
    o = O.oracle()
    lg = logits_case("normal", 3000, 4)
    base = o.sampling_probabilities(lg, 1.0)
    order = np.argsort(-base, kind="stable")
    for k in (1, 7, 100):
        p = o.sampling_probabilities(lg, 1.0, top_k=k)
        assert set(np.flatnonzero(p)) == set(order[:k])
        assert abs(p.astype(np.float64).sum() - 1.0) < 1e-5
    for top_p in (0.1, 0.5, 0.9):
        p = o.sampling_probabilities(lg, 1.0, top_p=top_p)
        keep = np.count_nonzero(p)
        run = np.cumsum(base[order].astype(np.float64))
        assert set(np.flatnonzero(p)) == set(order[:keep])
        assert run[keep - 1] >= top_p and (keep == 1 or run[keep - 2] < top_p)


def test_sample_is_the_inverse_cdf():
    """With the draw given, sample() is the first index whose running sum of
    the filtered probabilities reaches it (brute force over a small case)."""
    o = O.oracle()
    lg = np.array([0.3, -1.0, 2.0, 0.0, 1.5], np.float32)
    for top_k, top_p in [(0, 1.0), (3, 1.0), (0, 0.6)]:
        f = o.sampling_probabilities(lg, 0.9, top_k, top_p).astype(np.float64)
        run = np.cumsum(f)
        for t in np.linspace(0.0, 0.999, 41):
            assert o.sample_target(lg, 0.9, top_k, top_p, t) == int(np.argmax(run >= t))


class MT19937_64:
    """The generator as ISO C++ [rand.predef] defines std::mt19937_64."""

    def __init__(self, seed: int):
        self.mt = [seed & 0xFFFFFFFFFFFFFFFF]
        for i in range(1, 312):
            prev = self.mt[-1]
            self.mt.append((6364136223846793005 * (prev ^ (prev >> 62)) + i) & 0xFFFFFFFFFFFFFFFF)
        self.i = 312

    def __call__(self) -> int:
        if self.i >= 312:
            mt = self.mt
            for k in range(312):
                y = (mt[k] & 0xFFFFFFFF80000000) | (mt[(k + 1) % 312] & 0x7FFFFFFF)
                mt[k] = mt[(k + 156) % 312] ^ (y >> 1) ^ (0xB5026F5AA96619E9 if y & 1 else 0)
            self.i = 0
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y


def test_generator_and_uniform_mapping():
    g = MT19937_64(5489)
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042  # [rand.predef]: the 10000th output of a default-constructed engine
    for seed in (0, 7, 2**63 + 5):
        g = MT19937_64(seed)
        want = []
        for _ in range(400):
            x = float(g()) / 2.0**64  # double(x) rounds to nearest; / 2^64 is exact
            want.append(x if x < 1.0 else np.nextafter(1.0, 0.0))
        assert np.array_equal(O.oracle().draw_uniform(seed, 400), np.array(want))

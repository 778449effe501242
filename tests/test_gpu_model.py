"""GPU parity of the glue kernels and the device-resident model against the
compiled reference: glue vectors, the reference's 2-layer test models
(logits bit for bit), the KV-cache invariants of
tests/transformer_test.cpp, and greedy ids of the synthetic SmolLM2-135M
(Q8_0, 128 + 256 steps) and Qwen2.5-0.5B (Q4_0, 512 + 512 steps) models."""

import hashlib
import json
import os

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ----------------------------------------------------------------- glue
def test_glue_kernels_match_reference(golden):
    _, arrays = golden
    g = arrays["kernels"]
    lib = H.init()
    a = H.DeviceBuffer.from_array(g["dot_a"])
    b = H.DeviceBuffer.from_array(g["dot_b"])
    lens = H.DeviceBuffer.from_array(g["dot_n"].astype(np.int32))
    out = H.DeviceBuffer(4 * g["dot_n"].size)
    H.check(lib.llmi_hip_dot_dev(a.ptr, b.ptr, lens.ptr, g["dot_n"].size, out.ptr, None))
    H.synchronize()
    assert np.array_equal(bits(out.download(np.float32)), bits(g["dot_out"]))

    for n, eps, key in ((576, 1e-5, "rms_576"), (896, 1e-6, "rms_896")):
        x = H.DeviceBuffer.from_array(g["rms_x"][:n])
        w = H.DeviceBuffer.from_array(g["rms_w"][:n])
        y = H.DeviceBuffer(4 * n)
        H.check(lib.llmi_hip_rmsnorm_dev(x.ptr, w.ptr, 1, n, eps, y.ptr, None))
        H.synchronize()
        assert np.array_equal(bits(y.download(np.float32)), bits(g[key])), key

    sm = H.DeviceBuffer.from_array(g["softmax_in"])
    H.check(lib.llmi_hip_softmax_dev(sm.ptr, 1, g["softmax_in"].size, None))
    H.synchronize()
    assert np.array_equal(bits(sm.download(np.float32)), bits(g["softmax_out"]))

    si = H.DeviceBuffer.from_array(g["silu_in"])
    H.check(lib.llmi_hip_silu_dev(si.ptr, g["silu_in"].size, None))
    H.synchronize()
    assert np.array_equal(bits(si.download(np.float32)), bits(g["silu_out"]))


def test_device_expf_and_silu_match_host_libm_over_the_range():
    """SiLU exercises expf(-x); sweep every exponent range, including the
    subnormal-result and overflow ends, against the oracle (host libm)."""
    orc = O.oracle()
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.uniform(-110, 110, 1 << 20).astype(np.float32),
                        (rng.standard_normal(1 << 18) * 8).astype(np.float32),
                        np.array([0.0, -0.0, 88.0, -88.0, 87.3, -87.3, 103.9, -103.9, 1e-30, -1e-30], np.float32)])
    d = H.DeviceBuffer.from_array(x)
    H.check(H.init().llmi_hip_silu_dev(d.ptr, x.size, None))
    H.synchronize()
    got = d.download(np.float32)
    want = np.array([orc.silu(v) for v in x[:20000]] , dtype=np.float32)
    assert np.array_equal(bits(got[:20000]), bits(want))
    # The rest through softmax rows (expf of non-positive arguments).
    rows = x[20000:20000 + 64 * 1000].reshape(64, 1000)
    d2 = H.DeviceBuffer.from_array(rows)
    H.check(H.init().llmi_hip_softmax_dev(d2.ptr, 64, 1000, None))
    H.synchronize()
    got2 = d2.download(np.float32).reshape(64, 1000)
    for r in range(64):
        assert np.array_equal(bits(got2[r]), bits(orc.softmax(rows[r]))), r


def test_argmax_takes_the_first_maximum():
    lib = H.init()
    out = H.DeviceBuffer(4)
    for x, want in (([1, 3, 2, 3], 1), ([5.0], 0), ([-1, -1, -1], 0)):
        d = H.DeviceBuffer.from_array(np.array(x, np.float32))
        H.check(lib.llmi_hip_argmax_dev(d.ptr, len(x), out.ptr, None))
        H.synchronize()
        assert int(out.download(np.int32)[0]) == want
    big = synth.normal(3, 151936, 0.0, 1.0)
    big[[100, 90000, 150000]] = 9.0
    d = H.DeviceBuffer.from_array(big)
    H.check(lib.llmi_hip_argmax_dev(d.ptr, big.size, out.ptr, None))
    H.synchronize()
    assert int(out.download(np.int32)[0]) == 100


# ---------------------------------------------------------- tiny models
def test_tiny_models_match_reference(golden):
    rec, arrays = golden
    g = arrays["tiny_models"]
    for c in rec["tiny_models"]:  # F32, Q8_0 and Q4_0 weights
        m = H.Model(c["cfg"], synth.make_tensors(c["cfg"], c["seed"], c["convention"]), c["type"])
        cache = m.new_cache(len(g["prompt"]) + len(g["steps"]))
        pre = m.forward_cached(cache, g["prompt"], all_positions=True)
        assert np.array_equal(bits(pre), bits(g[c["key"] + "_prefill"])), c["key"]
        for i, s in enumerate(g["steps"]):
            assert np.array_equal(bits(m.forward_cached(cache, [s])), bits(g[c["key"] + "_steps"][i])), (c["key"], i)
        assert cache.length() == len(g["prompt"]) + len(g["steps"])
        ids = m.generate_greedy(np.array([1, 2, 3], np.int32), 12)
        assert np.array_equal(ids, g[c["key"] + "_greedy"]), c["key"]
        cache.free()
        m.free()


def test_kv_cache_invariants_and_causality():
    """transformer_test.cpp:322-381 and :201-218 on the device model."""
    for arch in (0, 1):
        cfg = synth.tiny(arch, True)
        for qt in (H.Q8_0, H.Q4_0):
            m = H.Model(cfg, synth.make_tensors(cfg, 11, "tiny"), qt)
            ids = np.array([2, 17, 4, 9, 21, 0, 13], np.int32)
            c1 = m.new_cache(len(ids))
            allpos = m.forward_cached(c1, ids, all_positions=True).reshape(len(ids), -1)
            # forward() without a cache (the model's own, reused and reset
            # between calls, also by a longer call in between) gives the same
            # logits, every time.
            for rep in range(2):
                assert np.array_equal(bits(m.forward(ids, all_positions=True)), bits(allpos.reshape(-1))), (arch, rep)
                assert np.array_equal(bits(m.forward(ids[:4])), bits(allpos[3])), (arch, rep)
                m.forward(np.arange(40, dtype=np.int32) % cfg["vocab_size"])
            c2 = m.new_cache(len(ids))
            for t, tok in enumerate(ids):
                assert np.array_equal(bits(m.forward_cached(c2, [tok])), bits(allpos[t])), (arch, qt, t)
            c3 = m.new_cache(len(ids))
            m.forward_cached(c3, ids[:3])
            for t in range(3, len(ids)):
                assert np.array_equal(bits(m.forward_cached(c3, [ids[t]])), bits(allpos[t]))
            other = ids.copy()
            other[4] = 1
            c4 = m.new_cache(len(ids))
            alt = m.forward_cached(c4, other, all_positions=True).reshape(len(ids), -1)
            assert np.array_equal(bits(alt[:4]), bits(allpos[:4]))
            assert not np.array_equal(alt[4:], allpos[4:])
            # Stop ids end generation right after the stop token.
            full = m.generate_greedy(np.array([1, 2], np.int32), 10)
            stop = int(full[2])
            first = int(np.argmax(full == stop))
            stopped = m.generate_greedy(np.array([1, 2], np.int32), 10, stop_ids=[stop])
            assert np.array_equal(stopped, full[:first + 1])
            for c in (c1, c2, c3, c4):
                c.free()
            m.free()


def test_bad_input_is_reported_like_the_reference():
    """transformer_test.cpp:242-250, :400-411."""
    cfg = synth.tiny(0, True)
    m = H.Model(cfg, synth.make_tensors(cfg, 6, "tiny"), H.Q8_0)
    other = H.Model(cfg, synth.make_tensors(cfg, 7, "tiny"), H.Q8_0)
    c = m.new_cache(3)
    for bad, msg in (([], "no tokens"), ([32], "out of range"), ([-1], "out of range")):
        with pytest.raises(H.HipError, match=msg):
            m.forward_cached(c, bad)
    with pytest.raises(H.HipError, match="not created by this model"):
        other.forward_cached(c, [1])
    m.forward_cached(c, [1, 2, 3])
    with pytest.raises(H.HipError, match="cache is full"):
        m.forward_cached(c, [4])
    c.reset()
    m.forward_cached(c, [1, 2, 3])
    with pytest.raises(H.HipError, match="max_len must be positive"):
        m.new_cache(0)
    for bad, msg in (([], "forward: no tokens"), ([32], "forward: token id 32 out of range"),
                     (list(range(65)), "forward: sequence longer than the model's context")):
        with pytest.raises(H.HipError, match=msg):
            m.forward([t % 32 for t in bad] if len(bad) > 1 else bad)
    with pytest.raises(H.HipError):
        H.Model(cfg, synth.make_tensors(cfg, 6, "tiny"), 7)  # not a weight type


def test_generation_past_the_context_fails_like_the_reference():
    """generate_greedy_cached (transformer.cpp:308-327) sizes its cache as
    min(prompt + max_new, max_position_embeddings) and fails with 'cache is
    full' at the first step that does not fit.  The tiny model's context is
    64: a 60-token prompt with 10 new tokens needs 69 positions and must
    fail (greedy and sampled, with and without stop ids); 5 new tokens need
    exactly 64 and must succeed, with the same ids as a run that stops
    early."""
    cfg = synth.tiny(1, True)
    assert cfg["max_position_embeddings"] == 64
    m = H.Model(cfg, synth.make_tensors(cfg, 8, "tiny"), H.Q4_0)
    prompt = synth.uniform_ids(3, 60, cfg["vocab_size"])
    with pytest.raises(H.HipError, match="cache is full"):
        m.generate_greedy(prompt, 10)
    with pytest.raises(H.HipError, match="cache is full"):
        m.generate_greedy(prompt, 10, stop_ids=[cfg["vocab_size"] + 5])  # never produced: the host-synced loop
    targets = np.linspace(0.05, 0.95, 10)
    with pytest.raises(H.HipError, match="cache is full"):
        m.generate_sampled(prompt, 10, H.Sampling(0.8, 0, 1.0), targets)
    ids5 = m.generate_greedy(prompt, 5)
    assert len(ids5) == 5
    assert np.array_equal(m.generate_greedy(prompt, 3), ids5[:3])
    # Sampled: the steps whose forward fits are queued on the device, the
    # rest run step by step, so a stop id drawn before the cache runs out
    # ends the run without the failure -- at a queued step (2) and at the
    # first step-by-step one (4).
    sc = H.Sampling(0.8, 0, 1.0)
    s5 = m.generate_sampled(prompt, 5, sc, targets)
    assert len(s5) == 5
    for at in (2, 4):
        got = m.generate_sampled(prompt, 10, sc, targets, stop_ids=[int(s5[at])])
        assert list(got) == list(s5[: list(s5).index(s5[at]) + 1])
    # The model is still usable after the failed calls.
    c = m.new_cache(64)
    logits = m.forward_cached(c, prompt)
    assert int(np.argmax(logits)) == int(ids5[0])
    c.free()
    m.free()


# ---------------------------------------------------- full-size models
@pytest.mark.parametrize("name", ["c3_smollm2_q8", "c4_qwen25_q4"])
def test_synthetic_model_greedy_ids_match_reference(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        rec = json.load(f)
    cfg = rec["cfg"]
    m = H.synthetic_model_dev(cfg, rec["seed"], rec["type"], rec["convention"])
    want_wb = {"c3_smollm2_q8": 151_289_856, "c4_qwen25_q4": 308_725_760}[name]
    assert m.weight_bytes() == want_wb
    prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
    cache = m.new_cache(rec["n_prompt"] + 1)
    logits = m.forward_cached(cache, prompt)
    assert sha(logits) == rec["first_logits_sha256"], (name, np.argsort(-logits)[:8], rec["first_logits_top"])
    cache.free()
    ids = m.generate_greedy(prompt, rec["n_steps"])
    want = np.array(rec["ids"], dtype=np.int32)
    if not np.array_equal(ids, want):
        k = int(np.argmax(ids != want))
        pytest.fail(f"{name}: first divergence at step {k} (margin there {rec['margins'][k]:.3g})")
    m.free()


@pytest.mark.parametrize("name", ["c3_smollm2_q8", "c4_qwen25_q4"])
def test_synthetic_model_step_logits_match_reference(name):
    """Per-step logits of the full-size synthetic models past the prefill
    (the reference pins per-step equality, tests/transformer_test.cpp:
    322-398): the one-token step fed the reference's greedy ids, its logits
    bit-identical (SHA-256) to the compiled reference's at the recorded
    steps (0 = the prefill's, 63, 127 and the last), and every step's argmax
    equal to the recorded id."""
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        rec = json.load(f)
    want = rec["step_logits_sha256"]
    cfg = rec["cfg"]
    m = H.synthetic_model_dev(cfg, rec["seed"], rec["type"], rec["convention"])
    prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
    n = rec["n_steps"]
    cache = m.new_cache(rec["n_prompt"] + n)
    logits = m.forward_cached(cache, prompt)
    checked = 0
    for s in range(n):
        if str(s) in want:
            assert sha(logits) == want[str(s)], (name, s, np.argsort(-logits)[:4])
            checked += 1
        assert int(np.argmax(logits)) == rec["ids"][s], (name, s)
        if s + 1 < n:
            logits = m.forward_cached(cache, [rec["ids"][s]])
    assert checked == len(want) >= 4
    cache.free()
    m.free()


def test_forward_trace_states():
    """ForwardTrace (transformer.hpp:14-19): embeddings, each layer, final
    norm; the embeddings are the dequantized rows and the head applied to
    the final state gives the logits, bit for bit."""
    orc = O.oracle()
    cfg = synth.tiny(1, True)
    tensors = synth.make_tensors(cfg, 21, "tiny")
    m = H.Model(cfg, tensors, H.Q8_0)
    c = m.new_cache(4)
    ids = np.array([3, 30, 7], np.int32)
    logits, states = m.forward_cached_trace(c, ids)
    assert states.shape == (cfg["num_layers"] + 2, 3, cfg["hidden_size"])
    data, scales = orc.quantize(tensors[0], cfg["vocab_size"], cfg["hidden_size"], H.Q8_0)
    for t, tok in enumerate(ids):
        want = orc.dequantize_row(data, scales, cfg["vocab_size"], cfg["hidden_size"], H.Q8_0, int(tok))
        assert np.array_equal(bits(states[0, t]), bits(want))
    head = orc.matmul(states[-1, 2], 1, cfg["hidden_size"], data, scales, H.Q8_0, cfg["vocab_size"])
    assert np.array_equal(bits(head), bits(logits))
    c2 = m.new_cache(4)
    assert np.array_equal(bits(m.forward_cached(c2, ids)), bits(logits))


# ------------------------------------------------ decode attention shapes
@pytest.mark.parametrize("hidden,heads,kv", [(256, 4, 2), (256, 2, 1), (448, 7, 1), (192, 3, 1)])
def test_decode_attention_matches_reference(hidden, heads, kv):
    """Head sizes 64 and 128 with GQA groups of 2, 3 and 7 take the two-kernel
    decode attention (scores over position tiles, then softmax + P.V per
    16-column slice); logits of every decode step up to 75 positions (all
    residues of the position padding) equal the reference's bit for bit."""
    cpu = O.reference() or O.oracle()
    cfg = dict(arch=1, vocab_size=64, hidden_size=hidden, intermediate_size=2 * hidden, num_layers=2,
               num_heads=heads, num_kv_heads=kv, max_position_embeddings=128, rms_norm_eps=1e-6,
               rope_theta=10000.0, tie_word_embeddings=1, qkv_bias=1)
    tensors = synth.make_tensors(cfg, hidden + heads, "bench")
    gm = H.Model(cfg, tensors, H.Q8_0)
    cm = O.CpuModel(cpu, cfg, tensors, O.Q8_0)
    ids = synth.uniform_ids(hidden, 75, cfg["vocab_size"])
    cache = gm.new_cache(80)
    assert cm.new_cache(80)
    assert np.array_equal(bits(gm.forward_cached(cache, ids[:5])), bits(cm.forward_cached(ids[:5])))
    for t in range(5, 75):
        got = gm.forward_cached(cache, ids[t:t + 1])
        want = cm.forward_cached(ids[t:t + 1])
        assert np.array_equal(bits(got), bits(want)), (hidden, heads, kv, t)
    cache.free()
    gm.free()
    cm.close()


@pytest.mark.parametrize("qt", [H.Q8_0, H.Q4_0])
@pytest.mark.parametrize("inter", [1536, 1560, 4864])
def test_decode_long_down_proj_matches_reference(qt, inter):
    """The one-token step's down_proj on rows of 48 to 152 blocks with
    SiLU(gate) * up staged by every workgroup (1560: a partial final block
    of 24 elements); every step's logits equal the reference's bit for
    bit."""
    cpu = O.reference() or O.oracle()
    cfg = dict(arch=1, vocab_size=80, hidden_size=128, intermediate_size=inter, num_layers=2, num_heads=2,
               num_kv_heads=1, max_position_embeddings=64, rms_norm_eps=1e-6, rope_theta=1e6,
               tie_word_embeddings=1, qkv_bias=1)
    tensors = synth.make_tensors(cfg, inter + qt, "bench")
    gm = H.Model(cfg, tensors, qt)
    cm = O.CpuModel(cpu, cfg, tensors, qt)
    ids = synth.uniform_ids(inter, 24, cfg["vocab_size"])
    cache = gm.new_cache(24)
    assert cm.new_cache(24)
    assert np.array_equal(bits(gm.forward_cached(cache, ids[:4])), bits(cm.forward_cached(ids[:4])))
    for t in range(4, 24):
        got = gm.forward_cached(cache, ids[t:t + 1])
        want = cm.forward_cached(ids[t:t + 1])
        assert np.array_equal(bits(got), bits(want)), (inter, qt, t)
    cache.free()
    gm.free()
    cm.close()


# ----------------------------------------------- prefill attention shapes
@pytest.mark.parametrize("hidden,heads,kv", [(64, 1, 1), (256, 4, 2), (192, 3, 1), (448, 7, 1), (576, 9, 3),
                                             (2048, 32, 1), (1024, 16, 1), (256, 2, 1), (80, 1, 1)])
def test_prefill_attention_matches_reference(hidden, heads, kv):
    """Multi-token forward passes after earlier ones (base > 0): head size 64
    with GQA groups of 1 to 32 takes the workgroup-per-(KV head, token tile)
    prefill attention (16 rows per workgroup up to groups of 16, 32 above),
    head sizes 128 and 80 the per-(head, token) kernel (80 also leaves a
    partial final quantization block in the q/k/v and fused gate/up
    products).  Chunk
    lengths leave ragged token tiles and end on and off the 64-position K/V
    tiles; every position's logits equal the reference's bit for bit."""
    cpu = O.reference() or O.oracle()
    cfg = dict(arch=1, vocab_size=64, hidden_size=hidden, intermediate_size=2 * hidden, num_layers=2,
               num_heads=heads, num_kv_heads=kv, max_position_embeddings=512, rms_norm_eps=1e-6,
               rope_theta=10000.0, tie_word_embeddings=1, qkv_bias=1)
    tensors = synth.make_tensors(cfg, hidden + 3 * heads, "bench")
    gm = H.Model(cfg, tensors, H.Q8_0)
    cm = O.CpuModel(cpu, cfg, tensors, O.Q8_0)
    chunks = [37, 1, 90, 64, 128, 23]
    ids = synth.uniform_ids(hidden + 1, sum(chunks), cfg["vocab_size"])
    cache = gm.new_cache(sum(chunks))
    assert cm.new_cache(sum(chunks))
    at = 0
    for n in chunks:
        got = gm.forward_cached(cache, ids[at:at + n], all_positions=True)
        want = cm.forward_cached(ids[at:at + n], all_positions=True)
        assert np.array_equal(bits(got), bits(want)), (hidden, heads, kv, at, n)
        at += n
    cache.free()
    gm.free()
    cm.close()


def test_prefill_attention_past_the_lds_scores():
    """The workgroup-per-tile kernel holds a 16-row tile's scores in LDS up to
    about 1850 positions: a first chunk of 1200 positions takes it, a second
    one reaching 2000 positions the per-(head, token) kernel; logits still
    equal the reference's."""
    cpu = O.reference() or O.oracle()
    cfg = dict(arch=0, vocab_size=64, hidden_size=128, intermediate_size=256, num_layers=1, num_heads=2,
               num_kv_heads=1, max_position_embeddings=2000, rms_norm_eps=1e-5, rope_theta=10000.0,
               tie_word_embeddings=1, qkv_bias=0)
    tensors = synth.make_tensors(cfg, 5, "bench")
    gm = H.Model(cfg, tensors, H.Q4_0)
    cm = O.CpuModel(cpu, cfg, tensors, O.Q4_0)
    ids = synth.uniform_ids(6, 2000, cfg["vocab_size"])
    cache = gm.new_cache(2000)
    assert cm.new_cache(2000)
    for a, b in ((0, 1200), (1200, 2000)):
        got = gm.forward_cached(cache, ids[a:b], all_positions=True)
        want = cm.forward_cached(ids[a:b], all_positions=True)
        assert np.array_equal(bits(got), bits(want)), (a, b)
    cache.free()
    gm.free()
    cm.close()

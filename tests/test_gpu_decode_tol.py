"""The tolerance-mode decode step (llmi_hip_model_set_decode_mode): attention
split over position chunks, merged in the o_proj launch's staging, and the
matmuls split over K (partial sums added atomically).  Its
logits are held to the path's floating-point contract against the exact
step, whose logits equal the reference's bit for bit (tests/test_gpu_model.py
pins them at the full-size models' recorded steps):

* per step, max|logits_tol - logits_exact| <= 1e-4 * max|logits_exact|
  (the relative-error bar the north star states for fp32-accumulate paths),
  fed the same tokens, on small models with head sizes 64 and 128, GQA groups
  1, 2, 3 and 7, two and three layers, and contexts from 1 to past 2048
  positions (one chunk of 64 up to sixteen chunks of 192), and on one-layer
  models with MLPs of 8192 and 16384 (every split width of the matmuls);
  an intermediate size that is not a multiple of 64 leaves gate and up as
  two matrices, and the tolerance mode then keeps the exact step;
* on the synthetic SmolLM2-135M and Qwen2.5-0.5B:
  the greedy ids of the first 64 steps equal the compiled reference's, and
  every step's logits, fed the reference's ids, are within the bar.
"""

import json
import os

import numpy as np
import pytest

import llmi_hip as H
import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4


def rel_err(a, b):
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    return float(np.abs(a64 - b64).max() / max(np.abs(b64).max(), 1e-30))


def cfg_of(hidden, heads, kv, arch=1, ctx=4096, layers=2, vocab=512):
    return dict(arch=arch, vocab_size=vocab, hidden_size=hidden, intermediate_size=2 * hidden, num_layers=layers,
                num_heads=heads, num_kv_heads=kv, max_position_embeddings=ctx, rms_norm_eps=1e-6,
                rope_theta=10000.0, tie_word_embeddings=1, qkv_bias=int(arch == 1))


@pytest.mark.parametrize("hidden,heads,kv,qt,layers,inter_pad",
                         [(128, 2, 2, H.Q8_0, 2, 0), (448, 7, 1, H.Q4_0, 2, 0), (576, 9, 3, H.Q8_0, 2, 0),
                          (256, 2, 1, H.Q4_0, 2, 0), (192, 3, 1, H.Q8_0, 3, 0), (128, 2, 1, H.Q4_0, 2, 16)])
def test_tolerance_steps_match_exact_steps(hidden, heads, kv, qt, layers, inter_pad):
    """Steps at positions 1..80 after a one-token prompt, then steps at
    positions ~1000-1100 and ~2100 after longer prompts (chunks of 64, 128 and
    192 positions); both modes fed the same tokens; two and three layers.
    The intermediate size 272 (not a multiple of 64: no fused gate|up
    matrix) keeps the exact step, so its logits are bit-identical."""
    cfg = cfg_of(hidden, heads, kv, layers=layers)
    cfg["intermediate_size"] += inter_pad
    m = H.Model(cfg, synth.make_tensors(cfg, 500 + hidden + heads, "bench"), qt)
    worst = 0.0
    for n_prompt, n_steps in ((1, 80), (1000, 100), (2100, 20)):
        prompt = synth.uniform_ids(n_prompt + hidden, n_prompt, cfg["vocab_size"])
        steps = synth.uniform_ids(n_steps + 7, n_steps, cfg["vocab_size"])
        ce, ct = m.new_cache(n_prompt + n_steps), m.new_cache(n_prompt + n_steps)
        m.set_decode_mode(H.DECODE_EXACT)
        le = m.forward_cached(ce, prompt)
        m.set_decode_mode(H.DECODE_TOLERANCE)
        lt = m.forward_cached(ct, prompt)
        if n_prompt > 1:
            assert np.array_equal(le, lt)  # the prompt's prefill is exact in both modes
        for i, tok in enumerate(steps):
            m.set_decode_mode(H.DECODE_EXACT)
            le = m.forward_cached(ce, [tok])
            m.set_decode_mode(H.DECODE_TOLERANCE)
            lt = m.forward_cached(ct, [tok])
            err = rel_err(lt, le)
            assert err <= TOL, (n_prompt, i, err)
            if inter_pad:
                assert err == 0.0, (n_prompt, i, err)
            worst = max(worst, err)
        ce.free()
        ct.free()
    m.free()
    print(f"hidden {hidden} heads {heads}/{kv}: worst relative logit error {worst:.3e}")


@pytest.mark.parametrize("inter,qt", [(8192, H.Q4_0), (16384, H.Q8_0)])
def test_wide_mlp_splits_match_exact_steps(inter, qt):
    """Matrices whose K splits take the wider per-workgroup block counts (8
    and 16 blocks: gate|up over 256 / 512 row tiles, down_proj over 256 / 512
    blocks), one layer, both modes fed the same tokens."""
    cfg = cfg_of(1024, 16, 4, layers=1)
    cfg["intermediate_size"] = inter
    m = H.synthetic_model_dev(cfg, 900 + inter % 7, qt, "bench")
    ce, ct = m.new_cache(40), m.new_cache(40)
    worst = 0.0
    for tok in synth.uniform_ids(inter, 32, cfg["vocab_size"]):
        m.set_decode_mode(H.DECODE_EXACT)
        le = m.forward_cached(ce, [tok])
        m.set_decode_mode(H.DECODE_TOLERANCE)
        lt = m.forward_cached(ct, [tok])
        err = rel_err(lt, le)
        assert err <= TOL, err
        worst = max(worst, err)
    ce.free()
    ct.free()
    m.free()
    print(f"intermediate {inter}: worst relative logit error {worst:.3e}")


def test_tolerance_mode_is_rejected_when_unknown():
    cfg = cfg_of(128, 2, 2)
    m = H.Model(cfg, synth.make_tensors(cfg, 3, "bench"), H.Q8_0)
    with pytest.raises(H.HipError, match="unknown mode"):
        m.set_decode_mode(7)
    m.free()


def test_head_size_without_a_tolerance_kernel_keeps_the_exact_step():
    """head_dim 16 (the reference's tiny test models): the tolerance mode
    falls back to the exact step, so its logits stay bit-identical."""
    cfg = synth.tiny(1, True)
    m = H.Model(cfg, synth.make_tensors(cfg, 8, "tiny"), H.Q4_0)
    ce, ct = m.new_cache(16), m.new_cache(16)
    for tok in [3, 9, 1, 30]:
        m.set_decode_mode(H.DECODE_EXACT)
        le = m.forward_cached(ce, [tok])
        m.set_decode_mode(H.DECODE_TOLERANCE)
        lt = m.forward_cached(ct, [tok])
        assert np.array_equal(le, lt)
    m.free()


@pytest.mark.parametrize("name", ["c3_smollm2_q8", "c4_qwen25_q4"])
def test_full_size_tolerance_decode(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        rec = json.load(f)
    cfg = rec["cfg"]
    m = H.synthetic_model_dev(cfg, rec["seed"], rec["type"], rec["convention"])
    prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
    m.set_decode_mode(H.DECODE_TOLERANCE)
    ids = m.generate_greedy(prompt, 64)
    assert list(ids) == rec["ids"][:64]
    # Every step fed the reference's ids: tolerance against exact.
    n = rec["n_steps"]
    ce, ct = m.new_cache(rec["n_prompt"] + n), m.new_cache(rec["n_prompt"] + n)
    m.set_decode_mode(H.DECODE_EXACT)
    le = m.forward_cached(ce, prompt)
    lt = m.forward_cached(ct, prompt)
    worst = 0.0
    for s in range(n - 1):
        tok = [rec["ids"][s]]
        m.set_decode_mode(H.DECODE_EXACT)
        le = m.forward_cached(ce, tok)
        m.set_decode_mode(H.DECODE_TOLERANCE)
        lt = m.forward_cached(ct, tok)
        err = rel_err(lt, le)
        assert err <= TOL, (name, s, err)
        worst = max(worst, err)
    ce.free()
    ct.free()
    m.free()
    print(f"{name}: worst relative logit error over {n - 1} steps {worst:.3e}")


def test_greedy_from_a_graph_equals_the_eager_loop():
    """generate_greedy in tolerance mode captures one step (argmax, the step
    with its positions read from device memory, the positions' advance) and
    replays it once per token.  With the graph and without, twice in a row
    with eager single steps between the runs, around the 8-step threshold
    below which it stays eager, and with stop ids (eager), the greedy ids
    are the reference's."""
    with open(os.path.join(GOLDEN, "c3_smollm2_q8.json")) as f:
        rec = json.load(f)
    cfg = rec["cfg"]
    m = H.synthetic_model_dev(cfg, rec["seed"], rec["type"], rec["convention"])
    prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
    want = rec["ids"]
    m.set_decode_mode(H.DECODE_TOLERANCE)
    for graph in (True, False, True, True):
        m.set_decode_graph(graph)
        assert list(m.generate_greedy(prompt, rec["n_steps"])) == want, graph
        c = m.new_cache(rec["n_prompt"] + 2)
        m.forward_cached(c, prompt)
        m.forward_cached(c, [want[0]])
        c.free()
    for n in (7, 8, 9, 40):
        assert list(m.generate_greedy(prompt, n)) == want[:n], n
    stop = want[-1]  # first reached late in the run
    assert list(m.generate_greedy(prompt, rec["n_steps"], stop_ids=[stop])) == want[:want.index(stop) + 1]
    m.free()


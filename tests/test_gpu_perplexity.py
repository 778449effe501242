"""GPU scoring of llmi-perplexity (apps/llmi-perplexity/main.cpp:146-168) through
llmi_hip_model_chunk_nll: with the exact lm_head every per-position NLL
equals the reference's formula applied to the reference's own all-positions
logits (to 1e-12 relative: only the double sum's order differs); with the
bf16-MFMA lm_head each NLL stays within the bound the logits' tolerance
implies (4e-2 of the row's max |logit|), at a toy shape and at the
Qwen2.5-0.5B lm_head shape (151936 x 896, 255 scored rows); with every
linear on the MFMA GEMM the per-token and mean NLL stay within stated
bounds of the exact path."""

import numpy as np
import pytest

import llmi_hip as H
import oracle as O
import synth

pytestmark = pytest.mark.gpu


def reference_nll(logits: np.ndarray, ids: np.ndarray, t_start: int) -> np.ndarray:
    """main.cpp:158-166 in numpy: float max, a sequential double sum of
    exp(double(row - max)), log(sum) + max, -(row[next] - lse)."""
    out = []
    for t in range(t_start, len(ids) - 1):
        row = logits[t]
        mx = np.float32(row.max())
        sum_exp = np.cumsum(np.exp((row - mx).astype(np.float64)))[-1]
        lse = np.log(sum_exp) + np.float64(mx)
        out.append(-(np.float64(row[ids[t + 1]]) - lse))
    return np.array(out)


def toy_cfg():
    return dict(arch=1, vocab_size=512, hidden_size=128, intermediate_size=256, num_layers=2, num_heads=2,
                num_kv_heads=1, max_position_embeddings=256, rms_norm_eps=1e-6, rope_theta=10000.0,
                tie_word_embeddings=1, qkv_bias=1)


@pytest.mark.parametrize("qt", [H.Q8_0, H.Q4_0])
def test_exact_head_matches_reference_formula(qt):
    cfg = toy_cfg()
    tensors = synth.make_tensors(cfg, 31 + qt, "bench")
    cpu = O.reference() or O.oracle()
    cm = O.CpuModel(cpu, cfg, tensors, qt)
    ids = synth.uniform_ids(77 + qt, 48, cfg["vocab_size"])
    assert cm.new_cache(64)
    logits = cm.forward_cached(ids, all_positions=True).reshape(len(ids), cfg["vocab_size"])
    cm.close()
    gm = H.Model(cfg, tensors, qt)
    for t_start in (0, 24, 46, 47, 60):
        got = gm.chunk_nll(ids, t_start, H.SCORE_EXACT)
        want = reference_nll(logits, ids, min(t_start, len(ids) - 1))
        assert got.shape == want.shape, t_start
        if want.size:
            assert np.all(np.abs(got - want) <= 1e-12 * np.maximum(1.0, np.abs(want))), t_start
    gm.free()


def test_mfma_head_within_the_logit_bound_toy():
    cfg = toy_cfg()
    tensors = synth.make_tensors(cfg, 40, "bench")
    gm = H.Model(cfg, tensors, H.Q8_0)
    ids = synth.uniform_ids(41, 100, cfg["vocab_size"])
    exact = gm.chunk_nll(ids, 10, H.SCORE_EXACT)
    fast = gm.chunk_nll(ids, 10, H.SCORE_MFMA_HEAD)
    c = gm.new_cache(128)
    logits = gm.forward_cached(c, ids, all_positions=True).reshape(len(ids), -1)[10:-1]
    bound = 4e-2 * np.abs(logits).max(axis=1)
    assert np.all(np.abs(fast - exact) <= bound)
    assert np.abs(fast - exact).mean() < 0.1 * bound.mean()  # typically far inside the bound
    c.free()
    gm.free()


def test_mfma_head_at_the_qwen_lm_head_shape():
    """Two Qwen2.5-0.5B-shaped layers (the full 151936 x 896 tied head),
    one 512-token chunk scored from position 256, as the app's default."""
    cfg = dict(arch=1, vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=2, num_heads=14,
               num_kv_heads=2, max_position_embeddings=32768, rms_norm_eps=1e-6, rope_theta=1e6,
               tie_word_embeddings=1, qkv_bias=1)
    gm = H.synthetic_model_dev(cfg, 5, H.Q4_0, "bench")
    ids = synth.uniform_ids(6, 512, cfg["vocab_size"])
    exact = gm.chunk_nll(ids, 256, H.SCORE_EXACT)
    fast = gm.chunk_nll(ids, 256, H.SCORE_MFMA_HEAD)
    assert exact.shape == (255,) and np.all(np.isfinite(exact))
    c = gm.new_cache(512)
    logits = gm.forward_cached(c, ids, all_positions=True).reshape(512, -1)[256:511]
    assert np.all(np.abs(fast - exact) <= 4e-2 * np.abs(logits).max(axis=1))
    c.free()
    gm.free()


@pytest.mark.parametrize("which", ["toy", "c3"])
def test_all_mfma_scoring_stays_close_to_exact(which):
    """Every linear on the bf16-MFMA GEMM (LLMI_SCORE_MFMA): per-token NLL
    within 0.1 and the chunk's mean NLL within 5e-3 of the exact path (the
    synthetic SmolLM2-135M, 30 layers: measured ~0.013 and ~2e-4)."""
    if which == "toy":
        cfg = toy_cfg()
        gm = H.Model(cfg, synth.make_tensors(cfg, 40, "bench"), H.Q4_0)
        ids, first = synth.uniform_ids(41, 100, cfg["vocab_size"]), 10
    else:
        import json
        import os
        with open(os.path.join(os.path.dirname(__file__), "golden", "c3_smollm2_q8.json")) as f:
            rec = json.load(f)
        cfg = rec["cfg"]
        gm = H.synthetic_model_dev(cfg, rec["seed"], rec["type"], rec["convention"])
        ids, first = synth.uniform_ids(6, 512, cfg["vocab_size"]), 256
    exact = gm.chunk_nll(ids, first, H.SCORE_EXACT)
    fast = gm.chunk_nll(ids, first, H.SCORE_MFMA)
    assert fast.shape == exact.shape and np.all(np.isfinite(fast))
    assert np.abs(fast - exact).max() <= 0.1
    assert abs(fast.mean() - exact.mean()) <= 5e-3
    gm.free()


def test_rejects_bad_input():
    cfg = toy_cfg()
    gm = H.Model(cfg, synth.make_tensors(cfg, 50, "bench"), H.Q8_0)
    with pytest.raises(H.HipError):
        gm.chunk_nll(np.array([1, 2, cfg["vocab_size"]], np.int32), 0)  # id out of range
    with pytest.raises(H.HipError):
        gm.chunk_nll(np.array([1, 2, 3], np.int32), 0, mode=7)
    gm.free()

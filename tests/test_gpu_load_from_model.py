"""Transformer::load(const Model&, quant::Type) run for real: each golden
tiny model (both architectures, tied and untied heads, F32 / Q8_0 / Q4_0) is
written as a Hugging Face model directory (config.json + model.safetensors),
read by the reference's own Model::load (src/model/model.cpp:210-240), handed
to this repository's host/integration/load_from_model.cpp and run on the GPU
by oracle/_ref/load_from_model_check (built from those sources by
oracle/Makefile).  Its prefill logits, step logits and greedy ids must be the
reference's golden ones bit for bit.  A bf16 checkpoint goes through the
reference's dtype conversion (read_float) and must give the logits of the
same weights rounded to bf16 and loaded directly."""

import json
import os
import struct
import subprocess

import numpy as np
import pytest

import llmi_hip as H
import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "oracle", "_ref", "load_from_model_check")
TYPES = {H.F32: "f32", H.Q8_0: "q8_0", H.Q4_0: "q4_0"}

needs_check = pytest.mark.skipif(not os.path.exists(CHECK),
                                 reason="oracle/_ref/load_from_model_check not built (no reference sources)")


def tensor_names(cfg):
    """The tensors of a Llama/Qwen2 checkpoint in load order."""
    names = ["model.embed_tokens.weight"]
    for i in range(cfg["num_layers"]):
        p = f"model.layers.{i}."
        names += [p + "input_layernorm.weight", p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                  p + "self_attn.v_proj.weight"]
        if cfg["qkv_bias"]:
            names += [p + "self_attn.q_proj.bias", p + "self_attn.k_proj.bias", p + "self_attn.v_proj.bias"]
        names += [p + "self_attn.o_proj.weight", p + "post_attention_layernorm.weight", p + "mlp.gate_proj.weight",
                  p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"]
    names.append("model.norm.weight")
    if not cfg["tie_word_embeddings"]:
        names.append("lm_head.weight")
    return names


def shapes(cfg):
    h, v, f = cfg["hidden_size"], cfg["vocab_size"], cfg["intermediate_size"]
    hd = h // cfg["num_heads"]
    q, kv = cfg["num_heads"] * hd, cfg["num_kv_heads"] * hd
    out = {"model.embed_tokens.weight": [v, h], "model.norm.weight": [h], "lm_head.weight": [v, h]}
    for i in range(cfg["num_layers"]):
        p = f"model.layers.{i}."
        out.update({p + "input_layernorm.weight": [h], p + "self_attn.q_proj.weight": [q, h],
                    p + "self_attn.k_proj.weight": [kv, h], p + "self_attn.v_proj.weight": [kv, h],
                    p + "self_attn.q_proj.bias": [q], p + "self_attn.k_proj.bias": [kv],
                    p + "self_attn.v_proj.bias": [kv], p + "self_attn.o_proj.weight": [h, q],
                    p + "post_attention_layernorm.weight": [h], p + "mlp.gate_proj.weight": [f, h],
                    p + "mlp.up_proj.weight": [f, h], p + "mlp.down_proj.weight": [h, f]})
    return out


def bf16_bits(a):
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def write_model(d, cfg, tensors, dtype="F32"):
    """A model directory as Hugging Face exports it: config.json and a
    safetensors file (8-byte header length, JSON header padded to 8 bytes,
    then the tensors' bytes)."""
    arch = "Qwen2ForCausalLM" if cfg["arch"] == 1 else "LlamaForCausalLM"
    conf = {"architectures": [arch], "vocab_size": cfg["vocab_size"], "hidden_size": cfg["hidden_size"],
            "intermediate_size": cfg["intermediate_size"], "num_hidden_layers": cfg["num_layers"],
            "num_attention_heads": cfg["num_heads"], "num_key_value_heads": cfg["num_kv_heads"],
            "max_position_embeddings": cfg["max_position_embeddings"], "rms_norm_eps": cfg["rms_norm_eps"],
            "rope_theta": cfg["rope_theta"], "tie_word_embeddings": bool(cfg["tie_word_embeddings"]),
            "hidden_act": "silu"}
    if cfg["arch"] == 0:
        conf["attention_bias"] = bool(cfg["qkv_bias"])
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(conf, f)
    shp = shapes(cfg)
    header, blobs, off = {}, [], 0
    for name, t in zip(tensor_names(cfg), tensors):
        b = bf16_bits(t).tobytes() if dtype == "BF16" else np.ascontiguousarray(t, np.float32).tobytes()
        assert len(b) == int(np.prod(shp[name])) * (2 if dtype == "BF16" else 4), name
        header[name] = {"dtype": dtype, "shape": shp[name], "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def run_check(d, qt, prompt, steps, out):
    r = subprocess.run([CHECK, d, TYPES[qt], out, ",".join(map(str, prompt)), ",".join(map(str, steps))],
                       capture_output=True, text=True, timeout=120)
    return r


def read_out(out, cfg, prompt, steps):
    V = cfg["vocab_size"]
    raw = open(out, "rb").read()
    n_log = (len(prompt) + len(steps)) * V
    logits = np.frombuffer(raw[: 4 * n_log], np.float32)
    ids = np.frombuffer(raw[4 * n_log:], np.int32)
    return logits[: len(prompt) * V], logits[len(prompt) * V:].reshape(len(steps), V), ids


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@needs_check
def test_reference_model_loader_runs_the_gpu_transformer(golden, tmp_path):
    rec, arrays = golden
    g = arrays["tiny_models"]
    prompt, steps = [int(i) for i in g["prompt"]], [int(i) for i in g["steps"]]
    for c in rec["tiny_models"]:
        d = str(tmp_path / c["key"])
        write_model(d, c["cfg"], synth.make_tensors(c["cfg"], c["seed"], c["convention"]))
        out = str(tmp_path / (c["key"] + ".bin"))
        r = run_check(d, c["type"], prompt, steps, out)
        assert r.returncode == 0, (c["key"], r.stderr)
        pre, st, ids = read_out(out, c["cfg"], prompt, steps)
        assert np.array_equal(bits(pre), bits(g[c["key"] + "_prefill"])), c["key"]
        for i in range(len(steps)):
            assert np.array_equal(bits(st[i]), bits(g[c["key"] + "_steps"][i])), (c["key"], i)
        assert np.array_equal(ids, g[c["key"] + "_greedy"]), c["key"]


@needs_check
def test_bf16_checkpoint_goes_through_the_reference_conversion(golden, tmp_path):
    rec, arrays = golden
    g = arrays["tiny_models"]
    prompt, steps = [int(i) for i in g["prompt"]], [int(i) for i in g["steps"]]
    c = next(c for c in rec["tiny_models"] if c["cfg"]["arch"] == 1 and c["type"] == H.Q8_0)
    tensors = synth.make_tensors(c["cfg"], c["seed"], c["convention"])
    d = str(tmp_path / "bf16")
    write_model(d, c["cfg"], tensors, dtype="BF16")
    out = str(tmp_path / "bf16.bin")
    r = run_check(d, c["type"], prompt, steps, out)
    assert r.returncode == 0, r.stderr
    pre, st, ids = read_out(out, c["cfg"], prompt, steps)
    rounded = [(bf16_bits(t).astype(np.uint32) << 16).view(np.float32) for t in tensors]
    m = H.Model(c["cfg"], rounded, c["type"])
    cache = m.new_cache(len(prompt) + len(steps))
    assert np.array_equal(bits(pre), bits(m.forward_cached(cache, prompt, all_positions=True)))
    for i, s in enumerate(steps):
        assert np.array_equal(bits(st[i]), bits(m.forward_cached(cache, [s])))
    assert np.array_equal(ids, m.generate_greedy(np.array([1, 2, 3], np.int32), 12))
    cache.free()
    m.free()


@needs_check
def test_loader_errors_come_back(golden, tmp_path):
    rec, _ = golden
    c = rec["tiny_models"][0]
    cfg = c["cfg"]
    tensors = synth.make_tensors(cfg, c["seed"], c["convention"])
    d = str(tmp_path / "missing")
    write_model(d, cfg, tensors)
    os.remove(os.path.join(d, "model.safetensors"))
    r = run_check(d, c["type"], [1, 2], [3], str(tmp_path / "x.bin"))
    assert r.returncode == 2 and "Model::load" in r.stderr
    # A prompt past the context: the reference's cache-full message through the host layer.
    d2 = str(tmp_path / "ok")
    write_model(d2, cfg, tensors)
    long_prompt = [1] * (cfg["max_position_embeddings"] + 1)
    r = run_check(d2, c["type"], long_prompt, [3], str(tmp_path / "y.bin"))
    assert r.returncode == 2

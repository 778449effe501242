"""The reference's own command-line apps on the GPU layer.

apps/llmi-generate/main.cpp and apps/llmi-perplexity/main.cpp are built
unchanged from their sources twice by oracle/Makefile: on the reference's CPU
engine (oracle/_ref/*-ref) and on this repository's host layer over
libllmi_hip.so (oracle/_ref/*-gpu, the drop-in a maintainer makes).  Both run
on the same Hugging Face model directories (config.json + model.safetensors,
read by the reference's Model::load); what they print must agree:

* llmi-generate --ids ... --max-new N [--kv-cache] --quant T --json
  (main.cpp:205-356, the JSON record of :339-345): generated_ids equal to the
  golden greedy ids of the compiled reference, with and without the KV cache,
  on every golden tiny model and on the full-size SmolLM2-135M
  for 64 steps;
* llmi-perplexity --ids-file F --ctx C --quant T (main.cpp:97-99, 146-168):
  the same printed mean NLL and perplexity as the reference's build, and the
  same mean NLL as this library's llmi_hip_model_chunk_nll over the chunks.
"""

import json
import os
import subprocess

import numpy as np
import pytest

import llmi_hip as H
import synth
from test_gpu_load_from_model import TYPES, write_model

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def app(name):
    return os.path.join(REF_DIR, name)


needs_apps = pytest.mark.skipif(
    not all(os.path.exists(app(f"{a}-{k}")) for a in ("llmi-generate", "llmi-perplexity") for k in ("gpu", "ref")),
    reason="oracle/_ref apps not built (no reference sources)")


def run(cmd, timeout=300):
    print("running:", " ".join(cmd[:2]), " ".join(c for c in cmd[2:] if not c[:1].isdigit())[:200], flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, (cmd[0], r.returncode, r.stderr[-2000:])
    return json.loads(r.stdout.strip().splitlines()[-1])


def generate(binary, d, ids, max_new, qt, kv_cache=True):
    cmd = [app(binary), d, "--ids", ",".join(str(int(i)) for i in ids), "--max-new", str(max_new),
           "--quant", TYPES[qt], "--json", "--ignore-eos"] + (["--kv-cache"] if kv_cache else [])
    return run(cmd)


@needs_apps
def test_llmi_generate_on_the_gpu_layer_tiny_models(golden, tmp_path):
    """Every golden tiny model (both architectures, tied and untied heads,
    F32 / Q8_0 / Q4_0): 12 greedy ids from the prompt 1,2,3 as the compiled
    reference recorded them, from the app on the GPU layer with and without
    --kv-cache, and from the app on the reference's engine."""
    rec, arrays = golden
    g = arrays["tiny_models"]
    for c in rec["tiny_models"]:
        d = str(tmp_path / c["key"])
        write_model(d, c["cfg"], synth.make_tensors(c["cfg"], c["seed"], c["convention"]))
        want = [int(i) for i in g[c["key"] + "_greedy"]]
        for kv in (True, False):
            out = generate("llmi-generate-gpu", d, [1, 2, 3], 12, c["type"], kv)
            assert out["generated_ids"] == want, (c["key"], kv)
            assert out["prompt_ids"] == [1, 2, 3]
        ref = generate("llmi-generate-ref", d, [1, 2, 3], 12, c["type"])
        assert ref["generated_ids"] == want, c["key"]
        assert out["weight_bytes"] == ref["weight_bytes"], c["key"]


@needs_apps
def test_llmi_generate_on_the_gpu_layer_smollm2(tmp_path):
    """configs[2] through the app: the synthetic SmolLM2-135M as a model
    directory, its 128-id prompt, 64 greedy steps with --kv-cache --quant
    q8_0: the golden ids of the compiled reference, and the reference's
    published weight bytes."""
    with open(os.path.join(GOLDEN, "c3_smollm2_q8.json")) as f:
        rec = json.load(f)
    cfg = rec["cfg"]
    d = str(tmp_path / "smollm2")
    write_model(d, cfg, synth.make_tensors(cfg, rec["seed"], rec["convention"]))
    prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
    out = generate("llmi-generate-gpu", d, prompt, 64, rec["type"])
    assert out["generated_ids"] == rec["ids"][:64]
    assert out["weight_bytes"] == 151_289_856


def perplexity(binary, d, ids_file, ctx, qt):
    return run([app(binary), d, "--ids-file", ids_file, "--ctx", str(ctx), "--quant", TYPES[qt]])


@needs_apps
def test_llmi_perplexity_on_the_gpu_layer(golden, tmp_path):
    """Windowed perplexity over 100 ids in chunks of 32 (scored from 16, the
    app's default half window) on one tiny model per architecture and weight
    type: the GPU build prints the reference build's numbers, and the mean
    NLL equals the library's own chunk scoring (llmi_hip_model_chunk_nll) to
    the printed precision."""
    rec, _ = golden
    ids = synth.uniform_ids(77, 100, rec["tiny_models"][0]["cfg"]["vocab_size"])
    ids_file = str(tmp_path / "ids.txt")
    with open(ids_file, "w") as f:
        f.write("\n".join(str(int(i)) for i in ids) + "\n")
    ctx = 32
    for c in rec["tiny_models"]:
        if not c["cfg"]["tie_word_embeddings"] and c["type"] != H.Q4_0:
            continue  # untied heads: Q4_0 only (the tied cases cover every type)
        d = str(tmp_path / c["key"])
        tensors = synth.make_tensors(c["cfg"], c["seed"], c["convention"])
        write_model(d, c["cfg"], tensors)
        gpu = perplexity("llmi-perplexity-gpu", d, ids_file, ctx, c["type"])
        ref = perplexity("llmi-perplexity-ref", d, ids_file, ctx, c["type"])
        for k in ("tokens", "scored_tokens", "ctx", "scored_from", "perplexity", "mean_nll", "weight_bytes"):
            assert gpu[k] == ref[k], (c["key"], k, gpu[k], ref[k])
        m = H.Model(c["cfg"], tensors, c["type"])
        nll = []
        for start in range(0, len(ids) - 1, ctx):
            chunk = ids[start:start + ctx]
            nll.append(m.chunk_nll(chunk, min(ctx // 2, len(chunk) - 1)))
        m.free()
        mean = float(np.concatenate(nll).mean())
        assert len(np.concatenate(nll)) == gpu["scored_tokens"]
        assert abs(mean - gpu["mean_nll"]) <= 1e-6, (c["key"], mean, gpu["mean_nll"])

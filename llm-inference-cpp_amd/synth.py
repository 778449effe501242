"""Deterministic synthetic inputs shared by the tests, the golden-fixture
generator and bench.py.

std::normal_distribution is implementation-defined (the reference hit this
between libstdc++ and libc++, tests/transformer_test.cpp:264-281), so nothing
here uses a library normal sampler.  Every value is produced from integer
hashing plus IEEE double additions and multiplications only, so the same
(seed, index) gives the same float32 on every host, in numpy, and in the
device generator (llmi_hip_synth_normal in csrc/synth.hip), which repeats
the same operations with non-contracted double arithmetic.

Generator "synth-v1":
  h(seed, c)  = splitmix64 output for counter c under key `seed`
                z = seed + (c + 1) * 0x9E3779B97F4A7C15 (mod 2^64), then the
                splitmix64 finaliser (shift-xor-multiply x2, shift-xor).
  element i of a normal stream uses h(seed, 2i) and h(seed, 2i + 1): their
  eight 16-bit lanes a_k give s = (sum a_k + 4) / 65536, a sum of eight
  uniforms on (0, 1); z = (s - 4) * sqrt(1.5) has mean 0 and variance 1
  (Irwin-Hall n=8, close to a Gaussian, bounded by +-4.9).
  value = float32(mean + std * z), each double operation rounded once.
  uniform integer ids in [0, n) use h(seed, i) mod n.
"""

from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
SQRT_1_5 = float(np.sqrt(np.float64(1.5)))  # IEEE sqrt: identical everywhere
GENERATOR = "synth-v1"

_CHUNK = 1 << 22


def _splitmix(seed: int, counters: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (counters + np.uint64(1)) * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        z = z ^ (z >> np.uint64(31))
    return z


def _lane_sum(h: np.ndarray) -> np.ndarray:
    m = np.uint64(0xFFFF)
    return ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m) + (h >> np.uint64(48)))


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0, offset: int = 0) -> np.ndarray:
    """float32[n]: elements offset .. offset+n-1 of the synth-v1 normal stream `seed`."""
    out = np.empty(n, dtype=np.float32)
    for lo in range(0, n, _CHUNK):
        hi = min(n, lo + _CHUNK)
        idx = np.arange(offset + lo, offset + hi, dtype=np.uint64)
        h0 = _splitmix(seed, idx * np.uint64(2))
        h1 = _splitmix(seed, idx * np.uint64(2) + np.uint64(1))
        total = (_lane_sum(h0) + _lane_sum(h1)).astype(np.float64)
        s = (total + 4.0) / 65536.0
        z = (s - 4.0) * SQRT_1_5
        v = np.float64(mean) + np.float64(std) * z
        out[lo:hi] = v.astype(np.float32)
    return out


def uniform_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    """int32[n] token ids in [0, vocab)."""
    idx = np.arange(n, dtype=np.uint64)
    h = _splitmix(seed, idx)
    return (h % np.uint64(vocab)).astype(np.int32)


def tensor_seed(base_seed: int, tensor_index: int) -> int:
    """Seed of the tensor_index-th tensor of a synthetic model built from base_seed."""
    return (base_seed * 1000003 + tensor_index * 7919 + 17) & 0xFFFFFFFFFFFFFFFF


# ---------------------------------------------------------------- models
# Architectures of BASELINE.json's configs (SmolLM2-135M: testdata/
# smollm2-135m/config.json of the reference; Qwen2.5-0.5B: the reference's
# docs/evidence/m1-weights-crosscheck.txt) plus the reference's 2-layer test
# model (tests/transformer_test.cpp:150-154).  Keys are llmi_model_config's.

SMOLLM2_135M = dict(arch=0, vocab_size=49152, hidden_size=576, intermediate_size=1536, num_layers=30, num_heads=9,
                    num_kv_heads=3, max_position_embeddings=8192, rms_norm_eps=1e-5, rope_theta=100000.0,
                    tie_word_embeddings=1, qkv_bias=0)
QWEN25_05B = dict(arch=1, vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=24, num_heads=14,
                  num_kv_heads=2, max_position_embeddings=32768, rms_norm_eps=1e-6, rope_theta=1000000.0,
                  tie_word_embeddings=1, qkv_bias=1)


def tiny(arch: int = 0, tied: bool = True) -> dict:
    return dict(arch=arch, vocab_size=32, hidden_size=16, intermediate_size=24, num_layers=2, num_heads=4,
                num_kv_heads=2, max_position_embeddings=64, rms_norm_eps=1e-6, rope_theta=10000.0,
                tie_word_embeddings=int(tied), qkv_bias=int(arch == 1))


def tensor_specs(cfg: dict) -> list:
    """(name, shape, kind) in the reference's expected_tensors() order
    (src/model/model.cpp:135-162); kind is 'matrix', 'norm' or 'bias'."""
    h = cfg["hidden_size"]
    hd = h // cfg["num_heads"]
    q = cfg["num_heads"] * hd
    kv = cfg["num_kv_heads"] * hd
    ff = cfg["intermediate_size"]
    v = cfg["vocab_size"]
    out = [("model.embed_tokens.weight", (v, h), "matrix")]
    for i in range(cfg["num_layers"]):
        p = f"model.layers.{i}."
        out.append((p + "input_layernorm.weight", (h,), "norm"))
        out.append((p + "self_attn.q_proj.weight", (q, h), "matrix"))
        out.append((p + "self_attn.k_proj.weight", (kv, h), "matrix"))
        out.append((p + "self_attn.v_proj.weight", (kv, h), "matrix"))
        if cfg["qkv_bias"]:
            out.append((p + "self_attn.q_proj.bias", (q,), "bias"))
            out.append((p + "self_attn.k_proj.bias", (kv,), "bias"))
            out.append((p + "self_attn.v_proj.bias", (kv,), "bias"))
        out.append((p + "self_attn.o_proj.weight", (h, q), "matrix"))
        out.append((p + "post_attention_layernorm.weight", (h,), "norm"))
        out.append((p + "mlp.gate_proj.weight", (ff, h), "matrix"))
        out.append((p + "mlp.up_proj.weight", (ff, h), "matrix"))
        out.append((p + "mlp.down_proj.weight", (h, ff), "matrix"))
    out.append(("model.norm.weight", (h,), "norm"))
    if not cfg["tie_word_embeddings"]:
        out.append(("lm_head.weight", (v, h), "matrix"))
    return out


# Value conventions of the synthetic models.  "bench": matrices, embeddings
# and biases N(0, 0.02), RMSNorm weights exactly 1.0.
# "tiny": N(0, 0.3) and norms 1 + 0.1 * N(0, 0.3), as the reference's own
# make_tiny (tests/transformer_test.cpp:179-181).
CONVENTIONS = {
    "bench": dict(std=0.02, norm_mean=1.0, norm_std=0.0),
    "tiny": dict(std=0.3, norm_mean=1.0, norm_std=0.03),
}


def tensor_params(cfg: dict, base_seed: int, convention: str = "bench") -> list:
    """Per tensor: (name, shape, seed, mean, std) of its synth-v1 stream."""
    conv = CONVENTIONS[convention]
    out = []
    for idx, (name, shape, kind) in enumerate(tensor_specs(cfg)):
        seed = tensor_seed(base_seed, idx)
        if kind == "norm":
            out.append((name, shape, seed, conv["norm_mean"], conv["norm_std"]))
        else:
            out.append((name, shape, seed, 0.0, conv["std"]))
    return out


def make_tensors(cfg: dict, base_seed: int, convention: str = "bench") -> list:
    """fp32 host arrays of every tensor (flattened), in expected order."""
    res = []
    for name, shape, seed, mean, std in tensor_params(cfg, base_seed, convention):
        n = int(np.prod(shape))
        if std == 0.0:
            res.append(np.full(n, np.float32(mean), dtype=np.float32))
        else:
            res.append(normal(seed, n, mean, std))
    return res

"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU oracle (liboracle.so,
our restatement of the reference algorithms in oracle.cpp) and, where it was
built, to the reference's own code (_ref/libllmi_ref.so, from
ref_shim.cpp + the reference sources).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  Both libraries expose the same call shapes, so `Cpu(lib)`
wraps either one.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# LLMI_ORACLE_SANITIZED=1 loads the AddressSanitizer/UBSan builds
# (make -C oracle sanitize) instead; the process must have libasan preloaded.
_SAN = os.environ.get("LLMI_ORACLE_SANITIZED") == "1"
ORACLE_SO = os.path.join(HERE, "_asan" if _SAN else "", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "asan" if _SAN else "", "libllmi_ref.so")

F32, Q8_0, Q4_0 = 0, 1, 2
BLOCK = 32


class ModelConfig(C.Structure):
    """Same layout as llmi_model_config in include/llmi_hip.h."""

    _fields_ = [
        ("arch", C.c_int32),
        ("vocab_size", C.c_uint32),
        ("hidden_size", C.c_uint32),
        ("intermediate_size", C.c_uint32),
        ("num_layers", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("max_position_embeddings", C.c_uint32),
        ("rms_norm_eps", C.c_double),
        ("rope_theta", C.c_double),
        ("tie_word_embeddings", C.c_int32),
        ("qkv_bias", C.c_int32),
    ]

    @classmethod
    def from_dict(cls, d: dict) -> "ModelConfig":
        return cls(**{k: d[k] for k, _ in cls._fields_})


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def row_bytes(n_in: int, qtype: int) -> int:
    return (n_in + 1) // 2 if qtype == Q4_0 else n_in


def nblocks(n_in: int) -> int:
    return (n_in + BLOCK - 1) // BLOCK


class Cpu:
    """One CPU implementation of the path: prefix 'oracle_' (restatement) or
    'ref_' (the compiled reference)."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.prefix = prefix
        self.lib = C.CDLL(path)
        L = self.lib
        f = lambda name: getattr(L, prefix + name)  # noqa: E731
        self._quantize = f("quantize")
        self._quantize.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p]
        self._dequant = f("dequantize_row")
        self._matmul = f("matmul")
        self._dot = f("dot")
        self._dot.restype = C.c_float
        self._dot.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        self._rmsnorm = f("rmsnorm")
        self._rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_float, C.c_void_p]
        self._rope = f("rope")
        self._rope.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        self._softmax = f("softmax")
        self._softmax.argtypes = [C.c_void_p, C.c_size_t]
        self._silu = f("silu")
        self._silu.restype = C.c_float
        self._silu.argtypes = [C.c_float]
        self._argmax = f("argmax")
        self._argmax.restype = C.c_size_t
        self._argmax.argtypes = [C.c_void_p, C.c_size_t]
        self._pool_workers = f("pool_workers")
        self._model_create = f("model_create")
        self._model_create.restype = C.c_void_p
        self._model_create.argtypes = [C.POINTER(ModelConfig), C.c_void_p, C.c_int]
        self._model_free = f("model_free")
        self._model_free.argtypes = [C.c_void_p]
        self._new_cache = f("model_new_cache")
        self._new_cache.argtypes = [C.c_void_p, C.c_size_t]
        self._cache_len = f("model_cache_length")
        self._cache_len.restype = C.c_size_t
        self._cache_len.argtypes = [C.c_void_p]
        self._fwd = f("model_forward_cached")
        self._fwd.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        self._greedy = f("generate_greedy_cached")
        self._greedy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]
        self._err = f("last_error")
        self._err.restype = C.c_char_p
        self._gguf = f("gguf_to_quantized")
        self._gguf.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p]

    def last_error(self) -> str:
        return self._err().decode()

    def pool_workers(self) -> int:
        return int(self._pool_workers())

    def set_pool_workers(self, n: int) -> None:
        """Oracle only: resize the restated thread pool."""
        self.lib.oracle_set_pool_workers(int(n))

    # -- quant ------------------------------------------------------------
    def quantize(self, w: np.ndarray, out: int, n_in: int, qtype: int):
        w = np.ascontiguousarray(w, dtype=np.float32)
        data = np.zeros(out * row_bytes(n_in, qtype), dtype=np.uint8)
        scales = np.zeros(out * nblocks(n_in), dtype=np.float32)
        self._quantize(_p(w), out, n_in, qtype, _p(data), _p(scales))
        return data, scales

    def gguf_to_quantized(self, raw: np.ndarray, out: int, n_in: int, gguf_type: int):
        """gguf::to_quantized on one tensor's raw ggml blocks (gguf.cpp:577-640):
        (data, scales) in the engine layout; ValueError with the message
        where the reference fails."""
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        qtype = Q8_0 if gguf_type == 8 else Q4_0
        data = np.zeros(max(1, out * row_bytes(n_in, qtype)), dtype=np.uint8)
        scales = np.zeros(max(1, out * nblocks(n_in)), dtype=np.float32)
        if self._gguf(_p(raw), raw.nbytes, out, n_in, gguf_type, _p(data), _p(scales)) != 0:
            raise ValueError(self.last_error())
        return data[:out * row_bytes(n_in, qtype)], scales[:out * nblocks(n_in)]

    def dequantize_row(self, data, scales, out: int, n_in: int, qtype: int, row: int) -> np.ndarray:
        dst = np.zeros(n_in, dtype=np.float32)
        if self.prefix == "ref_":
            self._dequant.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_int, C.c_size_t, C.c_void_p]
            self._dequant(_p(data), _p(scales), out, n_in, qtype, row, _p(dst))
        else:
            self._dequant.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_size_t, C.c_void_p]
            self._dequant(_p(data), _p(scales), n_in, qtype, row, _p(dst))
        return dst

    def matmul(self, x, rows: int, n_in: int, data, scales, qtype: int, out: int, bias=None, threads: int = 0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(rows * out, dtype=np.float32)
        if self.prefix == "ref_":
            self._matmul.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int, C.c_size_t,
                                     C.c_void_p, C.c_void_p]
            self._matmul(_p(x), rows, n_in, _p(data), _p(scales), qtype, out, _p(bias), _p(y))
        else:
            self._matmul.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int, C.c_size_t,
                                     C.c_void_p, C.c_void_p, C.c_int]
            self._matmul(_p(x), rows, n_in, _p(data), _p(scales), qtype, out, _p(bias), _p(y), threads)
        return y

    def qmatrix(self, data, scales, out: int, n_in: int, qtype: int) -> "QMatrix":
        """A packed matrix held across calls, so that a timing loop measures
        quant::matmul alone (the reference's QuantizedMatrix kept alive,
        ref_shim.cpp; the restatement reads the arrays in place)."""
        return QMatrix(self, data, scales, out, n_in, qtype)

    # -- glue kernels ------------------------------------------------------
    def dot(self, a, b) -> float:
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        return float(np.float32(self._dot(_p(a), _p(b), a.size)))

    def rmsnorm(self, x, w, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.zeros_like(x)
        self._rmsnorm(_p(x), _p(w), x.size, eps, _p(y))
        return y

    def rope(self, v, pos: int, inv_freq) -> np.ndarray:
        v = np.array(v, dtype=np.float32)
        inv = np.ascontiguousarray(inv_freq, np.float32)
        self._rope(_p(v), v.size, pos, _p(inv))
        return v

    def softmax(self, x) -> np.ndarray:
        x = np.array(x, dtype=np.float32)
        self._softmax(_p(x), x.size)
        return x

    def silu(self, v: float) -> np.float32:
        return np.float32(self._silu(float(v)))

    def argmax(self, x) -> int:
        x = np.ascontiguousarray(x, np.float32)
        return int(self._argmax(_p(x), x.size))

    # -- sampling (sampling.cpp) ----------------------------------------------
    def sampling_probabilities(self, logits, temperature: float, top_k: int = 0, top_p: float = 1.0) -> np.ndarray:
        x = np.ascontiguousarray(logits, np.float32)
        if x.size == 0:
            raise ValueError("sampling_probabilities: empty logits")
        out = np.empty_like(x)
        fn = getattr(self.lib, self.prefix + "sampling_probabilities")
        fn.argtypes = [C.c_void_p, C.c_size_t, C.c_float, C.c_size_t, C.c_float, C.c_void_p]
        fn(_p(x), x.size, float(temperature), int(top_k), float(top_p), _p(out))
        return out

    def sample_target(self, logits, temperature: float, top_k: int, top_p: float, target: float) -> int:
        """Oracle only: sample() with the uniform draw given."""
        x = np.ascontiguousarray(logits, np.float32)
        fn = self.lib.oracle_sample_target
        fn.restype = C.c_size_t
        fn.argtypes = [C.c_void_p, C.c_size_t, C.c_float, C.c_size_t, C.c_float, C.c_double]
        return int(fn(_p(x), x.size, float(temperature), int(top_k), float(top_p), float(target)))

    def draw_uniform(self, seed: int, count: int) -> np.ndarray:
        """Oracle only: the numbers successive sample() calls draw from
        std::mt19937_64(seed)."""
        out = np.empty(count, np.float64)
        fn = self.lib.oracle_draw_uniform
        fn.argtypes = [C.c_uint64, C.c_size_t, C.c_void_p]
        fn(int(seed), int(count), _p(out))
        return out

    def sample_sequence(self, logits, temperature: float, top_k: int, top_p: float, seed: int, count: int):
        """Reference only: `count` sample() calls on std::mt19937_64(seed) ->
        (ids, the number each call drew, -1 when it drew none)."""
        x = np.ascontiguousarray(logits, np.float32)
        ids = np.empty(count, np.int32)
        targets = np.empty(count, np.float64)
        fn = self.lib.ref_sample_sequence
        fn.argtypes = [C.c_void_p, C.c_size_t, C.c_float, C.c_size_t, C.c_float, C.c_uint64, C.c_size_t, C.c_void_p,
                       C.c_void_p]
        fn(_p(x), x.size, float(temperature), int(top_k), float(top_p), int(seed), int(count), _p(ids), _p(targets))
        return ids, targets

    # -- model -------------------------------------------------------------
    def model(self, cfg: dict, tensors: list, qtype: int) -> "CpuModel":
        return CpuModel(self, cfg, tensors, qtype)


class CpuModel:
    def __init__(self, cpu: Cpu, cfg: dict, tensors: list, qtype: int):
        self.cpu = cpu
        self.cfg = dict(cfg)
        self.c = ModelConfig.from_dict(cfg)
        arr = (C.c_void_p * len(tensors))(*[t.ctypes.data for t in tensors])
        self.h = cpu._model_create(C.byref(self.c), arr, qtype)
        if not self.h:
            raise RuntimeError(cpu.last_error())

    def close(self):
        if self.h:
            self.cpu._model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_cache(self, max_len: int) -> bool:
        return self.cpu._new_cache(self.h, max_len) == 0

    def cache_length(self) -> int:
        return int(self.cpu._cache_len(self.h))

    def forward_cached(self, tokens, all_positions: bool = False):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        n = max(1, toks.size if all_positions else 1)
        logits = np.zeros(n * self.cfg["vocab_size"], dtype=np.float32)
        if self.cpu._fwd(self.h, _p(toks), toks.size, int(all_positions), _p(logits)) != 0:
            return None
        return logits

    def generate_greedy(self, prompt, max_new: int):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        ids = np.zeros(max_new, dtype=np.int32)
        margins = np.zeros(max_new, dtype=np.float32)
        if self.cpu._greedy(self.h, _p(p), p.size, max_new, _p(ids), _p(margins)) != 0:
            raise RuntimeError(self.cpu.last_error())
        return ids, margins


_cache: dict = {}


class QMatrix:
    """Cpu.qmatrix: y = x W^T on a matrix that stays wrapped between calls."""

    def __init__(self, cpu: Cpu, data, scales, out: int, n_in: int, qtype: int):
        self.cpu, self.out, self.n_in, self.qtype = cpu, out, n_in, qtype
        self.data = np.ascontiguousarray(data, dtype=np.uint8)
        self.scales = np.ascontiguousarray(scales, dtype=np.float32)
        self.h = None
        if cpu.prefix == "ref_":
            L = cpu.lib
            L.ref_qmatrix_create.restype = C.c_void_p
            L.ref_qmatrix_create.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_int]
            L.ref_qmatrix_matmul.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]
            L.ref_qmatrix_free.argtypes = [C.c_void_p]
            self.h = L.ref_qmatrix_create(_p(self.data), _p(self.scales), out, n_in, qtype)

    def matmul(self, x: np.ndarray, rows: int, y: np.ndarray) -> np.ndarray:
        if self.h is not None:
            self.cpu.lib.ref_qmatrix_matmul(self.h, _p(x), rows, None, _p(y))
        else:
            self.cpu._matmul.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_int,
                                         C.c_size_t, C.c_void_p, C.c_void_p, C.c_int]
            self.cpu._matmul(_p(x), rows, self.n_in, _p(self.data), _p(self.scales), self.qtype, self.out, None,
                             _p(y), 0)
        return y

    def close(self) -> None:
        if self.h is not None:
            self.cpu.lib.ref_qmatrix_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


def oracle() -> Cpu:
    if "oracle" not in _cache:
        if not os.path.exists(ORACLE_SO):
            raise FileNotFoundError(f"{ORACLE_SO} is not built (run __graft_entry__.build())")
        _cache["oracle"] = Cpu(ORACLE_SO, "oracle_")
    return _cache["oracle"]


def reference() -> Cpu | None:
    """The compiled reference, or None where oracle/_ref was not built."""
    if "ref" not in _cache:
        _cache["ref"] = Cpu(REF_SO, "ref_") if os.path.exists(REF_SO) else None
    return _cache["ref"]

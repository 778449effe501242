"""ctypes binding of libllmi_hip.so (include/llmi_hip.h) for Python callers:
the tests, bench.py and __graft_entry__.smoke().

The product is the shared library; this module only declares the C
signatures and adds numpy conveniences.  It never falls back to another
implementation: if the library is missing or a call fails, it raises.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllmi_hip.so")

F32, Q8_0, Q4_0 = 0, 1, 2
GGUF_Q4_0, GGUF_Q8_0 = 2, 8  # GGUF tensor types (LLMI_GGUF_*)
SCORE_EXACT, SCORE_MFMA_HEAD, SCORE_MFMA = 0, 1, 2  # modes of llmi_hip_model_chunk_nll
BLOCK = 32
TYPE_NAMES = {F32: "f32", Q8_0: "q8_0", Q4_0: "q4_0"}

# Every symbol include/llmi_hip.h declares, with (restype, argtypes).
_sz, _vp, _i, _f, _d, _u64 = C.c_size_t, C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_uint64
SIGNATURES = {
    "llmi_hip_init": (_i, [_i]),
    "llmi_hip_shutdown": (_i, []),
    "llmi_hip_last_error": (C.c_char_p, []),
    "llmi_hip_version": (C.c_char_p, []),
    "llmi_hip_stream": (_vp, []),
    "llmi_hip_synchronize": (_i, []),
    "llmi_hip_malloc": (_i, [C.POINTER(_vp), _sz]),
    "llmi_hip_free": (_i, [_vp]),
    "llmi_hip_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "llmi_hip_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "llmi_hip_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "llmi_hip_memset_dev": (_i, [_vp, _i, _sz]),
    "llmi_hip_event_create": (_i, [C.POINTER(_vp)]),
    "llmi_hip_event_destroy": (_i, [_vp]),
    "llmi_hip_event_record": (_i, [_vp, _vp]),
    "llmi_hip_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "llmi_hip_graph_begin": (_i, []),
    "llmi_hip_graph_end": (_i, [C.POINTER(_vp)]),
    "llmi_hip_graph_launch": (_i, [_vp]),
    "llmi_hip_graph_destroy": (_i, [_vp]),
    "llmi_hip_synth_normal_dev": (_i, [_vp, _sz, _u64, _u64, _d, _d, _vp]),
    "llmi_hip_row_bytes": (_sz, [_sz, _i]),
    "llmi_hip_quantize": (_i, [_vp, _sz, _sz, _i, _vp, _vp]),
    "llmi_hip_quantize_dev": (_i, [_vp, _sz, _sz, _i, _vp, _vp, _vp]),
    "llmi_hip_weight_upload": (_i, [_vp, _vp, _sz, _sz, _i, C.POINTER(_vp)]),
    "llmi_hip_weight_quantize": (_i, [_vp, _sz, _sz, _i, C.POINTER(_vp)]),
    "llmi_hip_weight_quantize_dev": (_i, [_vp, _sz, _sz, _i, C.POINTER(_vp)]),
    "llmi_hip_weight_free": (_i, [_vp]),
    "llmi_hip_model_chunk_nll": (_i, [_vp, _vp, _sz, _sz, _i, _vp]),
    "llmi_hip_weight_from_gguf": (_i, [_vp, _sz, _sz, _sz, _i, C.POINTER(_vp)]),
    "llmi_hip_weight_download": (_i, [_vp, _vp, _vp]),
    "llmi_hip_weight_info": (_i, [_vp, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_i), C.POINTER(_sz)]),
    "llmi_hip_weight_device_bytes": (_sz, [_vp]),
    "llmi_hip_dequantize_row": (_i, [_vp, _sz, _vp]),
    "llmi_hip_dequantize_rows_dev": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "llmi_hip_matmul": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp]),
    "llmi_hip_matmul_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "llmi_hip_group_create": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, C.POINTER(_vp)]),
    "llmi_hip_group_launch": (_i, [_vp, _vp]),
    "llmi_hip_group_free": (None, [_vp]),
    "llmi_hip_matmul_mfma_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "llmi_hip_gemm_group_create": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, C.POINTER(_vp)]),
    "llmi_hip_gemm_group_launch": (_i, [_vp, _vp]),
    "llmi_hip_gemm_group_free": (None, [_vp]),
    "llmi_hip_matmul_tol_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "llmi_hip_tol_group_create": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, C.POINTER(_vp)]),
    "llmi_hip_tol_group_launch": (_i, [_vp, _vp]),
    "llmi_hip_tol_group_free": (None, [_vp]),
    "llmi_hip_dot_dev": (_i, [_vp, _vp, _vp, _sz, _vp, _vp]),
    "llmi_hip_rmsnorm_dev": (_i, [_vp, _vp, _sz, _sz, _f, _vp, _vp]),
    "llmi_hip_softmax_dev": (_i, [_vp, _sz, _sz, _vp]),
    "llmi_hip_silu_dev": (_i, [_vp, _sz, _vp]),
    "llmi_hip_argmax_dev": (_i, [_vp, _sz, _vp, _vp]),
    "llmi_hip_model_create": (_i, [_vp, _vp, _i, C.POINTER(_vp)]),
    "llmi_hip_model_create_dev": (_i, [_vp, _vp, _i, C.POINTER(_vp)]),
    "llmi_hip_model_free": (_i, [_vp]),
    "llmi_hip_model_weight_bytes": (_sz, [_vp]),
    "llmi_hip_model_new_cache": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "llmi_hip_cache_free": (_i, [_vp]),
    "llmi_hip_cache_length": (_sz, [_vp]),
    "llmi_hip_cache_capacity": (_sz, [_vp]),
    "llmi_hip_cache_reset": (_i, [_vp]),
    "llmi_hip_model_forward_cached": (_i, [_vp, _vp, _vp, _sz, _i, _vp]),
    "llmi_hip_model_forward_cached_trace": (_i, [_vp, _vp, _vp, _sz, _i, _vp, _vp]),
    "llmi_hip_model_forward": (_i, [_vp, _vp, _sz, _i, _vp, _vp]),
    "llmi_hip_matmul_mfma_noalloc_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "llmi_hip_model_generate_greedy": (_i, [_vp, _vp, _sz, _sz, _vp, _sz, _vp, C.POINTER(_sz)]),
    "llmi_hip_model_last_timing": (_i, [_vp, C.POINTER(_d), C.POINTER(_d)]),
    "llmi_hip_model_last_redraws": (_i, [_vp, C.POINTER(_sz)]),
    "llmi_hip_model_set_decode_mode": (_i, [_vp, _i]),
    "llmi_hip_model_set_decode_graph": (_i, [_vp, _i]),
    "llmi_hip_sample": (_i, [_vp, _sz, _vp, _d, C.POINTER(C.c_int32)]),
    "llmi_hip_sample_dev": (_i, [_vp, _sz, _vp, _d, C.POINTER(C.c_int32), _vp]),
    "llmi_hip_sampling_probabilities": (_i, [_vp, _sz, _vp, _vp]),
    "llmi_hip_sampling_set_exact_only": (_i, [_i]),
    "llmi_hip_sampling_last_paths": (_i, [C.POINTER(_i)]),
    "llmi_hip_model_forward_sample": (_i, [_vp, _vp, _vp, _sz, _vp, _d, C.POINTER(C.c_int32)]),
    "llmi_hip_model_generate_sampled": (_i, [_vp, _vp, _sz, _sz, _vp, _vp, _vp, _sz, _vp, C.POINTER(_sz)]),
}


class Sampling(C.Structure):
    """llmi_hip_sampling: SamplingConfig (include/llmi/model/sampling.hpp:20-24)."""

    _fields_ = [("temperature", C.c_float), ("top_k", C.c_size_t), ("top_p", C.c_float)]

    def __init__(self, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0):
        super().__init__(float(temperature), int(top_k), float(top_p))


DECODE_EXACT, DECODE_TOLERANCE = 0, 1


class HipError(RuntimeError):
    pass


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def row_bytes(n_in: int, qtype: int) -> int:
    return (n_in + 1) // 2 if qtype == Q4_0 else n_in


def nblocks(n_in: int) -> int:
    return (n_in + BLOCK - 1) // BLOCK


_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads the library and declares its signatures (no GPU call)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise HipError(f"llmi_hip error {rc}: {load().llmi_hip_last_error().decode()}")


_initialised = False


def init(device: int = 0) -> C.CDLL:
    global _initialised
    lib = load()
    if not _initialised:
        check(lib.llmi_hip_init(device))
        _initialised = True
    return lib


class DeviceBuffer:
    """A plain device allocation owned by Python."""

    def __init__(self, nbytes: int):
        self.lib = init()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(self.lib.llmi_hip_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(self.lib.llmi_hip_memcpy_h2d(self.ptr, _p(a), a.nbytes))

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        check(self.lib.llmi_hip_memcpy_d2h(_p(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(self.lib.llmi_hip_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A device-resident packed matrix (llmi_hip_weight)."""

    def __init__(self, handle: int, lib):
        self.h = handle
        self.lib = lib
        out, n_in, qt, bs = _sz(), _sz(), _i(), _sz()
        check(lib.llmi_hip_weight_info(self.h, C.byref(out), C.byref(n_in), C.byref(qt), C.byref(bs)))
        self.out, self.n_in, self.qtype, self.byte_size = out.value, n_in.value, qt.value, bs.value

    @classmethod
    def upload(cls, data: np.ndarray, scales: np.ndarray, out: int, n_in: int, qtype: int) -> "Weight":
        lib = init()
        h = C.c_void_p()
        check(lib.llmi_hip_weight_upload(_p(np.ascontiguousarray(data)), _p(np.ascontiguousarray(scales)), out, n_in,
                                         qtype, C.byref(h)))
        return cls(h.value, lib)

    @classmethod
    def from_gguf(cls, blocks: np.ndarray, out: int, n_in: int, gguf_type: int) -> "Weight":
        """A GGUF Q8_0/Q4_0 tensor's raw blocks (uint8) -> device weight."""
        lib = init()
        h = C.c_void_p()
        raw = np.ascontiguousarray(blocks, dtype=np.uint8)
        check(lib.llmi_hip_weight_from_gguf(_p(raw), raw.nbytes, out, n_in, gguf_type, C.byref(h)))
        return cls(h.value, lib)

    @classmethod
    def quantize(cls, w: np.ndarray, out: int, n_in: int, qtype: int) -> "Weight":
        lib = init()
        h = C.c_void_p()
        check(lib.llmi_hip_weight_quantize(_p(np.ascontiguousarray(w, dtype=np.float32)), out, n_in, qtype, C.byref(h)))
        return cls(h.value, lib)

    @classmethod
    def quantize_dev(cls, w_dev: int, out: int, n_in: int, qtype: int) -> "Weight":
        lib = init()
        h = C.c_void_p()
        check(lib.llmi_hip_weight_quantize_dev(w_dev, out, n_in, qtype, C.byref(h)))
        return cls(h.value, lib)

    def download(self):
        data = np.zeros(self.out * row_bytes(self.n_in, self.qtype), dtype=np.uint8)
        scales = np.zeros(self.out * nblocks(self.n_in), dtype=np.float32)
        check(self.lib.llmi_hip_weight_download(self.h, _p(data), _p(scales)))
        return data, scales

    def device_bytes(self) -> int:
        return int(self.lib.llmi_hip_weight_device_bytes(self.h))

    def dequantize_row(self, row: int) -> np.ndarray:
        dst = np.zeros(self.n_in, dtype=np.float32)
        check(self.lib.llmi_hip_dequantize_row(self.h, row, _p(dst)))
        return dst

    def matmul(self, x: np.ndarray, rows: int, bias: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(rows * self.out, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        check(self.lib.llmi_hip_matmul(self.h, _p(x), rows, self.n_in, self.out, _p(b), _p(y)))
        return y

    def matmul_dev(self, x_dev: int, rows: int, bias_dev: int | None, y_dev: int, stream=None) -> None:
        check(self.lib.llmi_hip_matmul_dev(self.h, x_dev, rows, bias_dev, y_dev, stream))

    def matmul_mfma_dev(self, x_dev: int, rows: int, bias_dev: int | None, y_dev: int, stream=None) -> None:
        check(self.lib.llmi_hip_matmul_mfma_dev(self.h, x_dev, rows, bias_dev, y_dev, stream))

    def matmul_tol_dev(self, x_dev: int, rows: int, bias_dev: int | None, y_dev: int, stream=None) -> None:
        check(self.lib.llmi_hip_matmul_tol_dev(self.h, x_dev, rows, bias_dev, y_dev, stream))

    def matmul_tol(self, x: np.ndarray, rows: int, bias: np.ndarray | None = None) -> np.ndarray:
        """The tolerance-mode Q4_0 product (matrix cores) on host arrays."""
        xd = DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
        yd = DeviceBuffer(max(1, rows * self.out) * 4)
        bd = None if bias is None else DeviceBuffer.from_array(np.ascontiguousarray(bias, dtype=np.float32))
        self.matmul_tol_dev(xd.ptr, rows, None if bd is None else bd.ptr, yd.ptr)
        synchronize()
        y = yd.download(np.float32, rows * self.out)
        for b in (xd, yd, bd):
            if b is not None:
                b.free()
        return y

    def matmul_mfma(self, x: np.ndarray, rows: int, bias: np.ndarray | None = None) -> np.ndarray:
        """The bf16-MFMA prefill product on host arrays (tolerance, not exact)."""
        xd = DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
        yd = DeviceBuffer(max(1, rows * self.out) * 4)
        bd = None if bias is None else DeviceBuffer.from_array(np.ascontiguousarray(bias, dtype=np.float32))
        self.matmul_mfma_dev(xd.ptr, rows, None if bd is None else bd.ptr, yd.ptr)
        synchronize()
        y = yd.download(np.float32, rows * self.out)
        for b in (xd, yd, bd):
            if b is not None:
                b.free()
        return y

    def free(self) -> None:
        if self.h:
            check(self.lib.llmi_hip_weight_free(self.h))
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def quantize(w: np.ndarray, out: int, n_in: int, qtype: int):
    """llmi_hip_quantize: planar (reference-layout) packed data and scales."""
    lib = init()
    w = np.ascontiguousarray(w, dtype=np.float32)
    data = np.zeros(out * row_bytes(n_in, qtype), dtype=np.uint8)
    scales = np.zeros(out * nblocks(n_in), dtype=np.float32)
    check(lib.llmi_hip_quantize(_p(w), out, n_in, qtype, _p(data), _p(scales)))
    return data, scales


def synth_normal_dev(buf: DeviceBuffer, n: int, seed: int, mean: float, std: float, offset: int = 0) -> None:
    lib = init()
    check(lib.llmi_hip_synth_normal_dev(buf.ptr, n, seed, offset, mean, std, None))


class Timer:
    """HIP events on the library stream."""

    def __init__(self):
        self.lib = init()
        a, b = C.c_void_p(), C.c_void_p()
        check(self.lib.llmi_hip_event_create(C.byref(a)))
        check(self.lib.llmi_hip_event_create(C.byref(b)))
        self.start_ev, self.stop_ev = a.value, b.value

    def start(self):
        check(self.lib.llmi_hip_event_record(self.start_ev, None))

    def stop(self) -> float:
        check(self.lib.llmi_hip_event_record(self.stop_ev, None))
        ms = C.c_float()
        check(self.lib.llmi_hip_event_elapsed_ms(self.start_ev, self.stop_ev, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            self.lib.llmi_hip_event_destroy(self.start_ev)
            self.lib.llmi_hip_event_destroy(self.stop_ev)
        except Exception:
            pass


class ModelConfig(C.Structure):
    """llmi_model_config (include/llmi_hip.h)."""

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


class Cache:
    def __init__(self, model: "Model", max_len: int):
        self.lib = model.lib
        h = C.c_void_p()
        check(self.lib.llmi_hip_model_new_cache(model.h, max_len, C.byref(h)))
        self.h = h.value

    def length(self) -> int:
        return int(self.lib.llmi_hip_cache_length(self.h))

    def capacity(self) -> int:
        return int(self.lib.llmi_hip_cache_capacity(self.h))

    def reset(self) -> None:
        check(self.lib.llmi_hip_cache_reset(self.h))

    def free(self) -> None:
        if self.h:
            check(self.lib.llmi_hip_cache_free(self.h))
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Model:
    """A device-resident quantized decoder (llmi_hip_model)."""

    def __init__(self, cfg: dict, tensors, qtype: int, on_device: bool = False):
        self.lib = init()
        self.cfg = dict(cfg)
        self.c = ModelConfig.from_dict(cfg)
        if on_device:
            ptrs = [int(t) for t in tensors]
        else:
            self._host = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
            ptrs = [t.ctypes.data for t in self._host]
        arr = (C.c_void_p * len(ptrs))(*ptrs)
        h = C.c_void_p()
        fn = self.lib.llmi_hip_model_create_dev if on_device else self.lib.llmi_hip_model_create
        check(fn(C.byref(self.c), arr, qtype, C.byref(h)))
        self._host = None
        self.h = h.value

    def weight_bytes(self) -> int:
        return int(self.lib.llmi_hip_model_weight_bytes(self.h))

    def new_cache(self, max_len: int) -> Cache:
        return Cache(self, max_len)

    def forward_cached(self, cache: Cache, tokens, all_positions: bool = False) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = toks.size if all_positions else 1
        logits = np.zeros(max(rows, 1) * self.cfg["vocab_size"], dtype=np.float32)
        check(self.lib.llmi_hip_model_forward_cached(self.h, cache.h, _p(toks), toks.size, int(all_positions),
                                                     _p(logits)))
        return logits

    def forward_cached_trace(self, cache: Cache, tokens, all_positions: bool = False):
        """(logits, states[(layers + 2), n, hidden])."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = toks.size if all_positions else 1
        logits = np.zeros(max(rows, 1) * self.cfg["vocab_size"], dtype=np.float32)
        states = np.zeros((self.cfg["num_layers"] + 2, toks.size, self.cfg["hidden_size"]), dtype=np.float32)
        check(self.lib.llmi_hip_model_forward_cached_trace(self.h, cache.h, _p(toks), toks.size, int(all_positions),
                                                           _p(logits), _p(states)))
        return logits, states

    def forward(self, tokens, all_positions: bool = False) -> np.ndarray:
        """Transformer::forward: the whole sequence, no caller's cache."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = toks.size if all_positions else 1
        logits = np.zeros(max(rows, 1) * self.cfg["vocab_size"], dtype=np.float32)
        check(self.lib.llmi_hip_model_forward(self.h, _p(toks), toks.size, int(all_positions), _p(logits), None))
        return logits

    def generate_greedy(self, prompt, max_new: int, stop_ids=()) -> np.ndarray:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        stop = np.ascontiguousarray(list(stop_ids), dtype=np.int32)
        ids = np.zeros(max(max_new, 1), dtype=np.int32)
        n = _sz()
        check(self.lib.llmi_hip_model_generate_greedy(self.h, _p(p), p.size, max_new, _p(stop) if stop.size else None,
                                                      stop.size, _p(ids), C.byref(n)))
        return ids[: n.value]

    def chunk_nll(self, tokens, t_start: int, mode: int = SCORE_EXACT) -> np.ndarray:
        """-log P(chunk[t+1] | chunk[..t]) for t in [t_start, n - 1) (float64)."""
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        rows = max(0, len(ids) - 1 - min(t_start, max(len(ids) - 1, 0)))
        out = np.zeros(max(rows, 1), dtype=np.float64)
        check(self.lib.llmi_hip_model_chunk_nll(self.h, _p(ids), len(ids), t_start, mode, _p(out)))
        return out[:rows]

    def forward_sample(self, cache: Cache, tokens, cfg: "Sampling", target: float) -> int:
        """forward_cached + sample() on the device; `target` is sample()'s draw."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = C.c_int32()
        check(self.lib.llmi_hip_model_forward_sample(self.h, cache.h, _p(toks), toks.size, C.byref(cfg),
                                                     float(target), C.byref(out)))
        return out.value

    def generate_sampled(self, prompt, max_new: int, cfg: "Sampling", targets, stop_ids=()) -> np.ndarray:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        t = np.ascontiguousarray(targets, dtype=np.float64)
        stop = np.ascontiguousarray(list(stop_ids), dtype=np.int32)
        ids = np.zeros(max(max_new, 1), dtype=np.int32)
        n = _sz()
        check(self.lib.llmi_hip_model_generate_sampled(self.h, _p(p), p.size, max_new, C.byref(cfg),
                                                       _p(t) if t.size else None, _p(stop) if stop.size else None,
                                                       stop.size, _p(ids), C.byref(n)))
        return ids[: n.value]

    def last_timing(self):
        """(prefill_ms, decode_ms) of the last generate_greedy / generate_sampled call."""
        a, b = _d(), _d()
        check(self.lib.llmi_hip_model_last_timing(self.h, C.byref(a), C.byref(b)))
        return a.value, b.value

    def last_redraws(self) -> int:
        """How many steps of the last generate_sampled call were redrawn with
        a host read-back of their own (0 when every step ran queued)."""
        v = _sz()
        check(self.lib.llmi_hip_model_last_redraws(self.h, C.byref(v)))
        return v.value

    def set_decode_mode(self, mode: int) -> None:
        """DECODE_EXACT (bit-identical, the default) or DECODE_TOLERANCE
        (position-chunked attention merged in o_proj; llmi_hip.h)."""
        check(self.lib.llmi_hip_model_set_decode_mode(self.h, int(mode)))

    def set_decode_graph(self, enable: bool) -> None:
        """Whether generate_greedy replays tolerance-mode steps from one
        captured graph (the default) or launches every kernel (llmi_hip.h)."""
        check(self.lib.llmi_hip_model_set_decode_graph(self.h, 1 if enable else 0))

    def free(self) -> None:
        if self.h:
            check(self.lib.llmi_hip_model_free(self.h))
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sample(logits, cfg: Sampling, target: float) -> int:
    """llmi::sample with its draw given (host logits)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = C.c_int32()
    check(init().llmi_hip_sample(_p(x), x.size, C.byref(cfg), float(target), C.byref(out)))
    return out.value


def sample_dev(logits: "DeviceBuffer", n: int, cfg: Sampling, target: float) -> int:
    out = C.c_int32()
    check(init().llmi_hip_sample_dev(logits.ptr, n, C.byref(cfg), float(target), C.byref(out), None))
    return out.value


def sampling_probabilities(logits, cfg: Sampling) -> np.ndarray:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty_like(x)
    check(init().llmi_hip_sampling_probabilities(_p(x), x.size, C.byref(cfg), _p(out)))
    return out


def sampling_set_exact_only(on: bool) -> None:
    check(init().llmi_hip_sampling_set_exact_only(int(on)))


def sampling_last_paths() -> int:
    v = C.c_int()
    check(init().llmi_hip_sampling_last_paths(C.byref(v)))
    return v.value


def synthetic_model_dev(cfg: dict, base_seed: int, qtype: int, convention: str = "bench") -> "Model":
    """Builds a synthetic model whose fp32 tensors are generated on the device
    by the synth-v1 generator (the same values synth.make_tensors gives)."""
    import synth

    bufs = []
    for name, shape, seed, mean, std in synth.tensor_params(cfg, base_seed, convention):
        n = int(np.prod(shape))
        b = DeviceBuffer(n * 4)
        if std == 0.0:
            b.upload(np.full(n, np.float32(mean), dtype=np.float32))
        else:
            synth_normal_dev(b, n, seed, mean, std)
        bufs.append(b)
    synchronize()
    m = Model(cfg, [b.ptr for b in bufs], qtype, on_device=True)
    for b in bufs:
        b.free()
    return m


class Group:
    """A fixed list of products (Weight, x device pointer, y device pointer,
    rows 1..8, optional bias device pointer) launched as one kernel."""

    _create, _launch, _free = "llmi_hip_group_create", "llmi_hip_group_launch", "llmi_hip_group_free"

    def __init__(self, items):
        self.lib = init()
        n = len(items)
        ws = (C.c_void_p * n)(*[it[0].h for it in items])
        xs = (C.c_void_p * n)(*[it[1] for it in items])
        ys = (C.c_void_p * n)(*[it[2] for it in items])
        rows = (C.c_size_t * n)(*[it[3] if len(it) > 3 else 1 for it in items])
        bs = (C.c_void_p * n)(*[it[4] if len(it) > 4 else None for it in items])
        h = C.c_void_p()
        check(getattr(self.lib, self._create)(ws, xs, rows, bs, ys, n, C.byref(h)))
        self.h = h

    def launch(self, stream=None) -> None:
        check(getattr(self.lib, self._launch)(self.h, stream))

    def free(self) -> None:
        if self.h:
            getattr(self.lib, self._free)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GemmGroup(Group):
    """A list of bf16-MFMA prefill products (Weight, x, y, rows, bias)
    launched together (llmi_hip_gemm_group_*)."""

    _create, _launch, _free = "llmi_hip_gemm_group_create", "llmi_hip_gemm_group_launch", "llmi_hip_gemm_group_free"


class TolGroup(Group):
    """A list of tolerance-mode Q4_0 products (Weight, x, y, rows, bias)
    launched together (llmi_hip_tol_group_*)."""

    _create, _launch, _free = "llmi_hip_tol_group_create", "llmi_hip_tol_group_launch", "llmi_hip_tol_group_free"


class Graph:
    """A captured sequence of _dev calls on the library stream."""

    def __init__(self, record):
        self.lib = init()
        check(self.lib.llmi_hip_graph_begin())
        try:
            record()
        finally:
            g = C.c_void_p()
            rc = self.lib.llmi_hip_graph_end(C.byref(g))
        check(rc)
        self.g = g.value

    def launch(self) -> None:
        check(self.lib.llmi_hip_graph_launch(self.g))

    def __del__(self):
        try:
            self.lib.llmi_hip_graph_destroy(self.g)
        except Exception:
            pass


def synchronize() -> None:
    check(init().llmi_hip_synchronize())

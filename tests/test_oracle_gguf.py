"""The oracle's restatement of gguf::to_quantized (src/model/gguf.cpp:577-640)
pinned three ways: the reference's own known-answer tests
(tests/gguf_test.cpp:389-453), the compiled reference on every fp16 scale
pattern and random codes, and the IEEE binary16 -> binary32 definition (via
numpy) for the scale conversion."""

import numpy as np
import pytest

import oracle as O
import synth

GGUF_Q4_0, GGUF_Q8_0 = 2, 8


def impls():
    out = [("oracle", O.oracle())]
    ref = O.reference()
    if ref is not None:
        out.append(("reference", ref))
    return out


def random_blocks(nblocks: int, gtype: int, seed: int, scales_u16=None) -> np.ndarray:
    """nblocks ggml blocks: fp16 scale (little endian) + codes."""
    qbytes = 32 if gtype == GGUF_Q8_0 else 16
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblocks, 2 + qbytes), dtype=np.uint8)
    if scales_u16 is not None:
        s = np.asarray(scales_u16, dtype=np.uint16)
        raw[:, 0] = (s & 0xFF).astype(np.uint8)
        raw[:, 1] = (s >> 8).astype(np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("name,cpu", impls())
def test_reference_known_answers(name, cpu):
    # gguf_test.cpp:389-416: one Q8_0 block, scale 1.0 (0x3C00), codes 0..31.
    raw = np.array([0x00, 0x3C] + list(range(32)), np.uint8)
    data, scales = cpu.gguf_to_quantized(raw, 1, 32, GGUF_Q8_0)
    assert scales[0] == 1.0
    assert list(cpu.dequantize_row(data, scales, 1, 32, O.Q8_0, 0)) == [float(i) for i in range(32)]
    # gguf_test.cpp:418-453: one Q4_0 block, scale 2.0 (0x4000), byte 0 = 0x91
    # (element 0 nibble 1, element 16 nibble 9), every other nibble 8.
    raw = np.array([0x00, 0x40, 0x91] + [0x88] * 15, np.uint8)
    data, scales = cpu.gguf_to_quantized(raw, 1, 32, GGUF_Q4_0)
    row = cpu.dequantize_row(data, scales, 1, 32, O.Q4_0, 0)
    assert row[0] == -14.0 and row[16] == 2.0
    assert np.count_nonzero(row) == 2


@pytest.mark.parametrize("name,cpu", impls())
def test_rejects_what_the_reference_rejects(name, cpu):
    raw = random_blocks(4, GGUF_Q8_0, 1)
    with pytest.raises(ValueError):
        cpu.gguf_to_quantized(raw, 2, 64, 0)  # F32 tensor type (gguf_test.cpp:455-460)
    if name == "oracle":
        # The boundary takes a byte count: more bytes than the shape needs is
        # an error there.  (Inside a GGUF file the reference sizes the tensor
        # from its shape, so trailing bytes never reach to_quantized.)
        with pytest.raises(ValueError):
            cpu.gguf_to_quantized(raw, 2, 64, GGUF_Q4_0)  # Q8_0-sized bytes declared Q4_0
    with pytest.raises(ValueError):
        cpu.gguf_to_quantized(raw[:-1], 2, 64, GGUF_Q8_0)  # one byte short
    with pytest.raises(ValueError):
        cpu.gguf_to_quantized(random_blocks(1, GGUF_Q8_0, 2), 1, 16, GGUF_Q8_0)  # in % 32 != 0


def test_scale_conversion_is_ieee_half_to_single():
    """Every fp16 pattern as a block scale: the oracle's fp32 scale equals
    numpy's exact conversion (non-NaN), and NaNs keep sign and payload
    (sign | 0x7F800000 | mantissa << 13, the reference's mapping)."""
    h = np.arange(65536, dtype=np.uint32)
    raw = random_blocks(65536, GGUF_Q8_0, 3, scales_u16=h)
    _, scales = O.oracle().gguf_to_quantized(raw, 2048, 32 * 32, GGUF_Q8_0)
    got = scales.view(np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    nan = ((h >> 10) & 0x1F == 0x1F) & (h & 0x3FF != 0)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(got[nan], ((h[nan] & 0x8000) << 16) | 0x7F800000 | ((h[nan] & 0x3FF) << 13))


def test_q4_nibble_placement_brute_force():
    """Each element of a Q4_0 block alone: byte j's low nibble is element j,
    the high nibble element j + 16; the engine keeps element e at byte e/2,
    low nibble when e is even."""
    cpu = O.oracle()
    for e in range(32):
        qs = np.full(16, 0x88, np.uint8)
        j = e % 16
        qs[j] = (qs[j] & 0xF0) | 0x3 if e < 16 else (qs[j] & 0x0F) | 0xD0
        raw = np.concatenate([np.array([0x00, 0x3C], np.uint8), qs])
        data, scales = cpu.gguf_to_quantized(raw, 1, 32, GGUF_Q4_0)
        row = cpu.dequantize_row(data, scales, 1, 32, O.Q4_0, 0)
        want = np.zeros(32, np.float32)
        want[e] = 3 - 8 if e < 16 else 0xD - 8
        assert np.array_equal(row, want), e


@pytest.mark.skipif(O.reference() is None, reason="oracle/_ref was not built (no reference sources)")
@pytest.mark.parametrize("gtype", [GGUF_Q8_0, GGUF_Q4_0])
def test_oracle_matches_compiled_reference(gtype):
    """Bit-exact against the reference's parse + to_quantized on all 65536
    fp16 scales and random codes, and on a Qwen2.5-shaped tensor."""
    orc, ref = O.oracle(), O.reference()
    for out, n_in, seed in ((2048, 32 * 32, 4), (896, 896, 5), (3, 64, 6)):
        nb = out * n_in // 32
        scales = np.arange(nb, dtype=np.uint32) % 65536 if nb >= 65536 else synth.uniform_ids(seed, nb, 65536)
        raw = random_blocks(nb, gtype, seed, scales_u16=scales)
        d1, s1 = orc.gguf_to_quantized(raw, out, n_in, gtype)
        d2, s2 = ref.gguf_to_quantized(raw, out, n_in, gtype)
        assert np.array_equal(d1, d2), (out, n_in)
        assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32)), (out, n_in)

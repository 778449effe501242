"""Device workloads shared by bench.py and the GPU tests, so that what the
bench times is what the tests check.

The shapes are those of BASELINE.json's configurations: the SmolLM2-135M
linear layers (configs[0]-[2]) and the Qwen2.5-0.5B ones (configs[3], [4]),
in the reference's per-layer order (src/model/transformer.cpp:245-291:
q, k, v, o, gate, up, down).
"""

from __future__ import annotations

import llmi_hip as H

SMOL_LAYER = [("q_proj", 576, 576), ("k_proj", 192, 576), ("v_proj", 192, 576), ("o_proj", 576, 576),
              ("gate_proj", 1536, 576), ("up_proj", 1536, 576), ("down_proj", 576, 1536)]
SMOL_HEAD = ("lm_head", 49152, 576)
QWEN_LAYER = [("q_proj", 896, 896), ("k_proj", 128, 896), ("v_proj", 128, 896), ("o_proj", 896, 896),
              ("gate_proj", 4864, 896), ("up_proj", 4864, 896), ("down_proj", 896, 4864)]
QWEN_HEAD = ("lm_head", 151936, 896)

# Which activation each product of a layer reads (transformer.cpp:245-291):
# the normalised state feeds q/k/v, the attention output o_proj, the second
# normalised state gate/up, and silu(gate) * up down_proj.
LAYER_INPUT = {"q_proj": "attn_in", "k_proj": "attn_in", "v_proj": "attn_in", "o_proj": "attn_out",
               "gate_proj": "mlp_in", "up_proj": "mlp_in", "down_proj": "mlp_act"}


def algo_bytes(out: int, n_in: int, qt: int, batch: int) -> int:
    """Packed codes + fp32 scales + x + y of one product, each counted once."""
    return out * H.row_bytes(n_in, qt) + 4 * out * H.nblocks(n_in) + 4 * batch * (n_in + out)


class PrefillProducts:
    """M rows of fp32 activations ~ N(0, 1) against
    every linear layer of `layers` Qwen2.5-0.5B layers, weights ~ N(0, 0.02)
    quantized to `qt` on the GPU.  Each layer has its own four activation
    matrices (LAYER_INPUT), so no two layers share an input; outputs are
    distinct buffers.  `items` are (Weight, x_ptr, y_ptr, rows) for
    H.GemmGroup, all layers in order; `per_layer` the same split by layer.
    `spec[i]` = (layer, name, out, in, x_seed, w_seed) says how product i
    was generated, so a checker can regenerate its operands on the host."""

    def __init__(self, M: int = 512, layers: int = 24, qt: int = H.Q8_0, seed: int = 7000):
        self.M, self.qt = M, qt
        self.weights, self.buffers, self.items, self.per_layer, self.spec = [], [], [], [], []
        self.ys = []
        stage = H.DeviceBuffer(max(o * i for _, o, i in QWEN_LAYER) * 4)
        for layer in range(layers):
            xs = {}
            for name, _, n_in in QWEN_LAYER:
                key = LAYER_INPUT[name]
                if key not in xs:
                    x_seed = seed + 100000 + 16 * layer + len(xs)
                    xb = H.DeviceBuffer(M * n_in * 4)
                    H.synth_normal_dev(xb, M * n_in, x_seed, 0.0, 1.0)
                    xs[key] = (xb, x_seed)
                    self.buffers.append(xb)
            li = []
            for j, (name, out, n_in) in enumerate(QWEN_LAYER):
                w_seed = seed + 16 * layer + j
                H.synth_normal_dev(stage, out * n_in, w_seed, 0.0, 0.02)
                w = H.Weight.quantize_dev(stage.ptr, out, n_in, qt)
                y = H.DeviceBuffer(M * out * 4)
                self.weights.append(w)
                self.buffers.append(y)
                self.ys.append(y)
                xb, x_seed = xs[LAYER_INPUT[name]]
                li.append((w, xb.ptr, y.ptr, M))
                self.spec.append((layer, name, out, n_in, x_seed, w_seed))
            self.items += li
            self.per_layer.append(li)
        stage.free()

    def flops(self) -> float:
        return 2.0 * self.M * sum(s[2] * s[3] for s in self.spec)

    def output(self, i: int):
        """The fp32 output of product i (host copy)."""
        import numpy as np

        return self.ys[i].download(np.float32)

    def free(self) -> None:
        for w in self.weights:
            w.free()
        for b in self.buffers:
            b.free()
        self.weights, self.buffers, self.items, self.per_layer, self.ys = [], [], [], [], []

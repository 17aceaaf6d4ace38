"""Party-local share GEMMs of a Qwen3 forward (Transformer::project_many /
project_joint_many, model.hpp:66-126; shapes model.hpp:63-64).

Per layer the reference runs four local products on one party's shares:

* joint q/k/v: x_attn [M][hidden] . [q | k | v]^T, out q_heads*head_dim + 2*kv_heads*head_dim
* o:           x_o [M][q_heads*head_dim] . W_o^T, out hidden
* joint gate/up: x_mlp [M][hidden] . [gate | up]^T, out 2*intermediate
* down:        x_down [M][intermediate] . W_down^T, out hidden

with weights stored [out][in] as in the reference's .npy files.  Between these
products the real chain runs two-party protocol steps (attention, SiLU,
truncation), so every product here gets its own seeded input shares.  Weights
are int8 (or int32 f12 words) with an exact per-output-channel left shift
``<< s_c mod 2^64`` standing in for a power-of-two scale.  All 4 x layers
products of a forward go to the device as one praghip_share_gemm_batch call.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from ._lib import GemmDesc, check, lib
from ._util import stream_handle
from . import synth


@dataclass(frozen=True)
class Qwen3Shape:
    layers: int = 28
    hidden: int = 1024
    q_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 3072

    def products(self):
        """(name, in_features, out_features) of one layer's local products."""
        q = self.q_heads * self.head_dim
        kv = self.kv_heads * self.head_dim
        return [("qkv", self.hidden, q + 2 * kv), ("o", q, self.hidden),
                ("gate_up", self.hidden, 2 * self.intermediate), ("down", self.intermediate, self.hidden)]

    def ops_per_layer(self, rows: int) -> int:
        return sum(2 * rows * k * n for _, k, n in self.products())


QWEN3_0_6B = Qwen3Shape()


class Qwen3LocalGemms:
    """Device-resident weights, shifts, input shares and outputs of every local
    product of a forward over `rows` tokens, with seeded synthetic contents."""

    def __init__(self, rows: int = 512, shape: Qwen3Shape = QWEN3_0_6B, seed: int = 0x5052414700000005,
                 mask_bits: int = 64, shifts: bool = True, device: str = "cuda"):
        import torch
        self.rows, self.shape, self.mask_bits = rows, shape, mask_bits
        self.device = torch.device(device)
        self.layers = []
        for layer in range(shape.layers):
            entry = {}
            for p, (name, k, n) in enumerate(shape.products()):
                s = seed + ((layer * 8 + p) << 8)
                x = torch.empty((rows, k), dtype=torch.int64, device=self.device)
                w = torch.empty((n, k), dtype=torch.int8, device=self.device)
                sh = torch.empty(n, dtype=torch.int8, device=self.device) if shifts else None
                y = torch.empty((rows, n), dtype=torch.int64, device=self.device)
                synth.fill_u64(x, s + 1)
                synth.fill_i8(w, s + 2)
                if sh is not None:
                    synth.fill_shift(sh, s + 3)
                entry[name] = (x, w, sh, y)
            self.layers.append(entry)
        descs = []
        for entry in self.layers:
            for name, _, _ in shape.products():
                x, w, sh, y = entry[name]
                descs.append(GemmDesc(x.data_ptr(), w.data_ptr(), None if sh is None else sh.data_ptr(),
                                      y.data_ptr(), rows, x.shape[1], w.shape[0], 8, mask_bits))
        self._descs = (GemmDesc * len(descs))(*descs)

    @property
    def ops(self) -> int:
        return self.shape.layers * self.shape.ops_per_layer(self.rows)

    def forward(self, stream=None):
        """Every local product of the forward, in layer order, on one stream."""
        check(lib().praghip_share_gemm_batch(self.device.index or 0, ctypes.cast(self._descs, ctypes.c_void_p),
                                             len(self._descs), stream_handle(stream)))

    def product(self, layer: int, name: str):
        """(x, w, shifts, y) tensors of one product."""
        return self.layers[layer][name]

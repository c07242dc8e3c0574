"""TurboQuant host-side configuration and tables (mirror of crates/fracture-core/src/
turboquant.rs): per-layer bit widths, packed sizes, Lloyd-Max codebooks and Haar rotations.

The tables come from libfracture_hip.so's host helpers, which restate the reference's CPU
code operation for operation (so the uploaded tables are the reference's tables).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib

BLOCK_SIZE = 16  # tokens per page (crates/fracture-engine/src/paged_kv_cache.rs:7)

# The reference validates {2, 4, 8} (turboquant.rs:37-57); this backend also packs 3-bit
# codes (the MSB-first bitstream), which the reference's solver supports but its kernels do
# not.
VALID_BITS = (2, 3, 4, 8)


@dataclass
class TurboQuantConfig:
    """TurboQuantConfig (turboquant.rs:7-151)."""

    key_bits: int = 4
    value_bits: int = 2
    protected_bits: int = 8
    protected_layers: int = 0
    residual_tokens: int = 0
    seed: int = 42

    def validate(self) -> None:
        for name in ("key_bits", "value_bits", "protected_bits"):
            v = getattr(self, name)
            if v not in VALID_BITS:
                raise ValueError(f"TurboQuant {name} must be one of {VALID_BITS}, got {v}")

    def is_protected(self, layer: int, num_layers: int) -> bool:
        return self.protected_layers > 0 and (
            layer < self.protected_layers or layer >= max(num_layers - self.protected_layers, 0))

    def key_bits_for_layer(self, layer: int, num_layers: int) -> int:
        return self.protected_bits if self.is_protected(layer, num_layers) else self.key_bits

    def value_bits_for_layer(self, layer: int, num_layers: int) -> int:
        return self.protected_bits if self.is_protected(layer, num_layers) else self.value_bits

    def distinct_bit_widths(self) -> list[int]:
        bits = {self.key_bits, self.value_bits}
        if self.protected_layers > 0:
            bits.add(self.protected_bits)
        return sorted(bits)

    @staticmethod
    def packed_dim_per_head(head_dim: int, bits: int) -> int:
        return int(_lib.load().fhip_tq_packed_dim_per_head(head_dim, bits))

    @staticmethod
    def bytes_per_block_layer(num_kv_heads: int, head_dim: int, key_bits: int,
                              value_bits: int) -> int:
        pk = TurboQuantConfig.packed_dim_per_head(head_dim, key_bits)
        pv = TurboQuantConfig.packed_dim_per_head(head_dim, value_bits)
        return BLOCK_SIZE * num_kv_heads * (pk + pv) + 2 * BLOCK_SIZE * num_kv_heads * 2

    def bytes_per_block_total(self, num_layers: int, num_kv_heads: int, head_dim: int) -> int:
        return sum(self.bytes_per_block_layer(num_kv_heads, head_dim,
                                              self.key_bits_for_layer(l, num_layers),
                                              self.value_bits_for_layer(l, num_layers))
                   for l in range(num_layers))

    def compute_num_blocks(self, gpu_available: int, scratch_reserve: int, num_layers: int,
                           num_kv_heads: int, head_dim: int) -> int:
        budget = max(gpu_available - scratch_reserve, 0)
        per = self.bytes_per_block_total(num_layers, num_kv_heads, head_dim)
        return budget // per if per else 0


def codebook(dim: int, bits: int):
    """LloydMaxCodebook::compute: (centroids f32[2^bits], boundaries f32[2^bits - 1])."""
    L = 1 << bits
    c = np.empty(L, np.float32)
    b = np.empty(max(L - 1, 1), np.float32)
    code = _lib.load().fhip_tq_codebook(dim, bits, c.ctypes.data, b.ctypes.data)
    if code != 0:
        raise ValueError(f"codebook(dim={dim}, bits={bits}) rejected")
    return c, b[: L - 1]


def rotation_matrix(d: int, seed: int) -> np.ndarray:
    """generate_rotation_matrix: row-major f32 [d, d]."""
    q = np.empty((d, d), np.float32)
    code = _lib.load().fhip_tq_rotation_matrix(d, seed, q.ctypes.data)
    if code != 0:
        raise ValueError(f"rotation_matrix(d={d}) rejected")
    return q


def rotation_seeds(base_seed: int, layer: int):
    k = C.c_uint64()
    v = C.c_uint64()
    _lib.load().fhip_tq_rotation_seeds(base_seed, layer, C.byref(k), C.byref(v))
    return k.value, v.value


def rope_freqs(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    _lib.load().fhip_rope_freqs(head_dim, theta, out.ctypes.data)
    return out

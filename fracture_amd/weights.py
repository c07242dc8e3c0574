"""Llama weights from a GGUF file onto a HipBackend, the way fracture-gguf's WeightStore
uploads them (crates/fracture-gguf/src/weight_store.rs:110-186): every tensor as an fp16 device
tensor in its stored [out_features, in_features] layout, with the Q and K projections'
llama.cpp RoPE interleave undone at load time (reverse_qk_permutation, weight_store.rs:139-159).

The GGUF reader covers the container (GGUF v2/v3: header, metadata, tensor infos, aligned data
section) and the F16 / F32 tensor types the engine's fp16 path uses.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from .backend import DType, DeviceTensor, HipBackend

_GGML_TYPES = {0: np.float32, 1: np.float16}
# metadata value types of the GGUF format
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
            11: "<q", 12: "<d"}


def read_gguf(path) -> tuple[dict, dict]:
    """(metadata, {tensor name: ndarray}) of a GGUF file; arrays are in row-major order
    (the file's ne[0] is the innermost dimension)."""
    raw = Path(path).read_bytes()
    if raw[:4] != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    off = 4

    def take(fmt):
        nonlocal off
        v = struct.unpack_from(fmt, raw, off)
        off += struct.calcsize(fmt)
        return v[0]

    def gstr():
        nonlocal off
        n = take("<Q")
        s = raw[off:off + n].decode("utf-8", errors="replace")
        off += n
        return s

    def value(t):
        if t in _SCALARS:
            return take(_SCALARS[t])
        if t == 8:
            return gstr()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        raise ValueError(f"GGUF metadata value type {t}")

    version = take("<I")
    if version not in (2, 3):
        raise ValueError(f"GGUF version {version}")
    n_tensors, n_kv = take("<Q"), take("<Q")
    meta = {}
    for _ in range(n_kv):
        k = gstr()
        meta[k] = value(take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = gstr()
        dims = [take("<Q") for _ in range(take("<I"))]
        infos.append((name, dims, take("<I"), take("<Q")))
    align = int(meta.get("general.alignment", 32))
    data0 = (off + align - 1) // align * align
    tensors = {}
    for name, dims, gt, toff in infos:
        if gt not in _GGML_TYPES:
            raise ValueError(f"tensor {name}: GGML type {gt} is not F16 or F32")
        n = int(np.prod(dims)) if dims else 1
        arr = np.frombuffer(raw, dtype=_GGML_TYPES[gt], count=n, offset=data0 + toff)
        tensors[name] = arr.reshape(list(reversed(dims))).copy()
    return meta, tensors


def reverse_qk_permutation(w: np.ndarray, num_heads: int, head_dim: int) -> np.ndarray:
    """Undo llama.cpp's RoPE interleave of a Q or K weight [num_heads * head_dim, hidden]:
    within each head, stored row 2i is row i and stored row 2i + 1 is row i + head_dim / 2
    (weight_store.rs:139-159)."""
    if w.shape[0] != num_heads * head_dim or head_dim % 2:
        raise ValueError(f"weight rows {w.shape[0]} != {num_heads} heads x {head_dim}")
    half = head_dim // 2
    h = w.reshape(num_heads, head_dim, -1)
    out = np.empty_like(h)
    out[:, :half] = h[:, 0::2]
    out[:, half:] = h[:, 1::2]
    return out.reshape(w.shape)


@dataclass
class LayerWeights:
    """One decoder layer's device tensors (weight_store.rs LayerWeights)."""

    attn_norm: DeviceTensor
    q_proj: DeviceTensor
    k_proj: DeviceTensor
    v_proj: DeviceTensor
    o_proj: DeviceTensor
    ffn_norm: DeviceTensor
    gate_proj: DeviceTensor
    up_proj: DeviceTensor
    down_proj: DeviceTensor


@dataclass
class LlamaWeights:
    token_embedding: DeviceTensor
    output_norm: DeviceTensor
    lm_head: DeviceTensor
    layers: list = field(default_factory=list)

    def tensors(self):
        yield from (self.token_embedding, self.output_norm, self.lm_head)
        for lw in self.layers:
            yield from vars(lw).values()


def upload_llama(backend: HipBackend, tensors: dict, num_layers: int, num_q_heads: int,
                 num_kv_heads: int, head_dim: int) -> LlamaWeights:
    """Upload GGUF-named llama tensors as fp16 device tensors. Q and K are un-permuted; the
    output head falls back to the token embedding when the file ties them."""

    def up(a: np.ndarray) -> DeviceTensor:
        a = np.ascontiguousarray(a, dtype=np.float16)
        t = backend.alloc(list(a.shape), DType.FP16)
        backend.copy_to_device(t, a)
        return t

    emb = tensors["token_embd.weight"]
    w = LlamaWeights(up(emb), up(tensors["output_norm.weight"]),
                     up(tensors.get("output.weight", emb)))
    for i in range(num_layers):
        g = lambda n: tensors[f"blk.{i}.{n}.weight"]  # noqa: E731
        w.layers.append(LayerWeights(
            attn_norm=up(g("attn_norm")),
            q_proj=up(reverse_qk_permutation(g("attn_q"), num_q_heads, head_dim)),
            k_proj=up(reverse_qk_permutation(g("attn_k"), num_kv_heads, head_dim)),
            v_proj=up(g("attn_v")), o_proj=up(g("attn_output")), ffn_norm=up(g("ffn_norm")),
            gate_proj=up(g("ffn_gate")), up_proj=up(g("ffn_up")), down_proj=up(g("ffn_down"))))
    return w

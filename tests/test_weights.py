"""GGUF reading and the load-time Q/K un-permutation (weight_store.rs:110-186), on the CPU.

The un-permutation is pinned by the reference's own dumps: with it, post_attn_norm · Wqᵀ and
post_attn_norm · Wkᵀ reproduce the fixture's q and k for every layer; without it they do not.
"""
import struct

import numpy as np
import pytest

from fracture_amd.weights import read_gguf, reverse_qk_permutation


def gguf_bytes(meta, tensors, align=32):
    """A GGUF v3 file: header, metadata, tensor infos, aligned data section."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta))
    for k, v in meta.items():
        out += s(k)
        if isinstance(v, str):
            out += struct.pack("<I", 8) + s(v)
        elif isinstance(v, list):
            out += struct.pack("<IIQ", 9, 4, len(v)) + b"".join(struct.pack("<I", e) for e in v)
        else:
            out += struct.pack("<II", 4, v)
    data, infos, at = b"", b"", 0
    for name, a in tensors.items():
        gt = {np.float32: 0, np.float16: 1}[a.dtype.type]
        infos += s(name) + struct.pack("<I", a.ndim)
        infos += b"".join(struct.pack("<Q", d) for d in reversed(a.shape))
        infos += struct.pack("<IQ", gt, at)
        blob = a.tobytes()
        pad = (-len(blob)) % align
        data += blob + b"\0" * pad
        at += len(blob) + pad
    out += infos
    out += b"\0" * ((-len(out)) % align)
    return out + data


def test_read_gguf_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    t = {"a.weight": rng.standard_normal((3, 5)).astype(np.float16),
         "b.bias": rng.standard_normal(7).astype(np.float32)}
    meta = {"general.architecture": "llama", "llama.block_count": 4, "x.list": [1, 2, 3]}
    p = tmp_path / "m.gguf"
    p.write_bytes(gguf_bytes(meta, t))
    m, got = read_gguf(p)
    assert m == meta
    for k, v in t.items():
        assert got[k].dtype == v.dtype and np.array_equal(got[k], v)
    p.write_bytes(b"NOPE" + p.read_bytes()[4:])
    with pytest.raises(ValueError):
        read_gguf(p)


def test_reverse_permutation_is_the_inverse_of_the_interleave():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((2 * 8, 5)).astype(np.float16)
    # llama.cpp's interleave: row i of a head goes to 2i, row i + half to 2i + 1
    inter = w.reshape(2, 2, 4, 5).transpose(0, 2, 1, 3).reshape(16, 5)
    assert np.array_equal(reverse_qk_permutation(inter, 2, 8), w)
    with pytest.raises(ValueError):
        reverse_qk_permutation(w, 3, 8)


@pytest.mark.parametrize("layer", [0, 1, 2, 3])
def test_unpermuted_projections_reproduce_the_reference_dumps(golden, layer):
    cfg = golden["config"]
    hd = cfg["head_dim"]
    x = golden[f"prompt_0/layer_{layer:02d}/post_attn_norm"][0].astype(np.float64)
    for name, key, heads in (("attn_q", "q", cfg["num_q_heads"]),
                             ("attn_k", "k", cfg["num_kv_heads"])):
        raw = golden[f"weights/blk.{layer}.{name}.weight"]
        want = golden[f"prompt_0/layer_{layer:02d}/{key}"][0]
        fixed = reverse_qk_permutation(raw, heads, hd).astype(np.float64)
        np.testing.assert_allclose(x @ fixed.T, want, rtol=5e-3, atol=5e-3)
        assert np.abs(x @ raw.astype(np.float64).T - want).max() > 1.0

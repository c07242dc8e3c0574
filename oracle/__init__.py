"""TEST INFRASTRUCTURE ONLY: numpy front end of the CPU oracle (``oracle.c``).

The oracle restates the reference's CPU arithmetic for the hot path (each C function
cites the reference file:line it follows). Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, as the checker or as the timed
CPU baseline; the product (``fracture_amd``) never does.

Parity status of each function and the checks that pin it are listed in the header of
``oracle.c``; ``build()`` compiles ``liboracle.so`` with the recipe in ``Makefile``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("FHIP_ORACLE_LIBRARY", HERE / "liboracle.so"))

_lib = None

F16, F32, BF16 = 0, 1, 2


def build() -> Path:
    """Compile liboracle.so with gcc (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p
I64 = C.c_int64


def _declare(L: C.CDLL) -> None:
    sig = {
        "o_f32_to_f16": (C.c_uint16, [C.c_float]),
        "o_f16_to_f32": (C.c_float, [C.c_uint16]),
        "o_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "o_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "o_f32_to_f16_array": (None, [P, P, I64]),
        "o_f16_to_f32_array": (None, [P, P, I64]),
        "o_add": (None, [P, P, P, I64, C.c_int]),
        "o_rmsnorm": (None, [P, P, C.c_float, P, I64, I64, C.c_int]),
        "o_add_rmsnorm": (None, [P, P, P, C.c_float, P, I64, I64, C.c_int]),
        "o_silu_mul": (None, [P, P, P, I64, C.c_int]),
        "o_rope_freqs": (None, [C.c_int, C.c_double, P]),
        "o_rope": (None, [P, P, P, I64, I64, I64, C.c_int]),
        "o_embedding": (None, [P, P, P, I64, I64, I64, C.c_int]),
        "o_argmax": (C.c_int, [P, I64, P]),
        "o_softmax": (None, [P, P, I64, C.c_float]),
        "o_softmax_rows": (None, [P, P, I64, I64, C.c_float]),
        "o_argmax_rows": (C.c_int, [P, I64, I64, P, P]),
        "o_lloyd_max": (C.c_int, [C.c_int, C.c_int, P, P]),
        "o_xoshiro_outputs": (None, [C.c_uint64, C.c_int, P]),
        "o_xoshiro_outputs_state": (None, [P, C.c_int, P]),
        "o_splitmix_state": (None, [C.c_uint64, P]),
        "o_gaussian_matrix": (None, [C.c_int, C.c_uint64, P]),
        "o_rotation": (None, [C.c_int, C.c_uint64, P]),
        "o_tq_code": (C.c_int, [C.c_float, P, C.c_int]),
        "o_tq_codes": (None, [P, I64, P, C.c_int, P]),
        "o_tq_pack_row": (None, [P, C.c_int, C.c_int, P]),
        "o_tq_pack_row_bitstream": (None, [P, C.c_int, C.c_int, P]),
        "o_tq_unpack": (C.c_int, [P, C.c_int, C.c_int]),
        "o_tq_quantize_pack": (None, [P, I64, C.c_int, P, C.c_int, C.c_int, P]),
        "o_tq_rotate": (None, [P, I64, C.c_int, P, P, P]),
        "o_tq_compress": (None, [P, I64, C.c_int, P, P, C.c_int, C.c_int, P, P, P]),
        "o_tq_dequant": (None, [P, P, I64, C.c_int, P, P, C.c_int, P]),
        "o_tq_attention": (None, [P, P, C.c_int, P, P, P, P, I64, I64, I64, I64, P, P, P, P,
                                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P]),
        "o_tq_attention_heads": (None, [P, P, C.c_int, P, P, P, P, I64, I64, I64, I64, P, P, P,
                                        P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.c_int, P]),
        "o_paged_attention": (None, [P, P, C.c_int, P, P, I64, I64, C.c_int, C.c_int, C.c_int,
                                     P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _dt(a: np.ndarray) -> int:
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:  # bf16 bit patterns
        return BF16
    raise TypeError(f"unsupported dtype {a.dtype}")


# -------------------------------------------------------------------------------------
# conversions
# -------------------------------------------------------------------------------------
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().o_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.array([lib().o_f32_to_bf16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------------------------------------
# elementwise
# -------------------------------------------------------------------------------------
def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b, dtype=a.dtype)
    out = np.empty_like(a)
    lib().o_add(_p(a), _p(b), _p(out), a.size, _dt(a))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=x.dtype)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().o_rmsnorm(_p(x), _p(w), eps, _p(out), x.size // cols, cols, _dt(x))
    return out


def add_rmsnorm(h: np.ndarray, d: np.ndarray, w: np.ndarray, eps: float):
    """Returns (new residual, normed)."""
    h = np.array(h, copy=True, order="C")
    d = np.ascontiguousarray(d, dtype=h.dtype)
    w = np.ascontiguousarray(w, dtype=h.dtype)
    cols = h.shape[-1]
    out = np.empty_like(h)
    lib().o_add_rmsnorm(_p(h), _p(d), _p(w), eps, _p(out), h.size // cols, cols, _dt(h))
    return h, out


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g)
    u = np.ascontiguousarray(u, dtype=g.dtype)
    out = np.empty_like(g)
    lib().o_silu_mul(_p(g), _p(u), _p(out), g.size, _dt(g))
    return out


def rope_freqs(hd: int, theta: float) -> np.ndarray:
    out = np.empty(hd // 2, np.float32)
    lib().o_rope_freqs(hd, theta, _p(out))
    return out


def rope(x: np.ndarray, positions: np.ndarray, freqs: np.ndarray) -> np.ndarray:
    """x [T, heads, hd]; returns the rotated copy."""
    x = np.array(x, copy=True, order="C")
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    fr = np.ascontiguousarray(freqs, dtype=np.float32)
    T, H, hd = x.shape
    lib().o_rope(_p(x), _p(pos), _p(fr), T, H, hd, _dt(x))
    return x


def embedding(table: np.ndarray, ids: np.ndarray) -> np.ndarray:
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    V, Hd = table.shape
    out = np.empty((ids.size, Hd), table.dtype)
    lib().o_embedding(_p(table), _p(ids), _p(out), ids.size, Hd, V, table.itemsize)
    return out


# -------------------------------------------------------------------------------------
# sampler
# -------------------------------------------------------------------------------------
ARGMAX_STATUS = {0: None, 1: "empty logits", 2: "NaN in logits", 3: "Inf in logits"}


def argmax(logits: np.ndarray):
    """Returns (index or -1, error message or None), as Sampler::sample's greedy branch."""
    l = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(1, np.int64)
    st = lib().o_argmax(_p(l), l.size, _p(idx))
    return (int(idx[0]) if st == 0 else -1), ARGMAX_STATUS[st]


def argmax_rows(logits: np.ndarray):
    l = np.ascontiguousarray(logits, dtype=np.float32)
    rows, cols = l.shape
    idx = np.empty(rows, np.int64)
    status = np.empty(rows, np.int32)
    lib().o_argmax_rows(_p(l), rows, cols, _p(idx), _p(status))
    return idx, status


def softmax_rows(logits: np.ndarray, temperature: float = 1.0) -> np.ndarray:
    l = np.ascontiguousarray(logits, dtype=np.float32)
    rows, cols = l.reshape(-1, l.shape[-1]).shape
    out = np.empty_like(l)
    lib().o_softmax_rows(_p(l), _p(out), rows, cols, temperature)
    return out


# -------------------------------------------------------------------------------------
# TurboQuant
# -------------------------------------------------------------------------------------
def lloyd_max(dim: int, bits: int):
    """(centroids f32[2^bits], boundaries f32[2^bits - 1], iterations)."""
    L = 1 << bits
    c = np.empty(L, np.float32)
    b = np.empty(max(L - 1, 1), np.float32)
    it = lib().o_lloyd_max(dim, bits, _p(c), _p(b))
    return c, b[: L - 1], it


def xoshiro_outputs(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().o_xoshiro_outputs(seed, n, _p(out))
    return out


def xoshiro_outputs_state(state, n: int) -> np.ndarray:
    st = np.ascontiguousarray(np.array(state, dtype=np.uint64))
    out = np.empty(n, np.uint64)
    lib().o_xoshiro_outputs_state(_p(st), n, _p(out))
    return out


def splitmix_state(seed: int) -> np.ndarray:
    out = np.empty(4, np.uint64)
    lib().o_splitmix_state(seed, _p(out))
    return out


def gaussian_matrix(d: int, seed: int) -> np.ndarray:
    g = np.empty((d, d), np.float32)
    lib().o_gaussian_matrix(d, seed, _p(g))
    return g


def rotation(d: int, seed: int) -> np.ndarray:
    q = np.empty((d, d), np.float32)
    lib().o_rotation(d, seed, _p(q))
    return q


def rotation_seeds(base: int, layer: int):
    return base + layer * 1000, base + layer * 1000 + 500


def packed_dim(hd: int, bits: int) -> int:
    return (hd * bits + 7) // 8


def tq_codes(y: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    out = np.empty(y.shape, np.uint8)
    lib().o_tq_codes(_p(y), y.size, _p(c), c.size, _p(out))
    return out


def tq_pack_rows(codes: np.ndarray, bits: int, bitstream: bool = False) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    rows, hd = codes.reshape(-1, codes.shape[-1]).shape
    pd = packed_dim(hd, bits)
    out = np.empty((rows, pd), np.uint8)
    fn = lib().o_tq_pack_row_bitstream if bitstream else lib().o_tq_pack_row
    flat = codes.reshape(rows, hd)
    for r in range(rows):
        fn(_p(flat[r]), hd, bits, _p(out[r]))
    return out


def tq_unpack_rows(packed: np.ndarray, hd: int, bits: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    rows = packed.shape[0]
    out = np.empty((rows, hd), np.uint8)
    for r in range(rows):
        row = packed[r]
        for d in range(hd):
            out[r, d] = lib().o_tq_unpack(_p(row), d, bits)
    return out


def tq_quantize_pack(y: np.ndarray, centroids: np.ndarray, bits: int) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    hd = y.shape[-1]
    rows = y.size // hd
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    out = np.empty((rows, packed_dim(hd, bits)), np.uint8)
    lib().o_tq_quantize_pack(_p(y), rows, hd, _p(c), c.size, bits, _p(out))
    return out


def tq_rotate(x16: np.ndarray, rot: np.ndarray):
    """x16 [..., hd] float16 -> (y f32 [rows, hd], norms f16 [rows])."""
    x = np.ascontiguousarray(x16, dtype=np.float16)
    hd = x.shape[-1]
    rows = x.size // hd
    r = np.ascontiguousarray(rot, dtype=np.float32)
    y = np.empty((rows, hd), np.float32)
    n = np.empty(rows, np.float16)
    lib().o_tq_rotate(_p(x), rows, hd, _p(r), _p(y), _p(n))
    return y, n


def tq_compress(x16: np.ndarray, rot: np.ndarray, centroids: np.ndarray, bits: int):
    """Returns (packed u8 [rows, pd], norms f16 [rows], y f32 [rows, hd])."""
    x = np.ascontiguousarray(x16, dtype=np.float16)
    hd = x.shape[-1]
    rows = x.size // hd
    r = np.ascontiguousarray(rot, dtype=np.float32)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    packed = np.empty((rows, packed_dim(hd, bits)), np.uint8)
    norms = np.empty(rows, np.float16)
    y = np.empty((rows, hd), np.float32)
    lib().o_tq_compress(_p(x), rows, hd, _p(r), _p(c), c.size, bits, _p(packed), _p(norms), _p(y))
    return packed, norms, y


def tq_dequant(packed: np.ndarray, norms: np.ndarray, rot: np.ndarray, centroids: np.ndarray,
               bits: int, hd: int) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    n = np.ascontiguousarray(norms, dtype=np.float16).ravel()
    rows = n.size
    r = np.ascontiguousarray(rot, dtype=np.float32)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    out = np.empty((rows, hd), np.float16)
    lib().o_tq_dequant(_p(p), _p(n), rows, hd, _p(r), _p(c), bits, _p(out))
    return out


def tq_attention(q16, block_table, causal_len, kp, kn, vp, vn, krot, vrot, kc, vc, kbits, vbits,
                 kvh, heads=None):
    """One query token: q16 [qh, hd] float16; pools as uint8 arrays [pages, ...].
    heads=(h0, h1) computes query heads h0..h1-1 only; the other output rows are zero."""
    q = np.ascontiguousarray(q16, dtype=np.float16)
    qh, hd = q.shape
    h0, h1 = (0, qh) if heads is None else heads
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    kp, kn, vp, vn = (np.ascontiguousarray(a) for a in (kp, kn, vp, vn))
    out = np.zeros((qh, hd), np.float16)
    lib().o_tq_attention_heads(
        _p(q), _p(bt), int(causal_len), _p(kp), _p(kn), _p(vp), _p(vn),
        kp[0].nbytes, kn[0].nbytes, vp[0].nbytes, vn[0].nbytes,
        _p(np.ascontiguousarray(krot, np.float32)), _p(np.ascontiguousarray(vrot, np.float32)),
        _p(np.ascontiguousarray(kc, np.float32)), _p(np.ascontiguousarray(vc, np.float32)),
        kbits, vbits, qh, kvh, hd, int(h0), int(h1), _p(out))
    return out


def paged_attention(q16, block_table, causal_len, kpool, vpool, kvh):
    """One query token over FP16 pages: q16 [qh, hd] float16; kpool/vpool [pages, 16, kvh, hd]
    float16 (any page shape whose rows are [16][kvh][hd])."""
    q = np.ascontiguousarray(q16, dtype=np.float16)
    qh, hd = q.shape
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    kp = np.ascontiguousarray(kpool, dtype=np.float16)
    vp = np.ascontiguousarray(vpool, dtype=np.float16)
    out = np.empty((qh, hd), np.float16)
    lib().o_paged_attention(_p(q), _p(bt), int(causal_len), _p(kp), _p(vp), kp[0].nbytes,
                            vp[0].nbytes, qh, kvh, hd, _p(out))
    return out

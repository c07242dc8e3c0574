"""ctypes binding of libfracture_hip.so (the C ABI declared in include/fracture_hip.h).

The library is built in-tree by ``python -m fracture_amd.build``. Loading fails loudly
when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("FHIP_LIBRARY", PKG / "libfracture_hip.so"))
HEADER = PKG.parent / "include" / "fracture_hip.h"

P = C.c_void_p
I = C.c_int
I64 = C.c_int64
U64 = C.c_uint64
SZ = C.c_size_t
F = C.c_float
D = C.c_double

MAX_DIMS = 8


class FhipTensor(C.Structure):
    """fhip_tensor: the C mirror of fracture_core::DeviceTensor."""

    _fields_ = [("id", U64), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", U64 * MAX_DIMS)]


TP = C.POINTER(FhipTensor)

SIGNATURES = {
    # raw launchers (ffi.rs counterparts)
    "fhip_launch_rmsnorm": (I, [P, P, P, F, I, I, P]),
    "fhip_launch_rope": (I, [P, P, P, P, I, I, I, I, P]),
    "fhip_launch_silu_mul": (I, [P, P, P, I, P]),
    "fhip_launch_embedding": (I, [P, P, P, I, I, I, P]),
    "fhip_launch_add": (I, [P, P, P, I, P]),
    "fhip_launch_turboquant_compress": (I, [P, P, P, P, P, I, I, I, I, I, I, P]),
    "fhip_launch_turboquant_decompress": (I, [P, P, P, P, P, I, I, I, I, I, P]),
    "fhip_launch_attention_paged_tq": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I,
                                           I, I, I, I, P]),
    "fhip_launch_paged_attention": (I, [P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "fhip_launch_attention": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "fhip_launch_matmul": (I, [P, P, P, I, I, I, P]),
    # additive raw launchers
    "fhip_launch_attention_paged_tq_ws": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I,
                                              I, I, I, I, P, SZ, P]),
    "fhip_launch_paged_attention_ws": (I, [P, P, P, P, P, I, I, I, I, I, I, I, P, SZ, P]),
    "fhip_launch_attention_paged_tq_noalloc": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I,
                                                   I, I, I, I, I, I, P]),
    "fhip_launch_rmsnorm_ex": (I, [P, P, P, F, I, I, I, P]),
    # measurement probes
    "fhip_probe_empty": (I, [I, P]),
    "fhip_probe_stream": (I, [P, I, P, I, I64, P, I, P]),
    "fhip_launch_add_ex": (I, [P, P, P, I64, I, P]),
    "fhip_launch_silu_mul_ex": (I, [P, P, P, I64, I, P]),
    "fhip_launch_rope_ex": (I, [P, P, P, P, I, I, I, I, I, P]),
    "fhip_launch_embedding_ex": (I, [P, P, P, I, I, I, I, P]),
    "fhip_launch_add_rmsnorm": (I, [P, P, P, F, P, I, I, I, P]),
    "fhip_rows_workspace_bytes": (SZ, [I, I]),
    "fhip_launch_softmax_rows": (I, [P, P, I, I, F, P, P]),
    "fhip_launch_argmax_rows": (I, [P, P, P, I, I, P, P]),
    "fhip_launch_softmax_argmax_rows": (I, [P, P, P, P, I, I, F, P, P]),
    "fhip_launch_tq_quantize_pack": (I, [P, P, I, I, P, I, I, I, P]),
    "fhip_launch_tq_rotate": (I, [P, P, P, P, I, I, P]),
    "fhip_launch_tq_compress_pages": (I, [P, P, P, I, I, P, P, I64, I64, P, I, I, I, I, I, P]),
    "fhip_launch_tq_dequant": (I, [P, P, P, P, I, P, I, I, I, I, I, P]),
    "fhip_launch_tq_compress_page_ptrs": (I, [P, P, P, I, I, P, P, P, I, I, I, I, I, P]),
    "fhip_launch_tq_compress_page_ptrs_planned": (I, [P, P, P, P, P, I, I, I, I, P]),
    "fhip_tq_plan_create": (I, [P, P, I, I, I, P, C.POINTER(P)]),
    "fhip_tq_plan_destroy": (None, [P]),
    "fhip_launch_tq_compress_planned": (I, [P, P, P, P, I, I, P]),
    "fhip_launch_tq_compress_pages_planned": (I, [P, P, P, P, I64, I64, P, I, I, I, I, P]),
    "fhip_launch_tq_dequant_planned": (I, [P, P, P, P, I, I, P]),
    "fhip_launch_tq_compress_kv_planned": (I, [P, P, P, P, P, P, P, P, I, I, P]),
    "fhip_launch_tq_compress_kv_page_ptrs_planned": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I,
                                                         P]),
    "fhip_launch_tq_dequant_kv_planned": (I, [P, P, P, P, P, P, P, P, I, I, P]),
    "fhip_attention_tq_workspace_bytes": (SZ, [I, I, I, I]),
    "fhip_launch_attention_tq_decode": (I, [P, P, P, P, I, I, I, P, P, P, P, I64, I64, I64, I64,
                                            P, P, P, P, I, I, I, I, I, P, P]),
    "fhip_launch_attention_tq_decode_ptrs": (I, [P, P, P, P, I, I, I, P, P, P, P, P, P, P, P, I,
                                                 I, I, I, I, P, P]),
    "fhip_attention_paged_workspace_bytes": (SZ, [I, I, I, I]),
    "fhip_launch_attention_paged_decode": (I, [P, P, P, P, I, I, I, P, P, I64, I64, I, I, I, P,
                                               P]),
    # handle runtime (Backend trait mirror)
    "fhip_last_error": (C.c_char_p, []),
    "fhip_backend_create": (I, [I, C.POINTER(P)]),
    "fhip_backend_destroy": (None, [P]),
    "fhip_get_ptr": (I, [P, U64, C.POINTER(P)]),
    "fhip_stream": (P, [P]),
    "fhip_precompute_rope_freqs": (I, [P, SZ, D]),
    "fhip_alloc": (I, [P, C.POINTER(U64), I, I, TP]),
    "fhip_free": (I, [P, TP]),
    "fhip_copy_to_device": (I, [P, TP, P, SZ]),
    "fhip_copy_to_host": (I, [P, TP, P, SZ]),
    "fhip_rmsnorm": (I, [P, TP, TP, D, TP]),
    "fhip_rope": (I, [P, TP, TP, P, SZ, D, SZ]),
    "fhip_silu_mul": (I, [P, TP, TP, TP]),
    "fhip_embedding": (I, [P, P, SZ, TP, TP]),
    "fhip_add": (I, [P, TP, TP, TP]),
    "fhip_copy_rows": (I, [P, TP, TP, SZ, SZ, SZ]),
    "fhip_attention": (I, [P, TP, TP, TP, SZ, SZ, TP]),
    "fhip_device_name": (C.c_char_p, [P]),
    "fhip_total_memory": (SZ, [P]),
    "fhip_available_memory": (SZ, [P]),
    "fhip_synchronize": (I, [P]),
    "fhip_create_timer": (I, [P, C.POINTER(U64)]),
    "fhip_start_timer": (I, [P, U64]),
    "fhip_stop_timer": (I, [P, U64, C.POINTER(F)]),
    "fhip_destroy_timer": (I, [P, U64]),
    "fhip_marker_push": (None, [P, C.c_char_p]),
    "fhip_marker_pop": (None, [P]),
    "fhip_turboquant_compress": (I, [P, TP, TP, TP, C.c_uint8, TP, TP]),
    "fhip_attention_paged_tq": (I, [P, TP, P, SZ, TP, TP, TP, TP, SZ, TP, TP, TP, TP,
                                    C.c_uint8, C.c_uint8, SZ, SZ, SZ, TP]),
    "fhip_attention_paged": (I, [P, TP, P, SZ, TP, TP, SZ, SZ, SZ, SZ, TP]),
    "fhip_matmul": (I, [P, TP, TP, TP]),
    "fhip_page_pool_create": (I, [P, TP, SZ, SZ, C.POINTER(U64)]),
    "fhip_page_pool_destroy": (I, [P, U64]),
    "fhip_attention_paged_pool": (I, [P, TP, P, SZ, U64, SZ, SZ, SZ, TP]),
    "fhip_attention_paged_tq_pool": (I, [P, TP, P, SZ, U64, TP, TP, TP, TP, C.c_uint8,
                                         C.c_uint8, SZ, SZ, SZ, TP]),
    "fhip_tq_append_kv": (I, [P, U64, TP, TP, TP, TP, TP, TP, C.c_uint8, C.c_uint8, P, SZ, SZ]),
    "fhip_attention_paged_tq_batched": (I, [P, TP, P, SZ, SZ, P, U64, TP, TP, TP, TP, C.c_uint8,
                                            C.c_uint8, SZ, TP]),
    "fhip_add_rmsnorm": (I, [P, TP, TP, TP, D, TP]),
    "fhip_rope_dev": (I, [P, TP, TP, TP, SZ, SZ]),
    "fhip_embedding_dev": (I, [P, TP, SZ, TP, TP]),
    "fhip_graph_begin": (I, [P]),
    "fhip_graph_end": (I, [P, C.POINTER(U64)]),
    "fhip_graph_launch": (I, [P, U64]),
    "fhip_graph_destroy": (I, [P, U64]),
    "fhip_softmax_rows": (I, [P, TP, F, TP]),
    "fhip_argmax_rows": (I, [P, TP, P, SZ]),
    "fhip_tq_dequantize": (I, [P, TP, TP, TP, TP, C.c_uint8, TP]),
    "fhip_tq_quantize_pack": (I, [P, TP, TP, C.c_uint8, TP]),
    # host helpers
    "fhip_tq_packed_dim_per_head": (SZ, [SZ, I]),
    "fhip_tq_codebook": (I, [I, I, P, P]),
    "fhip_tq_rotation_matrix": (I, [I, U64, P]),
    "fhip_tq_rotation_seeds": (None, [U64, U64, C.POINTER(U64), C.POINTER(U64)]),
    "fhip_rope_freqs": (None, [I, D, P]),
    "fhip_version": (C.c_char_p, []),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(fhip_\w+)\s*\(", text)) - {"fhip_tensor"})


def load() -> C.CDLL:
    """Load libfracture_hip.so and declare every entry point. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m fracture_amd.build` (hipcc, gfx950). "
            "fracture_amd has no CPU fallback.")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib

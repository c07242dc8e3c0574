"""Python mirror of Fracture's `Backend` trait over libfracture_hip.so's handle runtime.

``HipBackend`` exposes the trait's methods with the reference's names, argument meaning and
error behaviour (crates/fracture-core/src/backend.rs:8-223), the inherent ``CudaBackend``
API that callers use (new / get_ptr / stream / precompute_rope_freqs,
backends/fracture-cuda/src/lib.rs:76-161), and the additive ops of this backend
(fused add + RMSNorm, row softmax / argmax, TurboQuant dequantize / quantize-pack).
Every call goes through the C ABI; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _lib


class DType(enum.IntEnum):
    """fracture_core::DType (crates/fracture-core/src/dtype.rs:5-31)."""

    FP16 = 0
    FP32 = 1
    BF16 = 2
    INT8 = 3
    INT4 = 4

    def size_bytes(self) -> int:
        return {0: 2, 1: 4, 2: 2, 3: 1, 4: 1}[int(self)]

    def is_packed(self) -> bool:
        return self is DType.INT4

    def __str__(self) -> str:
        return self.name.lower()


@dataclass(frozen=True)
class TensorId:
    value: int


@dataclass
class DeviceTensor:
    """fracture_core::DeviceTensor (crates/fracture-core/src/tensor.rs:13-80)."""

    id: TensorId
    shape: tuple
    dtype: DType

    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    def size_bytes(self) -> int:
        if self.dtype.is_packed():
            return (self.numel() + 1) // 2
        return self.numel() * self.dtype.size_bytes()

    def reshape(self, new_shape: Sequence[int]) -> "DeviceTensor":
        n = 1
        for s in new_shape:
            n *= int(s)
        if n != self.numel():
            raise InvalidShape(
                f"cannot reshape tensor with {self.numel()} elements to shape "
                f"{list(new_shape)} ({n} elements)")
        return DeviceTensor(self.id, tuple(int(s) for s in new_shape), self.dtype)

    def _c(self) -> _lib.FhipTensor:
        if len(self.shape) > _lib.MAX_DIMS:
            raise InvalidShape(f"more than {_lib.MAX_DIMS} dimensions")
        t = _lib.FhipTensor()
        t.id = self.id.value
        t.dtype = int(self.dtype)
        t.ndim = len(self.shape)
        for i, s in enumerate(self.shape):
            t.shape[i] = int(s)
        return t


# ------------------------------------------------------------------------------------
# FractureError (crates/fracture-core/src/error.rs:6-51); str() is the Rust Display text.
# ------------------------------------------------------------------------------------
class FractureError(Exception):
    prefix = ""

    def __init__(self, payload: str):
        super().__init__(self.prefix + payload)
        self.payload = payload


class BackendError(FractureError):
    prefix = "backend error: "


class InvalidShape(FractureError):
    prefix = "invalid tensor shape: "


class TensorNotFound(FractureError):
    prefix = "tensor not found: "


class OutOfMemory(FractureError):
    prefix = "out of device memory: "


class UnsupportedDType(FractureError):
    prefix = "unsupported dtype: "


class GenerationError(FractureError):
    prefix = "generation error: "


_ERRORS = {1: BackendError, 2: InvalidShape, 3: TensorNotFound, 4: OutOfMemory,
           5: UnsupportedDType, 6: GenerationError}


def _check(code: int) -> None:
    if code != 0:
        msg = _lib.load().fhip_last_error().decode(errors="replace")
        raise _ERRORS.get(code, BackendError)(msg)


@dataclass(frozen=True)
class DeviceTimer:
    """fracture_core::DeviceTimer: an opaque timer id."""

    id: int


def _buf(obj, writable: bool = False):
    """(pointer, length) of a bytes-like object or numpy array."""
    if isinstance(obj, np.ndarray):
        if not obj.flags["C_CONTIGUOUS"]:
            raise InvalidShape("host buffer must be contiguous")
        return obj.ctypes.data, obj.nbytes
    if isinstance(obj, (bytes,)) and not writable:
        return C.cast(C.c_char_p(obj), C.c_void_p).value, len(obj)
    mv = memoryview(obj).cast("B")
    arr = np.frombuffer(mv, dtype=np.uint8)
    return arr.ctypes.data, arr.nbytes


class HipBackend:
    """The MI355X backend. ``HipBackend(0)`` is ``CudaBackend::new(0)``'s counterpart."""

    def __init__(self, device_id: int = 0):
        self._L = _lib.load()
        h = C.c_void_p()
        _check(self._L.fhip_backend_create(device_id, C.byref(h)))
        self._h = h
        self.device_id = device_id

    # -- lifetime -----------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.fhip_backend_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- inherent API (lib.rs) -------------------------------------------------------------
    def get_ptr(self, tid: TensorId) -> int:
        p = C.c_void_p()
        _check(self._L.fhip_get_ptr(self._h, tid.value, C.byref(p)))
        return p.value

    def stream(self) -> int:
        return self._L.fhip_stream(self._h) or 0

    def precompute_rope_freqs(self, head_dim: int, theta: float) -> None:
        _check(self._L.fhip_precompute_rope_freqs(self._h, head_dim, theta))

    # -- memory -------------------------------------------------------------------------------
    def alloc(self, shape: Sequence[int], dtype: DType) -> DeviceTensor:
        dims = (C.c_uint64 * max(1, len(shape)))(*[int(s) for s in shape])
        t = _lib.FhipTensor()
        _check(self._L.fhip_alloc(self._h, dims, len(shape), int(dtype), C.byref(t)))
        return DeviceTensor(TensorId(t.id), tuple(int(s) for s in shape), DType(dtype))

    def free(self, tensor: DeviceTensor) -> None:
        _check(self._L.fhip_free(self._h, C.byref(tensor._c())))

    def copy_to_device(self, dst: DeviceTensor, src) -> None:
        p, n = _buf(src)
        _check(self._L.fhip_copy_to_device(self._h, C.byref(dst._c()), p, n))

    def copy_to_host(self, src: DeviceTensor, dst) -> None:
        p, n = _buf(dst, writable=True)
        _check(self._L.fhip_copy_to_host(self._h, C.byref(src._c()), p, n))

    # -- compute (trait) ----------------------------------------------------------------------
    def rmsnorm(self, input: DeviceTensor, weight: DeviceTensor, eps: float,
                out: DeviceTensor) -> None:
        _check(self._L.fhip_rmsnorm(self._h, C.byref(input._c()), C.byref(weight._c()), eps,
                                    C.byref(out._c())))

    def rope(self, q: DeviceTensor, k: DeviceTensor, positions: Sequence[int], theta: float,
             head_dim: int) -> None:
        pos = np.ascontiguousarray(np.asarray(positions, dtype=np.uint32))
        _check(self._L.fhip_rope(self._h, C.byref(q._c()), C.byref(k._c()), pos.ctypes.data,
                                 pos.size, theta, head_dim))

    def attention(self, q: DeviceTensor, k_cache: DeviceTensor, v_cache: DeviceTensor,
                  num_kv_heads: int, start_pos: int, out: DeviceTensor) -> None:
        """Backend::attention over contiguous caches: not supported (the caches are paged)."""
        _check(self._L.fhip_attention(self._h, C.byref(q._c()), C.byref(k_cache._c()),
                                      C.byref(v_cache._c()), num_kv_heads, start_pos,
                                      C.byref(out._c())))

    def silu_mul(self, gate: DeviceTensor, up: DeviceTensor, out: DeviceTensor) -> None:
        _check(self._L.fhip_silu_mul(self._h, C.byref(gate._c()), C.byref(up._c()),
                                     C.byref(out._c())))

    def embedding(self, token_ids: Sequence[int], embedding_table: DeviceTensor,
                  out: DeviceTensor) -> None:
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
        _check(self._L.fhip_embedding(self._h, ids.ctypes.data, ids.size,
                                      C.byref(embedding_table._c()), C.byref(out._c())))

    def rope_dev(self, q: DeviceTensor, k: DeviceTensor, positions: DeviceTensor,
                 num_positions: int, head_dim: int) -> None:
        """rope with the positions read as uint32 from a device tensor (capturable)."""
        _check(self._L.fhip_rope_dev(self._h, C.byref(q._c()), C.byref(k._c()),
                                     C.byref(positions._c()), num_positions, head_dim))

    def embedding_dev(self, token_ids: DeviceTensor, num_tokens: int,
                      embedding_table: DeviceTensor, out: DeviceTensor) -> None:
        """embedding with the token ids read as uint32 from a device tensor (capturable)."""
        _check(self._L.fhip_embedding_dev(self._h, C.byref(token_ids._c()), num_tokens,
                                          C.byref(embedding_table._c()), C.byref(out._c())))

    def add(self, a: DeviceTensor, b: DeviceTensor, out: DeviceTensor) -> None:
        _check(self._L.fhip_add(self._h, C.byref(a._c()), C.byref(b._c()), C.byref(out._c())))

    def copy_rows(self, src: DeviceTensor, dst: DeviceTensor, src_offset: int, dst_offset: int,
                  count: int) -> None:
        _check(self._L.fhip_copy_rows(self._h, C.byref(src._c()), C.byref(dst._c()), src_offset,
                                      dst_offset, count))

    # -- device info ------------------------------------------------------------------------
    def device_name(self) -> str:
        return self._L.fhip_device_name(self._h).decode()

    def total_memory(self) -> int:
        return int(self._L.fhip_total_memory(self._h))

    def available_memory(self) -> int:
        return int(self._L.fhip_available_memory(self._h))

    def synchronize(self) -> None:
        _check(self._L.fhip_synchronize(self._h))

    # -- graph capture ------------------------------------------------------------------------
    def graph_begin(self) -> None:
        """Record this thread's following ops into a graph instead of running them."""
        _check(self._L.fhip_graph_begin(self._h))

    def graph_end(self) -> int:
        """End the capture; returns the id of the instantiated graph."""
        g = C.c_uint64()
        _check(self._L.fhip_graph_end(self._h, C.byref(g)))
        return g.value

    def graph_launch(self, graph: int) -> None:
        _check(self._L.fhip_graph_launch(self._h, graph))

    def graph_destroy(self, graph: int) -> None:
        _check(self._L.fhip_graph_destroy(self._h, graph))

    def capture(self, record) -> int:
        """Capture the ops `record()` issues into a graph and return its id; a failure inside
        ends the capture before it propagates."""
        self.graph_begin()
        try:
            record()
        except BaseException:
            try:
                self.graph_destroy(self.graph_end())
            except FractureError:
                pass
            raise
        return self.graph_end()

    # -- profiling ----------------------------------------------------------------------------
    def create_timer(self) -> DeviceTimer:
        tid = C.c_uint64()
        _check(self._L.fhip_create_timer(self._h, C.byref(tid)))
        return DeviceTimer(tid.value)

    def start_timer(self, timer: DeviceTimer) -> None:
        _check(self._L.fhip_start_timer(self._h, timer.id))

    def stop_timer(self, timer: DeviceTimer) -> float:
        ms = C.c_float()
        _check(self._L.fhip_stop_timer(self._h, timer.id, C.byref(ms)))
        return ms.value

    def destroy_timer(self, timer: DeviceTimer) -> None:
        _check(self._L.fhip_destroy_timer(self._h, timer.id))

    def marker_push(self, name: str) -> None:
        self._L.fhip_marker_push(self._h, name.encode())

    def marker_pop(self) -> None:
        self._L.fhip_marker_pop(self._h)

    # -- TurboQuant (trait) ----------------------------------------------------------------------
    def turboquant_compress(self, input: DeviceTensor, rotation_matrix: DeviceTensor,
                            centroids: DeviceTensor, bits: int, packed_out: DeviceTensor,
                            norms_out: DeviceTensor) -> None:
        _check(self._L.fhip_turboquant_compress(
            self._h, C.byref(input._c()), C.byref(rotation_matrix._c()),
            C.byref(centroids._c()), bits, C.byref(packed_out._c()), C.byref(norms_out._c())))

    def attention_paged_tq(self, q: DeviceTensor, block_table: Sequence[int],
                           k_packed: Sequence[DeviceTensor], k_norms: Sequence[DeviceTensor],
                           v_packed: Sequence[DeviceTensor], v_norms: Sequence[DeviceTensor],
                           k_rotation: DeviceTensor, v_rotation: DeviceTensor,
                           k_centroids: DeviceTensor, v_centroids: DeviceTensor, key_bits: int,
                           value_bits: int, num_kv_heads: int, kv_len: int, start_pos: int,
                           out: DeviceTensor) -> None:
        bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
        n = len(k_packed)
        if not (len(k_norms) == len(v_packed) == len(v_norms) == n):
            raise InvalidShape("k/v block tensor lists differ in length")
        arrs = [(_lib.FhipTensor * max(1, n))(*[t._c() for t in lst])
                for lst in (k_packed, k_norms, v_packed, v_norms)]
        _check(self._L.fhip_attention_paged_tq(
            self._h, C.byref(q._c()), bt.ctypes.data, bt.size, arrs[0], arrs[1], arrs[2],
            arrs[3], n, C.byref(k_rotation._c()), C.byref(v_rotation._c()),
            C.byref(k_centroids._c()), C.byref(v_centroids._c()), key_bits, value_bits,
            num_kv_heads, kv_len, start_pos, C.byref(out._c())))

    def matmul(self, a: DeviceTensor, b: DeviceTensor, out: DeviceTensor) -> None:
        """Backend::matmul as the CUDA backend implements it (cuda/src/backend.rs:75-128):
        out[M, N] = a[M, K] @ b[N, K]^T in fp16 with fp32 accumulation."""
        _check(self._L.fhip_matmul(self._h, C.byref(a._c()), C.byref(b._c()),
                                   C.byref(out._c())))

    def attention_paged(self, q: DeviceTensor, block_table: Sequence[int],
                        k_blocks: Sequence[DeviceTensor], v_blocks: Sequence[DeviceTensor],
                        num_kv_heads: int, kv_len: int, start_pos: int,
                        out: DeviceTensor) -> None:
        """Backend::attention_paged (backend.rs:74-88): causal GQA attention of q [T, qh, hd]
        fp16 over the pool's [16, kvh, hd] fp16 block tensors, indexed by physical block id."""
        bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
        n = len(k_blocks)
        if len(v_blocks) != n:
            raise InvalidShape("k/v block tensor lists differ in length")
        arrs = [(_lib.FhipTensor * max(1, n))(*[t._c() for t in lst])
                for lst in (k_blocks, v_blocks)]
        _check(self._L.fhip_attention_paged(
            self._h, C.byref(q._c()), bt.ctypes.data, bt.size, arrs[0], arrs[1], n,
            num_kv_heads, kv_len, start_pos, C.byref(out._c())))

    # -- registered page pools ------------------------------------------------------------------
    def page_pool_create(self, *block_lists: Sequence[DeviceTensor]) -> int:
        """Keep a KV pool's block addresses in device memory: lists (K, V) for
        attention_paged_pool, (K packed, K norms, V packed, V norms) for
        attention_paged_tq_pool. free() refuses a tensor while a pool holds it."""
        n = len(block_lists[0]) if block_lists else 0
        if not block_lists or any(len(l) != n for l in block_lists):
            raise InvalidShape("block lists differ in length")
        flat = [t._c() for lst in block_lists for t in lst]
        arr = (_lib.FhipTensor * max(1, len(flat)))(*flat)
        h = C.c_uint64()
        _check(self._L.fhip_page_pool_create(self._h, arr, len(block_lists), n, C.byref(h)))
        return h.value

    def page_pool_destroy(self, pool: int) -> None:
        _check(self._L.fhip_page_pool_destroy(self._h, pool))

    def attention_paged_pool(self, q: DeviceTensor, block_table: Sequence[int], pool: int,
                             num_kv_heads: int, kv_len: int, start_pos: int,
                             out: DeviceTensor) -> None:
        bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
        _check(self._L.fhip_attention_paged_pool(self._h, C.byref(q._c()), bt.ctypes.data,
                                                 bt.size, pool, num_kv_heads, kv_len, start_pos,
                                                 C.byref(out._c())))

    def attention_paged_tq_pool(self, q: DeviceTensor, block_table: Sequence[int], pool: int,
                                k_rotation: DeviceTensor, v_rotation: DeviceTensor,
                                k_centroids: DeviceTensor, v_centroids: DeviceTensor,
                                key_bits: int, value_bits: int, num_kv_heads: int, kv_len: int,
                                start_pos: int, out: DeviceTensor) -> None:
        bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
        _check(self._L.fhip_attention_paged_tq_pool(
            self._h, C.byref(q._c()), bt.ctypes.data, bt.size, pool, C.byref(k_rotation._c()),
            C.byref(v_rotation._c()), C.byref(k_centroids._c()), C.byref(v_centroids._c()),
            key_bits, value_bits, num_kv_heads, kv_len, start_pos, C.byref(out._c())))

    def tq_append_kv(self, pool: int, keys: DeviceTensor, values: DeviceTensor,
                     k_rotation: DeviceTensor, v_rotation: DeviceTensor,
                     k_centroids: DeviceTensor, v_centroids: DeviceTensor, key_bits: int,
                     value_bits: int, block_table: Sequence[int], start_pos: int) -> None:
        """QuantizedKvCacheManager::append_kv for one layer: compress keys / values
        [N, kv_heads, head_dim] and write token t into slot (start_pos + t) % 16 of block
        block_table[(start_pos + t) // 16] of a registered TurboQuant pool."""
        bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
        _check(self._L.fhip_tq_append_kv(
            self._h, pool, C.byref(keys._c()), C.byref(values._c()), C.byref(k_rotation._c()),
            C.byref(v_rotation._c()), C.byref(k_centroids._c()), C.byref(v_centroids._c()),
            key_bits, value_bits, bt.ctypes.data, bt.size, start_pos))

    def attention_paged_tq_batched(self, q: DeviceTensor, block_tables: Sequence[Sequence[int]],
                                   seq_lens: Sequence[int], pool: int, k_rotation: DeviceTensor,
                                   v_rotation: DeviceTensor, k_centroids: DeviceTensor,
                                   v_centroids: DeviceTensor, key_bits: int, value_bits: int,
                                   num_kv_heads: int, out: DeviceTensor) -> None:
        """Decode attention of q [B, qh, hd] (one query per sequence) over a registered
        TurboQuant pool in one call. block_tables: an int32 array [B, max_blocks], or rows of
        block ids (padded here to a common width)."""
        lens = np.ascontiguousarray(np.asarray(seq_lens, dtype=np.uint32))
        if isinstance(block_tables, np.ndarray) and block_tables.ndim == 2:
            bt = np.ascontiguousarray(block_tables, dtype=np.int32)
        else:
            width = max([len(r) for r in block_tables] + [1])
            bt = np.full((len(block_tables), width), -1, np.int32)
            for i, row in enumerate(block_tables):
                bt[i, :len(row)] = row
        width = bt.shape[1]
        nq = q.shape[0] if q.shape else 0
        if lens.ndim != 1 or lens.size != nq or bt.shape[0] != nq:
            raise InvalidShape(f"attention_paged_tq_batched: {lens.size} lengths and "
                               f"{bt.shape[0]} block-table rows for {nq} queries")
        _check(self._L.fhip_attention_paged_tq_batched(
            self._h, C.byref(q._c()), bt.ctypes.data, nq, width, lens.ctypes.data, pool,
            C.byref(k_rotation._c()), C.byref(v_rotation._c()), C.byref(k_centroids._c()),
            C.byref(v_centroids._c()), key_bits, value_bits, num_kv_heads, C.byref(out._c())))

    # -- additive ops ---------------------------------------------------------------------------
    def add_rmsnorm(self, residual: DeviceTensor, delta: DeviceTensor, weight: DeviceTensor,
                    eps: float, normed_out: DeviceTensor) -> None:
        """residual += delta (in place, rounded to the dtype); normed_out = rmsnorm(residual)."""
        _check(self._L.fhip_add_rmsnorm(self._h, C.byref(residual._c()), C.byref(delta._c()),
                                        C.byref(weight._c()), eps, C.byref(normed_out._c())))

    def softmax_rows(self, logits: DeviceTensor, temperature: float,
                     probs: DeviceTensor) -> None:
        _check(self._L.fhip_softmax_rows(self._h, C.byref(logits._c()), temperature,
                                         C.byref(probs._c())))

    def argmax_rows(self, logits: DeviceTensor) -> list[int]:
        """Greedy token per row; NaN / Inf rows raise GenerationError like Sampler::sample."""
        cols = logits.shape[-1] if logits.shape else 0
        rows = logits.numel() // cols if cols else 0
        out = np.zeros(max(rows, 1), np.uint32)
        _check(self._L.fhip_argmax_rows(self._h, C.byref(logits._c()), out.ctypes.data, rows))
        return [int(v) for v in out[:rows]]

    def tq_dequantize(self, packed: DeviceTensor, norms: DeviceTensor, rotation: DeviceTensor,
                      centroids: DeviceTensor, bits: int, out: DeviceTensor) -> None:
        _check(self._L.fhip_tq_dequantize(self._h, C.byref(packed._c()), C.byref(norms._c()),
                                          C.byref(rotation._c()), C.byref(centroids._c()),
                                          bits, C.byref(out._c())))

    def tq_quantize_pack(self, y: DeviceTensor, centroids: DeviceTensor, bits: int,
                         packed_out: DeviceTensor) -> None:
        _check(self._L.fhip_tq_quantize_pack(self._h, C.byref(y._c()), C.byref(centroids._c()),
                                             bits, C.byref(packed_out._c())))

    # -- numpy conveniences (tests) ----------------------------------------------------------
    _NP = {DType.FP16: np.float16, DType.FP32: np.float32, DType.BF16: np.uint16,
           DType.INT8: np.uint8, DType.INT4: np.uint8}

    def upload(self, arr: np.ndarray, dtype: DType | None = None) -> DeviceTensor:
        if dtype is None:
            dtype = {np.dtype(np.float16): DType.FP16, np.dtype(np.float32): DType.FP32,
                     np.dtype(np.uint8): DType.INT8, np.dtype(np.int8): DType.INT8,
                     np.dtype(np.int32): DType.FP32}[arr.dtype]
        t = self.alloc(arr.shape, dtype)
        self.copy_to_device(t, np.ascontiguousarray(arr))
        return t

    def download(self, t: DeviceTensor) -> np.ndarray:
        out = np.empty(t.size_bytes(), np.uint8)
        self.copy_to_host(t, out)
        if t.dtype.is_packed():
            return out
        return out.view(self._NP[t.dtype]).reshape(t.shape)

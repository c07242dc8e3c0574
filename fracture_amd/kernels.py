"""Raw launchers of libfracture_hip.so on torch device tensors.

These call the ``fhip_launch_*`` entry points with the tensors' device pointers on torch's
current HIP stream (torch is only the device-memory and stream plumbing here). Every
function checks device, dtype, contiguity and shapes on the host before it launches, so a
kernel never sees an operand that does not match its grid. Non-zero HIP codes raise.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib

_DT = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}


def _L():
    return _lib.load()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ok(code: int, name: str) -> None:
    if code != 0:
        raise RuntimeError(f"{name}: HIP error {code}")


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        _need(isinstance(t, torch.Tensor) and t.is_cuda, "operands must be HIP device tensors")
        _need(t.is_contiguous(), "operands must be contiguous")


def _p(t: torch.Tensor) -> int:
    return t.data_ptr()


# ---------------------------------------------------------------------------------------
# elementwise / norms
# ---------------------------------------------------------------------------------------
def add(out: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> None:
    _dev(out, a, b)
    _need(a.shape == b.shape and out.numel() == a.numel(), "add: shape mismatch")
    _need(a.dtype == b.dtype == out.dtype and a.dtype in _DT, "add: dtype")
    _ok(_L().fhip_launch_add_ex(_p(out), _p(a), _p(b), a.numel(), _DT[a.dtype], _stream()), "add")


def silu_mul(out: torch.Tensor, gate: torch.Tensor, up: torch.Tensor) -> None:
    _dev(out, gate, up)
    _need(gate.shape == up.shape and out.numel() == gate.numel(), "silu_mul: shape mismatch")
    _need(gate.dtype == up.dtype == out.dtype and gate.dtype in _DT, "silu_mul: dtype")
    _ok(_L().fhip_launch_silu_mul_ex(_p(out), _p(gate), _p(up), gate.numel(), _DT[gate.dtype],
                                     _stream()), "silu_mul")


def rmsnorm(out: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    _dev(out, x, weight)
    cols = x.shape[-1]
    _need(weight.numel() == cols and out.shape == x.shape, "rmsnorm: shape mismatch")
    _need(x.dtype == weight.dtype == out.dtype and x.dtype in _DT, "rmsnorm: dtype")
    _ok(_L().fhip_launch_rmsnorm_ex(_p(out), _p(x), _p(weight), eps, x.numel() // cols, cols,
                                    _DT[x.dtype], _stream()), "rmsnorm")


def add_rmsnorm(residual: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, eps: float,
                out: torch.Tensor) -> None:
    """residual = dtype(residual + delta) in place; out = rmsnorm(residual) * weight."""
    _dev(residual, delta, weight, out)
    cols = residual.shape[-1]
    _need(residual.shape == delta.shape == out.shape and weight.numel() == cols,
          "add_rmsnorm: shape mismatch")
    _need(residual.dtype == delta.dtype == weight.dtype == out.dtype and residual.dtype in _DT,
          "add_rmsnorm: dtype")
    _ok(_L().fhip_launch_add_rmsnorm(_p(residual), _p(delta), _p(weight), eps, _p(out),
                                     residual.numel() // cols, cols, _DT[residual.dtype],
                                     _stream()), "add_rmsnorm")


def rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, freqs: torch.Tensor) -> None:
    """In place on q [T, qh, hd] and k [T, kvh, hd]; positions int32/uint32 [T]; freqs f32."""
    _dev(q, k, positions, freqs)
    _need(q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2],
          "rope: q/k must be [T, heads, hd]")
    T, qh, hd = q.shape
    _need(positions.numel() == T and positions.dtype in (torch.int32, torch.uint32),
          "rope: positions")
    _need(freqs.dtype == torch.float32 and freqs.numel() == hd // 2, "rope: freqs")
    _need(q.dtype == k.dtype and q.dtype in _DT, "rope: dtype")
    _ok(_L().fhip_launch_rope_ex(_p(q), _p(k), _p(positions), _p(freqs), T, qh, k.shape[1], hd,
                                 _DT[q.dtype], _stream()), "rope")


def embedding(out: torch.Tensor, table: torch.Tensor, ids: torch.Tensor) -> None:
    _dev(out, table, ids)
    _need(table.dim() == 2 and ids.dtype in (torch.int32, torch.uint32), "embedding: args")
    V, H = table.shape
    _need(out.numel() == ids.numel() * H and out.dtype == table.dtype, "embedding: out")
    _ok(_L().fhip_launch_embedding_ex(_p(out), _p(table), _p(ids), ids.numel(), H, V,
                                      table.element_size(), _stream()), "embedding")


# ---------------------------------------------------------------------------------------
# row softmax / argmax
# ---------------------------------------------------------------------------------------
def rows_workspace(rows: int, cols: int, device="cuda") -> torch.Tensor:
    n = int(_L().fhip_rows_workspace_bytes(rows, cols))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def _rows(logits: torch.Tensor):
    _need(logits.dtype == torch.float32, "logits must be fp32")
    cols = logits.shape[-1]
    return logits.numel() // cols, cols


def softmax_rows(logits: torch.Tensor, probs: torch.Tensor, temperature: float = 1.0,
                 workspace: torch.Tensor | None = None) -> None:
    _dev(logits, probs)
    rows, cols = _rows(logits)
    _need(probs.shape == logits.shape and probs.dtype == torch.float32, "softmax: probs")
    ws = workspace if workspace is not None else rows_workspace(rows, cols, logits.device)
    _need(ws.numel() >= _L().fhip_rows_workspace_bytes(rows, cols), "softmax: workspace")
    _ok(_L().fhip_launch_softmax_rows(_p(logits), _p(probs), rows, cols, temperature, _p(ws),
                                      _stream()), "softmax_rows")


def argmax_rows(logits: torch.Tensor, index_out: torch.Tensor, flags_out: torch.Tensor,
                workspace: torch.Tensor | None = None) -> None:
    _dev(logits, index_out, flags_out)
    rows, cols = _rows(logits)
    _need(index_out.numel() == rows and index_out.dtype == torch.int32, "argmax: index_out")
    _need(flags_out.numel() == rows and flags_out.dtype in (torch.int32, torch.uint32),
          "argmax: flags_out")
    ws = workspace if workspace is not None else rows_workspace(rows, cols, logits.device)
    _need(ws.numel() >= _L().fhip_rows_workspace_bytes(rows, cols), "argmax: workspace")
    _ok(_L().fhip_launch_argmax_rows(_p(logits), _p(index_out), _p(flags_out), rows, cols, _p(ws),
                                     _stream()), "argmax_rows")


def softmax_argmax_rows(logits: torch.Tensor, probs: torch.Tensor, index_out: torch.Tensor,
                        flags_out: torch.Tensor, temperature: float = 1.0,
                        workspace: torch.Tensor | None = None) -> None:
    _dev(logits, probs, index_out, flags_out)
    rows, cols = _rows(logits)
    _need(probs.shape == logits.shape and probs.dtype == torch.float32, "probs")
    _need(index_out.numel() == rows and flags_out.numel() == rows, "index/flags")
    ws = workspace if workspace is not None else rows_workspace(rows, cols, logits.device)
    _need(ws.numel() >= _L().fhip_rows_workspace_bytes(rows, cols), "workspace")
    _ok(_L().fhip_launch_softmax_argmax_rows(_p(logits), _p(probs), _p(index_out), _p(flags_out),
                                             rows, cols, temperature, _p(ws), _stream()),
        "softmax_argmax_rows")


# ---------------------------------------------------------------------------------------
# TurboQuant
# ---------------------------------------------------------------------------------------
def packed_dim(head_dim: int, bits: int) -> int:
    return (head_dim * bits + 7) // 8


def _tq_common(x: torch.Tensor, rot: torch.Tensor):
    _need(x.dtype == torch.float16 and x.dim() >= 2, "tq: input must be fp16 [..., hd]")
    hd = x.shape[-1]
    _need(rot.dtype == torch.float32 and rot.shape == (hd, hd), "tq: rotation must be f32 [hd, hd]")
    return x.numel() // hd, hd


def tq_compress(x: torch.Tensor, rot: torch.Tensor, centroids: torch.Tensor, bits: int,
                packed: torch.Tensor, norms: torch.Tensor) -> None:
    """launch_turboquant_compress on x [N, kvh, hd] fp16."""
    _dev(x, rot, centroids, packed, norms)
    _need(x.dim() == 3, "tq_compress: input must be [N, kv_heads, hd]")
    rows, hd = _tq_common(x, rot)
    N, H = x.shape[0], x.shape[1]
    L = centroids.numel()
    pd = packed_dim(hd, bits)
    _need(centroids.dtype == torch.float32 and 1 <= L <= (1 << bits), "tq_compress: centroids")
    _need(packed.dtype == torch.uint8 and packed.numel() >= rows * pd, "tq_compress: packed")
    _need(norms.dtype == torch.float16 and norms.numel() >= rows, "tq_compress: norms")
    _ok(_L().fhip_launch_turboquant_compress(_p(x), _p(rot), _p(centroids), _p(packed), _p(norms),
                                             N, H, hd, L, bits, pd, _stream()), "tq_compress")


def tq_rotate(x: torch.Tensor, rot: torch.Tensor, y: torch.Tensor, norms: torch.Tensor) -> None:
    _dev(x, rot, y, norms)
    rows, hd = _tq_common(x, rot)
    _need(y.dtype == torch.float32 and y.numel() == rows * hd, "tq_rotate: y")
    _need(norms.dtype == torch.float16 and norms.numel() >= rows, "tq_rotate: norms")
    _ok(_L().fhip_launch_tq_rotate(_p(x), _p(rot), _p(y), _p(norms), rows, hd, _stream()),
        "tq_rotate")


def tq_quantize_pack(y: torch.Tensor, centroids: torch.Tensor, bits: int,
                     packed: torch.Tensor) -> None:
    _dev(y, centroids, packed)
    _need(y.dtype == torch.float32, "tq_quantize_pack: y must be fp32")
    hd = y.shape[-1]
    rows = y.numel() // hd
    L = centroids.numel()
    pd = packed_dim(hd, bits)
    _need(centroids.dtype == torch.float32 and 1 <= L <= (1 << bits), "centroids")
    _need(packed.dtype == torch.uint8 and packed.numel() >= rows * pd, "packed")
    _ok(_L().fhip_launch_tq_quantize_pack(_p(y), _p(centroids), L, bits, _p(packed), rows, hd, pd,
                                          _stream()), "tq_quantize_pack")


def tq_dequant(packed: torch.Tensor, norms: torch.Tensor, rot: torch.Tensor,
               centroids: torch.Tensor, bits: int, out: torch.Tensor) -> None:
    _dev(packed, norms, rot, centroids, out)
    _need(out.dtype == torch.float16 and out.dim() == 3, "tq_dequant: out [N, kvh, hd] fp16")
    N, H, hd = out.shape
    rows = N * H
    pd = packed_dim(hd, bits)
    L = centroids.numel()
    _need(rot.dtype == torch.float32 and rot.shape == (hd, hd), "rotation")
    _need(packed.dtype == torch.uint8 and packed.numel() >= rows * pd, "packed")
    _need(norms.dtype == torch.float16 and norms.numel() >= rows, "norms")
    _need(centroids.dtype == torch.float32 and 1 <= L <= (1 << bits), "centroids")
    _ok(_L().fhip_launch_tq_dequant(_p(packed), _p(norms), _p(rot), _p(centroids), L, _p(out), N,
                                    H, hd, bits, pd, _stream()), "tq_dequant")


def tq_compress_pages(x: torch.Tensor, rot: torch.Tensor, centroids: torch.Tensor, bits: int,
                      packed_pool: torch.Tensor, norms_pool: torch.Tensor,
                      page_ids: torch.Tensor, first_pos: int) -> None:
    """Compress x [T, kvh, hd] into pages: packed_pool [P, 16, kvh*pd] u8, norms_pool
    [P, 16, kvh] fp16; token t lands in page page_ids[(first_pos+t)//16]."""
    _dev(x, rot, centroids, packed_pool, norms_pool, page_ids)
    _need(x.dim() == 3, "tq_compress_pages: x [T, kvh, hd]")
    T, H, hd = x.shape
    pd = packed_dim(hd, bits)
    P = packed_pool.shape[0]
    _need(packed_pool.dtype == torch.uint8 and packed_pool.shape[1:] == (16, H * pd), "packed_pool")
    _need(norms_pool.dtype == torch.float16 and norms_pool.shape == (P, 16, H), "norms_pool")
    _need(page_ids.dtype == torch.int32 and page_ids.numel() * 16 >= first_pos + T, "page_ids")
    L = centroids.numel()
    _need(centroids.dtype == torch.float32 and 1 <= L <= (1 << bits), "centroids")
    _ok(_L().fhip_launch_tq_compress_pages(_p(x), _p(rot), _p(centroids), L, bits, _p(packed_pool),
                                           _p(norms_pool), packed_pool[0].nbytes if P else 16 * H * pd,
                                           norms_pool[0].nbytes if P else 32 * H, _p(page_ids), P,
                                           first_pos, T, H, hd, _stream()), "tq_compress_pages")


class TqPlan:
    """fhip_tq_plan for one rotation [hd, hd] f32 and codebook (head_dim 128): the quantizer
    tables and rotation fragments built once on the device (enqueued on the current
    stream). Freed when the object is."""

    def __init__(self, rot: torch.Tensor, centroids: torch.Tensor, bits: int):
        _dev(rot, centroids)
        hd = rot.shape[0]
        L = centroids.numel()
        _need(rot.dtype == torch.float32 and rot.shape == (hd, hd), "TqPlan: rotation")
        _need(centroids.dtype == torch.float32 and 1 <= L <= (1 << bits), "TqPlan: centroids")
        self._h = None
        h = C.c_void_p()
        _ok(_L().fhip_tq_plan_create(_p(rot), _p(centroids), L, bits, hd, _stream(),
                                     C.byref(h)), "tq_plan_create")
        self._h, self.head_dim, self.bits, self.n_levels = h, hd, bits, L
        self.packed_dim = packed_dim(hd, bits)

    def close(self) -> None:
        """Free the plan's device memory (waits for the device to idle)."""
        h, self._h = getattr(self, "_h", None), None
        if h:
            _lib.load().fhip_tq_plan_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library binding may be gone already
            pass


def tq_compress_planned(plan: TqPlan, x: torch.Tensor, packed: torch.Tensor,
                        norms: torch.Tensor) -> None:
    """tq_compress with a plan: x [N, kvh, hd] fp16."""
    _dev(x, packed, norms)
    _need(x.dtype == torch.float16 and x.dim() == 3 and x.shape[2] == plan.head_dim,
          "tq_compress_planned: x [N, kv_heads, hd] fp16")
    N, H = x.shape[0], x.shape[1]
    _need(packed.dtype == torch.uint8 and packed.numel() >= N * H * plan.packed_dim, "packed")
    _need(norms.dtype == torch.float16 and norms.numel() >= N * H, "norms")
    _ok(_L().fhip_launch_tq_compress_planned(plan._h, _p(x), _p(packed), _p(norms), N, H,
                                             _stream()), "tq_compress_planned")


def tq_compress_pages_planned(plan: TqPlan, x: torch.Tensor, packed_pool: torch.Tensor,
                              norms_pool: torch.Tensor, page_ids: torch.Tensor,
                              first_pos: int) -> None:
    """tq_compress_pages with a plan (same page layout and arguments)."""
    _dev(x, packed_pool, norms_pool, page_ids)
    _need(x.dtype == torch.float16 and x.dim() == 3 and x.shape[2] == plan.head_dim,
          "tq_compress_pages_planned: x [T, kvh, hd] fp16")
    T, H, _ = x.shape
    pd = plan.packed_dim
    P = packed_pool.shape[0]
    _need(packed_pool.dtype == torch.uint8 and packed_pool.shape[1:] == (16, H * pd), "packed_pool")
    _need(norms_pool.dtype == torch.float16 and norms_pool.shape == (P, 16, H), "norms_pool")
    _need(page_ids.dtype == torch.int32 and page_ids.numel() * 16 >= first_pos + T, "page_ids")
    _ok(_L().fhip_launch_tq_compress_pages_planned(
        plan._h, _p(x), _p(packed_pool), _p(norms_pool), packed_pool[0].nbytes if P else 16 * H * pd,
        norms_pool[0].nbytes if P else 32 * H, _p(page_ids), P, first_pos, T, H, _stream()),
        "tq_compress_pages_planned")


def tq_dequant_planned(plan: TqPlan, packed: torch.Tensor, norms: torch.Tensor,
                       out: torch.Tensor) -> None:
    """tq_dequant with a plan: out [N, kvh, hd] fp16."""
    _dev(packed, norms, out)
    _need(out.dtype == torch.float16 and out.dim() == 3 and out.shape[2] == plan.head_dim,
          "tq_dequant_planned: out [N, kvh, hd] fp16")
    N, H = out.shape[0], out.shape[1]
    _need(packed.dtype == torch.uint8 and packed.numel() >= N * H * plan.packed_dim, "packed")
    _need(norms.dtype == torch.float16 and norms.numel() >= N * H, "norms")
    _ok(_L().fhip_launch_tq_dequant_planned(plan._h, _p(packed), _p(norms), _p(out), N, H,
                                            _stream()), "tq_dequant_planned")


def tq_compress_kv_planned(kplan: TqPlan, vplan: TqPlan, k: torch.Tensor, v: torch.Tensor,
                           k_packed: torch.Tensor, k_norms: torch.Tensor,
                           v_packed: torch.Tensor, v_norms: torch.Tensor) -> None:
    """A layer's keys and values [N, kvh, hd] fp16 compressed in one launch."""
    _dev(k, v, k_packed, k_norms, v_packed, v_norms)
    _need(k.dtype == torch.float16 and k.dim() == 3 and k.shape == v.shape and
          v.dtype == torch.float16 and k.shape[2] == kplan.head_dim == vplan.head_dim,
          "tq_compress_kv_planned: k, v [N, kv_heads, hd] fp16")
    N, H = k.shape[0], k.shape[1]
    _need(k_packed.dtype == torch.uint8 and k_packed.numel() >= N * H * kplan.packed_dim, "k_packed")
    _need(v_packed.dtype == torch.uint8 and v_packed.numel() >= N * H * vplan.packed_dim, "v_packed")
    _need(k_norms.dtype == torch.float16 and k_norms.numel() >= N * H, "k_norms")
    _need(v_norms.dtype == torch.float16 and v_norms.numel() >= N * H, "v_norms")
    _ok(_L().fhip_launch_tq_compress_kv_planned(kplan._h, vplan._h, _p(k), _p(v), _p(k_packed),
                                                _p(k_norms), _p(v_packed), _p(v_norms), N, H,
                                                _stream()), "tq_compress_kv_planned")


def tq_dequant_kv_planned(kplan: TqPlan, vplan: TqPlan, k_packed: torch.Tensor,
                          k_norms: torch.Tensor, v_packed: torch.Tensor, v_norms: torch.Tensor,
                          k_out: torch.Tensor, v_out: torch.Tensor) -> None:
    """A layer's keys and values dequantized in one launch: outputs [N, kvh, hd] fp16."""
    _dev(k_packed, k_norms, v_packed, v_norms, k_out, v_out)
    _need(k_out.dtype == torch.float16 and k_out.dim() == 3 and k_out.shape == v_out.shape and
          v_out.dtype == torch.float16 and k_out.shape[2] == kplan.head_dim == vplan.head_dim,
          "tq_dequant_kv_planned: outputs [N, kvh, hd] fp16")
    N, H = k_out.shape[0], k_out.shape[1]
    _need(k_packed.dtype == torch.uint8 and k_packed.numel() >= N * H * kplan.packed_dim, "k_packed")
    _need(v_packed.dtype == torch.uint8 and v_packed.numel() >= N * H * vplan.packed_dim, "v_packed")
    _need(k_norms.dtype == torch.float16 and k_norms.numel() >= N * H, "k_norms")
    _need(v_norms.dtype == torch.float16 and v_norms.numel() >= N * H, "v_norms")
    _ok(_L().fhip_launch_tq_dequant_kv_planned(kplan._h, vplan._h, _p(k_packed), _p(k_norms),
                                               _p(v_packed), _p(v_norms), _p(k_out), _p(v_out),
                                               N, H, _stream()), "tq_dequant_kv_planned")


def attention_workspace(batch: int, qh: int, hd: int, max_blocks: int, device="cuda"):
    n = int(_L().fhip_attention_tq_workspace_bytes(batch, qh, hd, max_blocks))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def attention_tq_decode(out: torch.Tensor, q: torch.Tensor, block_table: torch.Tensor,
                        seq_lens: torch.Tensor, kp: torch.Tensor, kn: torch.Tensor,
                        vp: torch.Tensor, vn: torch.Tensor, krot: torch.Tensor,
                        vrot: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, key_bits: int,
                        value_bits: int, num_kv_heads: int,
                        workspace: torch.Tensor | None = None) -> None:
    """One query per sequence: q/out [B, qh, hd] fp16; block_table [B, max_blocks] int32;
    seq_lens [B] int32; pools kp [P, 16, kvh*pdk] u8, kn [P, 16, kvh] fp16, vp, vn."""
    _dev(out, q, block_table, seq_lens, kp, kn, vp, vn, krot, vrot, kc, vc)
    _need(q.dtype == torch.float16 and q.dim() == 3 and out.shape == q.shape, "q/out")
    B, qh, hd = q.shape
    _need(block_table.dtype == torch.int32 and block_table.dim() == 2 and
          block_table.shape[0] == B and block_table.shape[1] >= 1,
          "block_table [B, max_blocks >= 1]")
    _need(seq_lens.dtype == torch.int32 and seq_lens.numel() == B, "seq_lens")
    mb = block_table.shape[1]
    P = kp.shape[0]
    pdk, pdv = packed_dim(hd, key_bits), packed_dim(hd, value_bits)
    H = num_kv_heads
    _need(kp.dtype == torch.uint8 and kp.shape[1:] == (16, H * pdk), "k packed pool")
    _need(vp.dtype == torch.uint8 and vp.shape == (P, 16, H * pdv), "v packed pool")
    _need(kn.dtype == torch.float16 and kn.shape == (P, 16, H), "k norms pool")
    _need(vn.dtype == torch.float16 and vn.shape == (P, 16, H), "v norms pool")
    _need(krot.shape == (hd, hd) and vrot.shape == (hd, hd), "rotations")
    _need(kc.numel() >= (1 << key_bits) and vc.numel() >= (1 << value_bits), "centroids")
    ws = workspace if workspace is not None else attention_workspace(B, qh, hd, mb, q.device)
    _need(ws.numel() >= _L().fhip_attention_tq_workspace_bytes(B, qh, hd, mb), "workspace")
    _ok(_L().fhip_launch_attention_tq_decode(
        _p(out), _p(q), _p(block_table), _p(seq_lens), B, mb, P, _p(kp), _p(kn), _p(vp), _p(vn),
        kp[0].nbytes, kn[0].nbytes, vp[0].nbytes, vn[0].nbytes, _p(krot), _p(vrot), _p(kc),
        _p(vc), qh, H, hd, key_bits, value_bits, _p(ws), _stream()), "attention_tq_decode")


def attention_paged_workspace(batch: int, qh: int, hd: int, max_blocks: int, device="cuda"):
    n = int(_L().fhip_attention_paged_workspace_bytes(batch, qh, hd, max_blocks))
    return torch.empty(max(n, 16), dtype=torch.uint8, device=device)


def attention_paged_decode(out: torch.Tensor, q: torch.Tensor, block_table: torch.Tensor,
                           seq_lens: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           num_kv_heads: int, workspace: torch.Tensor | None = None) -> None:
    """One query per sequence over FP16 pages: q/out [B, qh, hd] fp16; block_table
    [B, max_blocks] int32; seq_lens [B] int32; k_pool/v_pool [P, 16, kvh, hd] fp16."""
    _dev(out, q, block_table, seq_lens, k_pool, v_pool)
    _need(q.dtype == torch.float16 and q.dim() == 3 and out.shape == q.shape and
          out.dtype == torch.float16, "q/out")
    B, qh, hd = q.shape
    _need(block_table.dtype == torch.int32 and block_table.dim() == 2 and
          block_table.shape[0] == B and block_table.is_contiguous() and
          block_table.shape[1] >= 1, "block_table [B, max_blocks >= 1]")
    _need(seq_lens.dtype == torch.int32 and seq_lens.numel() == B, "seq_lens")
    mb = block_table.shape[1]
    P = k_pool.shape[0]
    for t, name in ((k_pool, "k pool"), (v_pool, "v pool")):
        _need(t.dtype == torch.float16 and t.is_contiguous() and t.shape[0] == P and
              t[0].numel() == 16 * num_kv_heads * hd, name)
    ws = workspace if workspace is not None else attention_paged_workspace(B, qh, hd, mb,
                                                                           q.device)
    _need(ws.numel() >= _L().fhip_attention_paged_workspace_bytes(B, qh, hd, mb), "workspace")
    _ok(_L().fhip_launch_attention_paged_decode(
        _p(out), _p(q), _p(block_table), _p(seq_lens), B, mb, P, _p(k_pool), _p(v_pool),
        k_pool[0].nbytes, v_pool[0].nbytes, qh, num_kv_heads, hd, _p(ws), _stream()),
        "attention_paged_decode")


def paged_attention(out: torch.Tensor, q: torch.Tensor, block_table: torch.Tensor,
                    k_block_ptrs: torch.Tensor, v_block_ptrs: torch.Tensor, num_kv_heads: int,
                    kv_len: int, start_pos: int, workspace: torch.Tensor | None = None) -> None:
    """The reference interface (attention_paged.cu:172-185): T causal queries of one sequence;
    block_table [nblocks] int32; k/v_block_ptrs int64 device arrays of block addresses. With
    `workspace` (attention_paged_workspace(T, qh, hd, nblocks)) nothing is allocated."""
    _dev(out, q, block_table, k_block_ptrs, v_block_ptrs)
    _need(q.dtype == torch.float16 and q.dim() == 3 and out.shape == q.shape, "q/out")
    _need(block_table.dtype == torch.int32 and block_table.dim() == 1, "block_table")
    T, qh, hd = q.shape
    if workspace is None:
        _ok(_L().fhip_launch_paged_attention(
            _p(out), _p(q), _p(block_table), _p(k_block_ptrs), _p(v_block_ptrs), T, qh,
            num_kv_heads, hd, kv_len, start_pos, block_table.numel(), _stream()),
            "paged_attention")
        return
    _dev(workspace)
    _ok(_L().fhip_launch_paged_attention_ws(
        _p(out), _p(q), _p(block_table), _p(k_block_ptrs), _p(v_block_ptrs), T, qh,
        num_kv_heads, hd, kv_len, start_pos, block_table.numel(), _p(workspace),
        C.c_size_t(workspace.numel()), _stream()), "paged_attention")


def matmul(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> None:
    """c[M, N] = a[M, K] @ b[N, K]^T, fp16 in and out, fp32 accumulation
    (CudaBackend::matmul, cuda/src/backend.rs:75-128)."""
    _dev(c, a, b)
    _need(a.dtype == b.dtype == c.dtype == torch.float16, "fp16 operands")
    _need(a.dim() == 2 and b.dim() == 2 and a.shape[1] == b.shape[1] and
          tuple(c.shape) == (a.shape[0], b.shape[0]), "shapes")
    _ok(_L().fhip_launch_matmul(_p(c), _p(a), _p(b), a.shape[0], b.shape[0], a.shape[1],
                                _stream()), "matmul")


# ---------------------------------------------------------------------------------------
# Measurement probes (floors for the benchmark; no counterpart in the reference)
# ---------------------------------------------------------------------------------------
def probe_empty(grid: int) -> None:
    """An empty kernel of `grid` workgroups on torch's current stream."""
    _ok(_L().fhip_probe_empty(grid, _stream()), "probe_empty")


def probe_stream(inputs, outputs, nbytes: int, grid: int, sink: torch.Tensor | None = None) -> None:
    """Read `nbytes` of each input tensor and write their XOR to each output (device
    tensors of at least nbytes each): the memory traffic of a kernel, nothing else."""
    for t in list(inputs) + list(outputs):
        _need(t.is_cuda and t.numel() * t.element_size() >= nbytes, "probe buffer")
    ins = (C.c_void_p * 3)(*[_p(t) for t in inputs])
    outs = (C.c_void_p * 2)(*[_p(t) for t in outputs])
    _need(bool(outputs) or sink is not None, "a read-only probe needs a sink")
    _ok(_L().fhip_probe_stream(ins, len(inputs), outs, len(outputs), nbytes,
                               _p(sink) if sink is not None else None, grid, _stream()),
        "probe_stream")

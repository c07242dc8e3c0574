"""The Backend-trait mirror (HipBackend over the C-ABI handle runtime), following the
reference's backend tests (backends/fracture-cuda/src/tests.rs): memory management, error
mapping, every compute op through opaque tensor ids, timers and markers.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close
from fracture_amd import (BackendError, DType, DeviceTensor, GenerationError, HipBackend,
                          InvalidShape, TensorId, TensorNotFound)
from fracture_amd import turboquant as tq

pytestmark = pytest.mark.gpu


def up16(b, a):
    return b.upload(np.ascontiguousarray(a, np.float16))


def test_alloc_free_and_roundtrip(backend):
    t = backend.alloc([4, 8], DType.FP16)
    assert t.shape == (4, 8) and t.numel() == 32 and t.size_bytes() == 64
    data = (np.arange(32, dtype=np.float32) * 0.5).astype(np.float16)
    backend.copy_to_device(t, data)
    out = np.empty(32, np.float16)
    backend.copy_to_host(t, out)
    assert np.array_equal(out, data)
    backend.free(t)
    i4 = backend.alloc([5], DType.INT4)
    assert i4.size_bytes() == 3
    backend.free(i4)


def test_errors_match_reference(backend):
    fake = DeviceTensor(TensorId(999999), (1,), DType.FP16)
    with pytest.raises(TensorNotFound, match="tensor id 999999"):
        backend.free(fake)
    t = backend.alloc([4], DType.FP16)
    backend.free(t)
    with pytest.raises(TensorNotFound):
        backend.free(t)  # double free
    with pytest.raises(TensorNotFound):
        backend.copy_to_host(t, np.empty(4, np.float16))  # use after free
    with pytest.raises(BackendError, match="HIP error"):
        backend.alloc([1024 * 1024 * 1024, 256 * 8], DType.FP16)  # 4 TiB
    s = backend.alloc([8], DType.FP16)
    with pytest.raises(InvalidShape, match="source buffer too small"):
        backend.copy_to_device(s, np.zeros(4, np.float16))
    with pytest.raises(InvalidShape, match="destination buffer too small"):
        backend.copy_to_host(s, np.zeros(4, np.float16))
    backend.free(s)


def test_copy_rows(backend):
    src = up16(backend, np.arange(1, 9).reshape(4, 2))
    dst = up16(backend, np.zeros((4, 2)))
    backend.copy_rows(src, dst, 1, 2, 2)
    assert np.array_equal(backend.download(dst).astype(np.float32),
                          [[0, 0], [0, 0], [3, 4], [5, 6]])
    with pytest.raises(InvalidShape, match="exceeds src rows"):
        backend.copy_rows(src, dst, 3, 0, 2)
    with pytest.raises(InvalidShape, match="exceeds dst rows"):
        backend.copy_rows(src, dst, 0, 3, 2)
    other = up16(backend, np.zeros((4, 3)))
    with pytest.raises(InvalidShape, match="column shape"):
        backend.copy_rows(src, other, 0, 0, 1)
    f32 = backend.upload(np.zeros((4, 2), np.float32))
    with pytest.raises(InvalidShape, match="dtype"):
        backend.copy_rows(src, f32, 0, 0, 1)
    for t in (src, dst, other, f32):
        backend.free(t)


def test_small_tensor_arena(backend):
    """Tensors up to 64 KB share large chunks in size classes and are recycled on free: live
    tensors of every class never overlap (each keeps its own bytes through frees and
    reallocations around it), and a freed slot is handed out again."""
    rng = np.random.default_rng(3)
    sizes = [0, 1, 255, 256, 257, 4095, 8192, 65536, 65537, 100000]
    live = []

    def new(n):
        t = backend.alloc([n], DType.INT8)
        data = rng.integers(0, 256, n).astype(np.uint8)
        if n:
            backend.copy_to_device(t, data)
        live.append((t, data))

    for i in range(400):
        new(sizes[i % len(sizes)])
    freed = set()
    for t, _ in live[::3]:
        freed.add(backend.get_ptr(t.id))
        backend.free(t)
    live = [x for i, x in enumerate(live) if i % 3]
    reused = 0
    for i in range(200):
        new(sizes[i % len(sizes)])
        reused += backend.get_ptr(live[-1][0].id) in freed
    assert reused > 0
    for t, data in live:
        if len(data):
            assert np.array_equal(backend.download(t).reshape(-1).view(np.uint8), data)
    for t, _ in live:
        backend.free(t)


def test_device_info_timers_markers(backend):
    assert backend.device_name()
    assert backend.total_memory() > 0
    assert 0 < backend.available_memory() <= backend.total_memory()
    backend.synchronize()
    tm = backend.create_timer()
    backend.start_timer(tm)
    backend.marker_push("layer 0")
    x = up16(backend, np.ones((64, 4096)))
    w = up16(backend, np.ones(4096))
    o = backend.alloc([64, 4096], DType.FP16)
    backend.rmsnorm(x, w, 1e-5, o)
    backend.marker_pop()
    ms = backend.stop_timer(tm)
    assert ms >= 0.0
    backend.destroy_timer(tm)
    with pytest.raises(BackendError):
        backend.destroy_timer(tm)
    for t in (x, w, o):
        backend.free(t)


def test_elementwise_through_trait(backend):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((8, 64)).astype(np.float16)
    b = rng.standard_normal((8, 64)).astype(np.float16)
    ta, tb = up16(backend, a), up16(backend, b)
    out = backend.alloc([8, 64], DType.FP16)
    backend.add(ta, tb, out)
    assert np.array_equal(backend.download(out).view(np.uint16), oracle.add(a, b).view(np.uint16))
    backend.silu_mul(ta, tb, out)
    assert_close(backend.download(out).astype(np.float32),
                 oracle.silu_mul(a, b).astype(np.float32), 1e-3, 1e-3, "silu_mul")
    w = rng.uniform(0.5, 2.0, 64).astype(np.float16)
    tw = up16(backend, w)
    backend.rmsnorm(ta, tw, 1e-5, out)
    assert_close(backend.download(out).astype(np.float32),
                 oracle.rmsnorm(a, w, 1e-5).astype(np.float32), 1e-3, 1e-3, "rmsnorm")
    normed = backend.alloc([8, 64], DType.FP16)
    backend.add_rmsnorm(ta, tb, tw, 1e-5, normed)
    h2, n2 = oracle.add_rmsnorm(a, b, w, 1e-5)
    assert np.array_equal(backend.download(ta).view(np.uint16), h2.view(np.uint16))
    assert_close(backend.download(normed).astype(np.float32), n2.astype(np.float32), 1e-3,
                 1e-3, "add_rmsnorm")
    # shape errors (tests.rs:2924-2958)
    c = backend.alloc([8, 32], DType.FP16)
    with pytest.raises(InvalidShape, match="gate shape"):
        backend.silu_mul(ta, c, out)
    with pytest.raises(InvalidShape, match="a shape"):
        backend.add(ta, c, out)
    for t in (ta, tb, out, tw, normed, c):
        backend.free(t)


def test_embedding_through_trait(backend, golden):
    table = backend.upload(golden["weights/token_embd.weight"])
    ids = list(golden["prompt_0/token_ids"]) + [256, 10**6]
    out = backend.alloc([len(ids), 128], DType.FP16)
    backend.embedding(ids, table, out)
    got = backend.download(out).astype(np.float32)
    assert np.array_equal(got[:-2], golden["prompt_0/embeddings"].reshape(-1, 128))
    assert not got[-2:].any()
    backend.free(table)
    backend.free(out)


def test_rope_through_trait(golden):
    b = HipBackend(0)
    q = up16(b, np.ones((1, 4, 32)))
    k = up16(b, np.ones((1, 2, 32)))
    with pytest.raises(BackendError, match="precompute_rope_freqs"):
        b.rope(q, k, [3], 500000.0, 32)
    b.precompute_rope_freqs(32, 500000.0)
    cfg = golden["config"]
    qv = golden["prompt_1/layer_02/q"].reshape(-1, 4, 32).astype(np.float16)
    kv = golden["prompt_1/layer_02/k"].reshape(-1, 2, 32).astype(np.float16)
    tq_, tk = up16(b, qv), up16(b, kv)
    T = qv.shape[0]
    for _ in range(20):  # reuse of the staging ring across calls
        b.rope(tq_, tk, list(range(T)), cfg["rope_theta"], 32)
        tq_, tk = up16(b, qv), up16(b, kv)
    b.rope(tq_, tk, list(range(T)), cfg["rope_theta"], 32)
    assert_close(b.download(tq_).astype(np.float32),
                 golden["prompt_1/layer_02/q_rope"].reshape(qv.shape), 0.01, 0.025, "q_rope")
    with pytest.raises(InvalidShape):
        b.rope(tq_, tk, list(range(T)), cfg["rope_theta"], 64)  # table is for head_dim 32
    b.close()


def test_softmax_argmax_through_trait(backend, golden):
    l = np.ascontiguousarray(golden["prompt_0/logits"].reshape(-1, 256))
    tl = backend.upload(l)
    assert backend.argmax_rows(tl) == list(oracle.argmax_rows(l)[0])
    p = backend.alloc(list(l.shape), DType.FP32)
    backend.softmax_rows(tl, 1.0, p)
    assert_close(backend.download(p), oracle.softmax_rows(l), 1e-5, 1e-5, "softmax")
    bad = l.copy()
    bad[3, 7] = np.nan
    bad[5, 1] = np.inf
    tb = backend.upload(bad)
    with pytest.raises(GenerationError, match="NaN in logits"):
        backend.argmax_rows(tb)
    bad[3, 7] = 0
    backend.copy_to_device(tb, bad)
    with pytest.raises(GenerationError, match="Inf in logits"):
        backend.argmax_rows(tb)
    for t in (tl, p, tb):
        backend.free(t)


def test_turboquant_through_trait(backend):
    rng = np.random.default_rng(3)
    N, H, hd, bits = 40, 8, 128, 4
    x = rng.standard_normal((N, H, hd)).astype(np.float16)
    rot, cent = tq.rotation_matrix(hd, 42), tq.codebook(hd, bits)[0]
    tx, tr, tc = up16(backend, x), backend.upload(rot), backend.upload(cent)
    pd = tq.TurboQuantConfig.packed_dim_per_head(hd, bits)
    packed = backend.alloc([N, H * pd], DType.INT8)
    norms = backend.alloc([N, H], DType.FP16)
    backend.turboquant_compress(tx, tr, tc, bits, packed, norms)
    pk = backend.download(packed).reshape(N * H, pd)
    nv = backend.download(norms).reshape(-1)
    # bytes bit-exact given the same kernel's rotated vectors (quantize-pack entry)
    import torch

    from fracture_amd import kernels as K

    dev = torch.device("cuda:0")
    y = torch.empty((N * H, hd), dtype=torch.float32, device=dev)
    yn = torch.empty(N * H, dtype=torch.float16, device=dev)
    K.tq_rotate(torch.from_numpy(x).to(dev), torch.from_numpy(rot).to(dev), y, yn)
    torch.cuda.synchronize()
    assert np.array_equal(pk, oracle.tq_quantize_pack(y.cpu().numpy(), cent, bits))
    ty = backend.upload(y.cpu().numpy())
    p2 = backend.alloc([N * H, pd], DType.INT8)
    backend.tq_quantize_pack(ty, tc, bits, p2)
    assert np.array_equal(backend.download(p2), pk)
    out = backend.alloc([N, H, hd], DType.FP16)
    backend.tq_dequantize(packed, norms, tr, tc, bits, out)
    want = oracle.tq_dequant(pk, nv, rot, cent, bits, hd)
    assert_close(backend.download(out).reshape(-1, hd).astype(np.float32),
                 want.astype(np.float32), 1e-3, 1e-3, "dequant")
    with pytest.raises(InvalidShape):
        backend.turboquant_compress(tx, tr, tc, 3, packed, norms)  # 16 centroids for 3 bits
    for t in (tx, tr, tc, packed, norms, ty, p2, out):
        backend.free(t)


def test_attention_paged_tq_through_trait(backend):
    """Per-block tensors, as QuantizedKvCacheManager allocates them
    (crates/fracture-engine/src/quantized_paged_kv_cache.rs:82-133)."""
    rng = np.random.default_rng(4)
    qh, kvh, hd, kb, vb = 8, 2, 128, 4, 2
    kv_len = 50
    pdk, pdv = oracle.packed_dim(hd, kb), oracle.packed_dim(hd, vb)
    k = rng.standard_normal((kv_len, kvh, hd)).astype(np.float16)
    v = rng.standard_normal((kv_len, kvh, hd)).astype(np.float16)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc, vc = tq.codebook(hd, kb)[0], tq.codebook(hd, vb)[0]
    kp, kn, _ = oracle.tq_compress(k, krot, kc, kb)
    vp, vn, _ = oracle.tq_compress(v, vrot, vc, vb)
    pool = 6
    table = [4, 0, 5, 2]
    KP = np.zeros((pool, 16, kvh * pdk), np.uint8)
    KN = np.zeros((pool, 16, kvh), np.float16)
    VP = np.zeros((pool, 16, kvh * pdv), np.uint8)
    VN = np.zeros((pool, 16, kvh), np.float16)
    for t in range(kv_len):
        p, s = table[t // 16], t % 16
        KP[p, s], KN[p, s] = kp.reshape(kv_len, -1)[t], kn.reshape(kv_len, kvh)[t]
        VP[p, s], VN[p, s] = vp.reshape(kv_len, -1)[t], vn.reshape(kv_len, kvh)[t]
    kps = [backend.upload(KP[i]) for i in range(pool)]
    kns = [backend.upload(KN[i]) for i in range(pool)]
    vps = [backend.upload(VP[i]) for i in range(pool)]
    vns = [backend.upload(VN[i]) for i in range(pool)]
    q = rng.standard_normal((1, qh, hd)).astype(np.float16)
    tq_ = up16(backend, q)
    out = backend.alloc([1, qh, hd], DType.FP16)
    tkr, tvr, tkc, tvc = (backend.upload(a) for a in (krot, vrot, kc, vc))
    backend.attention_paged_tq(tq_, table, kps, kns, vps, vns, tkr, tvr, tkc, tvc, kb, vb, kvh,
                               kv_len, kv_len - 1, out)
    want = oracle.tq_attention(q[0], np.array(table, np.int32), kv_len, KP, KN, VP, VN, krot, vrot,
                               kc, vc, kb, vb, kvh)
    assert_close(backend.download(out)[0].astype(np.float32), want.astype(np.float32), 1e-3,
                 1e-3, "attention_paged_tq")
    with pytest.raises(InvalidShape, match="block id"):
        backend.attention_paged_tq(tq_, [4, 0, 9, 2], kps, kns, vps, vns, tkr, tvr, tkc, tvc, kb,
                                   vb, kvh, kv_len, kv_len - 1, out)
    for t in kps + kns + vps + vns + [tq_, out, tkr, tvr, tkc, tvc]:
        backend.free(t)


def test_attention_paged_through_trait(backend):
    """FP16 pool blocks as PagedKvCacheManager hands them to the backend
    (crates/fracture-engine/src/batched.rs:92-109): prefill of 5 tokens at start_pos 45."""
    rng = np.random.default_rng(5)
    qh, kvh, hd = 8, 2, 64
    kv_len, T = 50, 5
    pool = 6
    table = [4, 0, 5, 2]
    KP = rng.standard_normal((pool, 16, kvh, hd)).astype(np.float16)
    VP = rng.standard_normal((pool, 16, kvh, hd)).astype(np.float16)
    kbs = [backend.upload(KP[i]) for i in range(pool)]
    vbs = [backend.upload(VP[i]) for i in range(pool)]
    q = rng.standard_normal((T, qh, hd)).astype(np.float16)
    tq_ = up16(backend, q)
    out = backend.alloc([T, qh, hd], DType.FP16)
    backend.attention_paged(tq_, table, kbs, vbs, kvh, kv_len, kv_len - T, out)
    got = backend.download(out)
    for t in range(T):
        want = oracle.paged_attention(q[t], np.array(table, np.int32), kv_len - T + t + 1, KP,
                                      VP, kvh)
        assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"attention_paged token {t}")
    with pytest.raises(InvalidShape, match="block id"):
        backend.attention_paged(tq_, [4, 0, 9, 2], kbs, vbs, kvh, kv_len, kv_len - T, out)
    with pytest.raises(InvalidShape, match="block table"):
        backend.attention_paged(tq_, [4, 0], kbs, vbs, kvh, kv_len, kv_len - T, out)
    for t in kbs + vbs + [tq_, out]:
        backend.free(t)


def test_registered_page_pools(backend):
    """fhip_page_pool_create: pooled attention gives the per-call entries' exact outputs and
    stages only the block table; wrong pools are refused on the host."""
    rng = np.random.default_rng(6)
    qh, kvh, hd = 8, 2, 128
    kv_len, T = 70, 3
    pool = 7
    table = [5, 0, 6, 2, 3]
    KP = rng.standard_normal((pool, 16, kvh, hd)).astype(np.float16)
    VP = rng.standard_normal((pool, 16, kvh, hd)).astype(np.float16)
    kbs = [backend.upload(KP[i]) for i in range(pool)]
    vbs = [backend.upload(VP[i]) for i in range(pool)]
    q = rng.standard_normal((T, qh, hd)).astype(np.float16)
    tq_ = up16(backend, q)
    o1 = backend.alloc([T, qh, hd], DType.FP16)
    o2 = backend.alloc([T, qh, hd], DType.FP16)
    backend.attention_paged(tq_, table, kbs, vbs, kvh, kv_len, kv_len - T, o1)
    h = backend.page_pool_create(kbs, vbs)
    backend.attention_paged_pool(tq_, table, h, kvh, kv_len, kv_len - T, o2)
    assert np.array_equal(backend.download(o1), backend.download(o2))
    with pytest.raises(InvalidShape, match="block id"):
        backend.attention_paged_pool(tq_, [5, 0, 9, 2, 3], h, kvh, kv_len, kv_len - T, o2)

    # TurboQuant pool: (K packed, K norms, V packed, V norms)
    kb, vb = 4, 2
    pdk, pdv = oracle.packed_dim(hd, kb), oracle.packed_dim(hd, vb)
    lists = [rng.integers(0, 256, (pool, 16, kvh * pdk)).astype(np.uint8),
             np.full((pool, 16, kvh), np.float16(2.0)),
             rng.integers(0, 256, (pool, 16, kvh * pdv)).astype(np.uint8),
             np.full((pool, 16, kvh), np.float16(3.0))]
    tls = [[backend.upload(a[i]) for i in range(pool)] for a in lists]
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc, vc = tq.codebook(hd, kb)[0], tq.codebook(hd, vb)[0]
    tkr, tvr, tkc, tvc = (backend.upload(a) for a in (krot, vrot, kc, vc))
    with pytest.raises(InvalidShape, match="block lists"):  # the FP16 pool has 2 lists
        backend.attention_paged_tq_pool(tq_, table, h, tkr, tvr, tkc, tvc, kb, vb, kvh, kv_len,
                                        kv_len - T, o2)
    backend.attention_paged_tq(tq_, table, *tls, tkr, tvr, tkc, tvc, kb, vb, kvh, kv_len,
                               kv_len - T, o1)
    h4 = backend.page_pool_create(*tls)
    backend.attention_paged_tq_pool(tq_, table, h4, tkr, tvr, tkc, tvc, kb, vb, kvh, kv_len,
                                    kv_len - T, o2)
    assert np.array_equal(backend.download(o1), backend.download(o2))
    with pytest.raises(InvalidShape, match="need"):  # twice the kv heads: blocks too small
        backend.attention_paged_tq_pool(tq_, table, h4, tkr, tvr, tkc, tvc, kb, vb, 2 * kvh,
                                        kv_len, kv_len - T, o2)
    with pytest.raises(BackendError, match="registered page pool"):
        backend.free(kbs[0])  # still referenced by pool h
    backend.page_pool_destroy(h)
    backend.page_pool_destroy(h4)
    with pytest.raises(TensorNotFound):
        backend.page_pool_destroy(h)
    for t in kbs + vbs + [x for l in tls for x in l] + [tq_, o1, o2, tkr, tvr, tkc, tvc]:
        backend.free(t)

"""The TurboQuant KV cache manager's device path through the handle runtime, over per-block
tensors as QuantizedKvCacheManager allocates them (crates/fracture-engine/src/
quantized_paged_kv_cache.rs:82-133):

  * Backend::turboquant_compress / tq_dequantize through the backend's cached plans: bytes
    pinned against the oracle on the kernel's own rotated vectors, and the plan rebuilt after
    the rotation tensor is rewritten;
  * fhip_tq_append_kv (append_kv for one layer, quantized_paged_kv_cache.rs:404-500): the page
    bytes equal the oracle's quantize-pack of the kernel's rotated vectors, token by token in
    the reference's page layout, across page boundaries and successive appends; slots it must
    not write keep their contents;
  * fhip_attention_paged_tq_batched: a whole decode batch over a registered pool in one call,
    against the oracle and bit for bit against one fhip_attention_paged_tq_pool call per
    sequence (the engine's per-sequence dispatch, batched.rs:145-194); and the decode-attention
    benchmark workload (B=64, 32/8 heads, K4/V4, context U[1024,32768]) built with append_kv
    and checked against the oracle.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from fracture_amd import DType, InvalidShape
from fracture_amd import kernels as K
from fracture_amd import turboquant as tq

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def kernel_y(x16, rot):
    """The compress kernel's own fp32 rotated unit vectors for x16 [N, H, hd]."""
    dev = torch.device("cuda:0")
    N, H, hd = x16.shape
    y = torch.empty((N * H, hd), dtype=torch.float32, device=dev)
    yn = torch.empty(N * H, dtype=torch.float16, device=dev)
    K.tq_rotate(torch.from_numpy(np.ascontiguousarray(x16)).to(dev),
                torch.from_numpy(rot).to(dev), y, yn)
    torch.cuda.synchronize()
    return y.cpu().numpy(), yn.cpu().numpy()


@pytest.mark.parametrize("writer", ["copy_to_device", "add", "copy_rows"])
def test_planned_trait_compress_and_rebuild(backend, writer):
    """The backend's cached plan for a (rotation, codebook) pair is dropped by any op that
    writes either tensor: the next call rebuilds it from the new contents."""
    rng = np.random.default_rng(11)
    N, H, hd, bits = 70, 8, 128, 4
    x = (rng.standard_normal((N, H, hd)) * 3).astype(np.float16)
    r1, r2 = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    cent = tq.codebook(hd, bits)[0]
    tx, tr, tc = backend.upload(x), backend.upload(r1), backend.upload(cent)
    pd = K.packed_dim(hd, bits)
    packed = backend.alloc([N, H * pd], DType.INT8)
    norms = backend.alloc([N, H], DType.FP16)
    out = backend.alloc([N, H, hd], DType.FP16)
    for rot in (r1, r2):
        if rot is r2:  # same tensor id, new contents: the plan is rebuilt
            if writer == "copy_to_device":
                backend.copy_to_device(tr, rot)
            else:
                src = backend.upload(rot)
                if writer == "add":
                    zero = backend.upload(np.zeros_like(rot))
                    backend.add(src, zero, tr)  # exact in fp32
                    backend.free(zero)
                else:
                    backend.copy_rows(src, tr, 0, 0, hd)
                backend.synchronize()
                backend.free(src)
        for _ in range(2):  # second call reuses the cached plan
            backend.turboquant_compress(tx, tr, tc, bits, packed, norms)
            y, yn = kernel_y(x, rot)
            pk = backend.download(packed).reshape(N * H, pd)
            assert np.array_equal(pk, oracle.tq_quantize_pack(y, cent, bits))
            assert np.array_equal(backend.download(norms).reshape(-1).view(np.uint16),
                                  yn.view(np.uint16))
            backend.tq_dequantize(packed, norms, tr, tc, bits, out)
            want = oracle.tq_dequant(pk, yn, rot, cent, bits, hd)
            assert_close(backend.download(out).reshape(-1, hd).astype(np.float32),
                         want.astype(np.float32), 1e-3, 1e-3, "planned dequantize")
    for t in (tx, tr, tc, packed, norms, out):
        backend.free(t)


def make_pool(backend, P, kvh, hd, kb, vb, fill=0xA5):
    """P blocks of (K packed, K norms, V packed, V norms) per-block tensors, pre-filled."""
    pdk, pdv = K.packed_dim(hd, kb), K.packed_dim(hd, vb)
    shapes = [([16, kvh * pdk], DType.INT8), ([16, kvh], DType.FP16),
              ([16, kvh * pdv], DType.INT8), ([16, kvh], DType.FP16)]
    lists = []
    for shape, dt in shapes:
        lst = []
        for _ in range(P):
            t = backend.alloc(shape, dt)
            backend.copy_to_device(t, np.full(t.size_bytes(), fill, np.uint8))
            lst.append(t)
        lists.append(lst)
    return lists, backend.page_pool_create(*lists)


@pytest.mark.parametrize("hd,kb,vb", [(128, 4, 2), (64, 3, 3)])
def test_append_kv_into_pool(backend, hd, kb, vb):
    """Prefill of 37 tokens, one decode token, then 20 more (crossing two page boundaries):
    each token's page rows equal the oracle's quantize-pack of the kernel's rotated vectors;
    slots past the last token keep their fill."""
    rng = np.random.default_rng(hd + kb)
    kvh, P = 4, 7
    lists, pool = make_pool(backend, P, kvh, hd, kb, vb)
    table = [5, 1, 6, 0]
    krot, vrot = tq.rotation_matrix(hd, 42 + hd), tq.rotation_matrix(hd, 542 + hd)
    kc, vc = tq.codebook(hd, kb)[0], tq.codebook(hd, vb)[0]
    tkr, tvr, tkc, tvc = (backend.upload(a) for a in (krot, vrot, kc, vc))
    ks, vs = [], []
    pos = 0
    for n in (37, 1, 20):
        k = (rng.standard_normal((n, kvh, hd)) * np.exp(rng.normal(0, 0.5, (n, 1, 1)))).astype(np.float16)
        v = (rng.standard_normal((n, kvh, hd)) * 2).astype(np.float16)
        tk, tv = backend.upload(k), backend.upload(v)
        backend.tq_append_kv(pool, tk, tv, tkr, tvr, tkc, tvc, kb, vb, table, pos)
        backend.free(tk)
        backend.free(tv)
        ks.append(k)
        vs.append(v)
        pos += n
    k, v = np.concatenate(ks), np.concatenate(vs)
    pdk, pdv = K.packed_dim(hd, kb), K.packed_dim(hd, vb)
    blocks = [[backend.download(t) for t in lst] for lst in lists]
    for x, rot, cent, bits, pd, li in ((k, krot, kc, kb, pdk, 0), (v, vrot, vc, vb, pdv, 2)):
        y, yn = kernel_y(x, rot)
        want = oracle.tq_quantize_pack(y, cent, bits).reshape(pos, kvh * pd)
        wn = yn.reshape(pos, kvh)
        for t in range(pos):
            p, s = table[t // 16], t % 16
            assert np.array_equal(blocks[li][p].reshape(16, -1)[s], want[t]), f"token {t} codes"
            assert np.array_equal(blocks[li + 1][p].reshape(16, kvh).view(np.uint16)[s],
                                  wn[t].view(np.uint16)), f"token {t} norms"
        # untouched: slots after the last token, and blocks outside the table
        last = table[(pos - 1) // 16]
        assert (blocks[li][last].reshape(16, -1)[pos % 16:] == 0xA5).all()
        for p in set(range(P)) - set(table):
            assert (blocks[li][p] == 0xA5).all()
    with pytest.raises(InvalidShape, match="block table"):
        tk = backend.upload(k[:10])
        try:
            backend.tq_append_kv(pool, tk, tk, tkr, tvr, tkc, tvc, kb, vb, table, 60)
        finally:
            backend.free(tk)
    backend.page_pool_destroy(pool)
    for t in [x for l in lists for x in l] + [tkr, tvr, tkc, tvc]:
        backend.free(t)


def host_pool(lists, backend):
    return [np.stack([backend.download(t) for t in lst]) for lst in lists]


@pytest.mark.parametrize("hd,kb,vb", [(128, 4, 4), (128, 4, 2), (64, 3, 3)])
def test_attention_batched_pool(backend, hd, kb, vb):
    """One batched call over a registered pool equals the oracle and, bit for bit, one pooled
    call per sequence (T=1 at its last position); calls that alternate two batches for more
    than a turn of the host staging ring each repeat their batch's output bit for bit."""
    rng = np.random.default_rng(12)
    qh, kvh = 32, 8
    lens = [1, 17, 1030, 2100, 40, 3000]
    nbs = [(n + 15) // 16 for n in lens]
    P = sum(nbs) + 3
    perm = rng.permutation(P).tolist()
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at:at + nb])
        at += nb
    lists, pool = make_pool(backend, P, kvh, hd, kb, vb)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc, vc = tq.codebook(hd, kb)[0], tq.codebook(hd, vb)[0]
    tkr, tvr, tkc, tvc = (backend.upload(a) for a in (krot, vrot, kc, vc))
    for n, tab in zip(lens, tables):
        k = (rng.standard_normal((n, kvh, hd)) * np.exp(rng.normal(0, 0.5, (n, 1, 1)))).astype(np.float16)
        v = rng.standard_normal((n, kvh, hd)).astype(np.float16)
        tk, tv = backend.upload(k), backend.upload(v)
        backend.tq_append_kv(pool, tk, tv, tkr, tvr, tkc, tvc, kb, vb, tab, 0)
        backend.free(tk)
        backend.free(tv)
    B = len(lens)
    q = rng.standard_normal((B, qh, hd)).astype(np.float16)
    tq_ = backend.upload(q)
    out = backend.alloc([B, qh, hd], DType.FP16)
    backend.attention_paged_tq_batched(tq_, tables, lens, pool, tkr, tvr, tkc, tvc, kb, vb, kvh,
                                       out)
    got = backend.download(out)
    hp = host_pool(lists, backend)
    for b in range(B):
        q1, o1 = backend.upload(q[b:b + 1]), backend.alloc([1, qh, hd], DType.FP16)
        backend.attention_paged_tq_pool(q1, tables[b], pool, tkr, tvr, tkc, tvc, kb, vb, kvh,
                                        lens[b], lens[b] - 1, o1)
        one = backend.download(o1)[0]
        backend.free(q1)
        backend.free(o1)
        assert np.array_equal(got[b].view(np.uint16), one.view(np.uint16)), f"sequence {b}"
        tb = np.array(tables[b], np.int32)
        want = oracle.tq_attention(q[b], tb, lens[b], *hp, krot, vrot, kc, vc, kb, vb, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"sequence {b} (len {lens[b]})")
    with pytest.raises(InvalidShape, match="outside the pool"):
        bad = [list(t) for t in tables]
        bad[2][3] = P + 1
        backend.attention_paged_tq_batched(tq_, bad, lens, pool, tkr, tvr, tkc, tvc, kb, vb, kvh,
                                           out)
    # the C entry reads the host arrays only up to num_seqs, which must equal q's rows
    import ctypes as C
    from fracture_amd import _lib
    bt = np.full((B, max(nbs)), -1, np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    lens_u = np.array(lens, np.uint32)
    rc = _lib.load().fhip_attention_paged_tq_batched(
        backend._h, C.byref(tq_._c()), bt.ctypes.data, B - 1, bt.shape[1], lens_u.ctypes.data,
        pool, C.byref(tkr._c()), C.byref(tvr._c()), C.byref(tkc._c()), C.byref(tvc._c()), kb, vb,
        kvh, C.byref(out._c()))
    assert rc == 2 and b"sequences in the block tables" in _lib.load().fhip_last_error()
    # the block table and lengths travel through the backend's ring of 16 host staging slots,
    # read by the device in place: alternate two different batches for more than a turn of
    # the ring, queued back to back, and each call must give its batch's first output again
    lens2 = [3000, 1, 1030]
    tables2 = [tables[5], tables[0], tables[2]]
    q2 = backend.upload(q[:3])
    first = {}
    outs = []
    for i in range(20):
        o = backend.alloc([B if i % 2 == 0 else 3, qh, hd], DType.FP16)
        if i % 2 == 0:
            backend.attention_paged_tq_batched(tq_, tables, lens, pool, tkr, tvr, tkc, tvc, kb,
                                               vb, kvh, o)
        else:
            backend.attention_paged_tq_batched(q2, tables2, lens2, pool, tkr, tvr, tkc, tvc, kb,
                                               vb, kvh, o)
        outs.append(o)
    for i, o in enumerate(outs):
        h = backend.download(o).view(np.uint16)
        first.setdefault(i % 2, h)
        assert np.array_equal(h, first[i % 2]), f"call {i}"
        backend.free(o)
    assert np.array_equal(first[0], got.view(np.uint16))
    for j in range(3):
        tb = np.array(tables2[j], np.int32)
        want = oracle.tq_attention(q[j], tb, lens2[j], *hp, krot, vrot, kc, vc, kb, vb, kvh)
        assert_close(first[1][j].view(np.float16).astype(np.float32), want.astype(np.float32),
                     1e-3, 1e-3, f"second batch, sequence {j}")
    backend.free(q2)
    backend.page_pool_destroy(pool)
    for t in [x for l in lists for x in l] + [tq_, out, tkr, tvr, tkc, tvc]:
        backend.free(t)


def test_batched_pool_error_order(backend):
    """fhip_attention_paged_tq_batched names the first failing sequence in row order, whether
    its failure is a block id outside the pool or a length past the table's width; block ids
    past a sequence's used blocks are neither read nor checked; and after a rejected call
    (an id error is found once the table is staged, so it holds a slot of the staging ring)
    more than a turn of the ring later every call still gives the first call's output."""
    kvh, hd, qh, kb, vb, P = 2, 64, 4, 4, 4, 8
    lists, pool = make_pool(backend, P, kvh, hd, kb, vb)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc = tq.codebook(hd, kb)[0]
    tkr, tvr, tc = (backend.upload(a) for a in (krot, vrot, kc))
    rng = np.random.default_rng(3)
    q = backend.upload(rng.standard_normal((3, qh, hd)).astype(np.float16))
    out = backend.alloc([3, qh, hd], DType.FP16)
    good = np.array([[0, 1], [2, 3], [4, 5]], np.int32)
    lens = np.array([20, 32, 5], np.uint32)

    def call(table, ls):
        backend.attention_paged_tq_batched(q, table, ls, pool, tkr, tvr, tc, tc, kb, vb, kvh, out)

    call(good, lens)
    ref = backend.download(out).view(np.uint16).copy()
    bad = good.copy()
    bad[0, 1] = P  # sequence 0: an id outside the pool; sequence 1: 33 positions in 2 blocks
    with pytest.raises(InvalidShape, match=r"sequence 0: block id 8 outside the pool of 8"):
        call(bad, np.array([20, 33, 5], np.uint32))
    bad = good.copy()
    bad[1, 0] = -1  # sequence 0: 33 positions in 2 blocks; sequence 1: a negative id
    with pytest.raises(InvalidShape, match=r"sequence 0: 33 positions in 2 blocks"):
        call(bad, np.array([33, 32, 5], np.uint32))
    bad = good.copy()
    bad[2, 0] = P + 5  # the last sequence only
    with pytest.raises(InvalidShape, match=r"sequence 2: block id 13 outside the pool of 8"):
        call(bad, lens)
    loose = good.copy()
    loose[2, 1] = -7  # 5 positions use block 0 of the row only
    for i in range(20):
        call(loose, lens)
        assert np.array_equal(backend.download(out).view(np.uint16), ref), f"call {i}"
    backend.page_pool_destroy(pool)
    for t in [x for l in lists for x in l] + [q, out, tkr, tvr, tc]:
        backend.free(t)


def test_batched_pool_c5_workload(backend):
    """The decode-attention benchmark workload through the handle runtime, as the engine would
    drive it: per-block tensors registered as a pool, each sequence's K/V written with
    append_kv, then one batched decode call; every sequence checked against the oracle on a
    host copy of the pool (one query head per kv head, all heads for the two longest)."""
    lens = np.random.default_rng(5).integers(1024, 32769, 64).astype(np.int64)
    B, qh, kvh, hd = 64, 32, 8, 128
    nbs = (lens + 15) // 16
    P = int(nbs.sum())
    rng = np.random.default_rng(13)
    perm = rng.permutation(P)
    tables, at = [], 0
    for nb in nbs:
        tables.append(perm[at:at + nb].tolist())
        at += nb
    print(f"allocating {4 * P} block tensors", flush=True)
    lists = [[backend.alloc(shape, dt) for _ in range(P)] for shape, dt in
             (([16, kvh * 64], DType.INT8), ([16, kvh], DType.FP16),
              ([16, kvh * 64], DType.INT8), ([16, kvh], DType.FP16))]
    pool = backend.page_pool_create(*lists)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    cent = tq.codebook(hd, 4)[0]
    tkr, tvr, tc = (backend.upload(a) for a in (krot, vrot, cent))
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(14)
    # K/V written per sequence through append_kv, in chunks as prefill would
    print("appending K/V", flush=True)
    host = [np.zeros((P, 16, kvh * 64), np.uint8), np.zeros((P, 16, kvh), np.float16),
            np.zeros((P, 16, kvh * 64), np.uint8), np.zeros((P, 16, kvh), np.float16)]
    for b in range(B):
        n = int(lens[b])
        scale = torch.exp(torch.randn((n, 1, 1), generator=g, device=dev) * 0.5)
        kx = (torch.randn((n, kvh, hd), generator=g, device=dev) * scale).to(torch.float16)
        vx = (torch.randn((n, kvh, hd), generator=g, device=dev) * scale).to(torch.float16)
        tk, tv = backend.alloc([n, kvh, hd], DType.FP16), backend.alloc([n, kvh, hd], DType.FP16)
        backend.copy_to_device(tk, kx.cpu().numpy())
        backend.copy_to_device(tv, vx.cpu().numpy())
        backend.tq_append_kv(pool, tk, tv, tkr, tvr, tc, tc, 4, 4, tables[b], 0)
        # the oracle's copy of the pages: the same bytes from the flat compressor
        for x, rot, li in ((tk, tkr, 0), (tv, tvr, 2)):
            pk = backend.alloc([n, kvh * 64], DType.INT8)
            nm = backend.alloc([n, kvh], DType.FP16)
            backend.turboquant_compress(x, rot, tc, 4, pk, nm)
            pkh = backend.download(pk).reshape(n, -1)
            nmh = backend.download(nm).reshape(n, kvh)
            t = np.arange(n)
            pages = np.asarray(tables[b])[t // 16]
            host[li][pages, t % 16] = pkh
            host[li + 1][pages, t % 16] = nmh
            backend.free(pk)
            backend.free(nm)
        backend.free(tk)
        backend.free(tv)
    # spot check: the pool's own bytes for two blocks equal the host copy
    for p in (int(tables[0][0]), int(tables[-1][-1])):
        assert np.array_equal(backend.download(lists[0][p]).reshape(16, -1), host[0][p])
        assert np.array_equal(backend.download(lists[3][p]).reshape(16, kvh).view(np.uint16),
                              host[3][p].view(np.uint16))
    q = rng.standard_normal((B, qh, hd)).astype(np.float16)
    tq_ = backend.upload(q)
    out = backend.alloc([B, qh, hd], DType.FP16)
    print("batched decode", flush=True)
    backend.attention_paged_tq_batched(tq_, tables, lens.tolist(), pool, tkr, tvr, tc, tc, 4, 4,
                                       kvh, out)
    got = backend.download(out)
    full = set(np.argsort(lens)[-2:].tolist())

    def run(b):
        tb = np.asarray(tables[b], np.int32)
        ranges = [(0, qh)] if b in full else [(4 * gg + b % 4, 4 * gg + b % 4 + 1)
                                               for gg in range(kvh)]
        return b, [(h0, h1, oracle.tq_attention(q[b], tb, int(lens[b]), *host, krot, vrot, cent,
                                                cent, 4, 4, kvh, heads=(h0, h1)))
                   for h0, h1 in ranges]

    print("oracle", flush=True)
    with ThreadPoolExecutor(THREADS) as ex:
        for b, res in ex.map(run, range(B)):
            for h0, h1, want in res:
                assert_close(got[b, h0:h1].astype(np.float32), want[h0:h1].astype(np.float32),
                             1e-3, 1e-3, f"sequence {b} (len {lens[b]}) heads {h0}..{h1 - 1}")
    backend.page_pool_destroy(pool)
    print("freeing", flush=True)
    for t in [x for l in lists for x in l] + [tq_, out, tkr, tvr, tc]:
        backend.free(t)

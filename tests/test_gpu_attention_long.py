"""GPU parity of TurboQuant paged attention at long contexts against the oracle's restatement
of attention_paged_tq.cu:56-257 (fp16 output, |a - e| <= 1e-3 + 1e-3|e|).

  * the decode-attention benchmark workload itself: B=64, 32 q / 8 kv heads, head_dim 128,
    K4/V4, context lengths uniform in [1024, 32768] (the benchmark's seeded draw), pages
    scattered by a permuted block table; sequences past 16,384 positions exercise the split
    combine's second group of 16 splits;
  * the reference-signature launcher (per-page pointer arrays, the MFMA kernel's pointer-page
    form) at K4/V4 / head_dim 128 for decode and causal prefill beyond 16,384 positions, its
    caller-workspace form, and the same call through Backend::attention_paged_tq and a
    registered page pool;
  * head_dim 64 and 256 (the VALU split kernel; at 256 the combine reads the rotation from
    global memory).

Pages hold real compressed K/V: the GPU compressor writes them (its bytes are pinned against
the oracle in test_gpu_turboquant.py); the attention oracle then reads the same bytes. Slots
past a sequence's end and pages outside every block table hold random bytes, NaN norms
included: the kernels must never read them.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from fracture_amd import kernels as K
from fracture_amd import turboquant as tq

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def c5_lengths():
    """The decode-attention benchmark's context lengths (numpy seed 5)."""
    return np.random.default_rng(5).integers(1024, 32769, 64).astype(np.int32)


def gpu_pool(dev, seed, lens, kvh, hd, kbits, vbits, extra_pages=3):
    """K/V for every sequence compressed on the GPU into shared, permuted page pools.
    Returns device pools, host copies, the block table and the TurboQuant tables."""
    lens = np.asarray(lens, np.int64)
    rng = np.random.default_rng(seed)
    nbs = (lens + 15) // 16
    P = int(nbs.sum()) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    maxb = max(int(nbs.max()), 1)
    table = np.full((len(lens), maxb), -7, np.int32)
    dst = []
    at = 0
    for b, n in enumerate(lens):
        pages = perm[at:at + nbs[b]]
        at += nbs[b]
        table[b, :nbs[b]] = pages
        t = np.arange(n)
        dst.append(pages[t // 16].astype(np.int64) * 16 + t % 16)
    dst = torch.from_numpy(np.concatenate(dst)).to(dev)
    N = int(lens.sum())
    pdk, pdv = K.packed_dim(hd, kbits), K.packed_dim(hd, vbits)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc, vc = tq.codebook(hd, kbits)[0], tq.codebook(hd, vbits)[0]
    d = {n: torch.from_numpy(a).to(dev) for n, a in
         (("krot", krot), ("vrot", vrot), ("kc", kc), ("vc", vc))}
    pools = {}
    for name, rot, cent, bits, pd in (("K", d["krot"], d["kc"], kbits, pdk),
                                      ("V", d["vrot"], d["vc"], vbits, pdv)):
        # garbage everywhere first: random code bytes, random fp16 norms (NaN and Inf among them)
        packed = torch.randint(0, 256, (P, 16, kvh * pd), generator=g, device=dev,
                               dtype=torch.uint8)
        norms = torch.randint(-32768, 32767, (P, 16, kvh), generator=g, device=dev,
                              dtype=torch.int16).view(torch.float16)
        scale = torch.exp(torch.randn((N, 1, 1), generator=g, device=dev) * 0.5)
        x = (torch.randn((N, kvh, hd), generator=g, device=dev) * scale).to(torch.float16)
        fp = torch.empty((N, kvh * pd), dtype=torch.uint8, device=dev)
        fn = torch.empty((N, kvh), dtype=torch.float16, device=dev)
        K.tq_compress(x, rot, cent, bits, fp, fn)
        packed.view(P * 16, -1)[dst] = fp
        norms.view(P * 16, -1)[dst] = fn
        del x, fp, fn
        pools[name + "P"], pools[name + "N"] = packed, norms
    torch.cuda.synchronize()
    host = {k: v.cpu().numpy() for k, v in pools.items()}
    return dict(dev=pools, host=host, table=table, krot=krot, vrot=vrot, kc=kc, vc=vc, d=d,
                P=P, maxb=maxb)


def oracle_attention(pool, q, qi, clen, kbits, vbits, kvh, heads=None, table_row=None):
    h = pool["host"]
    row = pool["table"][qi] if table_row is None else table_row
    return oracle.tq_attention(q, row, clen, h["KP"], h["KN"], h["VP"], h["VN"], pool["krot"],
                               pool["vrot"], pool["kc"], pool["vc"], kbits, vbits, kvh, heads)


def test_c5_decode_workload_vs_oracle(dev):
    """The benchmark's K4/V4 decode-attention workload, checked sequence by sequence: all 32
    heads of the 6 longest sequences, and for every other sequence one query head of each kv
    head (head 4g + b % 4)."""
    lens = c5_lengths()
    assert lens.max() > 16 * 1024
    B, qh, kvh, hd = 64, 32, 8, 128
    pool = gpu_pool(dev, 50, lens, kvh, hd, 4, 4)
    g = torch.Generator(device=dev)
    g.manual_seed(51)
    q = torch.randn((B, qh, hd), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    p = pool["dev"]
    K.attention_tq_decode(out, q, torch.from_numpy(pool["table"]).to(dev),
                          torch.from_numpy(lens).to(dev), p["KP"], p["KN"], p["VP"], p["VN"],
                          pool["d"]["krot"], pool["d"]["vrot"], pool["d"]["kc"], pool["d"]["vc"],
                          4, 4, kvh)
    torch.cuda.synchronize()
    got, qn = out.cpu().numpy(), q.cpu().numpy()
    full = set(np.argsort(lens)[-6:].tolist())
    jobs = []
    for b in range(B):
        if b in full:
            jobs.append((b, [(0, qh)]))
        else:
            jobs.append((b, [(4 * gg + b % 4, 4 * gg + b % 4 + 1) for gg in range(kvh)]))

    def run(job):
        b, ranges = job
        res = []
        for h0, h1 in ranges:
            res.append((h0, h1, oracle_attention(pool, qn[b], b, int(lens[b]), 4, 4, kvh,
                                                 heads=(h0, h1))))
        return b, res

    with ThreadPoolExecutor(THREADS) as ex:
        for b, res in ex.map(run, jobs):
            for h0, h1, want in res:
                assert_close(got[b, h0:h1].astype(np.float32), want[h0:h1].astype(np.float32),
                             1e-3, 1e-3, f"sequence {b} (len {lens[b]}) heads {h0}..{h1 - 1}")


def _ptr_table(pool, dev):
    """Per-page device address arrays, as the reference passes them."""
    return [torch.tensor([t[i].data_ptr() for i in range(pool["P"])], dtype=torch.int64,
                         device=dev) for t in (pool["dev"]["KP"], pool["dev"]["KN"],
                                               pool["dev"]["VP"], pool["dev"]["VN"])]


@pytest.mark.parametrize("kv_len,T", [(17000, 1), (32768, 5), (16385, 3)])
def test_reference_interface_mfma_long(dev, kv_len, T):
    """fhip_launch_attention_paged_tq at K4/V4 / head_dim 128 (MFMA kernel, pointer pages):
    T queries at start_pos = kv_len - T, causal; beyond 16,384 positions. The caller-workspace
    form gives the same bytes."""
    qh, kvh, hd = 32, 8, 128
    pool = gpu_pool(dev, kv_len + T, [kv_len], kvh, hd, 4, 4, extra_pages=5)
    ptrs = _ptr_table(pool, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(T)
    q = torch.randn((T, qh, hd), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    out2 = torch.empty_like(q)
    table = torch.from_numpy(pool["table"][0]).to(dev)
    d = pool["d"]
    lib = K._L()
    s = torch.cuda.current_stream().cuda_stream
    start = kv_len - T
    args = (q.data_ptr(), table.data_ptr(), ptrs[0].data_ptr(), ptrs[1].data_ptr(),
            ptrs[2].data_ptr(), ptrs[3].data_ptr(), d["krot"].data_ptr(), d["vrot"].data_ptr(),
            d["kc"].data_ptr(), d["vc"].data_ptr(), T, qh, kvh, hd, kv_len, start, 4, 4, 64, 64)
    assert lib.fhip_launch_attention_paged_tq(out.data_ptr(), *args, s) == 0
    wsb = lib.fhip_attention_tq_workspace_bytes(T, qh, hd, (kv_len + 15) // 16)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    assert lib.fhip_launch_attention_paged_tq_ws(out2.data_ptr(), *args, ws.data_ptr(), wsb - 1,
                                                 s) != 0  # workspace too small: refused
    assert lib.fhip_launch_attention_paged_tq_ws(out2.data_ptr(), *args, ws.data_ptr(), wsb, s) == 0
    torch.cuda.synchronize()
    got, qn = out.cpu().numpy(), q.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), out2.cpu().numpy().view(np.uint16))

    def run(t):
        return t, oracle_attention(pool, qn[t], 0, min(start + t + 1, kv_len), 4, 4, kvh)

    with ThreadPoolExecutor(THREADS) as ex:
        for t, want in ex.map(run, range(T)):
            assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                         f"kv_len {kv_len} token {t}")


@pytest.mark.parametrize("qh,kvh,T,kv_len", [(32, 8, 40, 2060), (16, 8, 13, 1030),
                                             (8, 8, 20, 530), (64, 8, 6, 300),
                                             (32, 8, 131, 1500)])
@pytest.mark.parametrize("vbits", [4, 2])
def test_prefill_token_groups_vs_oracle(dev, qh, kvh, T, kv_len, vbits):
    """Causal prefill through fhip_launch_attention_paged_tq (K4 with V4 or V2, head_dim 128): the MFMA
    kernel gives 8 / G consecutive queries one set of MFMA columns (G = 4, 2 and 1; G = 8
    keeps one query per item), with a ragged last group and causal lengths that cross a
    1024-position block, a 256-position wave split or a page inside one group. At 131 x 32
    query vectors (at least 4096) the query rotation and the unrotation of the merged outputs
    run as batched MFMA products instead of the per-8-vector kernels."""
    hd = 128
    pool = gpu_pool(dev, 7 * T + kv_len + vbits, [kv_len], kvh, hd, 4, vbits, extra_pages=4)
    ptrs = _ptr_table(pool, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(T + qh)
    q = torch.randn((T, qh, hd), generator=g, device=dev).to(torch.float16)
    out = torch.empty_like(q)
    table = torch.from_numpy(pool["table"][0]).to(dev)
    d = pool["d"]
    start = kv_len - T
    assert K._L().fhip_launch_attention_paged_tq(
        out.data_ptr(), q.data_ptr(), table.data_ptr(), ptrs[0].data_ptr(), ptrs[1].data_ptr(),
        ptrs[2].data_ptr(), ptrs[3].data_ptr(), d["krot"].data_ptr(), d["vrot"].data_ptr(),
        d["kc"].data_ptr(), d["vc"].data_ptr(), T, qh, kvh, hd, kv_len, start, 4, vbits, 64,
        hd * vbits // 8,
        torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    got, qn = out.cpu().numpy(), q.cpu().numpy()

    def run(t):
        return t, oracle_attention(pool, qn[t], 0, min(start + t + 1, kv_len), 4, vbits, kvh)

    with ThreadPoolExecutor(THREADS) as ex:
        for t, want in ex.map(run, range(T)):
            assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                         f"qh {qh} token {t} (length {start + t + 1})")


def test_trait_and_pool_mfma_long(dev, backend):
    """Backend::attention_paged_tq over per-block tensors (the cache manager's layout,
    quantized_paged_kv_cache.rs:82-133) at K4/V4 / head_dim 128 and 17,000 positions, and the
    same blocks as a registered page pool: both equal the oracle, and each other exactly."""
    from fracture_amd import DType

    qh, kvh, hd, kv_len = 32, 8, 128, 17000
    pool = gpu_pool(dev, 77, [kv_len], kvh, hd, 4, 4, extra_pages=2)
    h = pool["host"]
    lists = [[backend.upload(np.ascontiguousarray(h[n][i])) for i in range(pool["P"])]
             for n in ("KP", "KN", "VP", "VN")]
    rng = np.random.default_rng(78)
    q = rng.standard_normal((1, qh, hd)).astype(np.float16)
    tq_ = backend.upload(q)
    o1 = backend.alloc([1, qh, hd], DType.FP16)
    o2 = backend.alloc([1, qh, hd], DType.FP16)
    tkr, tvr, tkc, tvc = (backend.upload(a) for a in (pool["krot"], pool["vrot"], pool["kc"],
                                                       pool["vc"]))
    table = [int(x) for x in pool["table"][0]]
    backend.attention_paged_tq(tq_, table, *lists, tkr, tvr, tkc, tvc, 4, 4, kvh, kv_len,
                               kv_len - 1, o1)
    hp = backend.page_pool_create(*lists)
    backend.attention_paged_tq_pool(tq_, table, hp, tkr, tvr, tkc, tvc, 4, 4, kvh, kv_len,
                                    kv_len - 1, o2)
    a, b = backend.download(o1), backend.download(o2)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    want = oracle_attention(pool, q[0], 0, kv_len, 4, 4, kvh)
    assert_close(a[0].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                 "Backend::attention_paged_tq K4/V4 17000")
    backend.page_pool_destroy(hp)
    for t in [x for l in lists for x in l] + [tq_, o1, o2, tkr, tvr, tkc, tvc]:
        backend.free(t)


@pytest.mark.parametrize("hd", [64, 256])
@pytest.mark.parametrize("kbits,vbits", [(4, 2), (3, 3)])
def test_decode_head_dims(dev, hd, kbits, vbits):
    """Batched decode at head_dim 64 and 256 (VALU split kernel, combine with the rotation in
    LDS at 64 and read from global memory at 256)."""
    lens = [1, 17, 1100, 2100]
    qh, kvh = 8, 2
    pool = gpu_pool(dev, hd + kbits, lens, kvh, hd, kbits, vbits)
    rng = np.random.default_rng(hd)
    q = rng.standard_normal((len(lens), qh, hd)).astype(np.float16)
    out = torch.empty((len(lens), qh, hd), dtype=torch.float16, device=dev)
    p, d = pool["dev"], pool["d"]
    K.attention_tq_decode(out, torch.from_numpy(q).to(dev),
                          torch.from_numpy(pool["table"]).to(dev),
                          torch.from_numpy(np.array(lens, np.int32)).to(dev), p["KP"], p["KN"],
                          p["VP"], p["VN"], d["krot"], d["vrot"], d["kc"], d["vc"], kbits, vbits,
                          kvh)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(len(lens)):
        want = oracle_attention(pool, q[b], b, lens[b], kbits, vbits, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"hd {hd} sequence {b} (len {lens[b]})")

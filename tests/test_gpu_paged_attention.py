"""GPU parity of FP16 paged attention against the oracle's restatement of attention_paged.cu
(fp16 output, |a - e| <= 1e-3 + 1e-3|e|).

Covers the batched decode entry over contiguous page pools (one query per sequence,
per-sequence lengths around page and 1024-position split edges, permuted block tables, GQA
groups of 1 to 12 q heads, head_dim 32 / 64 / 128 / 256 on the MFMA kernels and 16 / 20 / 80 /
96 on the generic kernel, masked pages, empty sequences) and the reference-interface entry with
per-block pointer arrays and causal prefill queries.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from fracture_amd import kernels as K

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def build_pool(rng, lens, kvh, hd, extra_pages=3):
    """Random fp16 K/V pages for each sequence in a shared, permuted pool; unused rows hold
    garbage (large values and NaN) that must never reach the output."""
    nbs = [(n + 15) // 16 for n in lens]
    P = sum(nbs) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    kp = rng.standard_normal((P, 16, kvh, hd)).astype(np.float16)
    vp = rng.standard_normal((P, 16, kvh, hd)).astype(np.float16)
    maxb = max(max(nbs), 1)
    table = np.full((len(lens), maxb), -7, np.int32)
    at = 0
    for b, n in enumerate(lens):
        pages = perm[at:at + nbs[b]]
        at += nbs[b]
        table[b, :nbs[b]] = pages
        if n % 16:  # rows past the sequence end in its last page
            kp[pages[-1], n % 16:] = np.float16(6e4)
            vp[pages[-1], n % 16:] = np.float16(np.nan)
    return kp, vp, table


def run_decode(dev, q, table, lens, kp, vp, kvh):
    out = torch.empty(q.shape, dtype=torch.float16, device=dev)
    K.attention_paged_decode(out, dev_t(q, dev), dev_t(table, dev),
                             dev_t(np.asarray(lens, np.int32), dev), dev_t(kp, dev),
                             dev_t(vp, dev), kvh)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("hd", [32, 64, 128, 256, 16, 20, 96])
@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 8), (16, 1), (24, 2)])
def test_decode_small_contexts(dev, hd, qh, kvh):
    rng = np.random.default_rng(hd * 100 + qh + kvh)
    lens = [1, 15, 16, 17, 33, 100]
    kp, vp, table = build_pool(rng, lens, kvh, hd)
    q = (rng.standard_normal((len(lens), qh, hd)) * 2).astype(np.float16)
    got = run_decode(dev, q, table, lens, kp, vp, kvh)
    for b, n in enumerate(lens):
        want = oracle.paged_attention(q[b], table[b], n, kp, vp, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"seq {b} len {n}")


@pytest.mark.parametrize("hd", [128, 64, 80])
def test_decode_split_edges(dev, hd):
    """Lengths around the 1024-position splits: the combine merges 1 to 3 splits."""
    rng = np.random.default_rng(7 + hd)
    qh, kvh = 16, 4
    lens = [1023, 1024, 1025, 2048, 2100, 3001]
    kp, vp, table = build_pool(rng, lens, kvh, hd)
    q = (rng.standard_normal((len(lens), qh, hd)) * 3).astype(np.float16)
    got = run_decode(dev, q, table, lens, kp, vp, kvh)
    for b, n in enumerate(lens):
        want = oracle.paged_attention(q[b], table[b], n, kp, vp, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"seq {b} len {n}")


def test_decode_long_contexts(dev):
    """Llama-3.1-8B heads (32 q / 8 kv, hd 128) at contexts up to 32768 positions."""
    rng = np.random.default_rng(11)
    qh, kvh, hd = 32, 8, 128
    lens = [32768, 20000, 5000, 1]
    kp, vp, table = build_pool(rng, lens, kvh, hd, extra_pages=1)
    q = (rng.standard_normal((len(lens), qh, hd)) * 3).astype(np.float16)
    got = run_decode(dev, q, table, lens, kp, vp, kvh)
    for b, n in enumerate(lens):
        want = oracle.paged_attention(q[b], table[b], n, kp, vp, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"seq {b} len {n}")


def test_decode_empty_sequence_and_masked_pages(dev):
    """Length 0 gives zeros; a page id outside the pool masks its 16 positions, which equals
    attending to the sequence without that page."""
    rng = np.random.default_rng(12)
    qh, kvh, hd = 8, 2, 128
    lens = [0, 80, 1100]
    kp, vp, table = build_pool(rng, lens, kvh, hd)
    P = kp.shape[0]
    table[1, 2] = P + 5          # page 2 of sequence 1 (positions 32..47)
    table[2, 10] = -3            # page 10 of sequence 2 (positions 160..175)
    q = (rng.standard_normal((len(lens), qh, hd)) * 2).astype(np.float16)
    got = run_decode(dev, q, table, lens, kp, vp, kvh)
    assert not got[0].any()
    keep1 = np.delete(table[1], 2)
    want1 = oracle.paged_attention(q[1], keep1, 80 - 16, kp, vp, kvh)
    assert_close(got[1].astype(np.float32), want1.astype(np.float32), 1e-3, 1e-3, "seq 1")
    keep2 = np.delete(table[2], 10)
    want2 = oracle.paged_attention(q[2], keep2, 1100 - 16, kp, vp, kvh)
    assert_close(got[2].astype(np.float32), want2.astype(np.float32), 1e-3, 1e-3, "seq 2")


@pytest.mark.parametrize("kv_len,T,start_pos,qh,kvh,hd", [
    (90, 6, 84, 8, 2, 64), (40, 5, 38, 8, 2, 64), (1030, 3, 1027, 8, 2, 64),
    (16, 1, 15, 8, 2, 64),
    # 8 / G queries per wave: ragged last groups, groups whose lengths straddle a page or
    # the 1024-position split edge, whole prefills from position 0
    (1050, 19, 1020, 4, 4, 128), (300, 13, 0, 8, 4, 32), (1100, 11, 1019, 6, 2, 256),
    (70, 70, 0, 8, 2, 128), (2100, 9, 2040, 16, 16, 64), (50, 7, 43, 16, 2, 64),
    # 16 / G queries per wave on the MFMA prefill kernel: G = 8 (2 queries), G = 1 (16)
    (2100, 33, 2067, 32, 4, 128), (600, 37, 563, 4, 4, 64), (1030, 21, 1010, 24, 3, 32),
    # the generic kernel (other head_dims): one query per wave
    (5, 5, 0, 4, 2, 16), (1040, 9, 1031, 8, 2, 96), (40, 17, 23, 6, 3, 20)])
def test_reference_interface_prefill_causal(dev, kv_len, T, start_pos, qh, kvh, hd):
    """fhip_launch_paged_attention: T queries at start_pos.. over per-block pointer arrays;
    query i attends to min(start_pos + i + 1, kv_len) positions."""
    rng = np.random.default_rng(kv_len + T)
    kp, vp, table = build_pool(rng, [kv_len], kvh, hd, extra_pages=2)
    P = kp.shape[0]
    tk, tv = dev_t(kp, dev), dev_t(vp, dev)
    kptr = torch.tensor([tk[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
    vptr = torch.tensor([tv[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
    q = (rng.standard_normal((T, qh, hd)) * 2).astype(np.float16)
    tq_ = dev_t(q, dev)
    out = torch.empty_like(tq_)
    tb = dev_t(table[0], dev)
    K.paged_attention(out, tq_, tb, kptr, vptr, kvh, kv_len, start_pos)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    # the caller-workspace form launches the same kernels
    ws = K.attention_paged_workspace(T, qh, hd, table.shape[1], dev)
    out2 = torch.empty_like(tq_)
    K.paged_attention(out2, tq_, tb, kptr, vptr, kvh, kv_len, start_pos, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out2.cpu().numpy().view(np.uint16), got.view(np.uint16))
    for t in range(T):
        clen = min(start_pos + t + 1, kv_len)
        want = oracle.paged_attention(q[t], table[0], clen, kp, vp, kvh)
        assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"token {t}")


def test_reference_interface_rejects_unsupported_head_dim(dev):
    q = torch.zeros((1, 4, 264), dtype=torch.float16, device=dev)
    out = torch.empty_like(q)
    bt = torch.zeros(1, dtype=torch.int32, device=dev)
    ptr = torch.zeros(1, dtype=torch.int64, device=dev)
    with pytest.raises(RuntimeError):
        K.paged_attention(out, q, bt, ptr, ptr, 4, 1, 0)


@pytest.mark.parametrize("qh,kvh,hd", [(32, 8, 128), (8, 8, 64), (12, 2, 256), (4, 2, 16)])
def test_reference_interface_prefill_masked_page_and_no_blocks(dev, qh, kvh, hd):
    """Causal prefill with a negative page id in the block table: its 16 positions are masked
    for every query whose causal length covers them, which equals attending without that page
    (queries whose length ends inside it see the positions before it). With no blocks at all,
    every query returns zeros."""
    rng = np.random.default_rng(qh + hd)
    kv_len, T, start_pos = 1090, 40, 1050
    kp, vp, table = build_pool(rng, [kv_len], kvh, hd, extra_pages=2)
    P = kp.shape[0]
    tk, tv = dev_t(kp, dev), dev_t(vp, dev)
    kptr = torch.tensor([tk[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
    vptr = torch.tensor([vp_.data_ptr() for vp_ in tv], dtype=torch.int64, device=dev)
    tab = table[0].copy()
    tab[3] = -1  # positions 48..63
    q = (rng.standard_normal((T, qh, hd)) * 2).astype(np.float16)
    tq_ = dev_t(q, dev)
    out = torch.empty_like(tq_)
    K.paged_attention(out, tq_, dev_t(tab, dev), kptr, vptr, kvh, kv_len, start_pos)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    keep = np.delete(tab, 3)
    for t in range(T):
        clen = min(start_pos + t + 1, kv_len)
        want = oracle.paged_attention(q[t], keep, clen - 16, kp, vp, kvh)
        assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"token {t}")
    empty = torch.full_like(tq_, 7.0)
    K.paged_attention(empty, tq_, dev_t(tab[:0], dev), kptr, vptr, kvh, 0, 0)
    torch.cuda.synchronize()
    assert not empty.cpu().numpy().any()

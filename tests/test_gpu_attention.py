"""GPU parity of TurboQuant paged decode attention against the oracle's restatement of
attention_paged_tq.cu (fp16 output, |a - e| <= 1e-3 + 1e-3|e|).

Covers the batched decode entry over contiguous page pools (one query per sequence,
per-sequence lengths, permuted block tables, split-K merging across 1024-position splits),
the reference-interface entry with per-block pointer arrays and causal prefill queries, and
several bit-width pairs.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from fracture_amd import kernels as K
from fracture_amd import turboquant as tq

pytestmark = pytest.mark.gpu


def dev_t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def build_pool(rng, lens, kvh, hd, kbits, vbits, extra_pages=3):
    """Compress random K/V for each sequence into a shared, permuted page pool."""
    pdk, pdv = oracle.packed_dim(hd, kbits), oracle.packed_dim(hd, vbits)
    nbs = [(n + 15) // 16 for n in lens]
    P = sum(nbs) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    krot, vrot = tq.rotation_matrix(hd, 42), tq.rotation_matrix(hd, 542)
    kc, vc = tq.codebook(hd, kbits)[0], tq.codebook(hd, vbits)[0]
    KP = rng.integers(0, 256, (P, 16, kvh * pdk)).astype(np.uint8)  # garbage in unused slots
    VP = rng.integers(0, 256, (P, 16, kvh * pdv)).astype(np.uint8)
    KN = np.full((P, 16, kvh), np.float16(3.0))
    VN = np.full((P, 16, kvh), np.float16(3.0))
    maxb = max(nbs)
    table = np.full((len(lens), maxb), -7, np.int32)
    at = 0
    for b, n in enumerate(lens):
        pages = perm[at:at + nbs[b]]
        at += nbs[b]
        table[b, :nbs[b]] = pages
        if n == 0:
            continue
        k = (rng.standard_normal((n, kvh, hd)) * np.exp(rng.normal(0, 0.5, (n, 1, 1)))).astype(np.float16)
        v = (rng.standard_normal((n, kvh, hd)) * np.exp(rng.normal(0, 0.5, (n, 1, 1)))).astype(np.float16)
        kp, kn, _ = oracle.tq_compress(k, krot, kc, kbits)
        vp, vn, _ = oracle.tq_compress(v, vrot, vc, vbits)
        for t in range(n):
            p, s = pages[t // 16], t % 16
            KP[p, s] = kp.reshape(n, -1)[t]
            KN[p, s] = kn.reshape(n, kvh)[t]
            VP[p, s] = vp.reshape(n, -1)[t]
            VN[p, s] = vn.reshape(n, kvh)[t]
    return dict(KP=KP, KN=KN, VP=VP, VN=VN, table=table, krot=krot, vrot=vrot, kc=kc, vc=vc)


@pytest.mark.parametrize("kbits,vbits", [(4, 4), (4, 2), (3, 3), (8, 2)])
@pytest.mark.parametrize("lens", [[1, 15, 16, 17], [300, 1024, 1025, 2100]])
def test_decode_attention_vs_oracle(dev, kbits, vbits, lens):
    rng = np.random.default_rng(sum(lens) + kbits * 10 + vbits)
    qh, kvh, hd = 8, 2, 128
    pool = build_pool(rng, lens, kvh, hd, kbits, vbits)
    B = len(lens)
    q = rng.standard_normal((B, qh, hd)).astype(np.float16)
    out = torch.empty((B, qh, hd), dtype=torch.float16, device=dev)
    K.attention_tq_decode(out, dev_t(q, dev), dev_t(pool["table"], dev),
                          dev_t(np.array(lens, np.int32), dev), dev_t(pool["KP"], dev),
                          dev_t(pool["KN"], dev), dev_t(pool["VP"], dev), dev_t(pool["VN"], dev),
                          dev_t(pool["krot"], dev), dev_t(pool["vrot"], dev),
                          dev_t(pool["kc"], dev), dev_t(pool["vc"], dev), kbits, vbits, kvh)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(B):
        want = oracle.tq_attention(q[b], pool["table"][b], lens[b], pool["KP"], pool["KN"],
                                   pool["VP"], pool["VN"], pool["krot"], pool["vrot"],
                                   pool["kc"], pool["vc"], kbits, vbits, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3,
                     f"sequence {b} (len {lens[b]})")


def test_decode_attention_llama_heads(dev):
    # Llama-3.1-8B head layout: 32 q heads over 8 kv heads, K4/V4
    rng = np.random.default_rng(8)
    lens = [37, 1500, 3000, 16]
    qh, kvh, hd = 32, 8, 128
    pool = build_pool(rng, lens, kvh, hd, 4, 4)
    q = rng.standard_normal((len(lens), qh, hd)).astype(np.float16)
    out = torch.empty((len(lens), qh, hd), dtype=torch.float16, device=dev)
    K.attention_tq_decode(out, dev_t(q, dev), dev_t(pool["table"], dev),
                          dev_t(np.array(lens, np.int32), dev), dev_t(pool["KP"], dev),
                          dev_t(pool["KN"], dev), dev_t(pool["VP"], dev), dev_t(pool["VN"], dev),
                          dev_t(pool["krot"], dev), dev_t(pool["vrot"], dev),
                          dev_t(pool["kc"], dev), dev_t(pool["vc"], dev), 4, 4, kvh)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for b in range(len(lens)):
        want = oracle.tq_attention(q[b], pool["table"][b], lens[b], pool["KP"], pool["KN"],
                                   pool["VP"], pool["VN"], pool["krot"], pool["vrot"],
                                   pool["kc"], pool["vc"], 4, 4, kvh)
        assert_close(got[b].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3, f"seq {b}")


def test_reference_interface_prefill_causal(dev):
    """fhip_launch_attention_paged_tq: T queries at start_pos.., per-block pointer arrays."""
    rng = np.random.default_rng(21)
    qh, kvh, hd, kbits, vbits = 4, 2, 128, 4, 2
    kv_len, T = 90, 6
    start_pos = kv_len - T
    pool = build_pool(rng, [kv_len], kvh, hd, kbits, vbits, extra_pages=2)
    P = pool["KP"].shape[0]
    tKP, tKN, tVP, tVN = (dev_t(pool[n], dev) for n in ("KP", "KN", "VP", "VN"))
    ptrs = [torch.tensor([t[i].data_ptr() for i in range(P)], dtype=torch.int64, device=dev)
            for t in (tKP, tKN, tVP, tVN)]
    q = rng.standard_normal((T, qh, hd)).astype(np.float16)
    tq_ = dev_t(q, dev)
    out = torch.empty_like(tq_)
    table = dev_t(pool["table"][0], dev)
    lib = K._L()
    krot, vrot = dev_t(pool["krot"], dev), dev_t(pool["vrot"], dev)
    kc, vc = dev_t(pool["kc"], dev), dev_t(pool["vc"], dev)
    code = lib.fhip_launch_attention_paged_tq(
        out.data_ptr(), tq_.data_ptr(), table.data_ptr(), ptrs[0].data_ptr(), ptrs[1].data_ptr(),
        ptrs[2].data_ptr(), ptrs[3].data_ptr(), krot.data_ptr(), vrot.data_ptr(), kc.data_ptr(),
        vc.data_ptr(), T, qh, kvh, hd, kv_len, start_pos, kbits, vbits,
        oracle.packed_dim(hd, kbits), oracle.packed_dim(hd, vbits),
        torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for t in range(T):
        clen = min(start_pos + t + 1, kv_len)
        want = oracle.tq_attention(q[t], pool["table"][0], clen, pool["KP"], pool["KN"],
                                   pool["VP"], pool["VN"], pool["krot"], pool["vrot"],
                                   pool["kc"], pool["vc"], kbits, vbits, kvh)
        assert_close(got[t].astype(np.float32), want.astype(np.float32), 1e-3, 1e-3, f"token {t}")

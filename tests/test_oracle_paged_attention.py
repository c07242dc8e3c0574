"""Pins the oracle's FP16 paged attention (attention_paged.cu:36-170) on the CPU.

Checks, chosen so that a dropped scale, a wrong GQA head mapping, a transposed operand or a
wrong page lookup fails at least one of them:
  - the textbook float64 softmax(q K^T / sqrt(d)) V over the gathered fp16 K/V rows;
  - one position: the output is that position's V row, bit for bit (p = 1 exactly);
  - equal keys: the output is the mean of the V rows;
  - the same logical sequence stored in different physical pages gives identical output;
  - causal length 0 gives zeros (the kernel's loops do not run).
"""
import numpy as np
import pytest

import oracle


def make_pool(rng, pages, kvh, hd):
    k = rng.standard_normal((pages, 16, kvh, hd)).astype(np.float16)
    v = rng.standard_normal((pages, 16, kvh, hd)).astype(np.float16)
    return k, v


def gather(pool, table, n):
    """[n, kvh, hd] rows of positions 0..n-1 through the block table."""
    return np.stack([pool[table[t // 16], t % 16] for t in range(n)]).astype(np.float64)


def textbook(q16, k_rows, v_rows):
    qh, hd = q16.shape
    kvh = k_rows.shape[1]
    G = qh // kvh
    out = np.empty((qh, hd))
    for h in range(qh):
        K = k_rows[:, h // G, :]
        V = v_rows[:, h // G, :]
        s = K @ q16[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("qh,kvh,hd,n", [(8, 2, 32, 37), (4, 4, 64, 16), (16, 2, 128, 100),
                                         (6, 3, 32, 1)])
def test_textbook_attention(qh, kvh, hd, n):
    rng = np.random.default_rng(qh * 1000 + n)
    pages = (n + 15) // 16 + 3
    kp, vp = make_pool(rng, pages, kvh, hd)
    table = rng.permutation(pages).astype(np.int32)
    q = rng.standard_normal((qh, hd)).astype(np.float16)
    got = oracle.paged_attention(q, table, n, kp, vp, kvh).astype(np.float64)
    want = textbook(q, gather(kp, table, n), gather(vp, table, n))
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-3)


def test_one_position_returns_its_value_row():
    rng = np.random.default_rng(1)
    kp, vp = make_pool(rng, 4, 2, 64)
    table = np.array([2, 0, 1, 3], np.int32)
    q = rng.standard_normal((4, 64)).astype(np.float16)
    got = oracle.paged_attention(q, table, 1, kp, vp, 2)
    for h in range(4):
        assert np.array_equal(got[h], vp[2, 0, h // 2])


def test_equal_keys_average_the_values():
    rng = np.random.default_rng(2)
    kp, vp = make_pool(rng, 3, 1, 32)
    kp[:] = kp[0, 0]
    q = rng.standard_normal((2, 32)).astype(np.float16)
    table = np.array([1, 2, 0], np.int32)
    n = 40
    got = oracle.paged_attention(q, table, n, kp, vp, 1).astype(np.float64)
    want = gather(vp, table, n)[:, 0, :].mean(0)
    np.testing.assert_allclose(got, np.broadcast_to(want, got.shape), rtol=1e-3, atol=1e-3)


def test_physical_placement_does_not_matter():
    rng = np.random.default_rng(3)
    kp, vp = make_pool(rng, 6, 2, 32)
    q = rng.standard_normal((4, 32)).astype(np.float16)
    t1 = np.array([0, 1, 2, 3, 4, 5], np.int32)
    perm = np.array([4, 2, 5, 0, 3, 1])
    kp2 = np.empty_like(kp)
    vp2 = np.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    t2 = perm[t1].astype(np.int32)
    a = oracle.paged_attention(q, t1, 90, kp, vp, 2)
    b = oracle.paged_attention(q, t2, 90, kp2, vp2, 2)
    assert np.array_equal(a, b)


def test_zero_length_gives_zeros():
    rng = np.random.default_rng(4)
    kp, vp = make_pool(rng, 2, 1, 32)
    q = rng.standard_normal((2, 32)).astype(np.float16)
    got = oracle.paged_attention(q, np.array([0, 1], np.int32), 0, kp, vp, 1)
    assert not got.any()


def test_a_planted_head_mapping_mistake_is_caught():
    """The textbook check tells a wrong GQA mapping (h % kvh instead of h // G) apart."""
    rng = np.random.default_rng(5)
    kp, vp = make_pool(rng, 3, 2, 32)
    table = np.array([0, 1, 2], np.int32)
    q = rng.standard_normal((4, 32)).astype(np.float16)
    k_rows, v_rows = gather(kp, table, 40), gather(vp, table, 40)
    good = textbook(q, k_rows, v_rows)
    swapped = textbook(q, k_rows[:, ::-1], v_rows[:, ::-1])  # head h on kv head 1 - h // 2
    got = oracle.paged_attention(q, table, 40, kp, vp, 2).astype(np.float64)
    assert np.abs(got - good).max() < 1e-2
    assert np.abs(got - swapped).max() > 0.1

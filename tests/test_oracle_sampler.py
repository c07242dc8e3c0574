"""Pins the oracle's greedy argmax and softmax (crates/fracture-generate/src/sampling.rs).

Checks: the sampler's own unit-test vector, the fixture logits -> greedy_token dumps,
brute force against numpy for ties (last index wins) and the NaN/Inf/empty errors, and
closed forms for softmax. CPU only.
"""
import numpy as np
import pytest

import oracle


def test_sampler_unit_vector():
    # sampling.rs:131-158: [1, 3, 2, 0.5, 0.1] -> 1
    assert oracle.argmax(np.array([1.0, 3.0, 2.0, 0.5, 0.1], np.float32)) == (1, None)


@pytest.mark.parametrize("case", ["prompt_0", "prompt_1", "decode_step_0"])
def test_fixture_greedy_token(golden, case):
    logits = golden[f"{case}/logits"].reshape(-1, 256)
    idx, err = oracle.argmax(logits[-1])
    assert err is None and idx == int(golden[f"{case}/greedy_token"][0])


def test_ties_take_the_last_index():
    l = np.array([1.0, 5.0, 2.0, 5.0, 5.0, -1.0], np.float32)
    assert oracle.argmax(l)[0] == 4
    # +0.0 and -0.0 compare equal, so the later one wins
    assert oracle.argmax(np.array([-1.0, 0.0, -0.0], np.float32))[0] == 2
    assert oracle.argmax(np.array([-1.0, -0.0, 0.0], np.float32))[0] == 2


def test_brute_force_random_with_ties():
    rng = np.random.default_rng(5)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        l = rng.integers(-5, 5, n).astype(np.float32)  # many ties
        want = n - 1 - int(np.argmax(l[::-1]))  # last maximal index
        assert oracle.argmax(l)[0] == want


def test_errors_nan_first_then_inf_then_empty():
    assert oracle.argmax(np.array([], np.float32)) == (-1, "empty logits")
    assert oracle.argmax(np.array([1, np.nan, 2], np.float32)) == (-1, "NaN in logits")
    assert oracle.argmax(np.array([1, np.inf, 2], np.float32)) == (-1, "Inf in logits")
    assert oracle.argmax(np.array([np.inf, np.nan], np.float32)) == (-1, "NaN in logits")
    assert oracle.argmax(np.array([-np.inf, 0], np.float32)) == (-1, "Inf in logits")


def test_softmax_closed_forms():
    rng = np.random.default_rng(6)
    l = (rng.standard_normal((4, 1000)) * 3).astype(np.float32)
    l[2, 77] += 20.0
    p = oracle.softmax_rows(l)
    l64 = l.astype(np.float64)
    want = np.exp(l64 - l64.max(1, keepdims=True))
    want /= want.sum(1, keepdims=True)
    # the sampler sums the exps sequentially in f32: relative error grows like n * 2^-24
    np.testing.assert_allclose(p, want, rtol=2e-5, atol=0)
    np.testing.assert_allclose(p.sum(1, dtype=np.float64), 1.0, atol=1e-5)
    # ratio p_i / p_j = exp(l_i - l_j)
    r = p[0, 3] / p[0, 9]
    assert abs(r / np.exp(l64[0, 3] - l64[0, 9]) - 1) < 1e-5
    assert p[2, 77] > 0.9  # the planted spike dominates


def test_softmax_temperature_divides():
    l = np.array([[1.0, 2.0, 3.0]], np.float32)
    p = oracle.softmax_rows(l, 0.5)
    want = np.exp(np.array([2.0, 4.0, 6.0]) - 6.0)
    np.testing.assert_allclose(p[0], want / want.sum(), rtol=1e-6)

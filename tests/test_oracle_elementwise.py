"""Pins the oracle's elementwise / normalisation / RoPE / embedding functions.

Checks against the reference's own PyTorch fixture dumps of the tiny model
(tests/reference-fixture, via tests/golden/tiny_llama_fixture.npz), the reference's
known-answer tests, and numpy's correctly rounded conversions. CPU only.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close

CASES = ["prompt_0", "prompt_1", "decode_step_0"]


# ---------------------------------------------------------------------------------------
# conversions: numpy's float16 cast is correctly rounded (RNE); bf16 RNE on the bits
# ---------------------------------------------------------------------------------------
def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 65536.0, -65520.0, 6.1035156e-05,
                  5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1e-10, np.inf,
                  -np.inf, 1.00048828125, 1.00146484375, 2049.0, 2051.0], np.float32),
    ]).astype(np.float32)
    got = oracle.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # and back
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(f)
    back = np.array([oracle.lib().o_f16_to_f32(int(b)) for b in bits[::97]], np.float32)
    assert np.array_equal(back[fin[::97]], f[::97][fin[::97]])


def test_bf16_conversion_rne():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(5000).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(x), want)
    # ties round to even: 0x3F808000 -> 0x3F80, 0x3F818000 -> 0x3F82
    t = np.array([0x3F808000, 0x3F818000], np.uint32).view(np.float32)
    assert list(oracle.f32_to_bf16_bits(t)) == [0x3F80, 0x3F82]


# ---------------------------------------------------------------------------------------
# reference fixture dumps
# ---------------------------------------------------------------------------------------
def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def residual_agreement(got, want):
    """(bit-exact fraction, fraction within the 5e-3 rule) of a residual sum vs the dump."""
    exact = np.mean(got == want)
    loose = np.mean(np.abs(got - want) <= 5e-3 + 5e-3 * np.abs(want))
    return exact, loose


# The dump script recomputes attn_output in FP32 after the FP16 forward
# (scripts/dump_reference.py:326-403), so input_hidden + attn_output reproduces the stored
# post_attn_residual exactly only where the recomputation agrees with the FP16 model: 77-96%
# of elements bit for bit in the prefill dumps. In the decode dump attn_output is recomputed
# over a different cache and does not sum to the residual at all, so it is not used here.
# The add formula itself is pinned bit-exactly by test_add_bit_exact_vs_exact_sum.
@pytest.mark.parametrize("case", ["prompt_0", "prompt_1"])
@pytest.mark.parametrize("layer", range(4))
def test_add_residual_fixture(golden, case, layer):
    h = golden[f"{case}/layer_{layer:02d}/input_hidden"].reshape(-1, 128)
    d = golden[f"{case}/layer_{layer:02d}/attn_output"].reshape(-1, 128)
    want = golden[f"{case}/layer_{layer:02d}/post_attn_residual"].reshape(-1, 128)
    got = oracle.add(_f16(h), _f16(d)).astype(np.float32)
    exact, loose = residual_agreement(got, want)
    assert exact >= 0.75 and loose >= 0.95, (exact, loose)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("layer", range(4))
def test_rmsnorm_fixture(golden, case, layer):
    L = f"{case}/layer_{layer:02d}"
    w_attn = golden[f"weights/blk.{layer}.attn_norm.weight"]
    w_ffn = golden[f"weights/blk.{layer}.ffn_norm.weight"]
    x = _f16(golden[f"{L}/input_hidden"].reshape(-1, 128))
    got = oracle.rmsnorm(x, w_attn, 1e-5).astype(np.float32)
    assert_close(got, golden[f"{L}/post_attn_norm"].reshape(-1, 128), 5e-3, 5e-3, "attn norm")
    x = _f16(golden[f"{L}/post_attn_residual"].reshape(-1, 128))
    got = oracle.rmsnorm(x, w_ffn, 1e-5).astype(np.float32)
    assert_close(got, golden[f"{L}/post_ffn_norm"].reshape(-1, 128), 5e-3, 5e-3, "ffn norm")


@pytest.mark.parametrize("case", CASES)
def test_final_norm_fixture(golden, case):
    x = _f16(golden[f"{case}/layer_03/output_hidden"].reshape(-1, 128))
    got = oracle.rmsnorm(x, golden["weights/output_norm.weight"], 1e-5).astype(np.float32)
    assert_close(got, golden[f"{case}/final_norm"].reshape(-1, 128), 5e-3, 5e-3, "final norm")


@pytest.mark.parametrize("case", ["prompt_0", "prompt_1"])
@pytest.mark.parametrize("layer", range(4))
def test_fused_add_rmsnorm_fixture(golden, case, layer):
    L = f"{case}/layer_{layer:02d}"
    h = _f16(golden[f"{L}/input_hidden"].reshape(-1, 128))
    d = _f16(golden[f"{L}/attn_output"].reshape(-1, 128))
    w = golden[f"weights/blk.{layer}.ffn_norm.weight"]
    res, normed = oracle.add_rmsnorm(h, d, w, 1e-5)
    exact, loose = residual_agreement(res.astype(np.float32),
                                      golden[f"{L}/post_attn_residual"].reshape(-1, 128))
    assert exact >= 0.75 and loose >= 0.95, (exact, loose)
    # the fused form equals add followed by rmsnorm of the rounded residual
    assert np.array_equal(normed.view(np.uint16), oracle.rmsnorm(res, w, 1e-5).view(np.uint16))


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("layer", range(4))
def test_silu_mul_fixture(golden, case, layer):
    L = f"{case}/layer_{layer:02d}"
    g = _f16(golden[f"{L}/gate"].reshape(-1, 256))
    u = _f16(golden[f"{L}/up"].reshape(-1, 256))
    got = oracle.silu_mul(g, u).astype(np.float32)
    assert_close(got, golden[f"{L}/silu_mul"].reshape(-1, 256), 1e-3, 1e-3, "silu_mul")


def _positions(golden, case, T):
    if case.startswith("decode"):
        return golden[f"{case}/position_index"].astype(np.uint32)
    return np.arange(T, dtype=np.uint32)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("layer", range(4))
def test_rope_fixture(golden, case, layer):
    cfg = golden["config"]
    L = f"{case}/layer_{layer:02d}"
    q = golden[f"{L}/q"].reshape(-1, cfg["num_q_heads"], cfg["head_dim"])
    k = golden[f"{L}/k"].reshape(-1, cfg["num_kv_heads"], cfg["head_dim"])
    T = q.shape[0]
    freqs = oracle.rope_freqs(cfg["head_dim"], cfg["rope_theta"])
    pos = _positions(golden, case, T)
    # rtol 0.01 / atol 0.025: the reference's own RoPE fixture tolerance
    # (tests/model-validation/tests/kernels.rs:1551-1552)
    assert_close(oracle.rope(_f16(q), pos, freqs).astype(np.float32),
                 golden[f"{L}/q_rope"].reshape(q.shape), 0.01, 0.025, "q_rope")
    assert_close(oracle.rope(_f16(k), pos, freqs).astype(np.float32),
                 golden[f"{L}/k_rope"].reshape(k.shape), 0.01, 0.025, "k_rope")


@pytest.mark.parametrize("case", CASES)
def test_embedding_fixture(golden, case):
    table = golden["weights/token_embd.weight"]
    ids = golden[f"{case}/token_ids"].astype(np.uint32)
    got = oracle.embedding(table, ids)
    assert np.array_equal(got.astype(np.float32), golden[f"{case}/embeddings"].reshape(-1, 128))


def test_embedding_oov_rows_are_zero():
    table = np.arange(8 * 4, dtype=np.float16).reshape(8, 4) + 1
    out = oracle.embedding(table, np.array([3, 8, 100, 0], np.uint32))
    assert np.array_equal(out[0], table[3]) and np.array_equal(out[3], table[0])
    assert not out[1].any() and not out[2].any()


# ---------------------------------------------------------------------------------------
# the reference's known-answer tests
# ---------------------------------------------------------------------------------------
def test_rmsnorm_known_answers():
    # [1,2,3,4] -> x / sqrt(7.5 + eps) (backends/fracture-cuda/src/tests.rs:183-212)
    x = np.array([[1, 2, 3, 4]], np.float32)
    got = oracle.rmsnorm(x, np.ones(4, np.float32), 1e-5)
    np.testing.assert_allclose(got, x / np.sqrt(7.5 + 1e-5), rtol=1e-6)
    # zeros stay zero (tests.rs:215-232)
    assert not oracle.rmsnorm(np.zeros((1, 4), np.float16), np.ones(4, np.float16), 1e-5).any()
    # 60000 everywhere -> 1.0 (tests.rs:663-690)
    x = np.full((2, 64), 60000, np.float16)
    np.testing.assert_allclose(oracle.rmsnorm(x, np.ones(64, np.float16), 1e-5).astype(np.float32),
                               1.0, atol=2e-3)
    # weights multiply through: w = [2, 0.5, 1, 3]
    w = np.array([2, 0.5, 1, 3], np.float32)
    got = oracle.rmsnorm(np.array([[1, 2, 3, 4]], np.float32), w, 1e-5)
    np.testing.assert_allclose(got[0], np.array([1, 2, 3, 4]) / np.sqrt(7.5 + 1e-5) * w, rtol=1e-6)


def test_silu_known_answers():
    # silu(0) = 0; silu(x) = x * sigmoid(x) in float64 (tests.rs:237-267)
    g = np.array([0.0, 1.0, -1.0, 2.0, 10.0, -10.0], np.float32)
    got = oracle.silu_mul(g, np.ones_like(g))
    want = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=0)
    assert got[0] == 0.0


def test_add_known_answer_and_fp16_rounding():
    a = np.array([1, 2, 3, 4], np.float16)
    b = np.array([10, 20, 30, 40], np.float16)
    assert list(oracle.add(a, b).astype(np.float32)) == [11, 22, 33, 44]
    # one rounding of the exact sum: 2048 + 1 ties to even (2048), 2048 + 3 -> 2052
    a = np.array([2048, 2048, 0.1], np.float16)
    b = np.array([1, 3, 0.2], np.float16)
    want = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
    assert np.array_equal(oracle.add(a, b).view(np.uint16), want.view(np.uint16))


def test_add_bit_exact_vs_exact_sum():
    # f16(f32(a) + f32(b)) (tests.rs:2051-2054) is the correctly rounded fp16 sum: the exact
    # float64 sum rounded once to fp16 must agree bit for bit, including ties and overflow.
    rng = np.random.default_rng(4)
    a = (rng.standard_normal(200000) * 10.0 ** rng.integers(-6, 5, 200000)).astype(np.float16)
    b = (rng.standard_normal(200000) * 10.0 ** rng.integers(-6, 5, 200000)).astype(np.float16)
    with np.errstate(over="ignore", invalid="ignore"):
        want = (a.astype(np.float64) + b.astype(np.float64)).astype(np.float16)
    got = oracle.add(a, b)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint16), want[fin].view(np.uint16))


def test_rope_freqs_closed_form():
    f = oracle.rope_freqs(128, 500000.0)
    want = (1.0 / (500000.0 ** (2.0 * np.arange(64) / 128.0)).astype(np.float32))
    assert np.array_equal(f, want.astype(np.float32))
    assert f[0] == 1.0


def test_rope_identity_and_position_one():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 4, 32)).astype(np.float32)
    freqs = oracle.rope_freqs(32, 10000.0)
    # position 0 is the identity (tests.rs:334-355)
    assert np.array_equal(oracle.rope(x, np.array([0], np.uint32), freqs), x)
    # position 1: rotation by freq[d] radians, closed form in float64 (tests.rs:2402-2444)
    got = oracle.rope(x, np.array([1], np.uint32), freqs)
    c, s = np.cos(freqs.astype(np.float64)), np.sin(freqs.astype(np.float64))
    x0, x1 = x[..., :16].astype(np.float64), x[..., 16:].astype(np.float64)
    np.testing.assert_allclose(got[..., :16], x0 * c - x1 * s, atol=1e-6)
    np.testing.assert_allclose(got[..., 16:], x0 * s + x1 * c, atol=1e-6)

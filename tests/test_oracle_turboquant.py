"""Pins the oracle's TurboQuant functions (crates/fracture-core/src/turboquant.rs and the
compress / decompress / attention kernels' semantics). CPU only.

No golden TurboQuant vectors exist in the reference, so each function is pinned by what
the mathematics fixes: the published xoshiro256** / SplitMix64 outputs, Max's (1960)
Gaussian quantizer tables, the QR factorisation properties of the rotation, brute-force
nearest-centroid search, the reference kernel's explicit 2/4/8-bit byte layouts, the
round-trip thresholds of the reference's tests, and float64 attention.
"""
import math

import numpy as np
import pytest

import oracle

SIG = 1.0 / math.sqrt(128.0)


# ---------------------------------------------------------------------------------------
# PRNG: published outputs
# ---------------------------------------------------------------------------------------
def test_xoshiro256starstar_reference_outputs():
    # xoshiro256** from state {1, 2, 3, 4}: the sequence of the authors' reference code
    got = oracle.xoshiro_outputs_state([1, 2, 3, 4], 4)
    assert [int(v) for v in got] == [11520, 0, 1509978240, 1215971899390074240]


def test_splitmix64_seeding():
    # The state words are consecutive SplitMix64 outputs; from seed 0 the first published
    # output is 0xe220a8397b1dcdaf, from seed 1234567 the sequence starts 6457827717110365317.
    assert int(oracle.splitmix_state(0)[0]) == 0xE220A8397B1DCDAF
    assert int(oracle.splitmix_state(1234567)[0]) == 6457827717110365317
    assert int(oracle.splitmix_state(1234567)[1]) == 3203168211198807973


def test_box_muller_first_pair():
    # g[0], g[1] from the first two generator outputs by the textbook transform in float64
    u = oracle.xoshiro_outputs(42, 2)
    u1 = max(float(int(u[0]) >> 11) / float(1 << 53), 1e-15)
    u2 = float(int(u[1]) >> 11) / float(1 << 53)
    r = math.sqrt(-2.0 * math.log(u1))
    th = 2.0 * math.pi * u2
    g = oracle.gaussian_matrix(4, 42)
    assert g[0, 0] == np.float32(r * math.cos(th)) and g[0, 1] == np.float32(r * math.sin(th))


def test_gaussian_matrix_statistics():
    g = oracle.gaussian_matrix(128, 7).astype(np.float64).ravel()
    assert abs(g.mean()) < 0.03 and abs(g.var() - 1.0) < 0.04
    # fourth moment of N(0,1) is 3
    assert abs(np.mean(g ** 4) - 3.0) < 0.25


# ---------------------------------------------------------------------------------------
# Rotation: orthogonal QR factor of the seeded Gaussian matrix with the diagonal sign rule
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("d,seed", [(16, 42), (64, 7), (128, 42), (128, 542)])
def test_rotation_is_qr_factor(d, seed):
    q = oracle.rotation(d, seed).astype(np.float64)
    g = oracle.gaussian_matrix(d, seed).astype(np.float64)
    assert np.abs(q.T @ q - np.eye(d)).max() < 1e-5  # turboquant.rs:662-736 uses 1e-4
    r = q.T @ g  # upper triangular up to rounding: Q spans G's leading columns in order
    scale = np.abs(np.diag(r)).min()
    assert np.abs(np.tril(r, -1)).max() < 1e-4 * scale
    # |R_ii| are the Gram-Schmidt column norms; the sign rule makes Q's diagonal >= 0
    assert (np.diag(q) >= 0).all()


def test_rotation_deterministic_and_seed_dependent():
    assert np.array_equal(oracle.rotation(32, 42), oracle.rotation(32, 42))
    assert not np.array_equal(oracle.rotation(16, 42), oracle.rotation(16, 43))


def test_rotation_seeds():
    assert oracle.rotation_seeds(42, 0) == (42, 542)
    assert oracle.rotation_seeds(42, 5) == (5042, 5542)


# ---------------------------------------------------------------------------------------
# Lloyd-Max codebook
# ---------------------------------------------------------------------------------------
# Max (1960), optimum quantizer outputs for N(0, 1), positive half.
MAX_1960 = {
    2: [0.4528, 1.5104],
    3: [0.2451, 0.7560, 1.3439, 2.1519],
    4: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326],
}


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_codebook_matches_max_tables(bits):
    c, b, it = oracle.lloyd_max(128, bits)
    pos = c[len(c) // 2:] / SIG
    np.testing.assert_allclose(pos, MAX_1960[bits], rtol=5e-4, atol=2e-4)


def test_codebook_iteration_counts():
    # An independent restatement of the solver converged (tol 1e-10) after 39 iterations at
    # 2 bits and 138 at 3 bits and stopped at the 200-iteration cap at 4 bits; the 4-bit
    # table therefore depends on the cap, which only an op-for-op restatement reproduces.
    assert oracle.lloyd_max(128, 2)[2] == 39
    assert oracle.lloyd_max(128, 3)[2] == 138
    assert oracle.lloyd_max(128, 4)[2] == 200


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_codebook_invariants(bits):
    c, b, _ = oracle.lloyd_max(128, bits)
    L = 1 << bits
    assert c.shape == (L,) and b.shape == (L - 1,)
    assert np.all(np.diff(c) > 0)
    assert np.all((b > c[:-1]) & (b < c[1:]))
    np.testing.assert_allclose(c + c[::-1], 0, atol=1e-5)
    assert np.abs(c).max() < 4.0 * SIG or bits == 8


def test_codebook_scales_with_dim():
    r = oracle.lloyd_max(64, 4)[0][-1] / oracle.lloyd_max(128, 4)[0][-1]
    assert abs(r - math.sqrt(2)) < 1e-3


# ---------------------------------------------------------------------------------------
# quantize + pack
# ---------------------------------------------------------------------------------------
def adversarial_y(c, rng, n=4000):
    c = c.astype(np.float32)
    mids = ((c[:-1].astype(np.float64) + c[1:]) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    special = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e30, -1e30, 3.0e38, 1e-40],
                       np.float32)
    return np.concatenate([rng.standard_normal(n).astype(np.float32) * SIG, c, mids, near,
                           special]).astype(np.float32)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
def test_codes_brute_force(bits):
    c = oracle.lloyd_max(128, bits)[0]
    y = adversarial_y(c, np.random.default_rng(bits))
    got = oracle.tq_codes(y, c)
    with np.errstate(invalid="ignore"):
        dist = np.abs(y[:, None] - c[None, :])  # float32, one rounding per element
    dist = np.where(np.isnan(dist), np.inf, dist)
    want = np.argmin(dist, axis=1)  # first minimum
    allinf = np.isinf(dist).all(axis=1)  # NaN / infinite y: no distance ever beats d[0]
    want[allinf] = 0
    assert np.array_equal(got, want.astype(np.uint8))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_reference_layouts_equal_bitstream(bits):
    rng = np.random.default_rng(10 + bits)
    for hd in (128, 96, 5, 3, 1):
        codes = rng.integers(0, 1 << bits, (7, hd)).astype(np.uint8)
        a = oracle.tq_pack_rows(codes, bits)
        b = oracle.tq_pack_rows(codes, bits, bitstream=True)
        assert np.array_equal(a, b)


def test_reference_4bit_and_2bit_byte_layout():
    c = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.uint8)
    assert list(oracle.tq_pack_rows(c, 4)[0]) == [0x12, 0x34, 0x56, 0x78]
    c = np.array([[1, 2, 3, 0, 3, 3, 3, 3]], np.uint8)
    assert list(oracle.tq_pack_rows(c, 2)[0]) == [0b01101100, 0xFF]
    # odd head_dim at 4 bits: the trailing low nibble is zero (turboquant_compress.cu:132-146)
    assert list(oracle.tq_pack_rows(np.array([[15, 1, 7]], np.uint8), 4)[0]) == [0xF1, 0x70]


@pytest.mark.parametrize("bits", [1, 3, 5, 6, 7])
def test_bitstream_roundtrip_other_widths(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (3, 128)).astype(np.uint8)
    packed = oracle.tq_pack_rows(codes, bits)
    assert packed.shape == (3, oracle.packed_dim(128, bits))
    assert np.array_equal(oracle.tq_unpack_rows(packed, 128, bits), codes)
    # 3 bits: the first 8 codes are one 24-bit big-endian word
    if bits == 3:
        w = 0
        for i in range(8):
            w = (w << 3) | int(codes[0, i])
        assert bytes(packed[0, :3]) == w.to_bytes(3, "big")


# ---------------------------------------------------------------------------------------
# compress / dequantize: round trips (turboquant.rs:1056-1101, 1224-1289;
# bins/fracture-server-cuda/tests/turboquant_gpu.rs thresholds)
# ---------------------------------------------------------------------------------------
def _cos(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, -1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1) + 1e-30)


@pytest.mark.parametrize("bits,min_cos", [(8, 0.999), (4, 0.95), (3, 0.93), (2, 0.80)])
def test_roundtrip_cosine(bits, min_cos):
    rng = np.random.default_rng(20 + bits)
    hd = 128
    x = (rng.standard_normal((64, hd)) * np.exp(rng.normal(0, 0.5, (64, 1)))).astype(np.float16)
    rot = oracle.rotation(hd, 42)
    c = oracle.lloyd_max(hd, bits)[0]
    packed, norms, y = oracle.tq_compress(x, rot, c, bits)
    out = oracle.tq_dequant(packed, norms, rot, c, bits, hd)
    cs = _cos(out, x)
    assert cs.min() > min_cos
    # stored norms within 2% (turboquant_gpu.rs:251-304); fp16 storage keeps them tighter
    n = np.linalg.norm(x.astype(np.float64), axis=1)
    assert np.abs(norms.astype(np.float64) / n - 1).max() < 2e-3


def test_rotate_matches_float64():
    rng = np.random.default_rng(30)
    x = rng.standard_normal((16, 128)).astype(np.float16)
    rot = oracle.rotation(128, 42)
    y, norms = oracle.tq_rotate(x, rot)
    x64 = x.astype(np.float64)
    want = (x64 / np.linalg.norm(x64, axis=1, keepdims=True)) @ rot.astype(np.float64).T
    np.testing.assert_allclose(y, want, atol=2e-6)


def test_zero_vector_compresses_without_nan():
    x = np.zeros((2, 128), np.float16)
    rot = oracle.rotation(128, 42)
    c = oracle.lloyd_max(128, 4)[0]
    packed, norms, y = oracle.tq_compress(x, rot, c, 4)
    out = oracle.tq_dequant(packed, norms, rot, c, 4, 128)
    assert not np.isnan(out.astype(np.float32)).any() and not out.astype(np.float32).any()


# ---------------------------------------------------------------------------------------
# attention over TurboQuant pages
# ---------------------------------------------------------------------------------------
def make_pages(rng, ctx, kvh, hd, kbits, vbits, n_pages, seed=42):
    """Random K/V, compressed by the oracle into shuffled pages."""
    k = (rng.standard_normal((ctx, kvh, hd)) * np.exp(rng.normal(0, 0.5, (ctx, 1, 1)))).astype(np.float16)
    v = (rng.standard_normal((ctx, kvh, hd)) * np.exp(rng.normal(0, 0.5, (ctx, 1, 1)))).astype(np.float16)
    krot, vrot = oracle.rotation(hd, seed), oracle.rotation(hd, seed + 500)
    kc, vc = oracle.lloyd_max(hd, kbits)[0], oracle.lloyd_max(hd, vbits)[0]
    pdk, pdv = oracle.packed_dim(hd, kbits), oracle.packed_dim(hd, vbits)
    kpk, kn, _ = oracle.tq_compress(k, krot, kc, kbits)
    vpk, vn, _ = oracle.tq_compress(v, vrot, vc, vbits)
    nb = (ctx + 15) // 16
    table = rng.permutation(n_pages)[:nb].astype(np.int32)
    KP = np.zeros((n_pages, 16, kvh * pdk), np.uint8)
    KN = np.zeros((n_pages, 16, kvh), np.float16)
    VP = np.zeros((n_pages, 16, kvh * pdv), np.uint8)
    VN = np.zeros((n_pages, 16, kvh), np.float16)
    for t in range(ctx):
        p, s = table[t // 16], t % 16
        KP[p, s] = kpk.reshape(ctx, kvh * pdk)[t]
        KN[p, s] = kn.reshape(ctx, kvh)[t]
        VP[p, s] = vpk.reshape(ctx, kvh * pdv)[t]
        VN[p, s] = vn.reshape(ctx, kvh)[t]
    deq_k = oracle.tq_dequant(kpk, kn, krot, kc, kbits, hd).reshape(ctx, kvh, hd)
    deq_v = oracle.tq_dequant(vpk, vn, vrot, vc, vbits, hd).reshape(ctx, kvh, hd)
    return dict(table=table, KP=KP, KN=KN, VP=VP, VN=VN, krot=krot, vrot=vrot, kc=kc, vc=vc,
                deq_k=deq_k, deq_v=deq_v, kpk=kpk, kn=kn, vpk=vpk, vn=vn)


def float64_attention(q, K, V, kvh):
    qh, hd = q.shape
    G = qh // kvh
    out = np.empty((qh, hd))
    for h in range(qh):
        kk = K[:, h // G].astype(np.float64)
        s = kk @ q[h].astype(np.float64) / math.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[:, h // G].astype(np.float64)
    return out


def test_attention_matches_float64_over_dequantized(rng=None):
    rng = np.random.default_rng(40)
    ctx, kvh, qh, hd = 77, 2, 8, 128
    pg = make_pages(rng, ctx, kvh, hd, 4, 4, n_pages=9)
    q = rng.standard_normal((qh, hd)).astype(np.float16)
    got = oracle.tq_attention(q, pg["table"], ctx, pg["KP"], pg["KN"], pg["VP"], pg["VN"],
                              pg["krot"], pg["vrot"], pg["kc"], pg["vc"], 4, 4, kvh)
    # Rotated-space scores and V accumulation are exact identities (turboquant.rs:1137-1220),
    # so the paged kernel equals plain attention over the dequantized K and V up to the fp16
    # rounding of the dequantized values.
    K = np.empty((ctx, kvh, hd))
    V = np.empty((ctx, kvh, hd))
    for t in range(ctx):
        for h in range(kvh):
            yk = pg["kc"][oracle.tq_unpack_rows(pg["kpk"][t * kvh + h][None], hd, 4)[0]].astype(np.float64)
            yv = pg["vc"][oracle.tq_unpack_rows(pg["vpk"][t * kvh + h][None], hd, 4)[0]].astype(np.float64)
            K[t, h] = pg["krot"].astype(np.float64).T @ yk * float(pg["kn"].reshape(-1)[t * kvh + h])
            V[t, h] = pg["vrot"].astype(np.float64).T @ yv * float(pg["vn"].reshape(-1)[t * kvh + h])
    want = float64_attention(q, K, V, kvh)
    np.testing.assert_allclose(got.astype(np.float64), want, rtol=2e-3, atol=2e-3)

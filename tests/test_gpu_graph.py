"""Graph capture of the handle runtime: a decode step's elementwise chain (embedding, add +
RMSNorm, RoPE, SwiGLU, add, RMSNorm, copy_rows; the per-layer sequence of engine.rs:621-706
without its GEMMs and attention) recorded once and replayed with fresh inputs. Every replay is
bit-identical to the same ops run eagerly, and every op of every replay matches the oracle on
that op's own inputs (bit-exact for the gather, the adds and the row copy; the 1e-3 rule for
RMSNorm, RoPE and SwiGLU). The ops that cannot be recorded are refused and record nothing."""
import numpy as np
import pytest

import oracle
from conftest import assert_close
from fracture_amd import BackendError, DType, HipBackend
from fracture_amd import turboquant as tq

pytestmark = pytest.mark.gpu

T, HID, VOCAB, QH, KVH, HD, FFN = 8, 512, 1000, 4, 2, 128, 1024
EPS = 1e-5


def _tensors(b):
    f16 = DType.FP16
    t = {
        "ids": b.alloc([T], DType.FP32),    # uint32 bytes
        "pos": b.alloc([T], DType.FP32),    # uint32 bytes
        "table": b.alloc([VOCAB, HID], f16),
        "w": b.alloc([HID], f16),
        "x": b.alloc([T, HID], f16),
        "h": b.alloc([T, HID], f16),
        "n1": b.alloc([T, HID], f16),
        "q": b.alloc([T, QH, HD], f16),
        "k": b.alloc([T, KVH, HD], f16),
        "gate": b.alloc([T, FFN], f16),
        "up": b.alloc([T, FFN], f16),
        "mid": b.alloc([T, FFN], f16),
        "h2": b.alloc([T, HID], f16),
        "n2": b.alloc([T, HID], f16),
        "save": b.alloc([2 * T, HID], f16),
    }
    rng = np.random.default_rng(0)
    b.copy_to_device(t["table"], (rng.standard_normal((VOCAB, HID)) * 0.5).astype(np.float16))
    b.copy_to_device(t["w"], rng.uniform(0.5, 1.5, HID).astype(np.float16))
    b.copy_to_device(t["save"], np.zeros((2 * T, HID), np.float16))
    return t


def _inputs(seed):
    rng = np.random.default_rng(100 + seed)
    ids = rng.integers(0, VOCAB, T).astype(np.uint32)
    ids[seed % T] = VOCAB + seed % 5  # one id past the vocabulary: a zero row
    pos = rng.integers(0, 8192, T).astype(np.uint32)
    h = rng.standard_normal((T, HID)).astype(np.float16)
    q = rng.standard_normal((T, QH, HD)).astype(np.float16)
    k = rng.standard_normal((T, KVH, HD)).astype(np.float16)
    gate = rng.standard_normal((T, FFN)).astype(np.float16)
    up = rng.standard_normal((T, FFN)).astype(np.float16)
    return {"ids": ids, "pos": pos, "h": h, "q": q, "k": k, "gate": gate, "up": up}


def _load(b, t, inp):
    for name, arr in inp.items():
        b.copy_to_device(t[name], arr)


def _chain(b, t):
    b.embedding_dev(t["ids"], T, t["table"], t["x"])
    b.add_rmsnorm(t["h"], t["x"], t["w"], EPS, t["n1"])
    b.rope_dev(t["q"], t["k"], t["pos"], T, HD)
    b.silu_mul(t["gate"], t["up"], t["mid"])
    b.add(t["h"], t["n1"], t["h2"])
    b.rmsnorm(t["h2"], t["w"], EPS, t["n2"])
    b.copy_rows(t["n2"], t["save"], 0, T, T)


OUTS = ("x", "h", "n1", "q", "k", "mid", "h2", "n2", "save")


def _read(b, t):
    return {n: b.download(t[n]).copy() for n in OUTS}


def _check_vs_oracle(got, inp, table, w, freqs, what):
    """Each op of one chain run against the oracle, fed the inputs that op saw on the GPU."""
    def same(a, b, name):
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"{what}: {name}"

    same(got["x"], oracle.embedding(table, inp["ids"]), "embedding")
    h_ref, n1_ref = oracle.add_rmsnorm(inp["h"], got["x"], w, EPS)
    same(got["h"], h_ref, "add+RMSNorm residual")
    assert_close(got["n1"], n1_ref, 1e-3, 1e-3, f"{what}: add+RMSNorm")
    assert_close(got["q"], oracle.rope(inp["q"], inp["pos"], freqs), 1e-3, 1e-3, f"{what}: RoPE q")
    assert_close(got["k"], oracle.rope(inp["k"], inp["pos"], freqs), 1e-3, 1e-3, f"{what}: RoPE k")
    assert_close(got["mid"], oracle.silu_mul(inp["gate"], inp["up"]), 1e-3, 1e-3, f"{what}: SwiGLU")
    same(got["h2"], oracle.add(got["h"], got["n1"]), "add")
    assert_close(got["n2"], oracle.rmsnorm(got["h2"], w, EPS), 1e-3, 1e-3, f"{what}: RMSNorm")
    same(got["save"][:T], np.zeros((T, HID), np.float16), "copy_rows (rows left alone)")
    same(got["save"][T:], got["n2"], "copy_rows")


def test_graph_replays_match_eager():
    with HipBackend(0) as b:
        b.precompute_rope_freqs(HD, 500000.0)
        t = _tensors(b)
        table = b.download(t["table"]).copy()
        w = b.download(t["w"]).copy()
        freqs = oracle.rope_freqs(HD, 500000.0)
        side = b.upload(np.random.default_rng(9).standard_normal((4, 3000)).astype(np.float32))
        probs = b.alloc([4, 3000], DType.FP32)
        _load(b, t, _inputs(0))
        g = b.capture(lambda: _chain(b, t))
        try:
            for it in range(4):
                inp = _inputs(it)
                _load(b, t, inp)
                b.graph_launch(g)
                b.synchronize()
                got = _read(b, t)
                _check_vs_oracle(got, inp, table, w, freqs, f"replay {it}")
                # eager work between replays, then the same ops eagerly on the same inputs
                b.softmax_rows(side, 1.0, probs)
                b.synchronize()
                _load(b, t, inp)
                _chain(b, t)
                b.synchronize()
                want = _read(b, t)
                for n in OUTS:
                    assert np.array_equal(got[n].view(np.uint16), want[n].view(np.uint16)), \
                        f"replay {it}: {n} differs from the eager run"
                # the graph's embedding gathered this replay's ids (zero rows past the vocab)
                ids = inp["ids"].astype(np.int64)
                rows = np.where((ids < VOCAB)[:, None], table[np.minimum(ids, VOCAB - 1)], 0)
                assert np.array_equal(got["x"].view(np.uint16),
                                      rows.astype(np.float16).view(np.uint16))
                assert (ids >= VOCAB).any() and (ids < VOCAB).any()
            # two replays back to back apply RoPE twice in place, like two eager passes
            inp = _inputs(7)
            _load(b, t, inp)
            b.graph_launch(g)
            b.graph_launch(g)
            b.synchronize()
            got_q = b.download(t["q"]).copy()
            _load(b, t, inp)
            _chain(b, t)
            _chain(b, t)
            b.synchronize()
            assert np.array_equal(got_q.view(np.uint16), b.download(t["q"]).view(np.uint16))
        finally:
            b.graph_destroy(g)


def test_dev_forms_equal_host_forms():
    with HipBackend(0) as b:
        b.precompute_rope_freqs(HD, 500000.0)
        t = _tensors(b)
        inp = _inputs(3)
        _load(b, t, inp)
        b.embedding_dev(t["ids"], T, t["table"], t["x"])
        b.rope_dev(t["q"], t["k"], t["pos"], T, HD)
        dev = _read(b, t)
        _load(b, t, inp)
        b.embedding([int(i) for i in inp["ids"]], t["table"], t["x"])
        b.rope(t["q"], t["k"], [int(p) for p in inp["pos"]], 500000.0, HD)
        host = _read(b, t)
        for n in ("x", "q", "k"):
            assert np.array_equal(dev[n].view(np.uint16), host[n].view(np.uint16)), n
        # ids past the vocabulary give zero rows, as in the host form
        assert (host["x"][inp["ids"] >= VOCAB] == 0).all()
        with pytest.raises(Exception, match="fewer than"):
            b.rope_dev(t["q"], t["k"], t["pos"], T + 1, HD)


def test_capture_refuses_host_bound_ops():
    with HipBackend(0) as b:
        b.precompute_rope_freqs(HD, 500000.0)
        t = _tensors(b)
        _load(b, t, _inputs(1))
        logits = b.upload(np.zeros((2, 64), np.float32))
        probs = b.alloc([2, 64], DType.FP32)
        a = b.upload(np.ones((4, 8), np.float16))
        w = b.upload(np.ones((8, 8), np.float16))
        c = b.alloc([4, 8], DType.FP16)
        host = np.zeros(T * HID, np.float16)
        refused = [
            lambda: b.rope(t["q"], t["k"], list(range(T)), 500000.0, HD),
            lambda: b.embedding(list(range(T)), t["table"], t["x"]),
            lambda: b.softmax_rows(logits, 1.0, probs),
            lambda: b.argmax_rows(logits),
            lambda: b.copy_to_host(t["x"], host),
            lambda: b.copy_to_device(t["x"], host),
            lambda: b.synchronize(),
            lambda: b.alloc([4], DType.FP16),
            lambda: b.free(c),
            lambda: b.matmul(a, w, c),
            lambda: b.graph_begin(),
        ]
        b.graph_begin()
        try:
            for i, op in enumerate(refused):
                with pytest.raises(BackendError, match="graph capture"):
                    op()
            b.silu_mul(t["gate"], t["up"], t["mid"])  # accepted, recorded
        finally:
            g = b.graph_end()
        b.graph_launch(g)
        b.synchronize()
        got = b.download(t["mid"]).copy()
        b.copy_to_device(t["mid"], np.zeros((T, FFN), np.float16))
        b.silu_mul(t["gate"], t["up"], t["mid"])
        assert np.array_equal(got.view(np.uint16), b.download(t["mid"]).view(np.uint16))
        b.graph_destroy(g)
        # after the capture, the refused ops run again
        b.rope(t["q"], t["k"], list(range(T)), 500000.0, HD)
        b.synchronize()
        with pytest.raises(BackendError, match="not found"):
            b.graph_launch(g)
        with pytest.raises(BackendError, match="no graph capture"):
            b.graph_end()


def test_capture_failure_inside_record_ends_capture():
    with HipBackend(0) as b:
        t = _tensors(b)

        def bad():
            b.silu_mul(t["gate"], t["up"], t["mid"])
            b.synchronize()  # refused

        with pytest.raises(BackendError, match="graph capture"):
            b.capture(bad)
        b.synchronize()  # the capture was ended: eager work runs again


def test_contiguous_attention_not_supported(backend):
    q = backend.alloc([1, 4, 64], DType.FP16)
    with pytest.raises(BackendError, match="not supported"):
        backend.attention(q, q, q, 2, 0, q)
    backend.free(q)


def test_free_refused_while_a_graph_uses_the_tensor():
    """A graph keeps the device addresses of the tensors it used: freeing one of them (whose
    block the next allocation could reuse) is refused until the graph is destroyed."""
    with HipBackend(0) as b:
        t = _tensors(b)
        _load(b, t, _inputs(2))
        g = b.capture(lambda: b.silu_mul(t["gate"], t["up"], t["mid"]))
        for name in ("gate", "up", "mid"):
            with pytest.raises(BackendError, match="captured graph"):
                b.free(t[name])
        b.free(t["x"])  # not used by the graph
        b.graph_launch(g)
        b.synchronize()
        b.graph_destroy(g)
        for name in ("gate", "up", "mid"):
            b.free(t[name])


def test_writing_plan_tables_refused_during_capture():
    """A TurboQuant plan cached from a rotation cannot be dropped under graph capture (that
    frees device memory), so an op writing that rotation is refused while capturing and
    records nothing; outside a capture the same write drops the plan."""
    rng = np.random.default_rng(3)
    with HipBackend(0) as b:
        t = _tensors(b)
        _load(b, t, _inputs(4))
        rot = b.upload(tq.rotation_matrix(128, 1))
        cent = b.upload(tq.codebook(128, 4)[0])
        x = b.upload(rng.standard_normal((4, 8, 128)).astype(np.float16))
        packed = b.alloc([4, 8 * 64], DType.INT8)
        norms = b.alloc([4, 8], DType.FP16)
        b.turboquant_compress(x, rot, cent, 4, packed, norms)  # builds and caches the plan
        before = b.download(packed).copy()
        zero = b.upload(np.zeros((128, 128), np.float32))
        b.graph_begin()
        try:
            with pytest.raises(BackendError, match="TurboQuant plan"):
                b.add(zero, zero, rot)
            b.silu_mul(t["gate"], t["up"], t["mid"])
        finally:
            g = b.graph_end()
        b.graph_launch(g)
        b.synchronize()
        b.graph_destroy(g)
        b.turboquant_compress(x, rot, cent, 4, packed, norms)
        assert np.array_equal(b.download(packed), before)  # rot was left alone
        b.add(zero, zero, rot)  # rot := 0 outside a capture: allowed, the plan is dropped
        b.turboquant_compress(x, rot, cent, 4, packed, norms)
        # every rotated coordinate is 0 now: each code is the one nearest 0
        c = tq.codebook(128, 4)[0]
        code0 = int(np.argmin(np.abs(c)))
        assert (b.download(packed) == (code0 << 4 | code0)).all()

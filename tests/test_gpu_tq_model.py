"""The same model over an FP16 paged KV cache and over a TurboQuant cache: logits compared.

This is the reference's end-to-end A/B test (bins/fracture-server-cuda/tests/turboquant_gpu.rs:
505-659): a random model (hidden 64, 2 layers, 4 / 2 heads, head_dim 16, ffn 128, vocab 256,
theta 1e4, every weight U(-0.1, 0.1) in fp16) runs a prompt through the paged forward once
with FP16 pages and once with TurboQuant pages, and the last token's logits must agree:
cosine > 0.95 for 8-bit keys and values (prompt [1, 2, 3, 4, 5]) and > 0.70 for the default
4-bit keys / 2-bit values (prompt [10, 20, 30]). The reference's weights come from an unseeded
generator, so its published cosines (0.999999 and 0.998995, docs/turboquant.md:200-207) are
context for the ones measured here, not an equality; the weights here are seeded.

The TurboQuant cache is the reference's QuantizedKvCacheManager for one sequence
(quantized_paged_kv_cache.rs:62-133, 404-500): per layer and block, K codes [16, kvh * pd]
(INT8), K norms [16, kvh] fp16 and the same for V; per-layer rotations from
rotation_seeds(42, layer); the Lloyd-Max codebook of each width. Writes go through
fhip_tq_append_kv over the layer's registered pool (the fused page writer), attention through
Backend::attention_paged_tq over the layer's block lists (prefill: causal over the prompt).
The same comparison runs on the tiny-llama fixture model (head_dim 32), whose FP16 forward is
pinned against the reference's dumps in test_gpu_model.py.
"""
import numpy as np
import pytest

from fracture_amd import DType
from fracture_amd import turboquant as tq
from fracture_amd.weights import LayerWeights, LlamaWeights, upload_llama
from test_gpu_model import PagedCache, forward

pytestmark = pytest.mark.gpu

E2E = {"hidden_size": 64, "num_layers": 2, "num_q_heads": 4, "num_kv_heads": 2, "head_dim": 16,
       "intermediate_size": 128, "vocab_size": 256, "rope_theta": 10000.0, "rms_norm_eps": 1e-5}


class TqCache:
    """One sequence's TurboQuant paged KV cache, blocks taken from the pool in a fixed
    scattered order (the same order as PagedCache)."""

    def __init__(self, backend, layers, kvh, hd, kbits, vbits, seed=42, pool=6,
                 order=(4, 1, 5, 0, 2, 3)):
        self.b, self.kvh, self.kbits, self.vbits = backend, kvh, kbits, vbits
        self.order = list(order)
        self.len = 0
        pk = tq.TurboQuantConfig.packed_dim_per_head(hd, kbits)
        pv = tq.TurboQuantConfig.packed_dim_per_head(hd, vbits)
        self.rot, self.lists, self.pools = [], [], []
        self.kcent = backend.upload(tq.codebook(hd, kbits)[0])
        self.vcent = backend.upload(tq.codebook(hd, vbits)[0])
        for layer in range(layers):
            ks, vs = tq.rotation_seeds(seed, layer)
            self.rot.append((backend.upload(tq.rotation_matrix(hd, ks)),
                             backend.upload(tq.rotation_matrix(hd, vs))))
            lists = ([backend.alloc([16, kvh * pk], DType.INT8) for _ in range(pool)],
                     [backend.alloc([16, kvh], DType.FP16) for _ in range(pool)],
                     [backend.alloc([16, kvh * pv], DType.INT8) for _ in range(pool)],
                     [backend.alloc([16, kvh], DType.FP16) for _ in range(pool)])
            self.lists.append(lists)
            self.pools.append(backend.page_pool_create(*lists))

    def table(self, n):
        return self.order[:(n + 15) // 16]

    def append(self, layer, k_mh, v_mh, start):
        kr, vr = self.rot[layer]
        n = start + k_mh.shape[0]
        self.b.tq_append_kv(self.pools[layer], k_mh, v_mh, kr, vr, self.kcent, self.vcent,
                            self.kbits, self.vbits, self.table(n), start)

    def attention(self, layer, q_mh, n, start, out_mh):
        kr, vr = self.rot[layer]
        kp, kn, vp, vn = self.lists[layer]
        self.b.attention_paged_tq(q_mh, self.table(n), kp, kn, vp, vn, kr, vr, self.kcent,
                                  self.vcent, self.kbits, self.vbits, self.kvh, n, start, out_mh)

    def free(self):
        for p in self.pools:
            self.b.page_pool_destroy(p)
        for lists in self.lists:
            for lst in lists:
                for t in lst:
                    self.b.free(t)
        for kr, vr in self.rot:
            self.b.free(kr)
            self.b.free(vr)
        self.b.free(self.kcent)
        self.b.free(self.vcent)


def random_model(backend, cfg, seed):
    """The reference's e2e weights (every tensor U(-0.1, 0.1) in fp16), seeded."""
    rng = np.random.default_rng(seed)
    hid, inter, kvd = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_kv_heads"] * cfg["head_dim"]

    def up(*shape):
        return backend.upload(rng.uniform(-0.1, 0.1, shape).astype(np.float16))

    emb = up(cfg["vocab_size"], hid)
    layers = [LayerWeights(attn_norm=up(hid), q_proj=up(hid, hid), k_proj=up(kvd, hid),
                           v_proj=up(kvd, hid), o_proj=up(hid, hid), ffn_norm=up(hid),
                           gate_proj=up(inter, hid), up_proj=up(inter, hid),
                           down_proj=up(hid, inter))
              for _ in range(cfg["num_layers"])]
    return LlamaWeights(token_embedding=emb, output_norm=up(hid), lm_head=up(cfg["vocab_size"], hid),
                        layers=layers)


def cosine(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def compare(backend, W, cfg, ids, kbits, vbits):
    """(cosine of the last token's logits, FP16 argmax, TurboQuant argmax)."""
    L, kvh, hd = cfg["num_layers"], cfg["num_kv_heads"], cfg["head_dim"]
    fp = PagedCache(backend, L, kvh, hd)
    tqc = TqCache(backend, L, kvh, hd, kbits, vbits)
    try:
        a = forward(backend, W, cfg, ids, fp, lambda *x: None)[-1]
        b = forward(backend, W, cfg, ids, tqc, lambda *x: None)[-1]
    finally:
        fp.free()
        tqc.free()
    assert np.isfinite(a).all() and np.isfinite(b).all()
    return cosine(a, b), int(np.argmax(a)), int(np.argmax(b))


@pytest.mark.parametrize("kbits,vbits,prompt,thr", [(8, 8, [1, 2, 3, 4, 5], 0.95),
                                                    (4, 2, [10, 20, 30], 0.70)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_model_tq_vs_fp16(backend, kbits, vbits, prompt, thr, seed):
    backend.precompute_rope_freqs(E2E["head_dim"], E2E["rope_theta"])
    W = random_model(backend, E2E, seed)
    try:
        c, am_fp, am_tq = compare(backend, W, E2E, prompt, kbits, vbits)
    finally:
        for t in W.tensors():
            backend.free(t)
    print(f"random model seed {seed}: K{kbits}/V{vbits} vs FP16 logit cosine {c:.6f}, "
          f"argmax {am_fp} / {am_tq}")
    assert c > thr, c


@pytest.mark.parametrize("kbits,vbits,thr", [(8, 8, 0.95), (4, 2, 0.70), (4, 4, 0.70)])
def test_tiny_llama_tq_vs_fp16(backend, golden, kbits, vbits, thr):
    cfg = golden["config"]
    tensors = {k[len("weights/"):]: v for k, v in golden.items() if k.startswith("weights/")}
    W = upload_llama(backend, tensors, cfg["num_layers"], cfg["num_q_heads"],
                     cfg["num_kv_heads"], cfg["head_dim"])
    backend.precompute_rope_freqs(cfg["head_dim"], cfg["rope_theta"])
    ids = [int(x) for x in golden["prompt_0/token_ids"].ravel()]
    try:
        c, am_fp, am_tq = compare(backend, W, cfg, ids, kbits, vbits)
    finally:
        for t in W.tensors():
            backend.free(t)
    print(f"tiny-llama prompt_0: K{kbits}/V{vbits} vs FP16 logit cosine {c:.6f}, "
          f"argmax {am_fp} / {am_tq}")
    assert am_fp == int(golden["prompt_0/greedy_token"][0])
    assert c > thr, c
    if kbits == 8:
        assert am_fp == am_tq

"""CPU check of every global-memory address that the MFMA decode-attention kernel
(tq_attn_mfma_kernel in fracture_amd/csrc/attention_tq.hip) and its combine kernel form,
against the buffers the launcher hands them.

The MFMA kernel's addresses come from its own index functions (fracture_amd/csrc/
tq_attn_index.h), called through their host build (libfracture_hip_index.so), for every
workgroup of the launch grid, every wave (one 512-position split of the workgroup's
1024-position block) and every 64-position chunk, with numpy over the 64 lanes. What they
compute:

  split pages        entry j = table[t_begin / 16 + j] for pages holding positions of the split,
                     in the pool; every other entry is the split's first valid page (no valid
                     page: the wave reads nothing)
  load_k             entry(j0 + n / 4) + ((4 (n % 4) + pt) kvh + g) 64 + 16 rg, 16 bytes
  dma_v              entry(j0 + i) + ((lane / 4) kvh + g) 64 + 16 ((lane % 4) ^ ((lane / 8) % 4)), 16 bytes
  load_norms         norm entry(j0 + lane / 16) + 2 ((lane % 16) kvh + g), 2 bytes
  Q (rotated)        (q qh + g G + head) hd + 32 rg + 4 s, 16 bytes, for column h = G t + head
                     of query q = tq0 + t
  partials           ((q qh + g G + head) nsplit + block) (2 | hd) + ..., written by the
                     workgroup's merge

In causal prefill (one block table shared by all queries, lengths from start_pos) a workgroup
item is a group of `tok` = 8 / G consecutive queries whose heads share the MFMA columns; in
decode tok = 1 and every query has its own table row.

and asserts that each access stays inside its pool AND inside the page it means to read
(an access past the page's rows reads a neighbouring page: in bounds, but wrong data).
The next chunk's loads are issued only while it starts before the split's end. No GPU is used.
"""
import numpy as np
import pytest

PAGE = 16
CHUNK = 64
SPLIT = 1024       # positions per partial (the MFMA kernel's workgroup block, the VALU kernel's split)
WAVE_SPLIT = 512   # positions per MFMA wave


def ws_layout(nq, qh, hd, max_tokens):
    ns = (max_tokens + SPLIT - 1) // SPLIT if max_tokens > 0 else 1
    al = lambda x: (x + 255) & ~255
    qrot = nq * qh * hd * 4
    ml = nq * qh * ns * 2 * 4
    acc = nq * qh * ns * hd * 4
    return ns, al(qrot), al(ml), al(acc)


def causal_len(seq_len, max_blocks):
    return max(0, min(int(seq_len), max_blocks * PAGE))


class Bounds:
    """Collects accesses [off, off + width) per buffer and checks them."""

    def __init__(self, sizes):
        self.sizes = sizes
        self.count = {k: 0 for k in sizes}

    def check(self, buf, off, width):
        off = np.asarray(off, dtype=np.int64).ravel()
        if off.size == 0:
            return
        lo, hi = int(off.min()), int(off.max()) + width
        assert lo >= 0 and hi <= self.sizes[buf], \
            f"{buf}: access [{lo}, {hi}) outside [0, {self.sizes[buf]})"
        self.count[buf] += off.size


class IndexLib:
    """The kernel's own index arithmetic (fracture_amd/csrc/tq_attn_index.h), host build."""

    def __init__(self):
        import ctypes as C
        from pathlib import Path
        path = Path(__file__).resolve().parents[1] / "fracture_amd" / "libfracture_hip_index.so"
        if not path.exists():
            pytest.fail(f"{path} is missing: run __graft_entry__.build()")
        self.C, self.lib = C, C.CDLL(str(path))
        L = self.lib
        L.fhip_idx_wg_item.argtypes = [C.c_int64, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int32)]
        L.fhip_idx_split.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int32), C.c_void_p,
                                     C.c_void_p]
        L.fhip_idx_chunk_first_page.argtypes = [C.c_int, C.c_int]
        L.fhip_idx_chunk_first_page.restype = C.c_int32
        L.fhip_idx_q_vectors.argtypes = [C.c_int] * 6 + [C.c_void_p, C.c_void_p]
        L.fhip_idx_partial_row.argtypes = [C.c_int] * 7
        L.fhip_idx_partial_row.restype = C.c_int64
        L.fhip_idx_lane_tables.argtypes = [C.c_int, C.c_int] + [C.c_void_p] * 6
        L.fhip_idx_v2_offsets.argtypes = [C.c_int, C.c_int, C.c_void_p]
        L.fhip_idx_split_grid_item.argtypes = [C.c_int64, C.c_int, C.c_int, C.c_int] + [C.POINTER(C.c_int32)] * 3
        self._tables = {}

    def lane_tables(self, kvh, g):
        key = (kvh, g)
        if key not in self._tables:
            k_off = np.zeros((4, 64), np.uint32)
            k_page = np.zeros(64, np.int32)
            v_off = np.zeros(64, np.uint32)
            n_off = np.zeros(64, np.uint32)
            n_page = np.zeros(64, np.int32)
            q_off = np.zeros((8, 64), np.int32)
            assert self.lib.fhip_idx_lane_tables(kvh, g, *(a.ctypes.data for a in (
                k_off, k_page, v_off, n_off, n_page, q_off))) == 0
            self._tables[key] = (k_off.astype(np.int64), k_page, v_off.astype(np.int64),
                                 n_off.astype(np.int64), n_page, q_off)
        return self._tables[key]

    def v2_offsets(self, kvh, g):
        out = np.zeros(64, np.uint32)
        assert self.lib.fhip_idx_v2_offsets(kvh, g, out.ctypes.data) == 0
        return out.astype(np.int64)

    def split_grid_item(self, lin, nsplit, kvh, nq):
        s, h, q = self.C.c_int32(), self.C.c_int32(), self.C.c_int32()
        assert self.lib.fhip_idx_split_grid_item(lin, nsplit, kvh, nq, self.C.byref(s), self.C.byref(h),
                                                 self.C.byref(q)) == 0
        return s.value, h.value, q.value

    def wg_item(self, wg, kvh):
        item, g = self.C.c_int64(), self.C.c_int32()
        assert self.lib.fhip_idx_wg_item(wg, kvh, self.C.byref(item), self.C.byref(g)) == 0
        return item.value, g.value

    def split(self, blk, wave, t_end):
        t_begin = self.C.c_int32()
        col = np.zeros(64, np.int32)
        ins = np.zeros(64, np.uint8)
        assert self.lib.fhip_idx_split(blk, wave, t_end, self.C.byref(t_begin), col.ctypes.data,
                                       ins.ctypes.data) == 0
        return t_begin.value, col, ins.astype(bool)

    def q_vectors(self, tq0, tok, G, nq, qh, g):
        vec = np.zeros(64, np.int64)
        live = np.zeros(64, np.uint8)
        assert self.lib.fhip_idx_q_vectors(tq0, tok, G, nq, qh, g, vec.ctypes.data,
                                           live.ctypes.data) == 0
        return vec, live.astype(bool)


_IDX = None


def index_lib():
    global _IDX
    if _IDX is None:
        _IDX = IndexLib()
    return _IDX


def model_mfma_kernel(lens, table, num_pages, qh, kvh, page_bytes, pool_bytes, tok=1, vbits=4):
    """Every access of tq_attn_mfma_kernel<PoolPages> for one launch (hd 128, K4 and V4 or V2),
    from the kernel's own index functions. With tok > 1, `table` has one row that every query
    reads (causal prefill). Walks every workgroup of the launcher's grid."""
    ix = index_lib()
    hd, pd = 128, 64
    B = len(lens)
    rows, max_blocks = table.shape
    stride = 0 if tok > 1 else max_blocks
    assert tok == 1 or rows == 1
    G = qh // kvh
    nsplit, _, ml_bytes, acc_bytes = ws_layout(B, qh, hd, max_blocks * PAGE)
    bnd = Bounds({"table": table.size * 4, "kp": pool_bytes["kp"], "kn": pool_bytes["kn"],
                  "vp": pool_bytes["vp"], "vn": pool_bytes["vn"], "qrot": B * qh * hd * 4,
                  "part_ml": ml_bytes, "part_acc": acc_bytes})
    items = (B + tok - 1) // tok
    wgs = (items * nsplit + 7) // 8 * 8 * kvh  # launch_mfma_split's grid
    seen = set()
    for wg in range(wgs):
        item, g = ix.wg_item(wg, kvh)
        assert 0 <= g < kvh and (item, g) not in seen, "workgroup index map is not one-to-one"
        seen.add((item, g))
        tq0, blk = (item // nsplit) * tok, item % nsplit
        if tq0 >= B:
            continue  # padding workgroup: leaves at once
        tq_last = min(tq0 + tok, B) - 1
        clen = causal_len(lens[tq_last], max_blocks)
        if blk * SPLIT >= clen:
            continue  # the workgroup leaves before building its tables
        k_off, k_page, v_off, n_off, n_page, q_off = ix.lane_tables(kvh, g)
        for k in range(4):
            assert (k_off[k] + 16 <= PAGE * kvh * pd).all() and (k_off[k] + 16 <= page_bytes["kp"]).all()
        vpd, vw = (pd, 16) if vbits == 4 else (pd // 2, 8)  # V row bytes, bytes per V load
        if vbits == 2:
            v_off = ix.v2_offsets(kvh, g)
        assert (v_off + vw <= min(PAGE * kvh * vpd, page_bytes["vp"])).all()
        for nm in ("kn", "vn"):
            assert (n_off + 2 <= min(PAGE * kvh * 2, page_bytes[nm])).all()
        for w in range(SPLIT // WAVE_SPLIT):
            t_begin, col, has = ix.split(blk, w, SPLIT * nsplit)
            if t_begin >= clen:
                continue  # empty state, nothing read
            t_end = min(clen, t_begin + WAVE_SPLIT)
            _, col, has = ix.split(blk, w, t_end)
            tidx = col[has]
            assert tidx.max() < max_blocks
            bnd.check("table", (tq0 * stride + tidx) * 4, 4)
            ids = np.full(64, -1, np.int64)
            ids[has] = table.reshape(-1)[tq0 * stride + tidx]
            ok = has & (ids >= 0) & (ids < num_pages)
            if not ok.any():
                continue
            entry = np.where(ok, ids, ids[np.flatnonzero(ok)[0]])[:WAVE_SPLIT // PAGE]
            assert ((entry >= 0) & (entry < num_pages)).all()
            for t0 in range(t_begin, t_end, CHUNK):
                j0 = ix.lib.fhip_idx_chunk_first_page(t0, t_begin)
                assert j0 + 3 < len(entry), "page entry index past the wave's table"
                for pt in range(4):  # K codes
                    bnd.check("kp", entry[j0 + k_page] * page_bytes["kp"] + k_off[pt], 16)
                for i in range(4):  # V copies: copy i reads entry j0 + i
                    bnd.check("vp", entry[j0 + i] * page_bytes["vp"] + v_off, vw)
                for nm in ("kn", "vn"):  # norms
                    bnd.check(nm, entry[j0 + n_page] * page_bytes[nm] + n_off, 2)
            vec, live = ix.q_vectors(tq0, tok, G, B, qh, g)
            assert (vec >= 0).all() and (vec < B * qh).all()
            for s8 in range(8):
                bnd.check("qrot", (vec * hd + q_off[s8]) * 4, 16)
        # the workgroup's merge: one partial per live column (query, head) of the group
        for h in range(tok * G):
            if tq0 + h // G >= B:
                continue
            prow = ix.lib.fhip_idx_partial_row(h, tq0, G, qh, g, nsplit, blk)
            bnd.check("part_ml", prow * 2 * 4, 8)
            bnd.check("part_acc", (prow * hd + np.arange(hd)) * 4, 4)
    assert len(seen) == wgs
    return bnd, nsplit


def model_combine(lens, max_blocks, qh, hd, nsplit, ml_bytes, acc_bytes):
    """tq_attn_combine_kernel: partial reads (clamped split index), rotation reads, output."""
    B = len(lens)
    nvec = B * qh
    bnd = Bounds({"part_ml": ml_bytes, "part_acc": acc_bytes, "vrot": hd * hd * 4,
                  "out": nvec * hd * 2})
    n16 = hd * hd // 4
    c0 = np.arange(256)[:, None] + 256 * np.arange(16)[None, :]
    bnd.check("vrot", 4 * np.minimum(c0, n16 - 1) * 4, 16)
    heads = np.arange(nvec)
    ns = np.array([(causal_len(lens[h // qh], max_blocks) + SPLIT - 1) // SPLIT for h in heads])
    assert ns.max() <= nsplit
    for hh, k in zip(heads, ns):
        sp = np.arange(k)
        bnd.check("part_ml", (hh * nsplit * 2 + 2 * sp) * 4, 8)
        clamp = np.minimum(np.arange(((k + 15) // 16) * 16), max(k - 1, 0))
        bnd.check("part_acc", ((hh * nsplit + clamp[:, None]) * hd + np.arange(hd)[None, :]) * 4, 4)
    bnd.check("out", heads * hd * 2, 2 * hd)
    return bnd


def c5_workload():
    """The decode-attention benchmark's lengths, block table and pool (seeded as bench.py)."""
    rng = np.random.default_rng(5)
    lens = rng.integers(1024, 32769, 64).astype(np.int32)
    nbs = (lens + 15) // 16
    P = int(nbs.sum())
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((64, int(nbs.max())), np.int32)
    at = 0
    for b in range(64):
        table[b, :nbs[b]] = perm[at:at + nbs[b]]
        at += nbs[b]
    return lens, table, P


def pools(P, kvh, pd=64):
    page = {"kp": PAGE * kvh * pd, "kn": PAGE * kvh * 2, "vp": PAGE * kvh * pd, "vn": PAGE * kvh * 2}
    return page, {k: v * P for k, v in page.items()}


@pytest.mark.parametrize("vbits", [4, 2])
@pytest.mark.parametrize("which", ["c5", "edges", "long"])
def test_mfma_decode_accesses_in_bounds(which, vbits):
    if which == "long":
        # a context of 270,000 positions (264 partial blocks) over a permuted table
        lens = np.array([270000, 5], np.int32)
        max_blocks = 270000 // 16
        rng = np.random.default_rng(4)
        P = max_blocks + 100
        table = np.full((len(lens), max_blocks), -1, np.int32)
        table[0] = rng.permutation(P)[:max_blocks]
        table[1, 0] = 7
    elif which == "c5":
        lens, table, P = c5_workload()
        assert lens.max() > 16 * SPLIT, "the workload must reach the combine's second 16-split step"
    else:
        # lengths at chunk, page and split edges; unused table slots hold ids outside the pool;
        # one sequence longer than its block table (clamped to max_blocks * 16)
        lens = np.array([1, 15, 16, 17, 63, 64, 65, 1023, 1024, 1025, 16384, 16385, 20000, 0,
                         33000], np.int32)
        max_blocks = 2048
        rng = np.random.default_rng(3)
        P = 2048 * 3
        table = np.full((len(lens), max_blocks), -7, np.int32)
        for b, n in enumerate(lens):
            nb = min((int(n) + 15) // 16, max_blocks)
            table[b, :nb] = rng.integers(0, P, nb)
        table[3, 1] = P + 5      # a page id past the pool: masked, never read
    qh, kvh = 32, 8
    page, pool = pools(P, kvh)
    if vbits == 2:  # V pages of 32-byte rows
        page["vp"] //= 2
        pool["vp"] //= 2
    bnd, nsplit = model_mfma_kernel(lens, table, P, qh, kvh, page, pool, vbits=vbits)
    assert bnd.count["kp"] > 0 and bnd.count["vp"] > 0
    _, _, ml, acc = ws_layout(len(lens), qh, 128, table.shape[1] * PAGE)
    model_combine(lens, table.shape[1], qh, 128, nsplit, ml, acc)


@pytest.mark.parametrize("qh,kvh,T,kv_len", [(32, 8, 37, 3000), (16, 8, 9, 1100), (8, 8, 20, 2100),
                                             (32, 8, 64, 64)])
def test_mfma_prefill_groups_in_bounds(qh, kvh, T, kv_len):
    """Causal prefill: groups of 8 / G consecutive queries over one shared block table (the
    reference interface's num_tokens > 1), ragged last group included."""
    G = qh // kvh
    tok = 8 // G if G < 8 else 1
    start_pos = kv_len - T
    lens = np.array([min(start_pos + t + 1, kv_len) for t in range(T)], np.int32)
    nb = (kv_len + 15) // 16
    rng = np.random.default_rng(T)
    P = nb + 5
    table = rng.permutation(P)[:nb].astype(np.int32)[None, :]
    page, pool = pools(P, kvh)
    bnd, nsplit = model_mfma_kernel(lens, table, P, qh, kvh, page, pool, tok=tok)
    assert bnd.count["kp"] > 0 and bnd.count["part_acc"] > 0
    _, _, ml, acc = ws_layout(T, qh, 128, nb * PAGE)
    model_combine(lens, nb, qh, 128, nsplit, ml, acc)


def test_page_stride_smaller_than_page_is_caught():
    """A page stride below the page size makes the model's in-page reads cross into the next
    page; the launcher rejects such strides (fhip_launch_attention_tq_decode)."""
    lens, table = np.array([48], np.int32), np.arange(3, dtype=np.int32)[None, :]
    page, pool = pools(3, 8)
    model_mfma_kernel(lens, table, 3, 32, 8, page, pool)
    for key in ("kp", "vn"):
        small = dict(page)
        small[key] //= 2
        with pytest.raises(AssertionError):
            model_mfma_kernel(lens, table, 3, 32, 8, small, pool)


def test_wg_item_balances_xcds():
    """The MFMA kernel's workgroup -> item map (wg_item) on the decode-attention benchmark's
    grid: workgroup wg runs on XCD wg % 8; every kv head of an item lands on one XCD (the L2 that
    holds their shared code lines), and the positions the 8 XCDs process are within 5% of their
    mean. Placing item i on XCD i % 8 instead puts every query's blocks b, b + 8, ... on one XCD
    (32 blocks per query here), and since later blocks exist only for longer sequences, that
    placement is off by more than 20%: the check tells the two apart."""
    ix = index_lib()
    lens, table, _ = c5_workload()
    kvh, max_blocks = 8, table.shape[1]
    nsplit = ws_layout(len(lens), 32, 128, max_blocks * PAGE)[0]
    assert nsplit % 8 == 0
    items = len(lens) * nsplit
    wgs = (items + 7) // 8 * 8 * kvh
    work = lambda it: (max(0, min(SPLIT, causal_len(lens[it // nsplit], max_blocks) - (it % nsplit) * SPLIT))
                       if it < items else 0)
    xcd_of_item, load, naive = {}, np.zeros(8), np.zeros(8)
    for wg in range(wgs):
        item, g = ix.wg_item(wg, kvh)
        assert xcd_of_item.setdefault(item, wg % 8) == wg % 8, "an item's kv heads on two XCDs"
        load[wg % 8] += work(item)
        naive[item % 8] += work(item)
    assert load.sum() == naive.sum() == kvh * sum(causal_len(n, max_blocks) for n in lens)
    assert load.max() / load.mean() < 1.05, load / load.mean()
    assert naive.max() / naive.mean() > 1.20, naive / naive.mean()


def test_split_grid_item_covers_grid_and_balances_xcds():
    """The VALU split kernel's workgroup map (split_grid_item, grid (nsplit, kvh, queries)):
    every (split, kv head, query) exactly once, on grids with and without a partial last group
    of 8 workgroups; and on the decode benchmark's lengths (32 splits per query) the positions
    the 8 XCDs process (workgroup lin on XCD lin % 8) are within 5% of their mean, where the
    grid's own order leaves them over 20% apart."""
    ix = index_lib()
    for nsplit, kvh, nq in [(32, 8, 3), (3, 1, 5), (7, 2, 3), (1, 1, 1), (8, 4, 9), (5, 3, 7)]:
        total = nsplit * kvh * nq
        got = {ix.split_grid_item(lin, nsplit, kvh, nq) for lin in range(total)}
        assert got == {(s, h, q) for s in range(nsplit) for h in range(kvh) for q in range(nq)}
    lens, _, _ = c5_workload()
    nsplit, kvh, nq = 32, 8, len(lens)
    assert (lens <= nsplit * SPLIT).all()
    work = lambda s, q: max(0, min(SPLIT, int(lens[q]) - s * SPLIT))
    load, naive = np.zeros(8), np.zeros(8)
    for lin in range(nsplit * kvh * nq):
        s, _, q = ix.split_grid_item(lin, nsplit, kvh, nq)
        load[lin % 8] += work(s, q)
        naive[lin % 8] += work(lin % nsplit, lin // (nsplit * kvh))
    assert load.sum() == naive.sum()
    assert load.max() / load.mean() < 1.05, load / load.mean()
    assert naive.max() / naive.mean() > 1.20, naive / naive.mean()

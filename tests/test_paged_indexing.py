"""CPU model of the work split of the FP16 paged-attention kernels (paged_attn_split_kernel
and paged_attn_prefill_mfma_kernel in fracture_amd/csrc/attention_paged.hip): which query rows
each wave reads and which split partials it writes, checked against the combine kernel's reads.

A wave item is (query group, kv head g, head block hb, split). In causal prefill over one
shared block table, a group is tok consecutive queries: 16 / G of them on the MFMA prefill
kernel (head_dim <= 128, G = qh / kvh <= 8), else 8 / G (G < 8); MFMA column c is head
g G + c % G of query tq0 + c / G. Otherwise tok = 1 and column c is head g G + 8 hb + c. Each
column scores positions below min(split end, its own causal length). The combine reads partial
(vector, split) for every split below the vector's causal length; the model asserts that each
of those is written by exactly one wave, with the causal length of that vector, and that
nothing else is read. No GPU is used.
"""
import numpy as np
import pytest

PAGE = 16
SPLIT = 1024
HEADS_MAX = 8
PF_WAVES = 4  # query groups per workgroup of the MFMA prefill kernel


def causal_len(qi, kv_len, start_pos, max_blocks, seq_lens=None):
    c = int(seq_lens[qi]) if seq_lens is not None else min(start_pos + qi + 1, kv_len)
    return max(0, min(c, max_blocks * PAGE))


def model_split_kernel(nq, qh, kvh, kv_len, start_pos, shared_table=True, seq_lens=None,
                       wrap=None, hd=128):
    G = qh // kvh
    wrap = G if wrap is None else wrap  # head count at which the acc loop's counter wraps
    nhb = (G + HEADS_MAX - 1) // HEADS_MAX
    max_blocks = (max(kv_len, int(max(seq_lens)) if seq_lens is not None else 0) + 15) // 16
    nsplit = max(1, (max_blocks * PAGE + SPLIT - 1) // SPLIT)
    prefill = seq_lens is None and shared_table and nq > 1
    mfma = prefill and hd <= 128 and G <= HEADS_MAX
    tok = (2 * HEADS_MAX // G if mfma else
           HEADS_MAX // G if prefill and G < HEADS_MAX else 1)
    NH = 16 if mfma else 4 if G * tok <= 4 else 8
    per_q = kvh * nhb * nsplit
    waves = []  # (tp0, tq0, ntok, g, hb, split, t_begin, t_end) of each wave that runs the loop
    if mfma:
        # workgroup (PF_WAVES groups, kv head, split); wave w takes the set's group w, and
        # all run the chunks of the set's longest causal length (uniform exits only)
        for wg in range(-(-(-(-nq // tok)) // PF_WAVES) * kvh * nsplit):
            tp0 = (wg // per_q) * PF_WAVES * tok
            if tp0 >= nq:
                continue
            g, split = wg % kvh, (wg // kvh) % nsplit
            clen = causal_len(min(tp0 + PF_WAVES * tok, nq) - 1, kv_len, start_pos, max_blocks,
                              seq_lens)
            t_begin = split * SPLIT
            if t_begin >= clen:
                continue
            for w in range(PF_WAVES):
                tq0 = tp0 + w * tok
                waves.append((tp0, tq0, max(0, min(tok, nq - tq0)), g, 0, split, t_begin,
                              min(clen, t_begin + SPLIT)))
    else:
        for item in range(-(-nq // tok) * per_q):
            tq0 = (item // per_q) * tok
            if tq0 >= nq:
                continue
            ntok = min(tok, nq - tq0)
            g = item % kvh
            hb = (item // kvh) % nhb
            split = (item // (kvh * nhb)) % nsplit
            clen = causal_len(tq0 + ntok - 1, kv_len, start_pos, max_blocks, seq_lens)
            t_begin = split * SPLIT
            if t_begin >= clen:
                continue
            waves.append((tq0, tq0, ntok, g, hb, split, t_begin, min(clen, t_begin + SPLIT)))
    written = {}
    q_rows = set()
    for tp0, tq0, ntok, g, hb, split, t_begin, t_end in waves:
        clen = t_end  # only its bound on the column lengths matters below
        h0 = g * G + hb * HEADS_MAX
        ncols = ntok * G if tok > 1 else min(HEADS_MAX, G - hb * HEADS_MAX)
        assert ncols <= NH
        # per lane column n (0..15): the Q row and the masking limit
        for n in range(16):
            col_ok = n < ncols
            ct = n // G if col_ok else 0
            hn = n - ct * G if col_ok else 0
            # a column past the queries reads the workgroup's first query row (unused)
            row = ((tq0 + ct) if col_ok else tp0) * qh + h0 + hn
            assert 0 <= row < nq * qh
            if not col_ok:
                continue
            assert tok > 1 or ct == 0
            col_len = causal_len(tq0 + ct, kv_len, start_pos, max_blocks, seq_lens) \
                if tok > 1 else t_end
            lim = min(t_end, col_len)
            q_rows.add(row)
            if mfma:
                # the MFMA kernel's partial write of product h, row 4 kg + e: column 8h + 4kg + e
                for col in range(ncols):
                    if col == n:
                        assert (tq0 + col // G) * qh + h0 + col % G == row
            else:
                # the partial write of lane n (== column n) and of the acc loop's column n
                hc, hh = 0, 0
                for h in range(NH):
                    if h == n:
                        assert (tq0 + hc) * qh + h0 + hh == row
                    hh += 1
                    if hh == wrap:
                        hh, hc = 0, hc + 1
            key = (row, split)
            assert key not in written, f"partial {key} written twice"
            written[key] = (lim, t_begin)
    # every partial the combine reads is written once, with that vector's own length
    for qi in range(nq):
        c = causal_len(qi, kv_len, start_pos, max_blocks, seq_lens)
        ns = (c + SPLIT - 1) // SPLIT
        for h in range(qh):
            for s in range(ns):
                lim, t_begin = written.pop((qi * qh + h, s))
                assert lim == min(c, t_begin + SPLIT), (qi, h, s, lim)
                assert lim > t_begin or c == 0
    # what is left was written past a vector's causal length and is never read
    for (row, s), (lim, t_begin) in written.items():
        assert lim <= t_begin
    assert len(q_rows) == sum(qh for qi in range(nq)
                              if causal_len(qi, kv_len, start_pos, max_blocks, seq_lens) > 0)
    return tok


@pytest.mark.parametrize("nq,qh,kvh,kv_len,start_pos,hd,tok", [
    (19, 4, 4, 1050, 1020, 128, 16), (13, 8, 4, 300, 0, 32, 8), (11, 6, 2, 1100, 1019, 256, 2),
    (11, 6, 2, 1100, 1019, 64, 5), (70, 8, 2, 70, 0, 128, 4), (9, 16, 16, 2100, 2040, 64, 16),
    (7, 16, 2, 50, 43, 64, 2), (37, 32, 8, 3000, 2963, 128, 4), (5, 24, 2, 1030, 1025, 128, 1),
    (1, 8, 8, 40, 39, 128, 1), (33, 32, 4, 2100, 2067, 128, 2), (21, 8, 8, 600, 579, 256, 8)])
def test_prefill_groups_cover_every_partial(nq, qh, kvh, kv_len, start_pos, hd, tok):
    assert model_split_kernel(nq, qh, kvh, kv_len, start_pos, hd=hd) == tok


def test_decode_rows_keep_one_query_per_wave():
    lens = np.array([5, 1030, 0, 2048, 17], np.int32)
    assert model_split_kernel(len(lens), 32, 8, 0, 0, shared_table=False, seq_lens=lens) == 1


def test_column_mapping_error_is_caught():
    """The model fails when the acc loop's column counter wraps at the wrong head count."""
    with pytest.raises(AssertionError):
        model_split_kernel(13, 8, 4, 300, 0, wrap=3, hd=256)

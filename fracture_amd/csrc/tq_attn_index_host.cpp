// Host build of the MFMA decode-attention kernel's index arithmetic (tq_attn_index.h), for the
// CPU bounds check of the kernel's global accesses. Each entry evaluates the same inline
// functions the kernel calls, over all 64 lanes where an index depends on the lane.
#include <stdint.h>

#include "tq_attn_index.h"

extern "C" {

// Per-lane tables for kv head g of kvh: K code offsets k_off[pt][lane] (pt = 0..3) and split
// page slots k_page[lane]; V copy offsets v_off[lane]; norm offsets n_off[lane] and slots
// n_page[lane]; query coordinate offsets q_off[s8][lane] (floats, s8 = 0..7).
int fhip_idx_lane_tables(int kvh, int g, uint32_t* k_off, int32_t* k_page, uint32_t* v_off,
                         uint32_t* n_off, int32_t* n_page, int32_t* q_off) {
    if (kvh < 1 || g < 0 || g >= kvh || !k_off || !k_page || !v_off || !n_off || !n_page || !q_off)
        return -1;
    for (int lane = 0; lane < 64; ++lane) {
        for (int pt = 0; pt < 4; ++pt)
            k_off[pt * 64 + lane] = fhip_idx::k_offset(lane, kvh, g) + pt * fhip_idx::k_tile_stride(kvh);
        k_page[lane] = fhip_idx::k_page(lane);
        v_off[lane] = fhip_idx::v_offset(lane, kvh, g);
        n_off[lane] = fhip_idx::norm_offset(lane, kvh, g);
        n_page[lane] = fhip_idx::norm_page(lane);
        for (int s8 = 0; s8 < 8; ++s8) q_off[s8 * 64 + lane] = fhip_idx::q_lane_offset(lane, s8);
    }
    return 0;
}

// 2-bit V codes: the per-lane load offsets v2_off[lane] for kv head g of kvh.
int fhip_idx_v2_offsets(int kvh, int g, uint32_t* v2_off) {
    if (kvh < 1 || g < 0 || g >= kvh || !v2_off) return -1;
    for (int lane = 0; lane < 64; ++lane) v2_off[lane] = fhip_idx::v2_offset(lane, kvh, g);
    return 0;
}

// Workgroup wg of a launch with kvh kv heads -> its item and kv head.
int fhip_idx_wg_item(int64_t wg, int kvh, int64_t* item, int32_t* g) {
    if (kvh < 1 || wg < 0 || !item || !g) return -1;
    int gg;
    fhip_idx::wg_item(wg, kvh, *item, gg);
    *g = gg;
    return 0;
}

// Workgroup lin of the VALU split kernel's grid (nsplit, kvh, nq) -> (split, kv head, query).
int fhip_idx_split_grid_item(int64_t lin, int nsplit, int kvh, int nq, int32_t* split,
                             int32_t* kvhead, int32_t* qi) {
    const int64_t total = (int64_t)nsplit * kvh * nq;
    if (nsplit < 1 || kvh < 1 || nq < 1 || lin < 0 || lin >= total || !split || !kvhead || !qi)
        return -1;
    int s, h, q;
    fhip_idx::split_grid_item(lin, total, nsplit, kvh, s, h, q);
    *split = s;
    *kvhead = h;
    *qi = q;
    return 0;
}

// Wave `wave` of block blk: its split's first position, and per lane the block-table column
// of split page `lane` and whether that page holds positions of [t_begin, t_end).
int fhip_idx_split(int blk, int wave, int t_end, int32_t* t_begin, int32_t* column,
                   uint8_t* in_split) {
    if (blk < 0 || wave < 0 || !t_begin || !column || !in_split) return -1;
    *t_begin = fhip_idx::split_begin(blk, wave);
    for (int lane = 0; lane < 64; ++lane) {
        int c;
        in_split[lane] = fhip_idx::split_page_column(*t_begin, t_end, lane, c) ? 1 : 0;
        column[lane] = c;
    }
    return 0;
}

// The first split page of the chunk starting at t0.
int32_t fhip_idx_chunk_first_page(int t0, int t_begin) {
    return fhip_idx::chunk_first_page(t0, t_begin);
}

// Per lane: the rotated-query vector its MFMA column reads, and whether the column is live.
int fhip_idx_q_vectors(int tq0, int tok, int G, int nq, int qh, int g, int64_t* vec, uint8_t* live) {
    if (G < 1 || tok < 1 || !vec || !live) return -1;
    for (int lane = 0; lane < 64; ++lane) {
        bool l;
        vec[lane] = fhip_idx::q_vector(lane, tq0, tok, G, nq, qh, g, l);
        live[lane] = l ? 1 : 0;
    }
    return 0;
}

// The partial row the merge writes for head column h of the item (query group tq0, kv head g,
// block blk).
int64_t fhip_idx_partial_row(int h, int tq0, int G, int qh, int g, int nsplit, int blk) {
    return fhip_idx::partial_row(fhip_idx::partial_vector(h, tq0, G, qh, g), nsplit, blk);
}

}  // extern "C"

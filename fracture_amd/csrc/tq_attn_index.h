// Index arithmetic of the MFMA decode-attention kernel (tq_attn_mfma_kernel, head_dim 128,
// 4-bit K codes, 4- or 2-bit V codes), shared by the kernel and by a host build of the functions
// (tq_attn_index_host.cpp). The CPU bounds check of every global access the kernel makes
// calls the host build, so it covers the arithmetic the kernel runs rather than a restatement
// of it. Page layout (quantized_paged_kv_cache.rs:86-128): a page holds 16 positions; its K
// codes are [16][kvh][64] bytes, its K norms [16][kvh] fp16, and the same for V.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define FHIP_IDX __host__ __device__ __forceinline__
#else
#define FHIP_IDX inline
#endif

namespace fhip_idx {

constexpr int kPageTokens = 16;      // positions per page
constexpr int kCodeRow = 64;         // bytes of one position's 4-bit codes for one kv head
constexpr int kChunk = 64;           // positions per chunk of a wave's loop
constexpr int kSplitPositions = 512; // positions per wave (one split)
constexpr int kBlockWaves = 2;       // waves per workgroup: one 1024-position block
constexpr int kXcdCount = 8;         // MI355X: workgroup b runs on XCD b % 8

// Workgroup wg -> (item, kv head g). An item is a (query group, block); the 8 kv heads of one
// item land on one XCD, whose L2 then holds the 128-byte lines that those heads' code rows share.
// Item i runs on XCD (i + i / 8) % 8: each group of 8 consecutive items is rotated by its group
// index. With XCD i % 8 instead, a query's blocks b, b + 8, b + 16, ... all land on XCD b % 8
// whenever the block count per query is a multiple of 8 (32 at 32768 positions), and as the
// later blocks exist only for the longer sequences, XCD 0 got up to 1.6x the work of XCD 7.
FHIP_IDX void wg_item(int64_t wg, int kvh, int64_t& item, int& g) {
    const int64_t per8 = (int64_t)kXcdCount * kvh;
    const int64_t a = wg / per8;              // the group of 8 items
    const int x = (int)(wg % kXcdCount);      // the XCD
    item = a * kXcdCount + (x - (int)(a % kXcdCount) + kXcdCount) % kXcdCount;
    g = (int)((wg % per8) / kXcdCount);
}

// The VALU split kernel's grid (nsplit, kvh, queries): workgroup `lin` in linear dispatch order
// (of `total`) -> (split, kv head, query). In the grid's own order split s of every (kv head,
// query) would run on XCD s % 8 whenever nsplit is a multiple of 8, loading XCD 0 most (later
// splits exist only for longer sequences). Each full group of 8 consecutive workgroups is
// rotated by its group index instead, as in wg_item; a partial last group keeps its order.
// The rotated index is then decoded split fastest.
FHIP_IDX void split_grid_item(int64_t lin, int64_t total, int nsplit, int kvh, int& split,
                              int& kvhead, int& qi) {
    const int64_t grp = lin / kXcdCount;
    const int64_t eff =
        (grp + 1) * kXcdCount <= total
            ? grp * kXcdCount + ((int)(lin % kXcdCount) - (int)(grp % kXcdCount) + kXcdCount) % kXcdCount
            : lin;
    split = (int)(eff % nsplit);
    kvhead = (int)((eff / nsplit) % kvh);
    qi = (int)(eff / ((int64_t)nsplit * kvh));
}

// First position of wave `wave`'s split in block blk.
FHIP_IDX int split_begin(int blk, int wave) { return (kBlockWaves * blk + wave) * kSplitPositions; }

// Lane j of a wave reads the block-table column of its split's page j, if that page holds
// positions of the split [t_begin, t_end).
FHIP_IDX bool split_page_column(int t_begin, int t_end, int lane, int& column) {
    column = t_begin / kPageTokens + lane;
    return t_begin + kPageTokens * lane < t_end;
}

// The split page (0..31) holding the first position of the chunk starting at t0.
FHIP_IDX int chunk_first_page(int t0, int t_begin) { return (t0 - t_begin) / kPageTokens; }

// K codes of a chunk: lane (n = lane & 15, rg = lane >> 4) reads split page
// chunk_first_page + k_page(lane), 16 bytes at k_offset + pt * k_tile_stride for pt = 0..3:
// position 4 (n & 3) + pt of the page, bytes [16 rg, 16 rg + 16) of kv head g's code row.
FHIP_IDX int k_page(int lane) { return (lane & 15) >> 2; }
FHIP_IDX uint32_t k_offset(int lane, int kvh, int g) {
    return (uint32_t)((4 * ((lane & 15) & 3) * kvh + g) * kCodeRow + 16 * (lane >> 4));
}
FHIP_IDX uint32_t k_tile_stride(int kvh) { return (uint32_t)(kvh * kCodeRow); }

// V codes of a chunk by LDS DMA: copy i (0..3) moves split page chunk_first_page + i; lane L
// copies position L / 4 of that page, 16-byte segment (L % 4) ^ ((L / 8) % 4) of kv head g's
// code row (the XOR swizzle spreads a transposed read of one dim range over the banks).
FHIP_IDX uint32_t v_offset(int lane, int kvh, int g) {
    return (uint32_t)(((lane >> 2) * kvh + g) * kCodeRow + 16 * ((lane & 3) ^ ((lane >> 3) & 3)));
}
// The same with 2-bit V codes (rows of kCodeRow / 2 bytes): lane L loads the 8 bytes that hold
// the codes of the 16-byte segment v_offset names, and widens them to it.
FHIP_IDX uint32_t v2_offset(int lane, int kvh, int g) {
    return (uint32_t)(((lane >> 2) * kvh + g) * (kCodeRow / 2) + 8 * ((lane & 3) ^ ((lane >> 3) & 3)));
}

// Norms of a chunk: lane L reads split page chunk_first_page + norm_page(L), the fp16 norm of
// position L % 16 and kv head g (K and V alike).
FHIP_IDX int norm_page(int lane) { return lane >> 4; }
FHIP_IDX uint32_t norm_offset(int lane, int kvh, int g) { return (uint32_t)(((lane & 15) * kvh + g) * 2); }

// The rotated query a lane's MFMA column reads: column h = lane & 7 is head h % G of query
// group member h / G; a column past the group's heads or queries reads the group's first
// vector (and is zeroed). Returns the vector index; *live tells whether the column is real.
FHIP_IDX int64_t q_vector(int lane, int tq0, int tok, int G, int nq, int qh, int g, bool& live) {
    const int h = lane & 7, ct = h / G, ch = h - ct * G;
    live = h < tok * G && tq0 + ct < nq;
    return (int64_t)(live ? tq0 + ct : tq0) * qh + (int64_t)g * G + (live ? ch : 0);
}
// Offset (floats) of the lane's 4 query coordinates of step s8 within its vector.
FHIP_IDX int q_lane_offset(int lane, int s8) { return 32 * (lane >> 4) + 4 * s8; }

// The partial the merge writes for head column h (< tok G) of the item's query group: vector
// (query tq0 + h / G, head G g + h % G), block blk; part_ml row and part_acc row of it.
FHIP_IDX int64_t partial_vector(int h, int tq0, int G, int qh, int g) {
    const int ht = h / G;
    return (int64_t)(tq0 + ht) * qh + (int64_t)g * G + (h - ht * G);
}
FHIP_IDX int64_t partial_row(int64_t vec, int nsplit, int blk) { return vec * nsplit + blk; }

}  // namespace fhip_idx

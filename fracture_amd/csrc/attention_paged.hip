// GQA decode / prefill attention over an FP16 paged KV cache, for gfx950.
//
// Semantics follow attention_paged.cu:36-170: query token i of a sequence attends to
// positions 0 .. min(start_pos + i + 1, kv_len) - 1 (or seq_lens[i] in the batched form);
// position t lives in page block_table[t / 16], row (t % 16), as a [16][kv_heads][head_dim]
// fp16 block; score = dot(q, k) / sqrt(head_dim) with fp32 accumulation, softmax in fp32,
// out = half(sum_t p_t v_t). The reference keeps a kv_len-float score row in shared memory
// (attention_paged.cu:58-59, 176); here the context is split into 1024-position pieces with an
// online softmax each, merged by a second kernel: up to 1,048,576 positions per sequence.
//
// Work split: one wave per (query, kv head, block of up to 8 of its q heads, split). Each K
// row crosses HBM once per (query, kv head) for up to 8 q heads. In causal prefill with fewer
// than 8 q heads per kv head, a wave takes 8 / G consecutive queries instead, its columns
// being (query, head) pairs each masked to its own causal length, so that a K or V row is
// read once for all of them. Per 32-position chunk (16 when head_dim is 256):
//   QK on v_mfma_f32_16x16x32_f16: A = K rows (row = position, 8 consecutive dims per lane,
//      exactly their memory layout), B = Q^T (column = q head): fp16 x fp16 products are
//      exact in fp32, the sums are fp32;
//   online softmax per head in log2 units, weights to LDS;
//   PV on the VALU in fp32: lane (dim group of 8, position subset) loads 16 bytes of a V row
//      and accumulates p_h * v for the wave's heads. V needs no transpose this way, and the
//      fp32 weights need no fp16 rounding.
// The kernel streams 4 * head_dim bytes per (position, kv head) and is bound by HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fhip_common.h"
#include "fracture_hip.h"

using namespace fhip;

namespace {

constexpr int kPSplit = 1024;  // positions per split: 64 pages, one per lane of the page cache
constexpr int kPWaves = 2;     // waves per workgroup (independent work items)
constexpr int kHeadsMax = 8;   // q heads per wave
// Longest context a block table may describe (the combine kernel keeps one weight per
// split in LDS: 4 KiB at this bound).
constexpr int64_t kMaxTokens = (int64_t)kPSplit * 1024;

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// Page sources: per-block pointer arrays (the reference's interface) or contiguous pools.
struct F16PtrPages {
    const uint8_t* const* k;
    const uint8_t* const* v;
    int num_pages;
    __device__ bool valid(int p) const { return p >= 0 && p < num_pages; }
    // Wave-wide page cache: lane j holds the pointers of page j of the current split; the
    // `_at` accessors read them back from lane j.
    struct Lane {
        const uint8_t *k, *v;
    };
    __device__ Lane lane_load(int p) const {
        if (!valid(p)) return Lane{nullptr, nullptr};
        return Lane{k[p], v[p]};
    }
    static __device__ const uint8_t* rl(const uint8_t* x, int j) {
        const uint64_t u = (uint64_t)x;
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, j);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
        return (const uint8_t*)(((uint64_t)hi << 32) | lo);
    }
    __device__ const uint8_t* k_at(const Lane& l, int j, int) const { return rl(l.k, j); }
    __device__ const uint8_t* v_at(const Lane& l, int j, int) const { return rl(l.v, j); }
    // one lane's own page (any page id per lane)
    __device__ const uint8_t* k_page(int p) const { return k[p]; }
    __device__ const uint8_t* v_page(int p) const { return v[p]; }
};
struct F16PoolPages {
    const uint8_t* k;
    const uint8_t* v;
    int64_t sk, sv;  // bytes between pages
    int num_pages;
    __device__ bool valid(int p) const { return p >= 0 && p < num_pages; }
    struct Lane {};
    __device__ Lane lane_load(int) const { return Lane{}; }
    __device__ const uint8_t* k_at(const Lane&, int, int p) const { return k + p * sk; }
    __device__ const uint8_t* v_at(const Lane&, int, int p) const { return v + p * sv; }
    __device__ const uint8_t* k_page(int p) const { return k + p * sk; }
    __device__ const uint8_t* v_page(int p) const { return v + p * sv; }
};

// Query i reads block-table row i (stride 0: one shared table) and attends to seq_lens[i]
// positions, or min(start_pos + i + 1, kv_len) when seq_lens is null; never more than the
// table holds.
struct PQueries {
    const int32_t* table;
    int64_t table_stride;
    int max_blocks;
    const int32_t* seq_lens;
    int kv_len, start_pos;
    int count;
    __device__ int causal_len(int qi) const {
        int c;
        if (seq_lens) {
            c = seq_lens[qi];
        } else {
            c = start_pos + qi + 1;
            if (c > kv_len) c = kv_len;
        }
        const int cap = max_blocks * FHIP_PAGE_TOKENS;
        if (c > cap) c = cap;
        return c < 0 ? 0 : c;
    }
};

// Split partials: per (query, q head, split) the running max m (natural log units), the sum
// l and the unnormalised accumulator acc[hd]. Splits at or past the causal length are not
// written; the combine kernel reads only the splits below it.
template <int HD, int NH, class Pages>
__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(2))) void
paged_attn_split_kernel(const uint16_t* __restrict__ q, PQueries qs, Pages pg, int qh, int kvh,
                        int nhb, float scale_log2, float* __restrict__ part_ml,
                        float* __restrict__ part_acc, int nsplit, int tok) {
    constexpr int kChunk = HD <= 128 ? 32 : 16;  // positions per chunk
    constexpr int kTiles = kChunk / 16;          // 16-position MFMA tiles (= pages) per chunk
    constexpr int kSteps = HD / 32;              // MFMA steps per tile
    constexpr int kDg = HD / 8;                  // lanes per V row, 8 dims each
    constexpr int kPpl = 64 / kDg;               // positions per V load
    constexpr int kVLoads = kChunk / kPpl;
    static_assert(kPpl <= 16 && 16 % kPpl == 0, "a V load stays inside one page");
    // Every lane writes its own slot of these buffers (columns / entries past the wave's
    // heads are written and never read): a store guarded by the lane index followed by reads
    // of every lane lets the compiler sink the reads into the guarded block, where they run
    // with the other lanes switched off (seen in a variant of this loop at head_dim 32).
    __shared__ __attribute__((aligned(16))) float pbuf[kPWaves][kChunk][16];
    __shared__ __attribute__((aligned(16))) float abuf[kPWaves][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t item = (int64_t)blockIdx.x * kPWaves + wave;
    const int64_t per_q = (int64_t)kvh * nhb * nsplit;
    // queries tq0 .. tq0 + ntok - 1 (tok > 1 only in causal prefill over one shared table
    // with nhb == 1, where causal lengths grow with the query index)
    const int tq0 = (int)(item / per_q) * tok;
    if (tq0 >= qs.count) return;
    const int ntok = min(tok, qs.count - tq0);
    // kv head fastest: waves of one workgroup read neighbouring rows of the same pages
    const int g = (int)(item % kvh);
    const int hb = (int)((item / kvh) % nhb);
    const int split = (int)((item / ((int64_t)kvh * nhb)) % nsplit);
    const int clen = qs.causal_len(tq0 + ntok - 1);
    const int t_begin = split * kPSplit;
    if (t_begin >= clen) return;
    const int t_end = min(clen, t_begin + kPSplit);
    const int G = qh / kvh;
    const int h0 = g * G + hb * kHeadsMax;
    // MFMA columns (<= NH): with tok == 1 heads h0 .. h0 + ncols - 1 of query tq0, else
    // column c is head h0 + c % G of query tq0 + c / G
    const int ncols = tok > 1 ? ntok * G : min(kHeadsMax, G - hb * kHeadsMax);
    const int32_t* table = qs.table + (int64_t)tq0 * qs.table_stride;

    // the split's pages, one per lane, read once
    static_assert(kPSplit == 64 * FHIP_PAGE_TOKENS, "one cached page per lane");
    const int split_page =
        t_begin + FHIP_PAGE_TOKENS * lane < t_end ? table[t_begin / FHIP_PAGE_TOKENS + lane] : -1;
    const typename Pages::Lane pl = pg.lane_load(split_page);

    // Q^T as the QK B operand: lane (column n, k group kg) holds dims 32 s + 8 kg + 0..7 of
    // column n's query row at step s; columns n >= ncols are zero and fully masked.
    const int n = lane & 15, kg = lane >> 4;
    const bool col_ok = n < ncols;
    const int ct = col_ok ? n / G : 0;  // 0 whenever tok == 1 (n < ncols <= G)
    const int hn = col_ok ? n - ct * G : 0;
    const int col_len = !col_ok ? 0 : tok > 1 ? qs.causal_len(tq0 + ct) : clen;
    const int lim = min(t_end, col_len);  // column n scores positions below lim
    u32x4 bq[kSteps];
    {
        const uint16_t* qrow = q + ((int64_t)(tq0 + ct) * qh + h0 + hn) * HD + 8 * kg;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const u32x4 v = ld16(qrow + 32 * s);
            bq[s] = col_ok ? v : u32x4{0u, 0u, 0u, 0u};
        }
    }
    // lane offsets inside a page: K row (lane & 15) segment kg; V row of position subset ps,
    // dims 8 dg .. 8 dg + 7
    const int64_t k_off = ((int64_t)(lane & 15) * kvh + g) * (HD * 2) + 16 * kg;
    const int dg = lane % kDg, ps = lane / kDg;
    const uint8_t* dummy = (const uint8_t*)q;  // >= 2 HD readable bytes, finite values

    float m_run = -__builtin_inff(), l_run = 0.0f;  // lanes n (any kg): head n
    float acc[NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;

    for (int t0 = t_begin; t0 < t_end; t0 += kChunk) {
        const int j0 = (t0 - t_begin) / FHIP_PAGE_TOKENS;
        // ---- every load of the chunk first: K rows, then V rows. Loads of positions past
        // the end or in invalid pages read `dummy` and are masked below.
        bool pok[kTiles];
        const uint8_t* kb[kTiles];
        const uint8_t* vb[kTiles];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt) {
            const int id = __builtin_amdgcn_readlane(split_page, j0 + tt);
            pok[tt] = pg.valid(id);
            kb[tt] = pok[tt] ? pg.k_at(pl, j0 + tt, id) : dummy;
            vb[tt] = pok[tt] ? pg.v_at(pl, j0 + tt, id) : dummy;
        }
        u32x4 kr[kTiles][kSteps];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt) {
            const bool ok = pok[tt] && t0 + 16 * tt + (lane & 15) < t_end;
            const uint8_t* src = ok ? kb[tt] + k_off : dummy;
#pragma unroll
            for (int s = 0; s < kSteps; ++s) kr[tt][s] = ld16(src + 64 * s);
        }
        u32x4 vr[kVLoads];
        bool vok[kVLoads];
#pragma unroll
        for (int j = 0; j < kVLoads; ++j) {
            const int pp = j * kPpl + ps;  // position in the chunk
            const int tt = (j * kPpl) / 16;
            vok[j] = pok[tt] && t0 + pp < t_end;
            const uint8_t* src =
                vok[j] ? vb[tt] + (((int64_t)(pp % 16) * kvh + g) * HD + 8 * dg) * 2 : dummy;
            vr[j] = ld16(src);
        }

        // ---- QK: lane (n, rg) gets positions 16 tt + 4 rg + e of head n
        float sc[kTiles][4];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt) {
            f4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kSteps; ++s)
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, kr[tt][s]),
                                                           __builtin_bit_cast(h8_t, bq[s]), d,
                                                           0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pos = t0 + 16 * tt + 4 * kg + e;
                sc[tt][e] = pok[tt] && pos < lim ? d[e] * scale_log2 : -__builtin_inff();
            }
        }
        // ---- online softmax per head (lanes n, n + 16, n + 32, n + 48 share head n)
        float cmax = -__builtin_inff();
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) cmax = fmaxf(cmax, sc[tt][e]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run, cmax);
        const float mref = m_new == -__builtin_inff() ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - mref);  // 0 while m_run is -inf
        float psum = 0.0f;
        // the previous chunk's reads of pbuf / abuf (other lanes' words) stay above these writes
        wave_lds_sync();
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = __builtin_amdgcn_exp2f(sc[tt][e] - mref);
                psum += p;
                pbuf[wave][16 * tt + 4 * kg + e][n] = p;
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        abuf[wave][lane] = alpha;
        // every lane's pbuf / abuf writes stay above the cross-lane reads below
        wave_lds_sync();

        // ---- PV
        float al[kHeadsMax];
        {
            const f4_t a0 = *(const f4_t*)&abuf[wave][0];
            const f4_t a1 = *(const f4_t*)&abuf[wave][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                al[i] = a0[i];
                al[4 + i] = a1[i];
            }
        }
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h][i] *= al[h];
#pragma unroll
        for (int j = 0; j < kVLoads; ++j) {
            const int pp = j * kPpl + ps;
            float pw[kHeadsMax];
            {
                const f4_t p0 = *(const f4_t*)&pbuf[wave][pp][0];
                const f4_t p1 = *(const f4_t*)&pbuf[wave][pp][4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pw[i] = p0[i];
                    pw[4 + i] = p1[i];
                }
            }
            float v[8];
            unpack16<TrF16>(vok[j] ? vr[j] : u32x4{0u, 0u, 0u, 0u}, v);
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(pw[h], v[i], acc[h][i]);
        }
    }

    // ---- partials: sum the position subsets (lanes with the same dim group), then lanes of
    // subset 0 write dims 8 dg .. 8 dg + 7 of each head
#pragma unroll
    for (int o = kDg; o < 64; o <<= 1)
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h][i] += __shfl_xor(acc[h][i], o);
    // column c's vector: (query tq0 + c / G, head h0 + c % G)
    if (lane < ncols) {  // lane == n here
        const int64_t v = (int64_t)(tq0 + ct) * qh + h0 + hn;
        part_ml[(v * nsplit + split) * 2 + 0] = m_run * 0.6931471805599453f;
        part_ml[(v * nsplit + split) * 2 + 1] = l_run;
    }
    if (ps == 0) {
        int hc = 0, hh = 0;  // column h is head h0 + hh of query tq0 + hc
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            if (h < ncols) {
                const int64_t v = (int64_t)(tq0 + hc) * qh + h0 + hh;
                float* dst = part_acc + (v * nsplit + split) * HD + 8 * dg;
                *(f4_t*)dst = f4_t{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
                *(f4_t*)(dst + 4) = f4_t{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
            }
            if (++hh == G) {
                hh = 0;
                ++hc;
            }
        }
    }
}

// Causal prefill groups with PV on the MFMA as well (head_dim 32 / 64 / 128, G <= 8 q heads per
// kv head): a wave takes 16 / G consecutive queries, MFMA column c being head c % G of query
// c / G. Per 32-position chunk:
//   QK as in paged_attn_split_kernel, over 16 columns;
//   PV on v_mfma_f32_16x16x32_f16, two products per 16-dim block: out[col][d] +=
//     P[col][slot] V[slot][d] for columns 0..7, then 8..15. Slot 8q + i of lane group q is
//     position 4q + i (i < 4) or 16 + 4q + i - 4: exactly the positions whose probabilities
//     that lane group holds after QK. In the product for columns 8h .. 8h + 7, A row m < 8 is
//     fp16(p) of column 8h + m and row 8 + m is fp16((p - fp16(p)) 2^12) of the same column
//     (one DPP row rotation by 8 brings each lane its partner column's p), and the output
//     is D[m] + 2^-12 D[8 + m]: fp32 weights to ~2^-22, V exact.
//   The kPfWaves waves of a workgroup take consecutive query groups over the same kv head and
//     split and share each chunk: the workgroup loads its K and V rows into LDS once and every
//     wave reads all of them (the chunk's K and V cross L2 once per kPfWaves x 16 / G queries);
//   B = V transposed: the chunk's V rows are staged in LDS row-major (rows padded so that the
//     four rows one transposed read gathers sit on different banks), and
//     ds_read_b64_tr_b16 gives lane (d, q) dim d of the 4 positions addressed by source
//     lanes a + 4k of its 16-lane group (destination lane 4a + b takes element b of each).
constexpr int kPfWaves = 4;  // prefill: waves (query groups) per workgroup sharing each chunk
template <int HD, class Pages>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(2))) void
paged_attn_prefill_mfma_kernel(const uint16_t* __restrict__ q, PQueries qs, Pages pg, int qh,
                               int kvh, float scale_log2, float* __restrict__ part_ml,
                               float* __restrict__ part_acc, int nsplit, int tok) {
    constexpr int kChunk = 32;
    constexpr int kTiles = 2;
    constexpr int kSteps = HD / 32;
    constexpr int kBlk = HD / 16;  // PV output dim blocks
    constexpr int kRow = HD * 2 + 32;   // bytes per staged V row
    constexpr int kRowK = HD * 2 + 16;  // per staged K row: 16 rows' reads of one segment
                                        // cover all banks
    static_assert(HD >= 32 && HD <= 128, "head_dim 32, 64 or 128");
    constexpr int kPieces = kChunk * HD / 8;  // 16-byte pieces of a chunk's K (and of its V)
    constexpr int kPer = (kPieces + 64 * kPfWaves - 1) / (64 * kPfWaves);
    __shared__ __attribute__((aligned(16))) uint8_t kbuf[kChunk * kRowK];
    __shared__ __attribute__((aligned(16))) uint8_t vbuf[kChunk * kRow];
    __shared__ __attribute__((aligned(16))) float abuf[kPfWaves][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroup (kPfWaves query groups, kv head, split); wave w takes the set's group w. Every
    // exit before the chunk loop is uniform over the workgroup (the loop has barriers).
    const int64_t wg = blockIdx.x;
    const int64_t per_p = (int64_t)kvh * nsplit;
    const int tp0 = (int)(wg / per_p) * kPfWaves * tok;  // the set's first query
    if (tp0 >= qs.count) return;
    const int tq0 = tp0 + wave * tok;
    const int ntok = max(0, min(tok, qs.count - tq0));  // 0: a wave past the last query
    const int g = (int)(wg % kvh);
    const int split = (int)((wg / kvh) % nsplit);
    // the set's longest causal length
    const int clen = qs.causal_len(min(tp0 + kPfWaves * tok, qs.count) - 1);
    const int t_begin = split * kPSplit;
    if (t_begin >= clen) return;
    const int t_end = min(clen, t_begin + kPSplit);
    const int G = qh / kvh;
    const int h0 = g * G;
    const int ncols = ntok * G;  // <= 16
    const int32_t* table = qs.table + (int64_t)tp0 * qs.table_stride;

    static_assert(kPSplit == 64 * FHIP_PAGE_TOKENS, "one cached page per lane");
    const int split_page =
        t_begin + FHIP_PAGE_TOKENS * lane < t_end ? table[t_begin / FHIP_PAGE_TOKENS + lane] : -1;
    const typename Pages::Lane pl = pg.lane_load(split_page);

    // column n is head h0 + n % G of query tq0 + n / G
    const int n = lane & 15, kg = lane >> 4;
    const bool col_ok = n < ncols;
    const int ct = col_ok ? n / G : 0;
    const int hn = col_ok ? n - ct * G : 0;
    const int lim = col_ok ? min(t_end, qs.causal_len(tq0 + ct)) : 0;
    u32x4 bq[kSteps];
    {
        const uint16_t* qrow = q + ((int64_t)(col_ok ? tq0 + ct : tp0) * qh + h0 + hn) * HD + 8 * kg;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const u32x4 v = ld16(qrow + 32 * s);
            bq[s] = col_ok ? v : u32x4{0u, 0u, 0u, 0u};
        }
    }
    const uint8_t* dummy = (const uint8_t*)q;
    uint8_t* vb = vbuf;
    // transposed-read source of this lane: row 4q + k (+16 for slots 4..7), dims 4a .. 4a + 3
    // of each 16-dim block (q = lane / 16, k = (lane / 4) % 4, a = lane % 4)
    const uint32_t tr_off =
        (uint32_t)((4 * (lane >> 4) + ((lane >> 2) & 3)) * kRow + 8 * (lane & 3));

    float m_run = -__builtin_inff(), l_run = 0.0f;
    f4_t acc[2][kBlk];  // columns 0..7, 8..15
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int b = 0; b < kBlk; ++b) acc[h][b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (int t0 = t_begin; t0 < t_end; t0 += kChunk) {
        const int j0 = (t0 - t_begin) / FHIP_PAGE_TOKENS;
        bool pok[kTiles];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt)
            pok[tt] = pg.valid(__builtin_amdgcn_readlane(split_page, j0 + tt));
        // ---- the chunk's K and V rows, 16-byte pieces spread over the workgroup: piece i is
        // row i / (HD / 8), segment i % (HD / 8). Rows past the end or in invalid pages read
        // `dummy` (finite); their V is staged as zeros (0 * NaN would poison PV).
        const uint8_t* kpg[kTiles];
        const uint8_t* vpg[kTiles];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt) {
            const int id = __builtin_amdgcn_readlane(split_page, j0 + tt);
            kpg[tt] = pok[tt] ? pg.k_at(pl, j0 + tt, id) : dummy;
            vpg[tt] = pok[tt] ? pg.v_at(pl, j0 + tt, id) : dummy;
        }
        u32x4 kr[kPer], vr[kPer];
        bool rok[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = min((int)threadIdx.x + 64 * kPfWaves * u, kPieces - 1);
            const int r = i / (HD / 8), sg = i % (HD / 8);
            rok[u] = pok[r / 16] && t0 + r < t_end;
            const int64_t off = ((int64_t)(r % 16) * kvh + g) * (HD * 2) + 16 * sg;
            kr[u] = ld16(rok[u] ? kpg[r / 16] + off : dummy);
            vr[u] = ld16(rok[u] ? vpg[r / 16] + off : dummy);
        }
        // ---- stage: every wave has finished reading the previous chunk
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = (int)threadIdx.x + 64 * kPfWaves * u;
            if (i < kPieces) {
                const int r = i / (HD / 8), sg = i % (HD / 8);
                *(u32x4*)(kbuf + r * kRowK + 16 * sg) = kr[u];
                *(u32x4*)(vb + r * kRow + 16 * sg) = rok[u] ? vr[u] : u32x4{0u, 0u, 0u, 0u};
            }
        }
        __syncthreads();

        // ---- QK: lane (n, kg) gets positions 16 tt + 4 kg + e of column n
        float sc[kTiles][4];
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt) {
            f4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < kSteps; ++st) {
                const u32x4 kv =
                    *(const u32x4*)(kbuf + (16 * tt + (lane & 15)) * kRowK + 64 * st + 16 * kg);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, kv),
                                                           __builtin_bit_cast(h8_t, bq[st]), d,
                                                           0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pos = t0 + 16 * tt + 4 * kg + e;
                sc[tt][e] = pok[tt] && pos < lim ? d[e] * scale_log2 : -__builtin_inff();
            }
        }
        // ---- online softmax per column (lanes n, n + 16, n + 32, n + 48)
        float cmax = -__builtin_inff();
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) cmax = fmaxf(cmax, sc[tt][e]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run, cmax);
        const float mref = m_new == -__builtin_inff() ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - mref);
        float psum = 0.0f;
        _Float16 a[2][8];  // A of the products for columns 0..7 and 8..15
#pragma unroll
        for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = __builtin_amdgcn_exp2f(sc[tt][e] - mref);
                psum += p;
                // p of column n ^ 8 (lane n of each 16-lane row takes lane n ^ 8)
                const float po = __int_as_float(
                    __builtin_amdgcn_mov_dpp(__float_as_int(p), 0x128, 0xF, 0xF, true));
                const _Float16 ph = (_Float16)p, oh = (_Float16)po;
                const _Float16 pl_ = (_Float16)((p - (float)ph) * 4096.0f);
                const _Float16 ol = (_Float16)((po - (float)oh) * 4096.0f);
                a[0][4 * tt + e] = n < 8 ? ph : ol;  // rows: hi of column n / lo of column n - 8
                a[1][4 * tt + e] = n < 8 ? oh : pl_;  // hi of column n + 8 / lo of column n
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        abuf[wave][lane] = alpha;
        wave_lds_sync();
        // ---- PV: rescale rows 4 kg + e (columns 8h + 4 (kg % 2) + e), then accumulate
        const f4_t al0 = *(const f4_t*)&abuf[wave][4 * (kg & 1)];
        const f4_t al1 = *(const f4_t*)&abuf[wave][8 + 4 * (kg & 1)];
        const h8_t av0 = {a[0][0], a[0][1], a[0][2], a[0][3], a[0][4], a[0][5], a[0][6], a[0][7]};
        const h8_t av1 = {a[1][0], a[1][1], a[1][2], a[1][3], a[1][4], a[1][5], a[1][6], a[1][7]};
#pragma unroll
        for (int b = 0; b < kBlk; ++b) {
            typedef short v4s_t __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;
            const uint8_t* base = vb + tr_off + 32 * b;
            const v4s_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_v4s_t*)(__attribute__((address_space(3))) uint8_t*)base);
            const v4s_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_v4s_t*)(__attribute__((address_space(3))) uint8_t*)(base + 16 * kRow));
            const h8_t bv = __builtin_bit_cast(
                h8_t, (short __attribute__((ext_vector_type(8)))){lo4[0], lo4[1], lo4[2], lo4[3],
                                                                  hi4[0], hi4[1], hi4[2], hi4[3]});
            acc[0][b] *= al0;
            acc[0][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av0, bv, acc[0][b], 0, 0, 0);
            acc[1][b] *= al1;
            acc[1][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av1, bv, acc[1][b], 0, 0, 0);
        }
    }

    // ---- partials: in product h, lanes kg < 2 hold rows 4 kg + e (column 8h + 4 kg + e,
    // fp16(p) part), lanes kg + 2 the matching 2^12 (p - fp16(p)) rows
    if (lane < ncols) {  // lane == n here
        const int64_t v = (int64_t)(tq0 + ct) * qh + h0 + hn;
        part_ml[(v * nsplit + split) * 2 + 0] = m_run * 0.6931471805599453f;
        part_ml[(v * nsplit + split) * 2 + 1] = l_run;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float o[kBlk][4];
#pragma unroll
        for (int b = 0; b < kBlk; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[b][e] = acc[h][b][e] + __shfl_xor(acc[h][b][e], 32) * (1.0f / 4096.0f);
        if (kg < 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int col = 8 * h + 4 * kg + e;
                if (col < ncols) {
                    const int cq = col / G;
                    const int64_t v = (int64_t)(tq0 + cq) * qh + h0 + (col - cq * G);
                    float* dst = part_acc + (v * nsplit + split) * HD + n;
#pragma unroll
                    for (int b = 0; b < kBlk; ++b) dst[16 * b] = o[b][e];
                }
            }
        }
    }
}

// Any other head_dim (1 .. 256; the reference kernel takes any width): one wave per (query,
// q head, 1024-position split), same partials as paged_attn_split_kernel. Per 64-position
// chunk, lane l scores position t0 + l against the query (fp32 dot over the dims in order,
// the query staged in LDS), the wave updates the online softmax (natural-log units), and each
// lane accumulates its dims l, l + 64, .. over the chunk's positions, their weights and row
// addresses broadcast from the lanes that scored them. A fallback for widths no model on this
// path uses at scale (the tiny test models' 16, odd widths): no MFMA, no vector loads.
constexpr int kGenWaves = 4;
template <class Pages>
__global__ __launch_bounds__(64 * kGenWaves) void paged_attn_generic_kernel(
    const uint16_t* __restrict__ q, PQueries qs, Pages pg, int qh, int kvh, int hd,
    float scale, float* __restrict__ part_ml, float* __restrict__ part_acc, int nsplit,
    int64_t items) {
    __shared__ float qbuf[kGenWaves][256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t item = (int64_t)blockIdx.x * kGenWaves + wave;
    if (item >= items) return;
    const int split = (int)(item % nsplit);
    const int64_t vec = item / nsplit;  // query qi, q head h
    const int qi = (int)(vec / qh), h = (int)(vec % qh);
    const int clen = qs.causal_len(qi);
    const int t_begin = split * kPSplit;
    if (t_begin >= clen) return;  // not read by the combine (splits below the length only)
    const int t_end = min(clen, t_begin + kPSplit);
    const int g = h / (qh / kvh);
    const int32_t* table = qs.table + (int64_t)qi * qs.table_stride;
    float* qv = qbuf[wave];
    for (int d = lane; d < hd; d += 64) qv[d] = h2f(q[vec * hd + d]);
    wave_lds_sync();  // every lane reads every dim below
    float m_run = -__builtin_inff(), l_run = 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // dims lane + 64 i
    const int64_t row_bytes = (int64_t)hd * 2;
    for (int t0 = t_begin; t0 < t_end; t0 += 64) {
        const int pos = t0 + lane;
        const int id = pos < t_end ? table[pos / FHIP_PAGE_TOKENS] : -1;
        const bool ok = pos < t_end && pg.valid(id);
        const int64_t roff = ((int64_t)(pos % FHIP_PAGE_TOKENS) * kvh + g) * row_bytes;
        const uint16_t* krow = ok ? (const uint16_t*)(pg.k_page(id) + roff) : nullptr;
        const uint16_t* vrow = ok ? (const uint16_t*)(pg.v_page(id) + roff) : nullptr;
        float s = -__builtin_inff();
        if (ok) {
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot = fmaf(qv[d], h2f(krow[d]), dot);
            s = dot * scale;
        }
        const float cmax = wave_max(s);
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = m_run == -__builtin_inff() ? 0.0f : expf(m_run - m_new);
        const float p = ok ? expf(s - m_new) : 0.0f;
        l_run = l_run * alpha + wave_sum(p);
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= alpha;
        const int n = min(64, t_end - t0);
        for (int j = 0; j < n; ++j) {
            const float pj = __shfl(p, j);
            const uint64_t vj = (uint64_t)__shfl((long long)(uintptr_t)vrow, j);
            if (vj == 0) continue;  // uniform: position j is masked
            const uint16_t* vr = (const uint16_t*)(uintptr_t)vj;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = lane + 64 * i;
                if (d < hd) acc[i] = fmaf(pj, h2f(vr[d]), acc[i]);
            }
        }
    }
    if (lane == 0) {
        part_ml[(vec * nsplit + split) * 2 + 0] = m_run;
        part_ml[(vec * nsplit + split) * 2 + 1] = l_run;
    }
    float* dst = part_acc + (vec * nsplit + split) * hd;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (lane + 64 * i < hd) dst[lane + 64 * i] = acc[i];
}

// Merge of the splits of one (query, q head) vector per workgroup:
// out = (sum_s w_s acc_s) / (sum_s w_s l_s), w_s = exp(m_s - max m); zeros when the query
// attends to no position. The split weights are computed once, in parallel, into LDS; each
// thread then sums its output dims over the splits with eight loads in flight at a time.
constexpr int kCombThreads = 128;
__global__ __launch_bounds__(kCombThreads) void paged_attn_combine_kernel(
    PQueries qs, const float* __restrict__ ml, const float* __restrict__ acc,
    uint16_t* __restrict__ out, int qh, int hd, int nsplit) {
    extern __shared__ float wts[];  // nsplit weights
    __shared__ float red[2][kCombThreads / kWave];
    const int64_t vec = blockIdx.x;
    const int qi = (int)(vec / qh);
    const int clen = qs.causal_len(qi);
    const int ns = (clen + kPSplit - 1) / kPSplit;
    const float* m = ml + vec * nsplit * 2;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    constexpr int kW = kCombThreads / kWave;
    float mx = -__builtin_inff();
    for (int s = tid; s < ns; s += kCombThreads) mx = fmaxf(mx, m[2 * s]);
    mx = wave_max(mx);
    if (lane == 0) red[0][wv] = mx;
    __syncthreads();
    float M = red[0][0];
#pragma unroll
    for (int w = 1; w < kW; ++w) M = fmaxf(M, red[0][w]);
    float ls = 0.0f;
    for (int s = tid; s < ns; s += kCombThreads) {
        const float w = M == -__builtin_inff() ? 0.0f : expf(m[2 * s] - M);
        wts[s] = w;
        ls += w * m[2 * s + 1];
    }
    ls = wave_sum(ls);
    if (lane == 0) red[1][wv] = ls;
    __syncthreads();
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) L += red[1][w];
    const float* a = acc + vec * nsplit * hd;
    for (int d = tid; d < hd; d += kCombThreads) {
        float o = 0.0f;
        int s = 0;
        for (; s + 8 <= ns; s += 8) {
            float av[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) av[j] = a[(int64_t)(s + j) * hd + d];
#pragma unroll
            for (int j = 0; j < 8; ++j) o = fmaf(wts[s + j], av[j], o);
        }
        for (; s < ns; ++s) o = fmaf(wts[s], a[(int64_t)s * hd + d], o);
        out[vec * hd + d] = (uint16_t)f2h(L > 0.0f ? o / L : 0.0f);
    }
}

// The same merge with one wave per vector, four vectors per workgroup, for launches with at
// most 8 splits per vector (contexts up to 8192 positions; causal prefill): lane s holds split
// s's (m, l) and the weights reach the dim loop by lane broadcasts, so no LDS and no barrier.
// A workgroup per vector spent most of its time being scheduled at prefill sizes.
constexpr int kCombWaveMaxSplits = 8;
__global__ __launch_bounds__(256) void paged_attn_combine_wave_kernel(
    PQueries qs, const float* __restrict__ ml, const float* __restrict__ acc,
    uint16_t* __restrict__ out, int qh, int hd, int nsplit, int64_t nvec) {
    const int lane = threadIdx.x & 63;
    const int64_t vec = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (vec >= nvec) return;
    const int clen = qs.causal_len((int)(vec / qh));
    const int ns = (clen + kPSplit - 1) / kPSplit;  // <= nsplit <= kCombWaveMaxSplits
    const float* m = ml + vec * nsplit * 2;
    const float ms = lane < ns ? m[2 * lane] : -__builtin_inff();
    const float ls = lane < ns ? m[2 * lane + 1] : 0.0f;
    const float M = wave_max(ms);
    const float w = lane < ns && M != -__builtin_inff() ? expf(ms - M) : 0.0f;
    const float L = wave_sum(w * ls);
    float ws[kCombWaveMaxSplits];
#pragma unroll
    for (int j = 0; j < kCombWaveMaxSplits; ++j) ws[j] = __shfl(w, j);
    const float* a = acc + vec * nsplit * hd;
    for (int d = lane; d < hd; d += 64) {
        float av[kCombWaveMaxSplits];
#pragma unroll
        for (int j = 0; j < kCombWaveMaxSplits; ++j) av[j] = j < ns ? a[(int64_t)j * hd + d] : 0.0f;
        float o = 0.0f;
#pragma unroll
        for (int j = 0; j < kCombWaveMaxSplits; ++j) o = fmaf(ws[j], av[j], o);
        out[vec * hd + d] = (uint16_t)f2h(L > 0.0f ? o / L : 0.0f);
    }
}

size_t paged_ws_layout(int nq, int qh, int hd, int max_tokens, size_t* off_acc, int* nsplit) {
    const int ns = max_tokens > 0 ? (max_tokens + kPSplit - 1) / kPSplit : 1;
    const size_t ml = (size_t)nq * qh * ns * 2 * sizeof(float);
    const size_t acc = (size_t)nq * qh * ns * hd * sizeof(float);
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    if (off_acc) *off_acc = al(ml);
    if (nsplit) *nsplit = ns;
    return al(ml) + al(acc);
}

// head_dim 32 / 64 / 128 / 256 run the MFMA kernels, any other width up to 256 the generic one
bool paged_shape_ok(int qh, int kvh, int hd) {
    return kvh > 0 && qh > 0 && qh % kvh == 0 && hd >= 1 && hd <= 256;
}

template <int HD, int NH, class Pages>
void launch_split_t(const uint16_t* q, const PQueries& qs, const Pages& pg, int qh, int kvh,
                    int nhb, float* ml, float* acc, int nsplit, int tok, int64_t groups,
                    hipStream_t s) {
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);
    hipLaunchKernelGGL((paged_attn_split_kernel<HD, NH, Pages>), dim3((unsigned)groups),
                       dim3(64 * kPWaves), 0, s, q, qs, pg, qh, kvh, nhb, scale_log2, ml, acc,
                       nsplit, tok);
}

template <int HD, class Pages>
void launch_split_hd(const uint16_t* q, const PQueries& qs, const Pages& pg, int qh, int kvh,
                     int nhb, float* ml, float* acc, int nsplit, int tok, int64_t groups,
                     hipStream_t s) {
    if constexpr (HD <= 128) {
        if (tok > 1) {
            // one workgroup per (kPfWaves query groups, kv head, split)
            const int64_t sets = ceil_div(ceil_div((int64_t)qs.count, tok), kPfWaves);
            const int64_t wgs = sets * kvh * nsplit;
            const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);
            hipLaunchKernelGGL((paged_attn_prefill_mfma_kernel<HD, Pages>), dim3((unsigned)wgs),
                               dim3(64 * kPfWaves), 0, s, q, qs, pg, qh, kvh, scale_log2, ml, acc,
                               nsplit, tok);
            return;
        }
    }
    if (qh / kvh * tok <= 4)
        launch_split_t<HD, 4>(q, qs, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
    else
        launch_split_t<HD, 8>(q, qs, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
}

template <class Pages>
int launch_paged(void* out, const void* q, const PQueries& qs, int nq, const Pages& pg, int qh,
                 int kvh, int hd, void* ws, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    size_t off_acc;
    int nsplit;
    paged_ws_layout(nq, qh, hd, qs.max_blocks * FHIP_PAGE_TOKENS, &off_acc, &nsplit);
    float* ml = (float*)ws;
    float* acc = (float*)((char*)ws + off_acc);
    const int G = qh / kvh;
    const int nhb = (G + kHeadsMax - 1) / kHeadsMax;
    // causal prefill over one shared table: 16 / G consecutive queries per wave on the MFMA
    // prefill kernel (head_dim <= 128, G <= 8), else 8 / G (G < 8)
    const bool prefill = !qs.seq_lens && qs.table_stride == 0 && nq > 1;
    const int tok = !prefill                          ? 1
                    : (hd <= 128 && G <= kHeadsMax)   ? 2 * kHeadsMax / G
                    : G < kHeadsMax                   ? kHeadsMax / G
                                                      : 1;
    const int64_t items = ceil_div((int64_t)nq, tok) * kvh * nhb * nsplit;
    const int64_t groups = ceil_div(items, kPWaves);
    if (groups > 0x7fffffff || (int64_t)nq * qh > 0x7fffffff) return hipErrorInvalidValue;
    PQueries q2 = qs;
    q2.count = nq;
    const uint16_t* qp = (const uint16_t*)q;
    if (hd != 32 && hd != 64 && hd != 128 && hd != 256) {
        const int64_t gitems = (int64_t)nq * qh * nsplit;
        const int64_t gwgs = ceil_div(gitems, kGenWaves);
        if (gwgs > 0x7fffffff) return hipErrorInvalidValue;
        hipLaunchKernelGGL((paged_attn_generic_kernel<Pages>), dim3((unsigned)gwgs),
                           dim3(64 * kGenWaves), 0, s, qp, q2, pg, qh, kvh, hd,
                           1.0f / sqrtf((float)hd), ml, acc, nsplit, gitems);
    } else {
    switch (hd) {
        case 32:
            launch_split_hd<32>(qp, q2, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
            break;
        case 64:
            launch_split_hd<64>(qp, q2, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
            break;
        case 128:
            launch_split_hd<128>(qp, q2, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
            break;
        default:
            launch_split_hd<256>(qp, q2, pg, qh, kvh, nhb, ml, acc, nsplit, tok, groups, s);
            break;
    }
    }
    const int64_t nvec = (int64_t)nq * qh;
    if (nsplit <= kCombWaveMaxSplits)
        hipLaunchKernelGGL(paged_attn_combine_wave_kernel, dim3((unsigned)ceil_div(nvec, 4)),
                           dim3(256), 0, s, q2, ml, acc, (uint16_t*)out, qh, hd, nsplit, nvec);
    else
        hipLaunchKernelGGL(paged_attn_combine_kernel, dim3((unsigned)nvec), dim3(kCombThreads),
                           (size_t)nsplit * sizeof(float), s, q2, ml, acc, (uint16_t*)out, qh,
                           hd, nsplit);
    return hipGetLastError();
}

}  // namespace

extern "C" {

size_t fhip_attention_paged_workspace_bytes(int batch, int num_q_heads, int head_dim,
                                            int max_blocks) {
    if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_blocks <= 0) return 0;
    return paged_ws_layout(batch, num_q_heads, head_dim, max_blocks * FHIP_PAGE_TOKENS, nullptr,
                           nullptr);
}

int fhip_launch_attention_paged_decode(void* output, const void* q, const int32_t* block_table,
                                       const int32_t* seq_lens, int batch, int max_blocks,
                                       int num_pages, const void* k_pool, const void* v_pool,
                                       int64_t page_k_bytes, int64_t page_v_bytes,
                                       int num_q_heads, int num_kv_heads, int head_dim,
                                       void* workspace, fhip_stream_t stream) {
    if (batch < 0 || max_blocks <= 0 || num_pages < 0 || page_k_bytes < 0 || page_v_bytes < 0 ||
        !paged_shape_ok(num_q_heads, num_kv_heads, head_dim) ||
        (int64_t)max_blocks * FHIP_PAGE_TOKENS > kMaxTokens)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (!output || !q || !block_table || !seq_lens || !k_pool || !v_pool || !workspace)
        return hipErrorInvalidValue;
    const PQueries qs{block_table, max_blocks, max_blocks, seq_lens, 0, 0, batch};
    const F16PoolPages pg{(const uint8_t*)k_pool, (const uint8_t*)v_pool, page_k_bytes,
                          page_v_bytes, num_pages};
    return launch_paged(output, q, qs, batch, pg, num_q_heads, num_kv_heads, head_dim, workspace,
                        fhip_host::as_stream(stream));
}

// The reference interface: one sequence, num_tokens queries at positions
// start_pos .. start_pos + num_tokens - 1, per-block pointer arrays indexed by the physical
// block ids of block_table[0 .. num_blocks_in_seq). `ws` holds the split partials
// (fhip_attention_paged_workspace_bytes(num_tokens, qh, hd, num_blocks_in_seq) bytes); null
// asks for a stream-ordered allocation freed on the same stream.
static int paged_attention_ref(void* output, const void* q, const int* block_table,
                               const void** k_block_ptrs, const void** v_block_ptrs,
                               int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                               int kv_len, int start_pos, int num_blocks_in_seq, void* ws,
                               size_t ws_bytes, hipStream_t s) {
    if (num_tokens < 0 || kv_len < 0 || start_pos < 0 || num_blocks_in_seq < 0 ||
        !paged_shape_ok(num_q_heads, num_kv_heads, head_dim) ||
        (int64_t)num_blocks_in_seq * FHIP_PAGE_TOKENS > kMaxTokens)
        return hipErrorInvalidValue;
    if (num_tokens == 0) return hipSuccess;
    if (!output || !q) return hipErrorInvalidValue;
    if (num_blocks_in_seq > 0 && (!block_table || !k_block_ptrs || !v_block_ptrs))
        return hipErrorInvalidValue;
    const int mb = num_blocks_in_seq > 0 ? num_blocks_in_seq : 1;
    // with no blocks every query attends to nothing: the table is never read
    const PQueries qs{(const int32_t*)block_table, 0, num_blocks_in_seq, nullptr, kv_len,
                      start_pos, num_tokens};
    const size_t bytes = paged_ws_layout(num_tokens, num_q_heads, head_dim,
                                         mb * FHIP_PAGE_TOKENS, nullptr, nullptr);
    const bool own = ws == nullptr;
    if (!own && ws_bytes < bytes) return hipErrorInvalidValue;
    if (own) {
        hipError_t e = hipMallocAsync(&ws, bytes, s);
        if (e != hipSuccess) return e;
    }
    const F16PtrPages pg{(const uint8_t* const*)k_block_ptrs, (const uint8_t* const*)v_block_ptrs,
                         0x7fffffff};
    int r = launch_paged(output, q, qs, num_tokens, pg, num_q_heads, num_kv_heads, head_dim, ws,
                         s);
    if (own) {
        hipError_t e2 = hipFreeAsync(ws, s);
        if (r == hipSuccess) r = e2;
    }
    return r;
}

int fhip_launch_paged_attention(void* output, const void* q, const int* block_table,
                                const void** k_block_ptrs, const void** v_block_ptrs,
                                int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                                int kv_len, int start_pos, int num_blocks_in_seq,
                                fhip_stream_t stream) {
    return paged_attention_ref(output, q, block_table, k_block_ptrs, v_block_ptrs, num_tokens,
                               num_q_heads, num_kv_heads, head_dim, kv_len, start_pos,
                               num_blocks_in_seq, nullptr, 0, fhip_host::as_stream(stream));
}

int fhip_launch_paged_attention_ws(void* output, const void* q, const int* block_table,
                                   const void** k_block_ptrs, const void** v_block_ptrs,
                                   int num_tokens, int num_q_heads, int num_kv_heads,
                                   int head_dim, int kv_len, int start_pos,
                                   int num_blocks_in_seq, void* workspace,
                                   size_t workspace_bytes, fhip_stream_t stream) {
    if (!workspace) return hipErrorInvalidValue;
    return paged_attention_ref(output, q, block_table, k_block_ptrs, v_block_ptrs, num_tokens,
                               num_q_heads, num_kv_heads, head_dim, kv_len, start_pos,
                               num_blocks_in_seq, workspace, workspace_bytes,
                               fhip_host::as_stream(stream));
}

// ffi.rs:172-184 `launch_attention`, attention over a contiguous KV cache: not supported. The
// engine's KV caches are paged (engine.rs:671-680 dispatches through the cache manager to the
// paged forms above), so this backend builds only those; the symbol exists so that a binding of
// the whole ffi.rs block links, and it launches nothing.
int fhip_launch_attention(void* output, const void* q, const void* k_cache, const void* v_cache,
                          int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                          int kv_len, int start_pos, fhip_stream_t stream) {
    (void)output, (void)q, (void)k_cache, (void)v_cache, (void)num_tokens, (void)num_q_heads;
    (void)num_kv_heads, (void)head_dim, (void)kv_len, (void)start_pos, (void)stream;
    return hipErrorNotSupported;
}

}  // extern "C"

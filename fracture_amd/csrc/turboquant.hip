// TurboQuant KV compression for gfx950: rotate (MFMA), L2 norm, Lloyd-Max quantize,
// MSB-first bit-pack, page scatter, and dequantize (MFMA).
//
// Rotation cost. Compress and dequantize each multiply every 128-wide vector by a dense
// 128x128 fp32 rotation, 2*128*128 flops per vector: 17.2 GFLOP per direction for one layer
// of K+V at 32768 tokens x 8 heads, against ~160-170 MB of HBM traffic (~21 us). On the VALU
// that is >100 us, so the rotation runs on MFMA (v_mfma_f32_32x32x16_f16) with fp32 accuracy
// recovered by splitting the fp32 operand into fp16 hi + 2^12-scaled fp16 lo parts:
//   compress:   y_raw = Pi x = 2^-12 (Pi_hi' x + Pi_lo' x)      Pi_hi' = 2^12 Pi_hi (exact),
//               both products in one fp32 accumulator; x is the raw fp16 input, exact as
//               an fp16 operand; the norm is applied after the product by linearity:
//               y = y_raw / (||x|| + 1e-8).
//   dequantize: x_hat = Pi^T yhat = Pi_hi^T c_hi + 2^-12 (Pi_lo'^T c_hi + Pi_hi^T c_lo')
// In compress each representation error is ~2^-22 relative, the level of the fp32 sums
// themselves. The dequantize runs its two correction products on fp8 MFMA (see there): ~2^-15
// of each term, under the fp16 output's own rounding.
//
// Work mapping (head_dim 128, 2/3/4/8 bits): one workgroup of 8 (compress) or 12
// (dequantize) waves per CU holds the rotation's hi/lo MFMA fragments in LDS (64 KB, staged
// once). Every wave then owns whole
// tiles of 32 vectors: it loads its tile's input straight into MFMA operand registers
// (prefetching the next tile while it computes), runs 4 blocks of 32 output coordinates x
// 8 K-steps of MFMA against the LDS fragments, and quantizes / packs / stores its own
// results. Waves never wait for one another after the staging barrier, and each keeps one
// tile of loads in flight, which is what hides HBM latency. The two lanes that hold the two
// halves of a 16-byte group exchange them with v_permlane32_swap.
// Other head dims and bit widths use a per-vector VALU path that follows the reference
// kernel's arithmetic.
#include <type_traits>

#include "fhip_internal.h"
#include "tq_quant.h"

using namespace fhip;

namespace {

constexpr int kTile = 32;        // vectors per MFMA tile
constexpr int kHd = 128;         // head_dim of the MFMA path
constexpr int kWavesC = 8;       // waves per workgroup of the MFMA compress (one group per CU)
constexpr int kWavesD = 12;      // waves per workgroup of the MFMA dequantize
constexpr float kLoScale = 4096.0f;
constexpr float kLoInv = 1.0f / 4096.0f;

// ---------------------------------------------------------------------------------------
// Destinations of the packed rows / norms: flat [rows, pd] + [rows], or 16-token pages.
// ---------------------------------------------------------------------------------------
struct FlatDst {
    uint8_t* packed;
    uint16_t* norms;
    int64_t pd;
    __device__ uint8_t* prow(int64_t m) const { return packed + m * pd; }
    __device__ uint16_t* nptr(int64_t m) const { return norms + m; }
};

// Token t = m / kvh, head m % kvh; logical position first_pos + t lives in page
// page_ids[pos / 16], slot pos % 16, with the page layout of
// quantized_paged_kv_cache.rs:86-128. Rows whose page id is outside [0, num_pages) are not
// written.
struct PageDst {
    uint8_t* pool;
    uint8_t* npool;
    int64_t page_bytes, page_norm_bytes;
    const int32_t* page_ids;
    int64_t first_pos;
    int kvh, num_pages;
    int64_t pd;
    __device__ bool slot(int64_t m, int64_t& page, int64_t& off) const {
        const int64_t t = m / kvh;
        const int64_t hh = m - t * kvh;
        const int64_t pos = first_pos + t;
        page = page_ids[pos / FHIP_PAGE_TOKENS];
        off = (pos % FHIP_PAGE_TOKENS) * kvh + hh;
        return page >= 0 && page < num_pages;
    }
    __device__ uint8_t* prow(int64_t m) const {
        int64_t page, off;
        if (!slot(m, page, off)) return nullptr;
        return pool + page * page_bytes + off * pd;
    }
    __device__ uint16_t* nptr(int64_t m) const {
        int64_t page, off;
        if (!slot(m, page, off)) return nullptr;
        return (uint16_t*)(npool + page * page_norm_bytes) + off;
    }
};

// The same page layout with one allocation per page, as QuantizedKvCacheManager allocates
// them (quantized_paged_kv_cache.rs:82-133): packed_pages[p] / norm_pages[p] are the device
// addresses of page p's packed rows and norms.
struct PtrPageDst {
    uint8_t* const* packed_pages;
    uint8_t* const* norm_pages;
    const int32_t* page_ids;
    int64_t first_pos;
    int kvh, num_pages;
    int64_t pd;
    __device__ bool slot(int64_t m, int64_t& page, int64_t& off) const {
        const int64_t t = m / kvh;
        const int64_t hh = m - t * kvh;
        const int64_t pos = first_pos + t;
        page = page_ids[pos / FHIP_PAGE_TOKENS];
        off = (pos % FHIP_PAGE_TOKENS) * kvh + hh;
        return page >= 0 && page < num_pages;
    }
    __device__ uint8_t* prow(int64_t m) const {
        int64_t page, off;
        if (!slot(m, page, off)) return nullptr;
        return packed_pages[page] + off * pd;
    }
    __device__ uint16_t* nptr(int64_t m) const {
        int64_t page, off;
        if (!slot(m, page, off)) return nullptr;
        return (uint16_t*)norm_pages[page] + off;
    }
};

// The wave's index in its workgroup, as a wave-uniform (scalar) value: the compiler cannot
// tell that threadIdx.x >> 6 is uniform, and would turn tile loops into divergent ones.
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------------------
// Rotation fragments in LDS. MFMA step s of a 32-coordinate block takes K = 16 coordinates;
// lane half h holds 8 of them (element e):
//   compress   (y = Pi x):      A[i][k] = Pi[32c + i][k], coordinate 16s + 8h + e. The two
//              lanes of an input row load adjacent 16-byte pieces of it in each step, so a
//              load instruction touches 32 cache lines, not 64 (the L1's per-line work was
//              what slowed the tiles while loads were in flight: 50.4 -> 46.4 us for a
//              layer's K+V);
//   back-rotation of fp32 rows (x = Pi^T y):  A[i][k] = Pi[k][32c + i], coordinate
//              64h + 8s + e (one contiguous half of the row per lane).
// frag[c][s][0|1][lane] = 8 fp16 of the hi / lo' part, lane = (i = lane & 31, h = lane >> 5).
// ---------------------------------------------------------------------------------------
struct RotLds {
    u32x4 frag[4][8][2][64];  // 64 KB
};

// Staging in two steps so the rotation's loads overlap the rest of a workgroup's set-up:
// load() issues this thread's reads of Pi into registers, store() converts them to the hi / lo'
// fragments and writes LDS. kThreads is the block size.
template <bool kTranspose, int kThreads, bool kHiScaled>
struct RotStage {
    static constexpr int kFrags = 4 * 8 * 64;
    static constexpr int kN = (kFrags + kThreads - 1) / kThreads;
    float v[kN][8];
    __device__ __forceinline__ void load(const float* __restrict__ rot) {
#pragma unroll
        for (int n = 0; n < kN; ++n) {
            const int idx = (int)threadIdx.x + n * kThreads;
            if (kFrags % kThreads != 0 && idx >= kFrags) break;
            const int lane = idx & 63, s = (idx >> 6) & 7, c = idx >> 9;
            const int row = 32 * c + (lane & 31);
            const int k0 = kTranspose ? 64 * (lane >> 5) + 8 * s : 16 * s + 8 * (lane >> 5);
            if constexpr (kTranspose) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[n][e] = rot[(k0 + e) * kHd + row];
            } else {
                const f32x4 a = *(const f32x4*)&rot[row * kHd + k0];
                const f32x4 b = *(const f32x4*)&rot[row * kHd + k0 + 4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[n][e] = a[e];
                    v[n][4 + e] = b[e];
                }
            }
        }
    }
    __device__ __forceinline__ void store(RotLds& L) const {
#pragma unroll
        for (int n = 0; n < kN; ++n) {
            const int idx = (int)threadIdx.x + n * kThreads;
            if (kFrags % kThreads != 0 && idx >= kFrags) break;
            const int lane = idx & 63, s = (idx >> 6) & 7, c = idx >> 9;
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
                uint32_t hb[2], lb[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float x = v[n][2 * e2 + t];
                    const _Float16 hi = (_Float16)x;
                    // x 2^12 is exact for an fp16 value of magnitude <= 1
                    hb[t] = __builtin_bit_cast(
                        uint16_t, kHiScaled ? (_Float16)((float)hi * kLoScale) : hi);
                    lb[t] = __builtin_bit_cast(uint16_t, (_Float16)((x - (float)hi) * kLoScale));
                }
                hw[e2] = hb[0] | (hb[1] << 16);
                lw[e2] = lb[0] | (lb[1] << 16);
            }
            L.frag[c][s][0][lane] = u32x4{hw[0], hw[1], hw[2], hw[3]};
            L.frag[c][s][1][lane] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        }
    }
};

__device__ __forceinline__ f16x8 frag(const RotLds& L, int c, int s, int hl, int lane) {
    return __builtin_bit_cast(f16x8, L.frag[c][s][hl][lane]);
}

// Lanes l and l^32: after swap_halves(v, w), lanes 0-31 hold (own v, partner's v) and lanes
// 32-63 hold (partner's w, own w) in (v, w) (v_permlane32_swap).
__device__ __forceinline__ void swap_halves(uint32_t& v, uint32_t& w) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, w, false, false);
    v = r[0];
    w = r[1];
}
__device__ __forceinline__ float partner_f(float x) {
    uint32_t v = __float_as_uint(x), w = v;
    swap_halves(v, w);  // lanes < 32: partner in w; lanes >= 32: partner in v
    return __uint_as_float((threadIdx.x & 32) ? v : w);
}

// Sum of squares of 8 fp16 values with fp32 accumulation (products of fp16 are exact).
__device__ __forceinline__ float sumsq8(const f16x8& b, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f16x2 p = {b[2 * e], b[2 * e + 1]};
        acc = __builtin_amdgcn_fdot2(p, p, acc, false);
    }
    return acc;
}

// Store n (2..64) bytes at dst, using the widest aligned stores the address allows.
template <int n>
__device__ __forceinline__ void store_bytes(uint8_t* dst, const uint32_t (&w)[16]) {
    const uintptr_t a = (uintptr_t)dst;
    if constexpr (n % 16 == 0) {
        if ((a & 15u) == 0) {
#pragma unroll
            for (int i = 0; i < n / 16; ++i)
                *(u32x4*)(dst + 16 * i) = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
            return;
        }
    }
    if constexpr (n % 8 == 0) {
        if ((a & 7u) == 0) {
#pragma unroll
            for (int i = 0; i < n / 8; ++i) *(u32x2*)(dst + 8 * i) = u32x2{w[2 * i], w[2 * i + 1]};
            return;
        }
    }
    if ((a & 3u) == 0) {
#pragma unroll
        for (int i = 0; i < n / 4; ++i) *(uint32_t*)(dst + 4 * i) = w[i];
        return;
    }
#pragma unroll
    for (int i = 0; i < n; ++i) dst[i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
}

// One lane's half of a 32 x 128 fp16 input tile: row r = lane & 31, coordinates
// 16s + 8h + 0..7 as MFMA B fragment s (s = 0..7). Rows past the end (or a tile past the last) read
// row 0 instead: their MFMA columns and results are discarded, and unconditional loads
// never make the compiler wait for a register's earlier loads before reusing it.
__device__ __forceinline__ const uint16_t* x_half_src(const uint16_t* __restrict__ in,
                                                     int64_t tile, int64_t ntiles,
                                                     int64_t rows) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int64_t m0 = tile * kTile;
    const bool ok = tile < ntiles && r < rows - m0;
    return in + (ok ? m0 * kHd + r * kHd : 0) + 8 * h;
}
__device__ __forceinline__ void load_x_half(const uint16_t* __restrict__ in, int64_t tile,
                                            int64_t ntiles, int64_t rows, f16x8 (&x)[8]) {
    const uint16_t* src = x_half_src(in, tile, ntiles, rows);
#pragma unroll
    for (int s = 0; s < 8; ++s) x[s] = __builtin_bit_cast(f16x8, ld16(src + 16 * s));
}

// ---------------------------------------------------------------------------------------
// MFMA compress / rotate of one tile by one wave (head_dim 128).
//   kMode 0: quantize + pack to Dst (kBits 2, 3, 4, 8);  kMode 1: fp32 y (and norms);
//   kMode 2: the raw fp32 product Pi x (no normalisation, no norms).
// Lane (r, h) ends block c holding coordinates 32c + 8g + 4h + e (g, e = 0..3) of vector r
// (accumulator element 4g + e); it quantizes them into half-groups (4 codes, 4*kBits bits,
// MSB first). After the 4 blocks lane h owns groups [8h, 8h+8) of row r: 8*kBits contiguous
// bytes at byte 8*kBits*h.
//
// The 32 MFMA steps (block c = q / 8, K-step s = q % 8) are software-pipelined, one
// scheduling region per step:
//   * the rotation fragments of step q + kAhead are read from LDS during step q;
//   * block c's MFMAs accumulate into set c % 2 while block c - 1 (the other set) is
//     quantized two values per step: in step s the bucket-table reads of values 2s, 2s + 1
//     are issued and the codes of values 2s - 2, 2s - 1 (read one step earlier) finish.
// ---------------------------------------------------------------------------------------
template <int kMode, int kBits, bool kUnitFast>
struct TileQuant {
    const Quantizer& qz;
    float scale, offset, jmax;  // the bucket map, held in registers
    float inv_s;
    float y[16];
    float2 ent[16];
    uint32_t hw[4];
    uint32_t (&half)[16];
    float* __restrict__ y_out;
    int64_t yrow;  // element offset of this lane's row in y_out, or -1 (kMode 1)

    // Phase A of value v (accumulator element v of block c): scale, and for the fast
    // quantizer issue the bucket-table read.
    __device__ __forceinline__ void a(const f32x16& acc, int c, int v) {
        y[v] = acc[v] * inv_s;
        if constexpr (kMode >= 1) {
            if ((v & 3) == 3 && yrow >= 0)
                *(f32x4*)&y_out[yrow + 32 * c + 8 * (v >> 2) + 4 * (threadIdx.x >> 5 & 1)] =
                    f32x4{y[v - 3], y[v - 2], y[v - 1], y[v]};
        } else if constexpr (kUnitFast) {
            // the quantizer's bucket map (bucket_of), with its table size known here: at most
            // 7 bits the table has at most 256 buckets; at 8 bits jmax tells which map it is
            const float jf = fmaf(y[v], scale, offset);
            int j;
            if constexpr (kBits <= 7)
                j = bucket_u8(jf);
            else
                j = jmax <= (float)(kBucketsU8 - 1) ? bucket_u8(jf) : bucket_wide(jf, jmax);
            ent[v] = qz.ent[j];
        }
    }
    // Phase B of value v: the code, packed MSB first into the half-group of group v / 4.
    __device__ __forceinline__ void b(int c, int v) {
        if constexpr (kMode == 0) {
            int code;
            if constexpr (kUnitFast)
                code = __float_as_int(ent[v].y) + (y[v] > ent[v].x ? 1 : 0);
            else
                code = quantize(qz, y[v]);
            const int g = v >> 2;
            hw[g] = ((v & 3) == 0 ? 0u : hw[g] << kBits) | (uint32_t)code;
            if ((v & 3) == 3) half[4 * c + g] = hw[g];
        }
    }
};

// pf / pf_src: the wave's prefetch of a later tile, issued one 16-byte load every fourth
// step so that a wave never stalls at issue behind a full memory queue before computing.
template <int kMode, int kBits, bool kUnitFast, class Dst>
__device__ __forceinline__ void compress_tile(const Quantizer& qz, const RotLds& L,
                                              const f16x8 (&x)[8], const Dst& dst,
                                              float* __restrict__ y_out, int64_t m0, int nvalid,
                                              f16x8 (&pf)[8], const uint16_t* pf_src) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    float ssq = 0.0f;  // this lane's half of vector r
#pragma unroll
    for (int s = 0; s < 8; ++s) ssq = sumsq8(x[s], ssq);
    const float nrm = sqrtf(ssq + partner_f(ssq));
    const float inv = 1.0f / (nrm + 1e-8f);
    const bool row_ok = r < nvalid;
    if (kMode != 2 && h == 0 && row_ok) {
        uint16_t* np = dst.nptr(m0 + r);
        if (np) *np = (uint16_t)f2h(nrm);
    }
    uint32_t half[16];  // kMode 0: half-group of group 4c + g held by this lane
    // Both fragment parts carry the factor 2^12 (hi stored as 2^12 Pi_hi), so hi and lo
    // products accumulate into one fp32 sum, 2^12 y_raw, scaled out with the norm.
    TileQuant<kMode, kBits, kUnitFast> tq{qz, qz.scale, qz.offset, qz.jmax,
                                          kMode == 2 ? kLoInv : inv * kLoInv,
                                          {}, {}, {}, half, y_out,
                                          row_ok ? (m0 + r) * kHd : -1};
    constexpr int kAhead = 2;
    constexpr int kRing = kAhead + 1;
    f16x8 fh[kRing], fl[kRing];
#pragma unroll
    for (int q = 0; q < kAhead; ++q) {
        fh[q] = frag(L, q >> 3, q & 7, 0, lane);
        fl[q] = frag(L, q >> 3, q & 7, 1, lane);
    }
    f32x16 acc[2];
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const int c = q >> 3, s = q & 7, b = c & 1;
        __builtin_amdgcn_sched_barrier(0);
        if ((q & 3) == 0) pf[q >> 2] = __builtin_bit_cast(f16x8, ld16(pf_src + 16 * (q >> 2)));
        if (q + kAhead < 32) {
            const int n = q + kAhead;
            fh[n % kRing] = frag(L, n >> 3, n & 7, 0, lane);
            fl[n % kRing] = frag(L, n >> 3, n & 7, 1, lane);
        }
        if (s == 0) acc[b] = f32x16{};
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[q % kRing], x[s], acc[b], 0, 0, 0);
        if (c > 0) {
            tq.a(acc[b ^ 1], c - 1, 2 * s);
            tq.a(acc[b ^ 1], c - 1, 2 * s + 1);
        }
        // the last two values of block c - 2 were looked up in block c - 1's final step
        if (c > 1 && s == 0) {
            tq.b(c - 2, 14);
            tq.b(c - 2, 15);
        }
        if (c > 0 && s > 0) {
            tq.b(c - 1, 2 * s - 2);
            tq.b(c - 1, 2 * s - 1);
        }
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fl[q % kRing], x[s], acc[b], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    tq.b(2, 14);
    tq.b(2, 15);
#pragma unroll
    for (int v = 0; v < 16; ++v) tq.a(acc[1], 3, v);
#pragma unroll
    for (int v = 0; v < 16; ++v) tq.b(3, v);
    if constexpr (kMode == 0) {
        // Group j (< 8) and group j + 8: lane h = 0 gets both halves of group j, lane h = 1
        // both halves of group j + 8, as (first half, second half) in (half[j], half[j+8]).
        uint32_t w[16] = {}, G[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v = half[j], u = half[j + 8];
            swap_halves(v, u);
            if constexpr (kBits == 4) {
                // the group's 4 bytes are v's two then u's two, most significant first
                w[j] = __builtin_amdgcn_perm(v, u, 0x00010405u);
            } else if constexpr (kBits == 8) {
                w[2 * j] = __builtin_amdgcn_perm(v, v, 0x00010203u);
                w[2 * j + 1] = __builtin_amdgcn_perm(u, u, 0x00010203u);
            } else {
                G[j] = (v << (4 * kBits)) | u;  // 8*kBits bits, MSB first
            }
        }
        if constexpr (kBits == 2 || kBits == 3) {
            // output dword m holds bytes 4m..4m+3 of the stream of groups, each group j's
            // kBits bytes most significant first: at most two groups per dword, one v_perm
#pragma unroll
            for (int m = 0; m < 2 * kBits; ++m) {
                const int j0 = 4 * m / kBits, j1 = min(j0 + 1, 7);
                uint32_t sel = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int b = 4 * m + i, j = b / kBits, k = b % kBits;
                    sel |= (uint32_t)((j == j0 ? 4 : 0) + (kBits - 1 - k)) << (8 * i);
                }
                w[m] = __builtin_amdgcn_perm(G[j0], G[j1], sel);
            }
        }
        if (row_ok) {
            uint8_t* prow = dst.prow(m0 + r);
            if (prow) store_bytes<8 * kBits>(prow + 8 * kBits * h, w);
        }
    }
}

// xa and xb hold the wave's first two tiles (loads issued before the workgroup's set-up).
template <int kMode, int kBits, bool kUnitFast, class Dst>
__device__ __forceinline__ void compress_waves(const Quantizer& qz, const RotLds& L,
                                               const uint16_t* __restrict__ in, const Dst& dst,
                                               float* __restrict__ y_out, int64_t rows,
                                               f16x8 (&xa)[8], f16x8 (&xb)[8], int64_t blk,
                                               int64_t nblk) {
    const int64_t ntiles = ceil_div(rows, kTile);
    const int64_t stride = nblk * kWavesC;
    int64_t tile = blk * kWavesC + wave_id();
    f16x8 xc[8];
    // Three register buffers in rotation, one tile per step: while a tile computes, the
    // loads of the next two are in flight.
    while (tile < ntiles) {
        compress_tile<kMode, kBits, kUnitFast>(qz, L, xa, dst, y_out, tile * kTile,
                                               (int)min<int64_t>(kTile, rows - tile * kTile), xc,
                                               x_half_src(in, tile + 2 * stride, ntiles, rows));
        tile += stride;
        if (tile >= ntiles) break;
        compress_tile<kMode, kBits, kUnitFast>(qz, L, xb, dst, y_out, tile * kTile,
                                               (int)min<int64_t>(kTile, rows - tile * kTile), xa,
                                               x_half_src(in, tile + 2 * stride, ntiles, rows));
        tile += stride;
        if (tile >= ntiles) break;
        compress_tile<kMode, kBits, kUnitFast>(qz, L, xc, dst, y_out, tile * kTile,
                                               (int)min<int64_t>(kTile, rows - tile * kTile), xb,
                                               x_half_src(in, tile + 2 * stride, ntiles, rows));
        tile += stride;
    }
}

// The general-quantizer tile loop (codebooks the fast bucket map cannot serve exactly), kept
// out of line so that its register needs do not constrain the fast path's allocation.
// It reloads the wave's first tiles, and takes the destination by value: a reference would
// move the kernel argument into private memory for the fast path too.
template <int kMode, int kBits, class Dst>
__device__ __noinline__ void compress_waves_general(const Quantizer& qz, const RotLds& L,
                                                    const uint16_t* __restrict__ in, Dst dst,
                                                    float* __restrict__ y_out, int64_t rows,
                                                    int64_t blk, int64_t nblk) {
    const int64_t first = blk * kWavesC + wave_id();
    const int64_t ntiles = ceil_div(rows, kTile);
    f16x8 xa[8], xb[8];
    load_x_half(in, first, ntiles, rows, xa);
    load_x_half(in, first + nblk * kWavesC, ntiles, rows, xb);
    compress_waves<kMode, kBits, false>(qz, L, in, dst, y_out, rows, xa, xb, blk, nblk);
}

// Copy of kBytes (a multiple of 16) from global memory into LDS by the whole block, in two
// steps so that other loads can be issued between them: load() puts every thread's chunks in
// flight, store() writes them to LDS.
template <int kThreads, int kBytes>
struct LdsCopy {
    static_assert(kBytes % 16 == 0, "16-byte chunks");
    static constexpr int kN = kBytes / 16, kPer = (kN + kThreads - 1) / kThreads;
    u32x4 v[kPer];
    __device__ __forceinline__ void load(const void* __restrict__ src) {
        const u32x4* s = (const u32x4*)src;
#pragma unroll
        for (int k = 0; k < kPer; ++k) v[k] = ld16(s + min((int)threadIdx.x + k * kThreads, kN - 1));
    }
    // Threads past the end rewrite the last chunk with its own value: no branch, which would
    // let the compiler sink the load into it and wait there for every older load.
    __device__ __forceinline__ void store(void* __restrict__ dst) const {
        u32x4* d = (u32x4*)dst;
#pragma unroll
        for (int k = 0; k < kPer; ++k) d[min((int)threadIdx.x + k * kThreads, kN - 1)] = v[k];
    }
};

struct TqPlanDev;
__device__ __forceinline__ const Quantizer& plan_quantizer(const TqPlanDev* p);
__device__ __forceinline__ const RotLds& plan_compress_frags(const TqPlanDev* p);

// The planned compress of one tensor by workgroup blk of nblk: the quantizer and the rotation
// fragments come ready-made from the plan (built once per rotation and codebook by
// tq_plan_kernel) and are only copied into LDS.
template <int kMode, int kBits, class Dst>
__device__ __forceinline__ void compress_planned(Quantizer& qz, RotLds& rl,
                                                 const uint16_t* __restrict__ in,
                                                 const TqPlanDev* __restrict__ plan,
                                                 const Dst& dst, float* __restrict__ y_out,
                                                 int64_t rows, int64_t blk, int64_t nblk) {
    // the plan's loads, then the first tile's (in flight through the copy's stores)
    const int64_t first = blk * kWavesC + wave_id();
    const int64_t ntiles = ceil_div(rows, kTile);
    LdsCopy<64 * kWavesC, (int)sizeof(Quantizer)> qc;
    LdsCopy<64 * kWavesC, (int)sizeof(RotLds)> rc;
    if constexpr (kMode == 0) qc.load(&plan_quantizer(plan));
    rc.load(&plan_compress_frags(plan));
    __builtin_amdgcn_sched_barrier(0);
    f16x8 xa[8], xb[8];
    load_x_half(in, first, ntiles, rows, xa);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kMode == 0) qc.store(&qz);
    rc.store(&rl);
    lds_barrier();
    load_x_half(in, first + nblk * kWavesC, ntiles, rows, xb);
    if (kMode >= 1 || qz.unit_fast)
        compress_waves<kMode, kBits, true>(qz, rl, in, dst, y_out, rows, xa, xb, blk, nblk);
    else
        compress_waves_general<kMode, kBits>(qz, rl, in, dst, y_out, rows, blk, nblk);
}

// kPlanned: the quantizer and the rotation fragments come from a plan; otherwise the
// workgroup builds them from rot and cent.
template <int kMode, int kBits, class Dst, bool kPlanned>
__global__ __launch_bounds__(64 * kWavesC) __attribute__((amdgpu_waves_per_eu(2))) void
tq_compress_mfma_kernel(const uint16_t* __restrict__ in, const float* __restrict__ rot,
                        const float* __restrict__ cent, int L, const TqPlanDev* __restrict__ plan,
                        Dst dst, float* __restrict__ y_out, int64_t rows) {
    __shared__ Quantizer qz;
    __shared__ RotLds rl;
    if constexpr (kPlanned) {
        compress_planned<kMode, kBits>(qz, rl, in, plan, dst, y_out, rows, blockIdx.x, gridDim.x);
        return;
    }
    // The centroids are loaded alone first (behind the chip-wide burst of the other loads
    // their latency is several times longer); then the rotation's loads and the wave's first
    // tile go out and stay in flight while wave 0 builds the quantizer. The second tile is only
    // requested after the set-up: a wave stalls at issue once its CU has too many bytes in
    // flight, and the set-up would wait behind it. The set-up's barriers order LDS only
    // (a full __syncthreads would drain the loads first).
    if constexpr (kMode == 0) {
        if (wave_id() == 0) {
            for (int i = (int)threadIdx.x; i < L; i += 64) qz.c[i] = cent[i];
        }
    }
    RotStage<false, 64 * kWavesC, true> rs;
    rs.load(rot);
    const int64_t first = (int64_t)blockIdx.x * kWavesC + wave_id();
    const int64_t ntiles = ceil_div(rows, kTile);
    f16x8 xa[8], xb[8];
    load_x_half(in, first, ntiles, rows, xa);
    // wave 0 builds the quantizer while the others stage the rotation
    if constexpr (kMode == 0) {
        if (wave_id() == 0) quantizer_finish<true>(qz, L);
    }
    rs.store(rl);
    lds_barrier();
    load_x_half(in, first + (int64_t)gridDim.x * kWavesC, ntiles, rows, xb);
    if (kMode >= 1 || qz.unit_fast)
        compress_waves<kMode, kBits, true>(qz, rl, in, dst, y_out, rows, xa, xb, blockIdx.x,
                                           gridDim.x);
    else
        compress_waves_general<kMode, kBits>(qz, rl, in, dst, y_out, rows, blockIdx.x,
                                             gridDim.x);
}

// Keys and values of one layer in one launch: even workgroups compress the keys, odd ones the
// values, each with its own plan, so the two tensors' load ramps and tails overlap on the
// chip instead of following one another. kKBits / kVBits: the two widths.
template <int kKBits, int kVBits, class Dst>
__global__ __launch_bounds__(64 * kWavesC) __attribute__((amdgpu_waves_per_eu(2))) void
tq_compress_kv_mfma_kernel(const uint16_t* __restrict__ k_in, const uint16_t* __restrict__ v_in,
                           const TqPlanDev* __restrict__ kplan,
                           const TqPlanDev* __restrict__ vplan, Dst kdst, Dst vdst,
                           int64_t rows) {
    __shared__ Quantizer qz;
    __shared__ RotLds rl;
    const int64_t blk = blockIdx.x >> 1, nblk = gridDim.x >> 1;
    if (blockIdx.x & 1)
        compress_planned<0, kVBits>(qz, rl, v_in, vplan, vdst, nullptr, rows, blk, nblk);
    else
        compress_planned<0, kKBits>(qz, rl, k_in, kplan, kdst, nullptr, rows, blk, nblk);
}

// ---------------------------------------------------------------------------------------
// Generic-head_dim compress / rotate on the VALU (turboquant_compress.cu:48-186 order):
// norm, normalise, sequential dot per output coordinate, quantize, pack.
// ---------------------------------------------------------------------------------------
template <int kMode, class Dst>
__global__ __launch_bounds__(256) void tq_compress_generic_kernel(
    const uint16_t* __restrict__ in, const float* __restrict__ rot,
    const float* __restrict__ cent, int L, int bits, Dst dst, float* __restrict__ y_out,
    int64_t rows, int hd) {
    __shared__ Quantizer qz;
    __shared__ float red[16];
    extern __shared__ float smem[];
    float* x = smem;         // [hd]
    float* yv = smem + hd;   // [hd]
    if constexpr (kMode == 0) quantizer_build(qz, cent, L);
    const int G = (hd + 7) / 8;
    const int64_t pd = ceil_div((int64_t)hd * bits, 8);
    for (int64_t m = blockIdx.x; m < rows; m += gridDim.x) {
        float ss = 0.0f;
        for (int d = threadIdx.x; d < hd; d += blockDim.x) {
            const float v = h2f(in[m * hd + d]);
            x[d] = v;
            ss += v * v;
        }
        ss = block_sum(ss, red);  // barriers also publish x[]
        const float nrm = sqrtf(ss);
        if (threadIdx.x == 0) {
            uint16_t* np = dst.nptr(m);
            if (np) *np = (uint16_t)f2h(nrm);
        }
        const float inv = 1.0f / (nrm + 1e-8f);
        for (int d = threadIdx.x; d < hd; d += blockDim.x) x[d] *= inv;
        __syncthreads();
        for (int i = threadIdx.x; i < hd; i += blockDim.x) {
            const float* pr = rot + (int64_t)i * hd;
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j) dot += pr[j] * x[j];
            yv[i] = dot;
            if constexpr (kMode == 1) y_out[m * hd + i] = dot;
        }
        __syncthreads();
        if constexpr (kMode == 0) {
            uint8_t* prow = dst.prow(m);
            for (int g = threadIdx.x; g < G && prow; g += blockDim.x) {
                int codes[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = 8 * g + e;
                    codes[e] = d < hd ? quantize(qz, yv[d]) : 0;
                }
                const int64_t nb = pd - (int64_t)g * bits;
                store_group(prow + (int64_t)g * bits, group_word(codes, bits), bits,
                            (int)(nb < bits ? nb : bits));
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// Quantize + pack of given fp32 y [rows, hd]: one lane per group of 8 coordinates.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tq_quantize_pack_kernel(const float* __restrict__ y,
                                                               const float* __restrict__ cent,
                                                               int L, int bits,
                                                               uint8_t* __restrict__ packed,
                                                               int64_t rows, int hd, int64_t pd) {
    __shared__ Quantizer qz;
    quantizer_build(qz, cent, L);
    const int G = (hd + 7) / 8;
    const int64_t total = rows * G;
    const bool vec = (hd % 8) == 0 && (((uintptr_t)y) & 15u) == 0;
    for (int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gi < total;
         gi += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = gi / G;
        const int g = (int)(gi - row * G);
        const float* yr = y + row * hd + 8 * g;
        float v[8];
        if (vec) {
            const f32x4 a = *(const f32x4*)yr, b = *(const f32x4*)(yr + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = a[e];
                v[4 + e] = b[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (8 * g + e < hd) ? yr[e] : 0.0f;
        }
        int codes[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) codes[e] = (8 * g + e < hd) ? quantize(qz, v[e]) : 0;
        const int64_t nb = pd - (int64_t)g * bits;
        store_group(packed + row * pd + (int64_t)g * bits, group_word(codes, bits), bits,
                    (int)(nb < bits ? nb : bits));
    }
}

// ---------------------------------------------------------------------------------------
// MFMA dequantize, head_dim 128 (turboquant_decompress.cu:21-94):
//   unpack -> c[idx] -> x_hat = Pi^T y_hat -> fp16(x_hat * float(norm)).
// ---------------------------------------------------------------------------------------
// x_hat = Pi_hi^T c_hi + 2^-12 (Pi_lo'^T c_hi + Pi_hi^T c_lo'). The main product runs on fp16
// MFMA (v_mfma_f32_32x32x16_f16, exact products). The two correction products, each ~2^-11
// of it, run on fp8 E4M3 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4: 64 coordinates per
// instruction at twice the fp16 rate), which cuts the kernel's MFMA time by a third. Their
// operands are prescaled by powers of two into fp8's normal range when the tables are built
// (f8_prescale); the instruction's E8M0 operand scales undo that exactly and apply the 2^-12,
// so the corrections accumulate straight into the main product's fp32 sum. fp8 rounds a
// correction term to 2^-4 of itself: ~2^-15 of the term |Pi||c|, against 2^-11 (half an
// fp16 ulp) for the stored output.
// fp8 operand u (0, 1) of lane (i or r, h) is 8 registers: byte b is coordinate 64h + 32u + b.
// The A and B operands use the same map, so the product sums over exactly those coordinates,
// in whatever order the instruction assigns them to K.
// ---------------------------------------------------------------------------------------
typedef int i32x8 __attribute__((ext_vector_type(8)));

// Power-of-two exponent that brings max |v| into [128, 256): fp8 E4M3's normal range, under
// its 448 maximum. 0 for a zero or non-finite maximum.
__device__ inline int f8_prescale(float maxabs) {
    if (!(maxabs > 0.0f) || !(maxabs <= 3.0e38f)) return 0;
    int e;
    (void)frexpf(maxabs, &e);  // maxabs = f 2^e, f in [0.5, 1)
    return min(max(8 - e, -120), 120);
}
// The instruction's E8M0 scale that undoes a prescale by 2^p and applies 2^-6, half of the
// corrections' 2^-12 (each product's two operand scales multiply): 2^(scale - 127) = 2^(-p-6).
// With p in [-120, 120] (f8_prescale) the scale stays in [1, 241].
__device__ __forceinline__ int f8_scale(int p) { return 127 - p - 6; }
// fp8 E4M3 bytes of 2^p a and 2^p b (v_cvt_pk_fp8_f32, round to nearest even), in the low
// (kHi = false) or high half of old.
template <bool kHi>
__device__ __forceinline__ uint32_t f8_pk(float a, float b, int p, uint32_t old) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(a, p), ldexpf(b, p), (int)old, kHi);
}

// Dequantize A operands (A[i][k] = Pi[k][32c + i]) for lane (i, h):
//   hi[c][s][lane]         8 fp16 of Pi_hi, coordinates 64h + 8s + 0..7;
//   f8[c][u][t][q][lane]   16 fp8 bytes of 2^p Pi_lo' (t = 0) or 2^p Pi_hi (t = 1),
//                          coordinates 64h + 32u + 16q + 0..15.
struct DeqLds {
    u32x4 hi[4][8][64];        // 32 KB
    u32x4 f8[4][2][2][2][64];  // 32 KB
};

// The dequantize's code-side tables and the four operand scales (E8M0).
enum { kScaleALo = 0, kScaleAHi = 1, kScaleBHi = 2, kScaleBLo = 3 };
struct DequantLds {
    // code -> fp16 c_hi | fp8 2^p c_hi << 16 | fp8 2^p' c_lo' << 24 (c = c_hi + 2^-12 c_lo')
    uint32_t tab[kMaxLevels];
    // 2, 3 or 4 bits: code pair b (codes b >> bits, b & (2^bits - 1); at 4 bits a code byte)
    // -> {the two fp16 c_hi, fp8 [hi, hi, lo', lo']}; 2^(2 bits) entries
    u32x2 pair[256];
    int scale[4];
};

// fp8 quad [hi(c0), hi(c1), lo'(c0), lo'(c1)] of two table entries.
__device__ __forceinline__ uint32_t f8_quad(uint32_t t0, uint32_t t1) {
    return __builtin_amdgcn_perm(t1, t0, 0x07030602u);
}
// fp16 hi pair of two table entries.
__device__ __forceinline__ uint32_t hi_pair(uint32_t t0, uint32_t t1) {
    return __builtin_amdgcn_perm(t1, t0, 0x05040100u);
}

// Maxima of non-negative floats across the workgroup (kN of them per thread): each wave's go
// to its own slots, and after the barrier every thread folds all of them. Compared as
// integers, so a NaN (any non-negative NaN pattern is above +inf) survives to the result.
template <int kN>
__device__ __forceinline__ void block_max(float (&m)[kN], int (*slots)[kN], int nwaves) {
    const int w = (int)(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < kN; ++j) {
        const int v = wave_max_int(__float_as_int(m[j]));
        if ((threadIdx.x & 63) == 0) slots[w][j] = v;
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < kN; ++j) {
        int v = 0;
        for (int k = 0; k < nwaves; ++k) v = max(v, slots[k][j]);
        m[j] = __int_as_float(v);
    }
}

// Staging of the dequantize A operands in two steps (load() issues this thread's reads of
// Pi, store() writes LDS), with the operand maxima in between. kThreads is the block size.
template <int kThreads>
struct DeqStage {
    static constexpr int kFrags = 4 * 8 * 64;
    static constexpr int kN = (kFrags + kThreads - 1) / kThreads;
    float v[kN][8];  // Pi[64h + 8s + e][32c + i] for fragment (c, s, lane = (i, h))
    __device__ __forceinline__ void load(const float* __restrict__ rot) {
#pragma unroll
        for (int n = 0; n < kN; ++n) {
            const int idx = (int)threadIdx.x + n * kThreads;
            if (kFrags % kThreads != 0 && idx >= kFrags) break;
            const int lane = idx & 63, s = (idx >> 6) & 7, c = idx >> 9;
            const int row = 32 * c + (lane & 31), k0 = 64 * (lane >> 5) + 8 * s;
#pragma unroll
            for (int e = 0; e < 8; ++e) v[n][e] = rot[(k0 + e) * kHd + row];
        }
    }
    // this thread's maxima of |Pi_lo'| and |Pi_hi|, folded into mlo and mhi
    __device__ __forceinline__ void maxima(float& mlo, float& mhi) const {
#pragma unroll
        for (int n = 0; n < kN; ++n) {
            const int idx = (int)threadIdx.x + n * kThreads;
            if (kFrags % kThreads != 0 && idx >= kFrags) break;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = v[n][e];
                const float hi = (float)(_Float16)x;
                mhi = fmaxf(mhi, fabsf(hi));
                mlo = fmaxf(mlo, fabsf((x - hi) * kLoScale));
            }
        }
    }
    // p_lo, p_hi: the prescales of Pi_lo' and Pi_hi (f8_prescale of their maxima)
    __device__ __forceinline__ void store(DeqLds& L, int p_lo, int p_hi) const {
#pragma unroll
        for (int n = 0; n < kN; ++n) {
            const int idx = (int)threadIdx.x + n * kThreads;
            if (kFrags % kThreads != 0 && idx >= kFrags) break;
            const int lane = idx & 63, s = (idx >> 6) & 7, c = idx >> 9;
            uint32_t hw[4], l8[2], h8[2];
            float hi[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 h = (_Float16)v[n][e];
                hi[e] = (float)h;
                lo[e] = (v[n][e] - hi[e]) * kLoScale;
            }
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2)
                hw[e2] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi[2 * e2]) |
                         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi[2 * e2 + 1]) << 16);
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                l8[d] = f8_pk<true>(lo[4 * d + 2], lo[4 * d + 3], p_lo,
                                    f8_pk<false>(lo[4 * d], lo[4 * d + 1], p_lo, 0u));
                h8[d] = f8_pk<true>(hi[4 * d + 2], hi[4 * d + 3], p_hi,
                                    f8_pk<false>(hi[4 * d], hi[4 * d + 1], p_hi, 0u));
            }
            L.hi[c][s][lane] = u32x4{hw[0], hw[1], hw[2], hw[3]};
            // coordinates 64h + 8s + 0..7 = chunk q = (s >> 1) & 1 of operand u = s >> 2, at
            // byte 8 (s & 1) of it
            const int u = s >> 2, q = (s >> 1) & 1, off = 2 * (s & 1);
            uint32_t* dl = (uint32_t*)&L.f8[c][u][0][q][lane] + off;
            uint32_t* dh = (uint32_t*)&L.f8[c][u][1][q][lane] + off;
            *(u32x2*)dl = u32x2{l8[0], l8[1]};
            *(u32x2*)dh = u32x2{h8[0], h8[1]};
        }
    }
};

// This thread's centroid's |c_hi| and |c_lo'| (zero past the codebook).
__device__ __forceinline__ void centroid_maxima(float c, float& mhi, float& mlo) {
    const float hi = (float)(_Float16)c;
    mhi = fabsf(hi);
    mlo = fabsf((c - hi) * kLoScale);
}
// Table entry of centroid c (DequantLds::tab) for prescales p_hi, p_lo of c_hi and c_lo'.
__device__ __forceinline__ uint32_t dq_tab_entry(float c, int p_hi, int p_lo) {
    const _Float16 h = (_Float16)c;
    const float hi = (float)h, lo = (c - hi) * kLoScale;
    const uint32_t f8 = f8_pk<false>(hi, 0.0f, p_hi, 0u) & 0xffu;
    const uint32_t l8 = f8_pk<false>(lo, 0.0f, p_lo, 0u) & 0xffu;
    return (uint32_t)__builtin_bit_cast(uint16_t, h) | (f8 << 16) | (l8 << 24);
}
// The workgroup's tables from the four maxima {|Pi_lo'|, |Pi_hi|, |c_hi|, |c_lo'|}: the
// scales, and the entry of centroid c_own for thread i < kMaxLevels (c_own = 0 past L).
// The 4-bit pair table needs the entries: build_pairs after a barrier.
__device__ __forceinline__ void dq_tables(DequantLds& t, const float (&m)[4], float c_own) {
    const int p_hi = f8_prescale(m[2]), p_lo = f8_prescale(m[3]);
    if (threadIdx.x == 0) {
        t.scale[kScaleALo] = f8_scale(f8_prescale(m[0]));
        t.scale[kScaleAHi] = f8_scale(f8_prescale(m[1]));
        t.scale[kScaleBHi] = f8_scale(p_hi);
        t.scale[kScaleBLo] = f8_scale(p_lo);
    }
    if ((int)threadIdx.x < kMaxLevels) t.tab[threadIdx.x] = dq_tab_entry(c_own, p_hi, p_lo);
}
// The pair table of a bits-wide code (2 to 4; none at other widths).
__device__ __forceinline__ void dq_pairs(DequantLds& t, int bits) {
    if (bits < 2 || bits > 4) return;
    const int n = 1 << (2 * bits), m = (1 << bits) - 1;
    for (int b = threadIdx.x; b < n; b += blockDim.x) {
        const uint32_t t0 = t.tab[b >> bits], t1 = t.tab[b & m];
        t.pair[b] = u32x2{hi_pair(t0, t1), f8_quad(t0, t1)};
    }
}

// One lane's codes of a tile: row r = lane & 31, groups [8h, 8h+8) (8*kBits bytes at byte
// 8*kBits*h of the row), and the row's norm.
template <int kBits>
struct CodeHalf {
    uint32_t w[2 * kBits];
    uint16_t norm;
};

template <int kBits>
__device__ __forceinline__ void load_code_half(const uint8_t* __restrict__ packed,
                                               const uint16_t* __restrict__ norms, int64_t tile,
                                               int64_t ntiles, int64_t rows, CodeHalf<kBits>& cw) {
    constexpr int pd = 16 * kBits;
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int64_t m0 = tile * kTile;
    const bool ok = tile < ntiles && r < rows - m0;
    // rows past the end read row 0 (their results are not stored); see load_x_half
    const int64_t row = ok ? m0 + r : 0;
    const uint8_t* src = packed + row * pd + 8 * kBits * h;
    if constexpr (kBits % 2 == 0) {  // 16, 32 or 64 bytes at a 16-byte aligned offset
#pragma unroll
        for (int i = 0; i < kBits / 2; ++i) {
            const u32x4 v = ld16(src + 16 * i);
#pragma unroll
            for (int t = 0; t < 4; ++t) cw.w[4 * i + t] = v[t];
        }
    } else {  // 24 bytes at an 8-byte aligned offset
#pragma unroll
        for (int i = 0; i < kBits; ++i) {
            const u32x2 v = *(const u32x2*)(src + 8 * i);
            cw.w[2 * i] = v[0];
            cw.w[2 * i + 1] = v[1];
        }
    }
    cw.norm = norms[row];
}

// The B operands of a tile's codes: bh[s] the fp16 c_hi of coordinates 64h + 8s + 0..7;
// b8[u][0 | 1] the fp8 c_hi / c_lo' of coordinates 64h + 32u + 0..31.
struct CodeOps {
    f16x8 bh[8];
    i32x8 b8[2][2];
};

// Group s (8 codes) of this lane's half into the B operands.
template <int kBits>
__device__ __forceinline__ void decode_group(const DequantLds& t, const CodeHalf<kBits>& cw,
                                             int s, CodeOps& ops) {
    uint32_t vh[4], fq[4];  // per code pair p: fp16 hi pair, fp8 quad
    if constexpr (kBits == 4) {
        const uint32_t g = cw.w[s];  // byte p: coordinates (2p, 2p+1) in (high, low) nibbles
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32x2 e = t.pair[(g >> (8 * p)) & 0xffu];
            vh[p] = e[0];
            fq[p] = e[1];
        }
    } else if constexpr (kBits == 2 || kBits == 3) {
        // big-endian group word of kBits bytes; codes 2p, 2p + 1 are its 2 kBits bits at
        // 2 kBits (3 - p), the pair table's index
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < kBits; ++k) {
            const int byte = s * kBits + k;
            word = (word << 8) | ((cw.w[byte >> 2] >> (8 * (byte & 3))) & 0xffu);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const u32x2 e =
                t.pair[(word >> (2 * kBits * (3 - p))) & ((1u << (2 * kBits)) - 1u)];
            vh[p] = e[0];
            fq[p] = e[1];
        }
    } else {
        uint64_t word = 0;  // big-endian group word of kBits bytes
#pragma unroll
        for (int k = 0; k < kBits; ++k) {
            const int byte = s * kBits + k;
            word = (word << 8) | ((cw.w[byte >> 2] >> (8 * (byte & 3))) & 0xffu);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t c0 = (uint32_t)(word >> (kBits * (7 - 2 * p))) & ((1u << kBits) - 1u);
            const uint32_t c1 = (uint32_t)(word >> (kBits * (6 - 2 * p))) & ((1u << kBits) - 1u);
            const uint32_t t0 = t.tab[c0], t1 = t.tab[c1];
            vh[p] = hi_pair(t0, t1);
            fq[p] = f8_quad(t0, t1);
        }
    }
    ops.bh[s] = __builtin_bit_cast(f16x8, u32x4{vh[0], vh[1], vh[2], vh[3]});
    const int u = s >> 2, j = 2 * (s & 3);  // registers j, j + 1 of operand u
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        ops.b8[u][0][j + d] = (int)__builtin_amdgcn_perm(fq[2 * d + 1], fq[2 * d], 0x05040100u);
        ops.b8[u][1][j + d] = (int)__builtin_amdgcn_perm(fq[2 * d + 1], fq[2 * d], 0x07060302u);
    }
}

// ---------------------------------------------------------------------------------------
// MFMA dequantize of one tile by one wave, head_dim 128 (turboquant_decompress.cu:21-94):
//   unpack -> c[idx] -> x_hat = Pi^T y_hat -> fp16(x_hat * float(norm)).
// Lane (r, h) ends block c holding coordinates 32c + 8g + 4h + e of row r; neighbouring
// chunks are exchanged with the partner lane so every lane stores 16 contiguous bytes.
// ---------------------------------------------------------------------------------------
// Block c of the lane's row: fp16(acc * nrm) to orow[32c .. 32c + 31].
__device__ __forceinline__ void store_block(const f32x16& acc, float nrm,
                                            uint16_t* __restrict__ orow, int c, bool row_ok) {
    uint32_t ch[4][2];  // chunk g: coordinates 32c + 8g + 4h + 0..3 as fp16 pairs
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 2; ++e)
            ch[g][e] = f2h(acc[4 * g + 2 * e] * nrm) | (f2h(acc[4 * g + 2 * e + 1] * nrm) << 16);
    // chunks (2m, 2m+1): lane h = 0 takes coordinates 16m + 0..7, lane h = 1 16m + 8..15
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int e = 0; e < 2; ++e) swap_halves(ch[2 * m][e], ch[2 * m + 1][e]);
        if (row_ok)
            *(u32x4*)&orow[32 * c + 16 * m] =
                u32x4{ch[2 * m][0], ch[2 * m][1], ch[2 * m + 1][0], ch[2 * m + 1][1]};
    }
}

// x = Pi^T y of the lane's row from the (hi, lo') fp16 B fragments of y (three fp16
// products per step), stored as fp16(x * nrm).
__device__ __forceinline__ void rotate_back_store(const RotLds& L, const f16x8 (&bh)[8],
                                                  const f16x8 (&bl)[8], float nrm,
                                                  uint16_t* __restrict__ out, int64_t m0,
                                                  int nvalid) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    uint16_t* orow = out + m0 * kHd + (r * kHd + 8 * h);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        __builtin_amdgcn_sched_barrier(0);  // keep each block's fragment loads within it
        f32x16 acc1 = {}, acc2 = {};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 ah = frag(L, c, s, 0, lane), al = frag(L, c, s, 1, lane);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh[s], acc1, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh[s], acc2, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl[s], acc2, 0, 0, 0);
        }
        f32x16 x;
#pragma unroll
        for (int v = 0; v < 16; ++v) x[v] = fmaf(acc2[v], kLoInv, acc1[v]);
        store_block(x, nrm, orow, c, r < nvalid);
    }
}

// fp8 A operand (u, t) of block c: 8 registers.
__device__ __forceinline__ i32x8 deq_a8(const DeqLds& L, int c, int u, int t, int lane) {
    const u32x4 a = L.f8[c][u][t][0][lane], b = L.f8[c][u][t][1][lane];
    return i32x8{(int)a[0], (int)a[1], (int)a[2], (int)a[3],
                 (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
}

template <int kBits>
__device__ __forceinline__ void dequant_tile(const DequantLds& t, const DeqLds& L,
                                             const CodeHalf<kBits>& cw,
                                             uint16_t* __restrict__ out, int64_t m0, int nvalid) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    CodeOps ops;
#pragma unroll
    for (int s = 0; s < 8; ++s) decode_group<kBits>(t, cw, s, ops);
    const int sa_lo = t.scale[kScaleALo], sa_hi = t.scale[kScaleAHi];
    const int sb_hi = t.scale[kScaleBHi], sb_lo = t.scale[kScaleBLo];
    const float nrm = h2f(cw.norm);
    uint16_t* orow = out + m0 * kHd + (r * kHd + 8 * h);
    // The 32 fp16 steps (block c = q / 8, step s = q % 8) run as one software pipeline: the
    // fp16 fragment of step q + 2 and the fp8 operand of the next odd step are read while step q
    // computes, and blocks alternate between two accumulators, so a block's stores overlap the
    // next block's products.
    constexpr int kAhead = 2;
    f16x8 fh[kAhead + 1];
    i32x8 f8r[2];
#pragma unroll
    for (int q = 0; q < kAhead; ++q) fh[q] = __builtin_bit_cast(f16x8, L.hi[q >> 3][q & 7][lane]);
    f8r[0] = deq_a8(L, 0, 0, 0, lane);
    f32x16 acc[2];
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const int c = q >> 3, s = q & 7, b = c & 1;
        __builtin_amdgcn_sched_barrier(0);
        if (q + kAhead < 32) {
            const int n = q + kAhead;
            fh[n % (kAhead + 1)] = __builtin_bit_cast(f16x8, L.hi[n >> 3][n & 7][lane]);
        }
        if ((q & 1) == 0 && (q >> 1) + 1 < 16) {  // fp8 operand j = q / 2 + 1 (odd step q + 1)
            const int j = (q >> 1) + 1;
            f8r[j & 1] = deq_a8(L, j >> 2, (j >> 1) & 1, j & 1, lane);
        }
        if (s == 0) acc[b] = f32x16{};
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fh[q % (kAhead + 1)], ops.bh[s], acc[b], 0, 0, 0);
        if (q & 1) {  // fp8 operand j = q / 2: block c, operand u = s / 4, part tt = s / 2 % 2
            const int j = q >> 1, u = s >> 2, tt = (s >> 1) & 1;
            if (tt == 0)  // Pi_lo' c_hi
                acc[b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    f8r[j & 1], ops.b8[u][0], acc[b], 0, 0, 0, sa_lo, 0, sb_hi);
            else  // Pi_hi c_lo'
                acc[b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    f8r[j & 1], ops.b8[u][1], acc[b], 0, 0, 0, sa_hi, 0, sb_lo);
        }
        // block c - 1's stores, two steps into block c (its last product has finished)
        if (c > 0 && s == 2) store_block(acc[b ^ 1], nrm, orow, c - 1, r < nvalid);
    }
    __builtin_amdgcn_sched_barrier(0);
    store_block(acc[1], nrm, orow, 3, r < nvalid);
}

// ---------------------------------------------------------------------------------------
// x = Pi^T y for fp32 rows y [rows, 128] -> fp16 (the attention combine's unrotation of the
// merged outputs, attention_paged_tq.cu:245-257, for batches of many vectors): each lane's
// 64 values of its row split into fp16 (hi, lo') operands (y = hi + 2^-12 lo'), then three
// fp16 products per step (rotate_back_store), fp32-accurate.
// ---------------------------------------------------------------------------------------
struct RowHalf {
    f32x4 v[16];  // coordinates 64 h + 4 i .. + 3 of the lane's row
};
__device__ __forceinline__ void load_row_half(const float* __restrict__ y, int64_t tile,
                                              int64_t ntiles, int64_t rows, RowHalf& rh) {
    const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
    const int64_t m0 = tile * kTile;
    // rows past the end read row 0 (their results are not stored)
    const int64_t row = tile < ntiles && r < rows - m0 ? m0 + r : 0;
    const float* src = y + row * kHd + 64 * h;
#pragma unroll
    for (int i = 0; i < 16; ++i) rh.v[i] = *(const f32x4*)(src + 4 * i);
}
__device__ __forceinline__ void rotate_back_tile(const RotLds& L, const RowHalf& rh,
                                                 uint16_t* __restrict__ out, int64_t m0,
                                                 int nvalid) {
    f16x8 bh[8], bl[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            uint32_t hb[2], lb[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float x = rh.v[2 * s + p / 2][2 * (p % 2) + e];
                const _Float16 hi = (_Float16)x;
                hb[e] = __builtin_bit_cast(uint16_t, hi);
                lb[e] = __builtin_bit_cast(uint16_t, (_Float16)((x - (float)hi) * kLoScale));
            }
            hw[p] = hb[0] | (hb[1] << 16);
            lw[p] = lb[0] | (lb[1] << 16);
        }
        bh[s] = __builtin_bit_cast(f16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
        bl[s] = __builtin_bit_cast(f16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
    }
    rotate_back_store(L, bh, bl, 1.0f, out, m0, nvalid);
}
constexpr int kWavesR = 4;  // waves per workgroup of the back-rotation (two workgroups per CU)
__global__ __launch_bounds__(64 * kWavesR) __attribute__((amdgpu_waves_per_eu(2))) void
tq_rotate_back_kernel(const float* __restrict__ y, const float* __restrict__ rot,
                      uint16_t* __restrict__ out, int64_t rows) {
    __shared__ RotLds rl;
    const int64_t ntiles = ceil_div(rows, kTile);
    const int64_t stride = (int64_t)gridDim.x * kWavesR;
    int64_t tile = (int64_t)blockIdx.x * kWavesR + wave_id();
    RotStage<true, 64 * kWavesR, false> rs;
    rs.load(rot);
    RowHalf ra;
    load_row_half(y, tile, ntiles, rows, ra);
    rs.store(rl);
    lds_barrier();
    while (tile < ntiles) {
        RowHalf rb;
        load_row_half(y, tile + stride, ntiles, rows, rb);
        rotate_back_tile(rl, ra, out, tile * kTile, (int)min<int64_t>(kTile, rows - tile * kTile));
        ra = rb;
        tile += stride;
    }
}

// The wave's tile loop: ca holds its first tile (loads issued); each tile's successor is in
// flight while it computes.
template <int kBits>
__device__ __forceinline__ void dequant_waves(const DequantLds& t, const DeqLds& rl,
                                              const uint8_t* __restrict__ packed,
                                              const uint16_t* __restrict__ norms,
                                              uint16_t* __restrict__ out, int64_t rows,
                                              int64_t tile, int64_t stride, int64_t ntiles,
                                              CodeHalf<kBits>& ca, CodeHalf<kBits>& cb) {
    while (tile < ntiles) {
        load_code_half<kBits>(packed, norms, tile + stride, ntiles, rows, cb);
        dequant_tile<kBits>(t, rl, ca, out, tile * kTile,
                            (int)min<int64_t>(kTile, rows - tile * kTile));
        tile += stride;
        if (tile >= ntiles) break;
        load_code_half<kBits>(packed, norms, tile + stride, ntiles, rows, ca);
        dequant_tile<kBits>(t, rl, cb, out, tile * kTile,
                            (int)min<int64_t>(kTile, rows - tile * kTile));
        tile += stride;
    }
}

// ---------------------------------------------------------------------------------------
// Plan: everything the MFMA kernels derive from one rotation and codebook, built once
// (tq_plan_kernel) in the layouts the kernels keep in LDS, plus the fp32 originals for the
// generic kernels.
// ---------------------------------------------------------------------------------------
struct TqPlanDev {
    RotLds comp;         // compress fragments (hi scaled by 2^12, lo')
    DeqLds deq;          // dequantize A operands (fp16 Pi_hi, fp8 Pi_lo' and Pi_hi)
    Quantizer qz;        // the built quantizer
    DequantLds dt;       // dequantize centroid tables
    float rot[kHd * kHd];
    float cent[kMaxLevels];
};
__device__ __forceinline__ const Quantizer& plan_quantizer(const TqPlanDev* p) { return p->qz; }
__device__ __forceinline__ const RotLds& plan_compress_frags(const TqPlanDev* p) {
    return p->comp;
}

// The planned dequantize of one tensor by workgroup blk of nblk: the tables and fragments are
// copied from the plan into LDS while the first tile's loads are in flight.
template <int kBits>
__device__ __forceinline__ void dequant_planned(DequantLds& t, DeqLds& rl,
                                                const uint8_t* __restrict__ packed,
                                                const uint16_t* __restrict__ norms,
                                                const TqPlanDev* __restrict__ plan,
                                                uint16_t* __restrict__ out, int64_t rows,
                                                int64_t blk, int64_t nblk) {
    const int64_t ntiles = ceil_div(rows, kTile);
    const int64_t stride = nblk * kWavesD;
    const int64_t tile = blk * kWavesD + wave_id();
    LdsCopy<64 * kWavesD, (int)sizeof(DequantLds)> tc;
    LdsCopy<64 * kWavesD, (int)sizeof(DeqLds)> rc;
    tc.load(&plan->dt);
    rc.load(&plan->deq);
    __builtin_amdgcn_sched_barrier(0);
    CodeHalf<kBits> ca, cb;
    load_code_half<kBits>(packed, norms, tile, ntiles, rows, ca);
    __builtin_amdgcn_sched_barrier(0);
    tc.store(&t);
    rc.store(&rl);
    lds_barrier();
    dequant_waves<kBits>(t, rl, packed, norms, out, rows, tile, stride, ntiles, ca, cb);
}

template <int kBits, bool kPlanned>
__global__ __launch_bounds__(64 * kWavesD) __attribute__((amdgpu_waves_per_eu(3))) void
tq_dequant_mfma_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ norms,
                       const float* __restrict__ rot, const float* __restrict__ cent, int L,
                       const TqPlanDev* __restrict__ plan, uint16_t* __restrict__ out,
                       int64_t rows) {
    __shared__ DequantLds t;
    __shared__ DeqLds rl;
    if constexpr (kPlanned) {
        dequant_planned<kBits>(t, rl, packed, norms, plan, out, rows, blockIdx.x, gridDim.x);
        return;
    }
    __shared__ int mx[kWavesD][4];
    const int64_t ntiles = ceil_div(rows, kTile);
    const int64_t stride = (int64_t)gridDim.x * kWavesD;
    int64_t tile = (int64_t)blockIdx.x * kWavesD + wave_id();
    // Loads go out in the order their data is needed: the centroids, the rotation, then the
    // first tile, which stays in flight through the set-up (whose barriers order LDS only).
    static_assert(kMaxLevels <= 64 * kWavesD, "one centroid per thread");
    const float c_own = (int)threadIdx.x < L ? cent[threadIdx.x] : 0.0f;
    DeqStage<64 * kWavesD> rs;
    rs.load(rot);
    CodeHalf<kBits> ca, cb;
    load_code_half<kBits>(packed, norms, tile, ntiles, rows, ca);
    float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // |Pi_lo'|, |Pi_hi|, |c_hi|, |c_lo'|
    rs.maxima(m[0], m[1]);
    centroid_maxima(c_own, m[2], m[3]);
    block_max(m, mx, kWavesD);
    dq_tables(t, m, c_own);
    rs.store(rl, f8_prescale(m[0]), f8_prescale(m[1]));
    lds_barrier();
    if constexpr (kBits >= 2 && kBits <= 4) {
        dq_pairs(t, kBits);
        lds_barrier();
    }
    dequant_waves<kBits>(t, rl, packed, norms, out, rows, tile, stride, ntiles, ca, cb);
}

// Keys and values of one layer in one launch: even workgroups dequantize the keys, odd ones
// the values (as the K+V compress kernel).
template <int kKBits, int kVBits>
__global__ __launch_bounds__(64 * kWavesD) __attribute__((amdgpu_waves_per_eu(3))) void
tq_dequant_kv_mfma_kernel(const uint8_t* __restrict__ k_packed, const uint16_t* __restrict__ k_norms,
                          const uint8_t* __restrict__ v_packed, const uint16_t* __restrict__ v_norms,
                          const TqPlanDev* __restrict__ kplan, const TqPlanDev* __restrict__ vplan,
                          uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out,
                          int64_t rows) {
    __shared__ DequantLds t;
    __shared__ DeqLds rl;
    const int64_t blk = blockIdx.x >> 1, nblk = gridDim.x >> 1;
    if (blockIdx.x & 1)
        dequant_planned<kVBits>(t, rl, v_packed, v_norms, vplan, v_out, rows, blk, nblk);
    else
        dequant_planned<kKBits>(t, rl, k_packed, k_norms, kplan, k_out, rows, blk, nblk);
}

// Build a plan (one workgroup): the quantizer exactly as the compress kernel builds it, both
// fragment layouts exactly as the kernels stage them, the dequantize tables, and copies of
// the fp32 rotation and centroids.
constexpr int kPlanThreads = 64 * kWavesC;
__global__ __launch_bounds__(kPlanThreads) void tq_plan_kernel(const float* __restrict__ rot,
                                                               const float* __restrict__ cent,
                                                               int L, int bits,
                                                               TqPlanDev* __restrict__ p) {
    __shared__ Quantizer qz;
    quantizer_build(qz, cent, L);
    {
        RotStage<false, kPlanThreads, true> rs;
        rs.load(rot);
        rs.store(p->comp);
    }
    {
        static_assert(kMaxLevels <= kPlanThreads, "one centroid per thread");
        __shared__ int mx[kPlanThreads / 64][4];
        DeqStage<kPlanThreads> ds;
        ds.load(rot);
        const float c_own = (int)threadIdx.x < L ? cent[threadIdx.x] : 0.0f;
        float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // |Pi_lo'|, |Pi_hi|, |c_hi|, |c_lo'|
        ds.maxima(m[0], m[1]);
        centroid_maxima(c_own, m[2], m[3]);
        block_max(m, mx, kPlanThreads / 64);
        ds.store(p->deq, f8_prescale(m[0]), f8_prescale(m[1]));
        dq_tables(p->dt, m, c_own);
    }
    for (int i = threadIdx.x; i < kHd * kHd; i += kPlanThreads) p->rot[i] = rot[i];
    for (int i = threadIdx.x; i < kMaxLevels; i += kPlanThreads) p->cent[i] = i < L ? cent[i] : 0.0f;
    __syncthreads();  // the table entries, written to the plan by other threads
    dq_pairs(p->dt, bits);
    __syncthreads();
    const uint32_t* q = (const uint32_t*)&qz;
    uint32_t* d = (uint32_t*)&p->qz;
    for (int i = threadIdx.x; i < (int)(sizeof(Quantizer) / 4); i += kPlanThreads) d[i] = q[i];
}

// Generic-head_dim dequantize on the VALU (turboquant_decompress.cu order).
__global__ __launch_bounds__(256) void tq_dequant_generic_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ norms,
    const float* __restrict__ rot, const float* __restrict__ cent, int bits,
    uint16_t* __restrict__ out, int64_t rows, int hd, int64_t pd) {
    extern __shared__ float yh[];  // [hd]
    const int G = (hd + 7) / 8;
    for (int64_t m = blockIdx.x; m < rows; m += gridDim.x) {
        for (int g = threadIdx.x; g < G; g += blockDim.x) {
            int codes[8];
            const int64_t nb = pd - (int64_t)g * bits;
            load_group(packed + m * pd + (int64_t)g * bits, bits, (int)(nb < bits ? nb : bits),
                       codes);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (8 * g + e < hd) yh[8 * g + e] = cent[codes[e]];
        }
        __syncthreads();
        const float nrm = h2f(norms[m]);
        for (int i = threadIdx.x; i < hd; i += blockDim.x) {
            float dot = 0.0f;
            for (int j = 0; j < hd; ++j) dot += rot[(int64_t)j * hd + i] * yh[j];
            out[m * hd + i] = (uint16_t)f2h(dot * nrm);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------
int tq_grid(int64_t work_units, int cap) {
    return (int)(work_units < cap ? (work_units > 0 ? work_units : 1) : cap);
}

bool tq_args_ok(int n_levels, int bits) {
    return bits >= 1 && bits <= 8 && n_levels >= 1 && n_levels <= (1 << bits) &&
           n_levels <= kMaxLevels;
}

// Grid of the MFMA kernels: one workgroup per CU (each stages the rotation once), never
// more workgroups than needed to give every wave a tile.
int mfma_grid(int64_t ntiles, int waves) {
    const int64_t need = ceil_div(ntiles, waves);
    const int64_t cus = fhip_host::cu_count();
    return (int)(need < cus ? (need > 0 ? need : 1) : cus);
}

// plan: non-null for the planned kernels (rot and cent then point into the plan).
template <int kMode, class Dst>
int launch_compress(const void* input, const float* rot, const float* cent, int L, int bits,
                    Dst dst, float* y_out, int64_t rows, int hd, hipStream_t s,
                    const TqPlanDev* plan = nullptr) {
    if (rows == 0) return hipSuccess;
    const bool mfma_bits = kMode >= 1 || bits == 2 || bits == 3 || bits == 4 || bits == 8;
    if (hd == kHd && mfma_bits && fhip_host::aligned16(input) &&
        (kMode == 0 || fhip_host::aligned16(y_out))) {
        auto pick = [&](auto planned) {
            constexpr bool kP = decltype(planned)::value;
            auto kern = tq_compress_mfma_kernel<kMode, 4, Dst, kP>;
            if constexpr (kMode == 0) {
                switch (bits) {
                    case 2: kern = tq_compress_mfma_kernel<kMode, 2, Dst, kP>; break;
                    case 3: kern = tq_compress_mfma_kernel<kMode, 3, Dst, kP>; break;
                    case 8: kern = tq_compress_mfma_kernel<kMode, 8, Dst, kP>; break;
                    default: break;
                }
            }
            return kern;
        };
        auto kern = plan ? pick(std::true_type{}) : pick(std::false_type{});
        hipLaunchKernelGGL(kern, dim3(mfma_grid(ceil_div(rows, kTile), kWavesC)),
                           dim3(64 * kWavesC), 0, s, (const uint16_t*)input, rot, cent, L, plan,
                           dst, y_out, rows);
    } else if constexpr (kMode == 2) {
        return hipErrorInvalidValue;  // the raw product exists for head_dim 128 only
    } else {
        const int grid = tq_grid(rows, 2048);
        const size_t lds = 2 * (size_t)hd * sizeof(float);
        hipLaunchKernelGGL((tq_compress_generic_kernel<kMode, Dst>), dim3(grid), dim3(256), lds,
                           s, (const uint16_t*)input, rot, cent, L, bits, dst, y_out, rows, hd);
    }
    return hipGetLastError();
}

int launch_dequant(const void* packed_in, const void* norms_in, const float* rotation,
                   const float* centroids, int L, void* output, int64_t rows, int head_dim,
                   int bits, int packed_dim_per_head, hipStream_t s,
                   const TqPlanDev* plan = nullptr) {
    const bool mfma_bits = bits == 2 || bits == 3 || bits == 4 || bits == 8;
    if (head_dim == kHd && mfma_bits && packed_dim_per_head == 16 * bits &&
        fhip_host::aligned16(output) && fhip_host::aligned16(packed_in) &&
        (((uintptr_t)norms_in) & 1u) == 0) {
        auto pick = [&](auto planned) {
            constexpr bool kP = decltype(planned)::value;
            auto kern = tq_dequant_mfma_kernel<4, kP>;
            switch (bits) {
                case 2: kern = tq_dequant_mfma_kernel<2, kP>; break;
                case 3: kern = tq_dequant_mfma_kernel<3, kP>; break;
                case 8: kern = tq_dequant_mfma_kernel<8, kP>; break;
                default: break;
            }
            return kern;
        };
        auto kern = plan ? pick(std::true_type{}) : pick(std::false_type{});
        hipLaunchKernelGGL(kern, dim3(mfma_grid(ceil_div(rows, kTile), kWavesD)),
                           dim3(64 * kWavesD), 0, s, (const uint8_t*)packed_in,
                           (const uint16_t*)norms_in, rotation, centroids, L, plan,
                           (uint16_t*)output, rows);
    } else {
        const int grid = tq_grid(rows, 2048);
        hipLaunchKernelGGL(tq_dequant_generic_kernel, dim3(grid), dim3(256),
                           (size_t)head_dim * sizeof(float), s, (const uint8_t*)packed_in,
                           (const uint16_t*)norms_in, rotation, centroids, bits,
                           (uint16_t*)output, rows, head_dim, (int64_t)packed_dim_per_head);
    }
    return hipGetLastError();
}

// Grid of the K+V kernels: one workgroup per CU in all (half per tensor), never more per
// tensor than gives every wave a tile.
int mfma_grid_kv(int64_t ntiles, int waves) {
    const int64_t need = ceil_div(ntiles, waves);
    const int64_t half = fhip_host::cu_count() >= 2 ? fhip_host::cu_count() / 2 : 1;
    return 2 * (int)(need < half ? (need > 0 ? need : 1) : half);
}

// Both tensors in one launch where a K+V kernel exists for the two widths (equal widths of
// 2, 3, 4 or 8 bits, or 4-bit keys with 2-bit values); false otherwise, nothing launched.
template <class Dst>
bool launch_compress_kv(const TqPlanDev* kp, const TqPlanDev* vp, int kbits, int vbits,
                        const void* kin, const void* vin, Dst kd, Dst vd, int64_t rows,
                        hipStream_t s) {
    if (!fhip_host::aligned16(kin) || !fhip_host::aligned16(vin)) return false;
    auto kern = tq_compress_kv_mfma_kernel<4, 4, Dst>;
    if (kbits == 4 && vbits == 4) kern = tq_compress_kv_mfma_kernel<4, 4, Dst>;
    else if (kbits == 3 && vbits == 3) kern = tq_compress_kv_mfma_kernel<3, 3, Dst>;
    else if (kbits == 2 && vbits == 2) kern = tq_compress_kv_mfma_kernel<2, 2, Dst>;
    else if (kbits == 8 && vbits == 8) kern = tq_compress_kv_mfma_kernel<8, 8, Dst>;
    else if (kbits == 4 && vbits == 2) kern = tq_compress_kv_mfma_kernel<4, 2, Dst>;
    else return false;
    hipLaunchKernelGGL(kern, dim3(mfma_grid_kv(ceil_div(rows, kTile), kWavesC)),
                       dim3(64 * kWavesC), 0, s, (const uint16_t*)kin, (const uint16_t*)vin, kp,
                       vp, kd, vd, rows);
    return true;
}

bool launch_dequant_kv(const TqPlanDev* kp, const TqPlanDev* vp, int kbits, int vbits,
                       const void* kpk, const void* knm, const void* vpk, const void* vnm,
                       void* kout, void* vout, int64_t rows, hipStream_t s) {
    if (!fhip_host::aligned16(kpk) || !fhip_host::aligned16(vpk) || !fhip_host::aligned16(kout) ||
        !fhip_host::aligned16(vout) || (((uintptr_t)knm) & 1u) || (((uintptr_t)vnm) & 1u))
        return false;
    auto kern = tq_dequant_kv_mfma_kernel<4, 4>;
    if (kbits == 4 && vbits == 4) kern = tq_dequant_kv_mfma_kernel<4, 4>;
    else if (kbits == 3 && vbits == 3) kern = tq_dequant_kv_mfma_kernel<3, 3>;
    else if (kbits == 2 && vbits == 2) kern = tq_dequant_kv_mfma_kernel<2, 2>;
    else if (kbits == 8 && vbits == 8) kern = tq_dequant_kv_mfma_kernel<8, 8>;
    else if (kbits == 4 && vbits == 2) kern = tq_dequant_kv_mfma_kernel<4, 2>;
    else return false;
    hipLaunchKernelGGL(kern, dim3(mfma_grid_kv(ceil_div(rows, kTile), kWavesD)),
                       dim3(64 * kWavesD), 0, s, (const uint8_t*)kpk, (const uint16_t*)knm,
                       (const uint8_t*)vpk, (const uint16_t*)vnm, kp, vp, (uint16_t*)kout,
                       (uint16_t*)vout, rows);
    return true;
}

}  // namespace

extern "C" {

int fhip_launch_turboquant_compress(const void* input, const float* rotation,
                                    const float* centroids, void* packed_out, void* norms_out,
                                    int num_tokens, int num_kv_heads, int head_dim, int n_levels,
                                    int bits, int packed_dim_per_head, fhip_stream_t stream) {
    if (num_tokens < 0 || num_kv_heads < 0 || head_dim <= 0 || head_dim > 8192 ||
        !tq_args_ok(n_levels, bits) ||
        packed_dim_per_head != (int)ceil_div((int64_t)head_dim * bits, 8))
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !rotation || !centroids || !packed_out || !norms_out) return hipErrorInvalidValue;
    FlatDst dst{(uint8_t*)packed_out, (uint16_t*)norms_out, packed_dim_per_head};
    return launch_compress<0>(input, rotation, centroids, n_levels, bits, dst, nullptr, rows,
                              head_dim, fhip_host::as_stream(stream));
}

}  // extern "C"

namespace fhip_internal {

int tq_rotate_rows(const void* input, const float* rotation, float* out, int64_t rows,
                   hipStream_t stream) {
    if (rows < 0 || !input || !rotation || !out || !fhip_host::aligned16(input) ||
        !fhip_host::aligned16(out))
        return hipErrorInvalidValue;
    FlatDst dst{nullptr, nullptr, 0};
    return launch_compress<2>(input, rotation, nullptr, 0, 8, dst, out, rows, kHd, stream);
}

int tq_rotate_back_rows(const float* input, const float* rotation, void* out, int64_t rows,
                        hipStream_t stream) {
    if (rows < 0 || !input || !rotation || !out || !fhip_host::aligned16(input) ||
        !fhip_host::aligned16(out))
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const int64_t need = ceil_div(ceil_div(rows, kTile), kWavesR);
    const int64_t cap = 2 * (int64_t)fhip_host::cu_count();
    hipLaunchKernelGGL(tq_rotate_back_kernel, dim3((unsigned)(need < cap ? need : cap)),
                       dim3(64 * kWavesR), 0, stream, input, rotation, (uint16_t*)out, rows);
    return hipGetLastError();
}

}  // namespace fhip_internal

extern "C" {

int fhip_launch_tq_rotate(const void* input, const float* rotation, float* y_out,
                          void* norms_out, int rows, int head_dim, fhip_stream_t stream) {
    if (rows < 0 || head_dim <= 0 || head_dim > 8192) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!input || !rotation || !y_out || !norms_out) return hipErrorInvalidValue;
    FlatDst dst{nullptr, (uint16_t*)norms_out, 0};
    return launch_compress<1>(input, rotation, nullptr, 0, 8, dst, y_out, rows, head_dim,
                              fhip_host::as_stream(stream));
}

int fhip_launch_tq_compress_pages(const void* input, const float* rotation,
                                  const float* centroids, int n_levels, int bits,
                                  void* packed_pool, void* norms_pool, int64_t page_packed_bytes,
                                  int64_t page_norm_bytes, const int32_t* page_ids, int num_pages,
                                  int first_pos, int num_tokens, int num_kv_heads, int head_dim,
                                  fhip_stream_t stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim > 8192 ||
        first_pos < 0 || num_pages < 0 || !tq_args_ok(n_levels, bits))
        return hipErrorInvalidValue;
    const int64_t pd = ceil_div((int64_t)head_dim * bits, 8);
    if (page_packed_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * pd ||
        page_norm_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * 2)
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !rotation || !centroids || !packed_pool || !norms_pool || !page_ids)
        return hipErrorInvalidValue;
    PageDst dst{(uint8_t*)packed_pool, (uint8_t*)norms_pool, page_packed_bytes, page_norm_bytes,
                page_ids, first_pos, num_kv_heads, num_pages, pd};
    return launch_compress<0>(input, rotation, centroids, n_levels, bits, dst, nullptr, rows,
                              head_dim, fhip_host::as_stream(stream));
}

int fhip_launch_tq_compress_page_ptrs(const void* input, const float* rotation,
                                      const float* centroids, int n_levels, int bits,
                                      void* const* packed_pages, void* const* norm_pages,
                                      const int32_t* page_ids, int num_pages, int first_pos,
                                      int num_tokens, int num_kv_heads, int head_dim,
                                      fhip_stream_t stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim > 8192 ||
        first_pos < 0 || num_pages < 0 || !tq_args_ok(n_levels, bits))
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !rotation || !centroids || !packed_pages || !norm_pages || !page_ids)
        return hipErrorInvalidValue;
    const int64_t pd = ceil_div((int64_t)head_dim * bits, 8);
    PtrPageDst dst{(uint8_t* const*)packed_pages, (uint8_t* const*)norm_pages, page_ids,
                   first_pos, num_kv_heads, num_pages, pd};
    return launch_compress<0>(input, rotation, centroids, n_levels, bits, dst, nullptr, rows,
                              head_dim, fhip_host::as_stream(stream));
}

int fhip_launch_tq_quantize_pack(const float* y, const float* centroids, int n_levels, int bits,
                                 void* packed_out, int rows, int head_dim,
                                 int packed_dim_per_head, fhip_stream_t stream) {
    if (rows < 0 || head_dim <= 0 || !tq_args_ok(n_levels, bits) ||
        packed_dim_per_head != (int)ceil_div((int64_t)head_dim * bits, 8))
        return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!y || !centroids || !packed_out) return hipErrorInvalidValue;
    const int64_t groups = (int64_t)rows * ((head_dim + 7) / 8);
    const int grid = tq_grid(ceil_div(groups, 256), 2048);
    hipLaunchKernelGGL(tq_quantize_pack_kernel, dim3(grid), dim3(256), 0,
                       fhip_host::as_stream(stream), y, centroids, n_levels, bits,
                       (uint8_t*)packed_out, (int64_t)rows, head_dim,
                       (int64_t)packed_dim_per_head);
    return hipGetLastError();
}

int fhip_launch_tq_dequant(const void* packed_in, const void* norms_in, const float* rotation,
                           const float* centroids, int n_levels, void* output, int num_tokens,
                           int num_kv_heads, int head_dim, int bits, int packed_dim_per_head,
                           fhip_stream_t stream) {
    if (num_tokens < 0 || num_kv_heads < 0 || head_dim <= 0 || head_dim > 8192 ||
        !tq_args_ok(n_levels, bits) ||
        packed_dim_per_head != (int)ceil_div((int64_t)head_dim * bits, 8))
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!packed_in || !norms_in || !rotation || !centroids || !output)
        return hipErrorInvalidValue;
    return launch_dequant(packed_in, norms_in, rotation, centroids, n_levels, output, rows,
                          head_dim, bits, packed_dim_per_head, fhip_host::as_stream(stream));
}

int fhip_launch_turboquant_decompress(const void* packed_in, const void* norms_in,
                                      const float* rotation, const float* centroids,
                                      void* output, int num_tokens, int num_kv_heads,
                                      int head_dim, int bits, int packed_dim_per_head,
                                      fhip_stream_t stream) {
    if (bits < 1 || bits > 8) return hipErrorInvalidValue;
    return fhip_launch_tq_dequant(packed_in, norms_in, rotation, centroids, 1 << bits, output,
                                  num_tokens, num_kv_heads, head_dim, bits, packed_dim_per_head,
                                  stream);
}

struct fhip_tq_plan {
    TqPlanDev* dev;
    int n_levels, bits, head_dim;
};

int fhip_tq_plan_create(const float* rotation, const float* centroids, int n_levels, int bits,
                        int head_dim, fhip_stream_t stream, fhip_tq_plan** out) {
    if (!out) return hipErrorInvalidValue;
    *out = nullptr;
    if (!rotation || !centroids || head_dim != kHd || !tq_args_ok(n_levels, bits))
        return hipErrorInvalidValue;
    TqPlanDev* dev = nullptr;
    hipError_t e = hipMalloc((void**)&dev, sizeof(TqPlanDev));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(tq_plan_kernel, dim3(1), dim3(kPlanThreads), 0,
                       fhip_host::as_stream(stream), rotation, centroids, n_levels, bits, dev);
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return e;
    }
    *out = new fhip_tq_plan{dev, n_levels, bits, head_dim};
    return hipSuccess;
}

void fhip_tq_plan_destroy(fhip_tq_plan* plan) {
    if (!plan) return;
    (void)hipFree(plan->dev);  // hipFree waits for work that may still use the plan
    delete plan;
}

int fhip_launch_tq_compress_planned(const fhip_tq_plan* plan, const void* input,
                                    void* packed_out, void* norms_out, int num_tokens,
                                    int num_kv_heads, fhip_stream_t stream) {
    if (!plan || num_tokens < 0 || num_kv_heads < 0) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !packed_out || !norms_out) return hipErrorInvalidValue;
    const int64_t pd = ceil_div((int64_t)plan->head_dim * plan->bits, 8);
    FlatDst dst{(uint8_t*)packed_out, (uint16_t*)norms_out, pd};
    const TqPlanDev* p = plan->dev;
    return launch_compress<0>(input, p->rot, p->cent, plan->n_levels, plan->bits, dst, nullptr,
                              rows, plan->head_dim, fhip_host::as_stream(stream), p);
}

int fhip_launch_tq_compress_pages_planned(const fhip_tq_plan* plan, const void* input,
                                          void* packed_pool, void* norms_pool,
                                          int64_t page_packed_bytes, int64_t page_norm_bytes,
                                          const int32_t* page_ids, int num_pages, int first_pos,
                                          int num_tokens, int num_kv_heads,
                                          fhip_stream_t stream) {
    if (!plan || num_tokens < 0 || num_kv_heads <= 0 || first_pos < 0 || num_pages < 0)
        return hipErrorInvalidValue;
    const int64_t pd = ceil_div((int64_t)plan->head_dim * plan->bits, 8);
    if (page_packed_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * pd ||
        page_norm_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * 2)
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !packed_pool || !norms_pool || !page_ids) return hipErrorInvalidValue;
    PageDst dst{(uint8_t*)packed_pool, (uint8_t*)norms_pool, page_packed_bytes, page_norm_bytes,
                page_ids, first_pos, num_kv_heads, num_pages, pd};
    const TqPlanDev* p = plan->dev;
    return launch_compress<0>(input, p->rot, p->cent, plan->n_levels, plan->bits, dst, nullptr,
                              rows, plan->head_dim, fhip_host::as_stream(stream), p);
}

int fhip_launch_tq_compress_page_ptrs_planned(const fhip_tq_plan* plan, const void* input,
                                              void* const* packed_pages,
                                              void* const* norm_pages, const int32_t* page_ids,
                                              int num_pages, int first_pos, int num_tokens,
                                              int num_kv_heads, fhip_stream_t stream) {
    if (!plan || num_tokens < 0 || num_kv_heads <= 0 || first_pos < 0 || num_pages < 0)
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!input || !packed_pages || !norm_pages || !page_ids) return hipErrorInvalidValue;
    const int64_t pd = ceil_div((int64_t)plan->head_dim * plan->bits, 8);
    PtrPageDst dst{(uint8_t* const*)packed_pages, (uint8_t* const*)norm_pages, page_ids,
                   first_pos, num_kv_heads, num_pages, pd};
    const TqPlanDev* p = plan->dev;
    return launch_compress<0>(input, p->rot, p->cent, plan->n_levels, plan->bits, dst, nullptr,
                              rows, plan->head_dim, fhip_host::as_stream(stream), p);
}

int fhip_launch_tq_dequant_planned(const fhip_tq_plan* plan, const void* packed_in,
                                   const void* norms_in, void* output, int num_tokens,
                                   int num_kv_heads, fhip_stream_t stream) {
    if (!plan || num_tokens < 0 || num_kv_heads < 0) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!packed_in || !norms_in || !output) return hipErrorInvalidValue;
    const int pd = (int)ceil_div((int64_t)plan->head_dim * plan->bits, 8);
    const TqPlanDev* p = plan->dev;
    return launch_dequant(packed_in, norms_in, p->rot, p->cent, plan->n_levels, output, rows,
                          plan->head_dim, plan->bits, pd, fhip_host::as_stream(stream), p);
}

// K+V entries: one launch for a layer's keys and values (plans of head_dim 128), falling back
// to one launch per tensor for width pairs without a K+V kernel.
int fhip_launch_tq_compress_kv_planned(const fhip_tq_plan* kplan, const fhip_tq_plan* vplan,
                                       const void* k_input, const void* v_input,
                                       void* k_packed_out, void* k_norms_out,
                                       void* v_packed_out, void* v_norms_out, int num_tokens,
                                       int num_kv_heads, fhip_stream_t stream) {
    if (!kplan || !vplan || num_tokens < 0 || num_kv_heads < 0) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!k_input || !v_input || !k_packed_out || !k_norms_out || !v_packed_out || !v_norms_out)
        return hipErrorInvalidValue;
    const hipStream_t s = fhip_host::as_stream(stream);
    const int64_t kpd = ceil_div((int64_t)kplan->head_dim * kplan->bits, 8);
    const int64_t vpd = ceil_div((int64_t)vplan->head_dim * vplan->bits, 8);
    FlatDst kd{(uint8_t*)k_packed_out, (uint16_t*)k_norms_out, kpd};
    FlatDst vd{(uint8_t*)v_packed_out, (uint16_t*)v_norms_out, vpd};
    if (kplan->head_dim == kHd && vplan->head_dim == kHd &&
        launch_compress_kv(kplan->dev, vplan->dev, kplan->bits, vplan->bits, k_input, v_input,
                           kd, vd, rows, s))
        return hipGetLastError();
    int r = fhip_launch_tq_compress_planned(kplan, k_input, k_packed_out, k_norms_out,
                                            num_tokens, num_kv_heads, stream);
    if (r) return r;
    return fhip_launch_tq_compress_planned(vplan, v_input, v_packed_out, v_norms_out,
                                           num_tokens, num_kv_heads, stream);
}

int fhip_launch_tq_compress_kv_page_ptrs_planned(
    const fhip_tq_plan* kplan, const fhip_tq_plan* vplan, const void* k_input,
    const void* v_input, void* const* k_packed_pages, void* const* k_norm_pages,
    void* const* v_packed_pages, void* const* v_norm_pages, const int32_t* page_ids,
    int num_pages, int first_pos, int num_tokens, int num_kv_heads, fhip_stream_t stream) {
    if (!kplan || !vplan || num_tokens < 0 || num_kv_heads <= 0 || first_pos < 0 ||
        num_pages < 0)
        return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!k_input || !v_input || !k_packed_pages || !k_norm_pages || !v_packed_pages ||
        !v_norm_pages || !page_ids)
        return hipErrorInvalidValue;
    const hipStream_t s = fhip_host::as_stream(stream);
    const int64_t kpd = ceil_div((int64_t)kplan->head_dim * kplan->bits, 8);
    const int64_t vpd = ceil_div((int64_t)vplan->head_dim * vplan->bits, 8);
    PtrPageDst kd{(uint8_t* const*)k_packed_pages, (uint8_t* const*)k_norm_pages, page_ids,
                  first_pos, num_kv_heads, num_pages, kpd};
    PtrPageDst vd{(uint8_t* const*)v_packed_pages, (uint8_t* const*)v_norm_pages, page_ids,
                  first_pos, num_kv_heads, num_pages, vpd};
    if (kplan->head_dim == kHd && vplan->head_dim == kHd &&
        launch_compress_kv(kplan->dev, vplan->dev, kplan->bits, vplan->bits, k_input, v_input,
                           kd, vd, rows, s))
        return hipGetLastError();
    int r = fhip_launch_tq_compress_page_ptrs_planned(kplan, k_input, k_packed_pages,
                                                      k_norm_pages, page_ids, num_pages,
                                                      first_pos, num_tokens, num_kv_heads, stream);
    if (r) return r;
    return fhip_launch_tq_compress_page_ptrs_planned(vplan, v_input, v_packed_pages,
                                                     v_norm_pages, page_ids, num_pages, first_pos,
                                                     num_tokens, num_kv_heads, stream);
}

int fhip_launch_tq_dequant_kv_planned(const fhip_tq_plan* kplan, const fhip_tq_plan* vplan,
                                      const void* k_packed_in, const void* k_norms_in,
                                      const void* v_packed_in, const void* v_norms_in,
                                      void* k_output, void* v_output, int num_tokens,
                                      int num_kv_heads, fhip_stream_t stream) {
    if (!kplan || !vplan || num_tokens < 0 || num_kv_heads < 0) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)num_tokens * num_kv_heads;
    if (rows == 0) return hipSuccess;
    if (!k_packed_in || !k_norms_in || !v_packed_in || !v_norms_in || !k_output || !v_output)
        return hipErrorInvalidValue;
    if (kplan->head_dim == kHd && vplan->head_dim == kHd &&
        launch_dequant_kv(kplan->dev, vplan->dev, kplan->bits, vplan->bits, k_packed_in,
                          k_norms_in, v_packed_in, v_norms_in, k_output, v_output, rows,
                          fhip_host::as_stream(stream)))
        return hipGetLastError();
    int r = fhip_launch_tq_dequant_planned(kplan, k_packed_in, k_norms_in, k_output, num_tokens,
                                           num_kv_heads, stream);
    if (r) return r;
    return fhip_launch_tq_dequant_planned(vplan, v_packed_in, v_norms_in, v_output, num_tokens,
                                          num_kv_heads, stream);
}

}  // extern "C"

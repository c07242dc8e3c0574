// TurboQuant KV compression for gfx950: rotate (MFMA), L2 norm, Lloyd-Max quantize,
// MSB-first bit-pack, page scatter, and dequantize (MFMA).
//
// Rotation cost. Compress and dequantize each multiply every 128-wide vector by a dense
// 128x128 fp32 rotation, 2*128*128 flops per vector: 17.2 GFLOP per direction for one layer
// of K+V at 32768 tokens x 8 heads, against ~160-170 MB of HBM traffic (~21 us). On the VALU
// that is >100 us, so the rotation runs on MFMA (v_mfma_f32_32x32x16_f16) with fp32 accuracy
// recovered by splitting the fp32 operand into fp16 hi + 2^12-scaled fp16 lo parts:
//   compress:   y_raw = Pi x = Pi_hi x + 2^-12 (Pi_lo' x)       x is the raw fp16 input,
//               exact as an fp16 operand; the norm is applied after the product by
//               linearity: y = y_raw / (||x|| + 1e-8).
//   dequantize: x_hat = Pi^T yhat = Pi_hi^T c_hi + 2^-12 (Pi_lo'^T c_hi + Pi_hi^T c_lo')
// Each representation error is ~2^-22 relative, the level of the fp32 sums themselves.
//
// Work mapping (head_dim 128): a 256-lane workgroup (4 waves) takes tiles of 32 vectors;
// wave w owns rotated coordinates [32w, 32w+32) and keeps its 32x128 slice of the rotation
// (hi and lo) in registers for the workgroup's lifetime. The tile is staged once in LDS and
// shared by the four waves. Other head dims use a per-vector VALU path that follows the
// reference kernel's arithmetic.
#include "tq_quant.h"

using namespace fhip;

namespace {

constexpr int kTile = 32;        // vectors per MFMA tile
constexpr int kHd = 128;         // head_dim of the MFMA path
constexpr int kXStride = 136;    // fp16 elements per LDS row (128 + 8 pad, conflict-free)
constexpr int kCStride = 132;    // bytes per LDS code row (128 + 4 pad)
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

struct CompressLds {
    uint16_t x[kTile * kXStride];
    float ssp[4][kTile];
    uint8_t codes[kTile * kCStride];
};

// Load the rotation slice of wave `wave` as MFMA A fragments, split hi/lo.
// kTranspose = false: A[i][k] = Pi[32w + i][k]   (compress: y = Pi x)
// kTranspose = true : A[i][k] = Pi[k][32w + i]   (dequantize: x = Pi^T y)
template <bool kTranspose>
__device__ __forceinline__ void load_rotation(const float* __restrict__ rot, int wave, int r,
                                              int h, f16x8 (&ahi)[8], f16x8 (&alo)[8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        float v[8];
        if constexpr (!kTranspose) {
            const float* p = rot + (32 * wave + r) * kHd + 16 * s + 8 * h;
            const f32x4 p0 = *(const f32x4*)p;
            const f32x4 p1 = *(const f32x4*)(p + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = p0[e];
                v[4 + e] = p1[e];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = rot[(16 * s + 8 * h + e) * kHd + 32 * wave + r];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const _Float16 hi = (_Float16)v[e];
            ahi[s][e] = hi;
            alo[s][e] = (_Float16)((v[e] - (float)hi) * kLoScale);
        }
    }
}

// ---------------------------------------------------------------------------------------
// MFMA compress / rotate, head_dim 128.
//   kMode 0: quantize + pack to Dst;  kMode 1: write fp32 y (and norms) for verification.
// ---------------------------------------------------------------------------------------
template <int kMode, class Dst>
__global__ __launch_bounds__(256) void tq_compress_mfma_kernel(
    const uint16_t* __restrict__ in, const float* __restrict__ rot,
    const float* __restrict__ cent, int L, int bits, Dst dst, float* __restrict__ y_out,
    int64_t rows) {
    __shared__ Quantizer qz;
    __shared__ CompressLds sh;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 31, h = lane >> 5;

    f16x8 ahi[8], alo[8];
    load_rotation<false>(rot, wave, r, h, ahi, alo);
    if constexpr (kMode == 0) quantizer_build(qz, cent, L);

    const int64_t ntiles = ceil_div(rows, kTile);
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * kTile;
        const int nvalid = (int)(rows - m0 < kTile ? rows - m0 : kTile);
        // Stage the 32 x 128 fp16 tile (8 KB): 16 lanes per row, 16 bytes each.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx >> 4, c16 = idx & 15;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (row < nvalid) v = ld16(in + (m0 + row) * kHd + c16 * 8);
            *(u32x4*)&sh.x[row * kXStride + c16 * 8] = v;
        }
        __syncthreads();

        f32x16 acc_hi = {}, acc_lo = {};
        float ssq = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 b = *(const f16x8*)&sh.x[r * kXStride + 16 * s + 8 * h];
            acc_hi = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[s], b, acc_hi, 0, 0, 0);
            acc_lo = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[s], b, acc_lo, 0, 0, 0);
            if ((s >> 1) == wave) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xe = (float)b[e];
                    ssq += xe * xe;
                }
            }
        }
        ssq += __shfl_xor(ssq, 32);
        if (h == 0) sh.ssp[wave][r] = ssq;
        __syncthreads();
        const float ss = sh.ssp[0][r] + sh.ssp[1][r] + sh.ssp[2][r] + sh.ssp[3][r];
        const float nrm = sqrtf(ss);
        const float inv = 1.0f / (nrm + 1e-8f);
        if (wave == 0 && h == 0 && r < nvalid) {
            uint16_t* np = dst.nptr(m0 + r);
            if (np) *np = (uint16_t)f2h(nrm);
        }
        // Lane (r, h) holds coordinates 32*wave + 8g + 4h + e of vector r.
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                y[e] = (acc_hi[4 * g + e] + acc_lo[4 * g + e] * kLoInv) * inv;
            const int i0 = 32 * wave + 8 * g + 4 * h;
            if constexpr (kMode == 1) {
                if (r < nvalid) {
                    f32x4 yv = {y[0], y[1], y[2], y[3]};
                    *(f32x4*)&y_out[(m0 + r) * kHd + i0] = yv;
                }
            } else {
                uint32_t word = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) word |= (uint32_t)quantize(qz, y[e]) << (8 * e);
                *(uint32_t*)&sh.codes[r * kCStride + i0] = word;
            }
        }
        if constexpr (kMode == 0) {
            __syncthreads();
            // Pack: 32 rows x 16 groups of 8 codes, 2 groups per lane; consecutive lanes
            // write consecutive bytes of the tile's packed rows.
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int idx = tid + 256 * i;
                const int row = idx >> 4, g = idx & 15;
                if (row < nvalid) {
                    uint8_t* prow = dst.prow(m0 + row);
                    if (prow) {
                        const uint32_t* cp = (const uint32_t*)&sh.codes[row * kCStride + 8 * g];
                        const uint32_t w0 = cp[0], w1 = cp[1];
                        int codes[8];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            codes[e] = (w0 >> (8 * e)) & 0xff;
                            codes[4 + e] = (w1 >> (8 * e)) & 0xff;
                        }
                        store_group(prow + g * bits, group_word(codes, bits), bits, bits);
                    }
                }
            }
        }
        __syncthreads();
    }
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
struct DequantLds {
    uint16_t chi[kMaxLevels], clo[kMaxLevels];
    uint16_t yhi[kTile * kXStride], ylo[kTile * kXStride];
};

__global__ __launch_bounds__(256) void tq_dequant_mfma_kernel(const uint8_t* __restrict__ packed,
                                                              const uint16_t* __restrict__ norms,
                                                              const float* __restrict__ rot,
                                                              const float* __restrict__ cent,
                                                              int L, int bits,
                                                              uint16_t* __restrict__ out,
                                                              int64_t rows, int64_t pd) {
    __shared__ DequantLds sh;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 31, h = lane >> 5;
    for (int i = tid; i < kMaxLevels; i += 256) {
        const float c = i < L ? cent[i] : 0.0f;
        const _Float16 hi = (_Float16)c;
        sh.chi[i] = __builtin_bit_cast(uint16_t, hi);
        sh.clo[i] = __builtin_bit_cast(uint16_t, (_Float16)((c - (float)hi) * kLoScale));
    }
    f16x8 ahi[8], alo[8];
    load_rotation<true>(rot, wave, r, h, ahi, alo);
    __syncthreads();
    const int64_t ntiles = ceil_div(rows, kTile);
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * kTile;
        const int nvalid = (int)(rows - m0 < kTile ? rows - m0 : kTile);
        // Decode 32 rows x 16 groups into fp16 hi/lo operand tiles, 2 groups per lane.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx >> 4, g = idx & 15;
            uint32_t whi[4] = {0u, 0u, 0u, 0u}, wlo[4] = {0u, 0u, 0u, 0u};
            if (row < nvalid) {
                int codes[8];
                load_group(packed + (m0 + row) * pd + (int64_t)g * bits, bits, bits, codes);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    whi[e] = (uint32_t)sh.chi[codes[2 * e]] | ((uint32_t)sh.chi[codes[2 * e + 1]] << 16);
                    wlo[e] = (uint32_t)sh.clo[codes[2 * e]] | ((uint32_t)sh.clo[codes[2 * e + 1]] << 16);
                }
            }
            u32x4 vh = {whi[0], whi[1], whi[2], whi[3]}, vl = {wlo[0], wlo[1], wlo[2], wlo[3]};
            *(u32x4*)&sh.yhi[row * kXStride + 8 * g] = vh;
            *(u32x4*)&sh.ylo[row * kXStride + 8 * g] = vl;
        }
        __syncthreads();
        f32x16 acc1 = {}, acc2 = {};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const f16x8 bh = *(const f16x8*)&sh.yhi[r * kXStride + 16 * s + 8 * h];
            const f16x8 bl = *(const f16x8*)&sh.ylo[r * kXStride + 16 * s + 8 * h];
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[s], bh, acc1, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[s], bh, acc2, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[s], bl, acc2, 0, 0, 0);
        }
        if (r < nvalid) {
            const float nrm = h2f(norms[m0 + r]);
            uint16_t* orow = out + (m0 + r) * kHd;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint32_t w[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float x0 = (acc1[4 * g + 2 * e] + acc2[4 * g + 2 * e] * kLoInv) * nrm;
                    const float x1 =
                        (acc1[4 * g + 2 * e + 1] + acc2[4 * g + 2 * e + 1] * kLoInv) * nrm;
                    w[e] = f2h(x0) | (f2h(x1) << 16);
                }
                u32x2 wv = {w[0], w[1]};
                *(u32x2*)&orow[32 * wave + 8 * g + 4 * h] = wv;
            }
        }
        __syncthreads();
    }
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

template <int kMode, class Dst>
int launch_compress(const void* input, const float* rot, const float* cent, int L, int bits,
                    Dst dst, float* y_out, int64_t rows, int hd, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (hd == kHd && fhip_host::aligned16(input) && fhip_host::aligned16(rot) &&
        (kMode == 0 || fhip_host::aligned16(y_out))) {
        const int grid = tq_grid(ceil_div(rows, kTile), 1024);
        hipLaunchKernelGGL((tq_compress_mfma_kernel<kMode, Dst>), dim3(grid), dim3(256), 0, s,
                           (const uint16_t*)input, rot, cent, L, bits, dst, y_out, rows);
    } else {
        const int grid = tq_grid(rows, 2048);
        const size_t lds = 2 * (size_t)hd * sizeof(float);
        hipLaunchKernelGGL((tq_compress_generic_kernel<kMode, Dst>), dim3(grid), dim3(256), lds,
                           s, (const uint16_t*)input, rot, cent, L, bits, dst, y_out, rows, hd);
    }
    return hipGetLastError();
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
    hipStream_t s = fhip_host::as_stream(stream);
    const int L = n_levels;
    if (head_dim == kHd && fhip_host::aligned16(output) && fhip_host::aligned16(rotation)) {
        const int grid = tq_grid(ceil_div(rows, kTile), 1024);
        hipLaunchKernelGGL(tq_dequant_mfma_kernel, dim3(grid), dim3(256), 0, s,
                           (const uint8_t*)packed_in, (const uint16_t*)norms_in, rotation,
                           centroids, L, bits, (uint16_t*)output, rows,
                           (int64_t)packed_dim_per_head);
    } else {
        const int grid = tq_grid(rows, 2048);
        hipLaunchKernelGGL(tq_dequant_generic_kernel, dim3(grid), dim3(256),
                           (size_t)head_dim * sizeof(float), s, (const uint8_t*)packed_in,
                           (const uint16_t*)norms_in, rotation, centroids, bits,
                           (uint16_t*)output, rows, head_dim, (int64_t)packed_dim_per_head);
    }
    return hipGetLastError();
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

}  // extern "C"

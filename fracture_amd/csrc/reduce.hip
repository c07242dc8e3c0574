// Row softmax and argmax over fp32 logits [rows, cols] for gfx950.
//
// The reference does both on the CPU after copying the logits to the host
// (crates/fracture-generate/src/sampling.rs:45-82, crates/fracture-engine/src/engine.rs:728-738).
// A 128,256-wide row is 513 KB, more than one CU's LDS, and a decode batch has few rows, so
// each row is split into 4096-element chunks, one workgroup per (chunk, row), which fills
// the chip. Pass 1 reduces each chunk to a record {max, sum exp(x - max), argmax, flags};
// pass 2 combines the row's records (every workgroup of a row in the same order, so all of
// them agree on the row max and sum) and writes exp(x/T - M) / S for its chunk, the second
// read being served mostly by the 256 MB MALL.
#include "fhip_common.h"

using namespace fhip;

namespace {

constexpr int kBlock = 256;
constexpr int kPerLane = 16;                  // 4 x 16-byte loads per lane
constexpr int kChunk = kBlock * kPerLane;     // 4096 elements per workgroup

struct alignas(16) RowPart {
    float m;         // chunk max of the scaled logits (-inf if none)
    float s;         // sum of exp(x - m) over the chunk
    float bv;        // largest value, ties to the last index
    int bi;          // its index (-1 if none)
    uint32_t flags;  // FHIP_ROW_HAS_NAN | FHIP_ROW_HAS_INF
    uint32_t pad[3];
};

int num_chunks(int cols) { return (int)ceil_div(cols, kChunk); }

// (value, index) order of the greedy sampler: larger value wins, equal values go to the
// larger index (Iterator::max_by keeps the last maximum); NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i > bi);
}

__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
}

template <bool kVec>
__device__ __forceinline__ void load_chunk(const float* row, int cols, int base, float T,
                                           float (&v)[kPerLane], bool (&ok)[kPerLane]) {
#pragma unroll
    for (int u = 0; u < kPerLane / 4; ++u) {
        const int e0 = base + u * (kBlock * 4) + threadIdx.x * 4;
        if constexpr (kVec) {
            if (e0 + 3 < cols) {
                const u32x4 w = ld16(row + e0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[4 * u + i] = __uint_as_float(w[i]) / T;
                    ok[4 * u + i] = true;
                }
                continue;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = e0 + i;
            ok[4 * u + i] = e < cols;
            v[4 * u + i] = e < cols ? row[e] / T : 0.0f;
        }
    }
}

// Pass 1: one RowPart per (chunk, row).
template <bool kVec>
__global__ __launch_bounds__(kBlock) void row_partials_kernel(const float* __restrict__ logits,
                                                              int cols, float T,
                                                              RowPart* __restrict__ parts) {
    __shared__ float sm[4], ss[4], sbv[4];
    __shared__ int sbi[4];
    __shared__ uint32_t sfl[4];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const int base = chunk * kChunk;
    const float* r = logits + (int64_t)row * cols;
    float v[kPerLane];
    bool ok[kPerLane];
    load_chunk<kVec>(r, cols, base, T, v, ok);

    float m = -__builtin_inff(), bv = -__builtin_inff();
    int bi = -1;
    uint32_t fl = 0;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        if (!ok[j]) continue;
        const float x = v[j];
        const int idx = base + (j / 4) * (kBlock * 4) + threadIdx.x * 4 + (j & 3);
        m = fmaxf(m, x);
        if (x != x) fl |= FHIP_ROW_HAS_NAN;
        if (__builtin_isinf(x)) fl |= FHIP_ROW_HAS_INF;
        if (better(x, idx, bv, bi)) {
            bv = x;
            bi = idx;
        }
    }
    float s = 0.0f;
    if (m != -__builtin_inff()) {
#pragma unroll
        for (int j = 0; j < kPerLane; ++j)
            if (ok[j]) s += expf(v[j] - m);
    }
    // wave combine
    const float mw = wave_max(m);
    const float sw = wave_sum(mw == -__builtin_inff() || m == -__builtin_inff()
                                  ? 0.0f
                                  : s * expf(m - mw));
    wave_argmax(bv, bi);
    const uint32_t any_nan = __ballot(fl & FHIP_ROW_HAS_NAN) != 0 ? FHIP_ROW_HAS_NAN : 0u;
    const uint32_t any_inf = __ballot(fl & FHIP_ROW_HAS_INF) != 0 ? FHIP_ROW_HAS_INF : 0u;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sm[wave] = mw;
        ss[wave] = sw;
        sbv[wave] = bv;
        sbi[wave] = bi;
        sfl[wave] = any_nan | any_inf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float M = sm[0];
        for (int w = 1; w < kBlock / 64; ++w) M = fmaxf(M, sm[w]);
        float S = 0.0f, BV = sbv[0];
        int BI = sbi[0];
        uint32_t F = sfl[0];
        for (int w = 0; w < kBlock / 64; ++w) {
            if (sm[w] != -__builtin_inff()) S += ss[w] * expf(sm[w] - M);
            if (w > 0) {
                if (better(sbv[w], sbi[w], BV, BI)) {
                    BV = sbv[w];
                    BI = sbi[w];
                }
                F |= sfl[w];
            }
        }
        RowPart p;
        p.m = M;
        p.s = S;
        p.bv = BV;
        p.bi = BI;
        p.flags = F;
        p.pad[0] = p.pad[1] = p.pad[2] = 0;
        parts[(int64_t)row * gridDim.x + chunk] = p;
    }
}

// Combine a row's records in chunk order (identical in every workgroup of the row).
__device__ __forceinline__ void combine_row(const RowPart* __restrict__ parts, int nchunks,
                                            float& M, float& S) {
    M = -__builtin_inff();
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, parts[c].m);
    S = 0.0f;
    for (int c = 0; c < nchunks; ++c)
        if (parts[c].m != -__builtin_inff()) S += parts[c].s * expf(parts[c].m - M);
}

__device__ __forceinline__ void argmax_row(const RowPart* __restrict__ parts, int nchunks,
                                           int32_t* index_out, uint32_t* flags_out) {
    float BV = parts[0].bv;
    int BI = parts[0].bi;
    uint32_t F = parts[0].flags;
    for (int c = 1; c < nchunks; ++c) {
        if (better(parts[c].bv, parts[c].bi, BV, BI)) {
            BV = parts[c].bv;
            BI = parts[c].bi;
        }
        F |= parts[c].flags;
    }
    *index_out = BI;
    *flags_out = F;
}

// Pass 2: probabilities for one (chunk, row); chunk 0 also writes the row's argmax.
template <bool kVec>
__global__ __launch_bounds__(kBlock) void softmax_write_kernel(
    const float* __restrict__ logits, float* __restrict__ probs, int cols, float T,
    const RowPart* __restrict__ parts, int32_t* __restrict__ index_out,
    uint32_t* __restrict__ flags_out) {
    __shared__ float sMS[2];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const RowPart* rp = parts + (int64_t)row * gridDim.x;
    if (threadIdx.x == 0) {
        float M, S;
        combine_row(rp, gridDim.x, M, S);
        sMS[0] = M;
        sMS[1] = S;
        if (chunk == 0 && index_out) argmax_row(rp, gridDim.x, index_out + row, flags_out + row);
    }
    const int base = chunk * kChunk;
    const float* r = logits + (int64_t)row * cols;
    float v[kPerLane];
    bool ok[kPerLane];
    load_chunk<kVec>(r, cols, base, T, v, ok);
    __syncthreads();
    const float M = sMS[0], S = sMS[1];
    float* o = probs + (int64_t)row * cols;
#pragma unroll
    for (int u = 0; u < kPerLane / 4; ++u) {
        const int e0 = base + u * (kBlock * 4) + threadIdx.x * 4;
        if (kVec && e0 + 3 < cols) {
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(expf(v[4 * u + i] - M) / S);
            st16_stream(o + e0, w);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (ok[4 * u + i]) o[e0 + i] = expf(v[4 * u + i] - M) / S;
        }
    }
}

// Argmax only: one lane per row folds the row's records.
__global__ __launch_bounds__(kBlock) void argmax_finalize_kernel(const RowPart* __restrict__ parts,
                                                                 int rows, int nchunks,
                                                                 int32_t* __restrict__ index_out,
                                                                 uint32_t* __restrict__ flags_out) {
    const int row = blockIdx.x * kBlock + threadIdx.x;
    if (row < rows)
        argmax_row(parts + (int64_t)row * nchunks, nchunks, index_out + row, flags_out + row);
}

int check_rows(const float* logits, int rows, int cols, void* ws) {
    if (rows < 0 || cols <= 0 || rows > 65535) return hipErrorInvalidValue;
    if (rows > 0 && (!logits || !ws)) return hipErrorInvalidValue;
    return hipSuccess;
}

int launch_partials(const float* logits, int rows, int cols, float T, RowPart* parts,
                    hipStream_t s, bool& vec) {
    vec = cols % 4 == 0 && fhip_host::aligned16(logits);
    dim3 grid(num_chunks(cols), rows);
    if (vec)
        hipLaunchKernelGGL(row_partials_kernel<true>, grid, dim3(kBlock), 0, s, logits, cols, T,
                           parts);
    else
        hipLaunchKernelGGL(row_partials_kernel<false>, grid, dim3(kBlock), 0, s, logits, cols, T,
                           parts);
    return hipGetLastError();
}

}  // namespace

extern "C" {

size_t fhip_rows_workspace_bytes(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    return (size_t)rows * num_chunks(cols) * sizeof(RowPart);
}

int fhip_launch_softmax_argmax_rows(const float* logits, float* probs, int32_t* index_out,
                                    uint32_t* flags_out, int rows, int cols, float temperature,
                                    void* workspace, fhip_stream_t stream) {
    int e = check_rows(logits, rows, cols, workspace);
    if (e != hipSuccess) return e;
    if (rows > 0 && !probs) return hipErrorInvalidValue;
    if ((index_out == nullptr) != (flags_out == nullptr)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    hipStream_t s = fhip_host::as_stream(stream);
    RowPart* parts = (RowPart*)workspace;
    bool vec;
    e = launch_partials(logits, rows, cols, temperature, parts, s, vec);
    if (e != hipSuccess) return e;
    vec = vec && fhip_host::aligned16(probs);
    dim3 grid(num_chunks(cols), rows);
    if (vec)
        hipLaunchKernelGGL(softmax_write_kernel<true>, grid, dim3(kBlock), 0, s, logits, probs,
                           cols, temperature, parts, index_out, flags_out);
    else
        hipLaunchKernelGGL(softmax_write_kernel<false>, grid, dim3(kBlock), 0, s, logits, probs,
                           cols, temperature, parts, index_out, flags_out);
    return hipGetLastError();
}

int fhip_launch_softmax_rows(const float* logits, float* probs, int rows, int cols,
                             float temperature, void* workspace, fhip_stream_t stream) {
    return fhip_launch_softmax_argmax_rows(logits, probs, nullptr, nullptr, rows, cols,
                                           temperature, workspace, stream);
}

int fhip_launch_argmax_rows(const float* logits, int32_t* index_out, uint32_t* flags_out,
                            int rows, int cols, void* workspace, fhip_stream_t stream) {
    int e = check_rows(logits, rows, cols, workspace);
    if (e != hipSuccess) return e;
    if (rows > 0 && (!index_out || !flags_out)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    hipStream_t s = fhip_host::as_stream(stream);
    RowPart* parts = (RowPart*)workspace;
    bool vec;
    e = launch_partials(logits, rows, cols, 1.0f, parts, s, vec);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)ceil_div(rows, kBlock)),
                       dim3(kBlock), 0, s, parts, rows, num_chunks(cols), index_out, flags_out);
    return hipGetLastError();
}

}  // extern "C"

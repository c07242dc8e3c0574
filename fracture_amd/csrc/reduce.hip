// Row softmax and argmax over fp32 logits [rows, cols] for gfx950.
//
// The reference does both on the CPU after copying the logits to the host
// (crates/fracture-generate/src/sampling.rs:45-82, crates/fracture-engine/src/engine.rs:728-738).
// A 128,256-wide row is 513 KB, more than one CU's LDS, and a decode batch has few rows, so
// each row is split into 4096-element chunks, one workgroup per (chunk, row), which fills
// the chip with one wave of loads.
//
// Pass 1 (row_stats_kernel) reduces each chunk to a record {max, sum exp(x - max), argmax,
// flags}. argmax then folds each row's records with one wave per row (argmax_fold_kernel);
// softmax reads the logits again in softmax_write_kernel (each XCD in the reverse of pass 1's
// order, which measured faster), where
// every workgroup of a row folds the row's records in the same fixed order (so all agree on
// the row's max and sum) while its logits loads are in flight, and writes exp(x/T - M) / S.
// No atomics or cross-workgroup fences: a device-scope fence on gfx9 writes back the L2.
//
// exp is evaluated as exp2((s - m) * log2(e)) on the hardware exp2; over the logit range of a
// sampler (|s - m| < 100) that is within 1e-5 relative of expf.
#include "fhip_common.h"

using namespace fhip;

namespace {

constexpr int kBlock = 256;
constexpr int kPerLane = 16;                  // 4 x 16-byte loads per lane
constexpr int kChunk = kBlock * kPerLane;     // 4096 elements per workgroup
constexpr float kLog2e = 1.4426950408889634f;

enum : int { kStatsSoftmax = 1, kStatsArgmax = 2 };

struct alignas(16) RowPart {
    float m;         // chunk max of the scaled logits (-inf if none)
    float s;         // sum of exp(s - m) over the chunk
    float bv;        // largest raw logit, ties to the last index
    int bi;          // its index (-1 if none)
    uint32_t flags;  // FHIP_ROW_HAS_NAN | FHIP_ROW_HAS_INF
    uint32_t pad[3];
};

// Workspace: RowPart[rows][nchunks].
int num_chunks(int cols) { return (int)ceil_div(cols, kChunk); }

// (value, index) order of the greedy sampler: larger value wins, equal values go to the
// larger index (Iterator::max_by keeps the last maximum); NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i > bi);
}

// Wave argmax of per-lane (value, index) pairs under better(): the largest value, then the
// largest index among the lanes that hold it. Lanes without a candidate hold (-inf, -1).
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
    const float wm = wave_max(bv);
    bi = wave_max_int(bv == wm ? bi : -1);
    bv = wm;
}

// exp(s - m) for the softmax; s == m gives exactly 1.
__device__ __forceinline__ float exp_diff(float s, float m) {
    return __builtin_amdgcn_exp2f((s - m) * kLog2e);
}

// Wave combine of per-lane (max, sum-of-exp) pairs.
__device__ __forceinline__ void wave_softmax_pair(float& m, float& s) {
    const float mw = wave_max(m);
    const float part = (m == -__builtin_inff()) ? 0.0f : s * exp_diff(m, mw);
    s = wave_sum(part);
    m = mw;
}

// This lane's kPerLane elements of the chunk at base (element j at elem_index(base, j)).
// Positions past the row's end read the row's last element or vector instead (every caller
// ignores them), so the loads carry no branches and are all in flight at once: a guarded
// load makes the compiler wait for the previous one before it. kVec: cols % 4 == 0.
template <bool kVec>
__device__ __forceinline__ void load_chunk(const float* row, int cols, int base,
                                           float (&v)[kPerLane]) {
#pragma unroll
    for (int u = 0; u < kPerLane / 4; ++u) {
        const int e0 = base + u * (kBlock * 4) + threadIdx.x * 4;
        if constexpr (kVec) {
            const u32x4 w = ld16(row + min(e0, cols - 4));
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * u + i] = __uint_as_float(w[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * u + i] = row[min(e0 + i, cols - 1)];
        }
    }
}

__device__ __forceinline__ int elem_index(int base, int j) {
    return base + (j / 4) * (kBlock * 4) + threadIdx.x * 4 + (j & 3);
}

// One lane's pass over its chunk elements: non-finite screen (nf), running max of x * inv_t
// (m), and the argmax (bv, bi). The lane visits its indices in increasing order, so `>=`
// keeps the last maximum. kFull: the whole chunk lies inside the row. Selects rather than
// branches keep this straight-line code.
template <int kMode, bool kFull>
__device__ __forceinline__ void scan_lane(const float (&v)[kPerLane], int base, int nvalid,
                                          float inv_t, float& nf, float& m, float& bv, int& bi) {
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
        const int idx = elem_index(base, j);
        const bool ok = kFull || idx - base < nvalid;
        const float x = v[j];
        nf = ok ? fmaf(x, 0.0f, nf) : nf;
        if constexpr (kMode & kStatsArgmax) {
            const bool t = ok && x >= bv;
            bv = t ? x : bv;
            bi = t ? idx : bi;
        }
        if constexpr (kMode & kStatsSoftmax) m = ok ? fmaxf(m, x * inv_t) : m;
    }
}

// Pass 1. kMode: kStatsSoftmax and/or kStatsArgmax.
template <int kMode, bool kVec>
__global__ __launch_bounds__(kBlock) void row_stats_kernel(const float* __restrict__ logits,
                                                           int cols, float inv_t,
                                                           RowPart* __restrict__ parts) {
    __shared__ float sm[4], ss[4], sbv[4];
    __shared__ int sbi[4];
    __shared__ uint32_t sfl[4];
    const int chunk = blockIdx.x, row = blockIdx.y, nchunks = gridDim.x;
    const int base = chunk * kChunk;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* r = logits + (int64_t)row * cols;
    float v[kPerLane];
    load_chunk<kVec>(r, cols, base, v);
    const int nvalid = cols - base;  // elements of this chunk: indices base .. base + nvalid-1

    // Non-finite screen: x * 0 is NaN exactly for NaN and +-inf.
    float nf = 0.0f;
    float m = -__builtin_inff(), s = 0.0f, bv = -__builtin_inff();
    int bi = -1;
    const bool full = nvalid >= kChunk;  // uniform: only a row's last chunk can be partial
    if (full)
        scan_lane<kMode, true>(v, base, nvalid, inv_t, nf, m, bv, bi);
    else
        scan_lane<kMode, false>(v, base, nvalid, inv_t, nf, m, bv, bi);
    if constexpr (kMode & kStatsSoftmax) {
        if (m != -__builtin_inff()) {
#pragma unroll
            for (int j = 0; j < kPerLane; ++j) {
                const float e = exp_diff(v[j] * inv_t, m);
                s += (full || elem_index(base, j) - base < nvalid) ? e : 0.0f;
            }
        }
    }
    uint32_t fl = 0;
    if (nf != nf) {  // rare: classify exactly
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            if (elem_index(base, j) - base >= nvalid) continue;
            const float x = v[j];
            if (x != x) fl |= FHIP_ROW_HAS_NAN;
            if (__builtin_isinf(x)) fl |= FHIP_ROW_HAS_INF;
        }
    }
    if constexpr (kMode & kStatsSoftmax) wave_softmax_pair(m, s);
    if constexpr (kMode & kStatsArgmax) wave_argmax(bv, bi);  // NaN never enters bv
    const uint32_t any_nan = __ballot(fl & FHIP_ROW_HAS_NAN) != 0 ? FHIP_ROW_HAS_NAN : 0u;
    const uint32_t any_inf = __ballot(fl & FHIP_ROW_HAS_INF) != 0 ? FHIP_ROW_HAS_INF : 0u;
    if (lane == 0) {
        sm[wave] = m;
        ss[wave] = s;
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
            if (sm[w] != -__builtin_inff()) S += ss[w] * exp_diff(sm[w], M);
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
        parts[(int64_t)row * nchunks + chunk] = p;
    }
}

// Fold one row's records on one wave (chunk c on lane c mod 64, a fixed order, so every
// caller of the same row gets the same M and S).
template <int kMode>
__device__ __forceinline__ void fold_row(const RowPart* __restrict__ rp, int nchunks, float& M,
                                         float& S, float& BV, int& BI, uint32_t& F) {
    const int lane = threadIdx.x & 63;
    M = -__builtin_inff();
    S = 0.0f;
    BV = -__builtin_inff();
    BI = -1;
    uint32_t fl = 0;
    for (int c = lane; c < nchunks; c += 64) {
        const RowPart p = rp[c];
        fl |= p.flags;
        if constexpr (kMode & kStatsArgmax) {
            if (better(p.bv, p.bi, BV, BI)) {
                BV = p.bv;
                BI = p.bi;
            }
        }
        if constexpr (kMode & kStatsSoftmax) {
            if (p.m != -__builtin_inff()) {
                const float mn = fmaxf(M, p.m);
                S = (M == -__builtin_inff() ? 0.0f : S * exp_diff(M, mn)) +
                    p.s * exp_diff(p.m, mn);
                M = mn;
            }
        }
    }
    if constexpr (kMode & kStatsSoftmax) wave_softmax_pair(M, S);
    if constexpr (kMode & kStatsArgmax) wave_argmax(BV, BI);
    const uint32_t fn = __ballot(fl & FHIP_ROW_HAS_NAN) != 0 ? FHIP_ROW_HAS_NAN : 0u;
    const uint32_t fi = __ballot(fl & FHIP_ROW_HAS_INF) != 0 ? FHIP_ROW_HAS_INF : 0u;
    F = fn | fi;
}

// argmax pass 2: one wave per row.
__global__ __launch_bounds__(kBlock) void argmax_fold_kernel(const RowPart* __restrict__ parts,
                                                             int rows, int nchunks,
                                                             int32_t* __restrict__ index_out,
                                                             uint32_t* __restrict__ flags_out) {
    const int row = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    float M, S, BV;
    int BI;
    uint32_t F;
    fold_row<kStatsArgmax>(parts + (int64_t)row * nchunks, nchunks, M, S, BV, BI, F);
    if ((threadIdx.x & 63) == 0) {
        index_out[row] = BI;
        flags_out[row] = F;
    }
}

// Pass 2: probabilities for one (chunk, row); chunk 0 also writes the row's argmax.
template <int kMode, bool kVec>
__global__ __launch_bounds__(kBlock) void softmax_write_kernel(
    const float* __restrict__ logits, float* __restrict__ probs, int cols, float inv_t,
    const RowPart* __restrict__ parts, int32_t* __restrict__ index_out,
    uint32_t* __restrict__ flags_out) {
    __shared__ float sMS[2];
    // Pass 1 ran workgroup w (w = chunk + nchunks row) on XCD w % 8, in order of w. Here each
    // XCD takes the same chunks in the reverse order, so its re-reads start with the lines pass
    // 1 read last. Measured at [64, 128256] fp32: 15.6 -> 13.6 us, with the same L2 miss bytes
    // (FETCH_SIZE), so the gain is in how fast the misses are served, not in L2 hits.
    const int nchunks = gridDim.x;
    const int w = blockIdx.x + blockIdx.y * nchunks, nw = nchunks * gridDim.y;
    const int pw = nw % 8 == 0 ? (nw / 8 - 1 - w / 8) * 8 + w % 8 : w;
    const int chunk = pw % nchunks, row = pw / nchunks;
    const int base = chunk * kChunk;
    const float* r = logits + (int64_t)row * cols;
    float v[kPerLane];
    load_chunk<kVec>(r, cols, base, v);
    if (threadIdx.x < 64) {
        float M, S, BV;
        int BI;
        uint32_t F;
        fold_row<kMode>(parts + (int64_t)row * nchunks, nchunks, M, S, BV, BI, F);
        if (threadIdx.x == 0) {
            sMS[0] = M;
            sMS[1] = 1.0f / S;
            if constexpr (kMode & kStatsArgmax) {
                if (chunk == 0) {
                    index_out[row] = BI;
                    flags_out[row] = F;
                }
            }
        }
    }
    __syncthreads();
    const float M = sMS[0], invS = sMS[1];
    float* o = probs + (int64_t)row * cols;
#pragma unroll
    for (int u = 0; u < kPerLane / 4; ++u) {
        const int e0 = base + u * (kBlock * 4) + threadIdx.x * 4;
        if (kVec && e0 + 3 < cols) {
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = __float_as_uint(exp_diff(v[4 * u + i] * inv_t, M) * invS);
            st16_stream(o + e0, w);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (e0 + i < cols) o[e0 + i] = exp_diff(v[4 * u + i] * inv_t, M) * invS;
        }
    }
}

int check_rows(const float* logits, int rows, int cols, void* ws) {
    if (rows < 0 || cols <= 0 || rows > 65535) return hipErrorInvalidValue;
    if (rows > 0 && (!logits || !ws)) return hipErrorInvalidValue;
    return hipSuccess;
}

template <int kMode>
int launch_stats(const float* logits, int rows, int cols, float inv_t, RowPart* parts,
                 hipStream_t s) {
    const bool vec = cols % 4 == 0 && fhip_host::aligned16(logits);
    dim3 grid(num_chunks(cols), rows);
    if (vec)
        hipLaunchKernelGGL((row_stats_kernel<kMode, true>), grid, dim3(kBlock), 0, s, logits, cols,
                           inv_t, parts);
    else
        hipLaunchKernelGGL((row_stats_kernel<kMode, false>), grid, dim3(kBlock), 0, s, logits,
                           cols, inv_t, parts);
    return hipGetLastError();
}

template <int kMode>
void launch_write(const float* logits, float* probs, int rows, int cols, float inv_t,
                  const RowPart* parts, int32_t* index_out, uint32_t* flags_out, hipStream_t s) {
    const bool vec = cols % 4 == 0 && fhip_host::aligned16(logits) && fhip_host::aligned16(probs);
    dim3 grid(num_chunks(cols), rows);
    if (vec)
        hipLaunchKernelGGL((softmax_write_kernel<kMode, true>), grid, dim3(kBlock), 0, s, logits,
                           probs, cols, inv_t, parts, index_out, flags_out);
    else
        hipLaunchKernelGGL((softmax_write_kernel<kMode, false>), grid, dim3(kBlock), 0, s, logits,
                           probs, cols, inv_t, parts, index_out, flags_out);
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
    const float inv_t = 1.0f / temperature;
    if (index_out) {
        e = launch_stats<kStatsSoftmax | kStatsArgmax>(logits, rows, cols, inv_t, parts, s);
        if (e != hipSuccess) return e;
        launch_write<kStatsSoftmax | kStatsArgmax>(logits, probs, rows, cols, inv_t, parts,
                                                   index_out, flags_out, s);
    } else {
        e = launch_stats<kStatsSoftmax>(logits, rows, cols, inv_t, parts, s);
        if (e != hipSuccess) return e;
        launch_write<kStatsSoftmax>(logits, probs, rows, cols, inv_t, parts, nullptr, nullptr, s);
    }
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
    e = launch_stats<kStatsArgmax>(logits, rows, cols, 1.0f, parts, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_fold_kernel, dim3((unsigned)ceil_div(rows, kBlock / 64)),
                       dim3(kBlock), 0, s, parts, rows, num_chunks(cols), index_out, flags_out);
    return hipGetLastError();
}

}  // extern "C"

// TurboQuant scalar quantizer and bit packer, shared by the compress, quantize-pack and
// page-writer kernels.
//
// Reference semantics (turboquant_compress.cu:120-130): the code of a coordinate y is the
// FIRST index i minimising fabsf(y - c[i]) in fp32, scanning i = 0..L-1 with a strict `<`.
// A linear scan costs ~5 VALU ops per level, which at 4 bits is several times the HBM time
// of the whole compress. This quantizer returns the same index in ~7 ops and one LDS read:
//
//  * With sorted, distinct, finite centroids, d_i(y) = |fl(y - c_i)| is non-increasing in i
//    while c_i <= y and non-decreasing once c_i > y (fl() is monotone). If, in addition,
//    |y| + max|c| <= min_gap * 2^20, two different exact differences never round to the
//    same float, so the decreasing part is strict and the first minimum equals
//    #{q : d_q(y) > d_{q+1}(y)}.
//  * Each predicate P_q(y) = d_q(y) > d_{q+1}(y) is monotone in y, so it equals y > t_q for
//    an exact float threshold t_q, found by bisection over the float ordering.
//  * A bucket map j(y) = clamp(int(fma(y, s, o))) is monotone, so thresholds in lower
//    buckets are < y and in higher buckets > y; with at most one threshold per bucket,
//    code = base[j] + (y > t[j]). J = 2L buckets span the thresholds (at least 16): for the
//    Lloyd-Max codebooks of 2-8 bits no bucket then holds two. With at most 256 buckets the
//    map is one saturating float-to-byte conversion (v_cvt_pk_u8_f32: round, clamp to
//    [0, 255], NaN to 0) over a table of 256 entries; larger tables clamp, then truncate.
//    At 4 bits the 32 entries of 8 bytes cover the 64 LDS banks once, so the lanes of a
//    lookup never conflict.
//  Anything outside those conditions (NaN, +-inf, huge |y|, unsorted or repeated centroids,
//  a bucket holding two thresholds) takes the reference's linear scan.
#pragma once

#include "fhip_common.h"

namespace fhip {

constexpr int kMaxLevels = 256;
constexpr int kMaxBuckets = 1024;

struct alignas(16) Quantizer {
    float c[kMaxLevels];             // centroids
    float t[kMaxLevels];             // exact thresholds t_q, q < L-1
    int jt[kMaxLevels];              // bucket of t_q
    float2 ent[kMaxBuckets];         // {threshold in bucket or +inf, base count (int bits)}
    float ybound, scale, offset, jmax;
    int L, J;
    int unit_fast;  // quantize_unit is exact for every |y| <= 4 and for NaN
    float red_f[2][16];
    int red_i[16];
};

__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ofloat(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Thresholds. t_q is the largest float y in [c_q, c_q+1) with
// fabsf(y - c_q) <= fabsf(y - c_q+1): the predicate is monotone in y, so order keys (floats
// mapped to monotone unsigned integers) can be searched.
// The threshold found by a whole wave (c0, c1 uniform; every lane returns it): each
// round tests 64 evenly spaced order keys between a key where the predicate holds (lo) and
// one where it fails (hi) and keeps the crossing, so about 6 rounds replace the 32 serial
// steps of the bisection. Used for the pairs the short walk cannot settle, e.g. c0 = -c1,
// whose fp32 midpoint 0 lies ~2^30 keys below the threshold.
__device__ inline float exact_threshold_wave(float c0, float c1) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t lo = okey(c0), hi = okey(c1);  // P(lo) holds, P(hi) fails
    while (hi - lo > 1u) {
        const uint32_t span = hi - lo;
        // lane l tests lo + ceil(span (l + 1) / 64): increasing in l, lane 63 tests hi
        const uint32_t k = lo + (uint32_t)(((uint64_t)span * (lane + 1u) + 63u) >> 6);
        const float y = ofloat(k);
        const bool p = k < hi && fabsf(y - c0) <= fabsf(y - c1);
        const uint64_t m = __ballot(p);
        // P is monotone in the key: lanes [0, n) hold, lanes [n, 64) fail
        const int n = m == 0 ? 0 : 64 - __builtin_clzll(m);
        const uint32_t nlo = n == 0 ? lo : __builtin_amdgcn_readlane(k, n - 1);
        const uint32_t nhi = n == 64 ? hi : __builtin_amdgcn_readlane(k, n);
        lo = nlo;
        hi = nhi;
    }
    return ofloat(lo);
}

// Short walk from the fp32 midpoint (the threshold is within a step of it except for
// pairs like c0 = -c1); NaN when it does not settle within 4 steps.
__device__ inline float threshold_walk4(float c0, float c1) {
    const float m = c0 + 0.5f * (c1 - c0);
    if (!(m > c0 && m < c1)) return __builtin_nanf("");
    uint32_t k = okey(m);
    const bool up = fabsf(m - c0) <= fabsf(m - c1);
#pragma unroll 1
    for (int it = 0; it < 4; ++it) {
        if (up) {  // P(k) holds: advance while P(k + 1) holds
            const float n = ofloat(k + 1u);
            if (!(n < c1) || fabsf(n - c0) > fabsf(n - c1)) return ofloat(k);
            ++k;
        } else {  // P(k) fails: step down until it holds
            --k;
            const float n = ofloat(k);
            if (!(n > c0) || fabsf(n - c0) <= fabsf(n - c1)) return n > c0 ? n : c0;
        }
    }
    return __builtin_nanf("");
}

constexpr int kBucketsU8 = 256;  // tables of at most this many buckets use bucket_u8
__device__ __forceinline__ int bucket_u8(float jf) {
    return (int)__builtin_amdgcn_cvt_pk_u8_f32(jf, 0u, 0u);
}
__device__ __forceinline__ int bucket_wide(float jf, float jmax) {
    return (int)__builtin_amdgcn_fmed3f(jf, 0.0f, jmax);
}
__device__ __forceinline__ int bucket_of(const Quantizer& q, float y) {
    const float jf = fmaf(y, q.scale, q.offset);
    return q.J <= kBucketsU8 ? bucket_u8(jf) : bucket_wide(jf, q.jmax);
}

// The reference's linear scan.
__device__ inline int slow_code(float y, const float* c, int L) {
    float best = fabsf(y - c[0]);
    int idx = 0;
    for (int i = 1; i < L; ++i) {
        const float d = fabsf(y - c[i]);
        if (d < best) {
            best = d;
            idx = i;
        }
    }
    return idx;
}

// Fast path for the rotated unit vectors of TurboQuant (|y| <= 1 up to rounding, or NaN when
// the input held NaN/inf): valid when q.unit_fast is set, i.e. ybound >= 4 and no bucket
// holds two thresholds. NaN clamps to bucket 0 and takes its base, code 0, which is what the
// reference's scan returns for NaN (no distance compares below the first).
__device__ __forceinline__ int quantize_unit(const Quantizer& q, float y) {
    const float2 e = q.ent[bucket_of(q, y)];
    return __float_as_int(e.y) + (y > e.x ? 1 : 0);
}

__device__ __forceinline__ int quantize(const Quantizer& q, float y) {
    int code = -1;
    if (fabsf(y) <= q.ybound) {
        const float2 e = q.ent[bucket_of(q, y)];
        const int base = __float_as_int(e.y);
        if (base >= 0) code = base + (y > e.x ? 1 : 0);
    }
    if (code < 0) code = slow_code(y, q.c, q.L);
    return code;
}

// Ordering point between the phases of the quantizer build: a workgroup barrier (LDS
// only: outstanding global loads of the caller stay in flight) or, when one wave builds
// alone, a wavefront fence: a wave's LDS accesses are performed in program order, so the
// fence only has to stop the compiler from moving them across.
template <bool kOneWave>
__device__ __forceinline__ void build_sync() {
    if constexpr (kOneWave) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    } else {
        lds_barrier();
    }
}

// Build the quantizer for L centroids in LDS once q.c[0, L) holds them.
//   kOneWave = false: every thread of the block calls it (blockDim.x a multiple of 64);
//   kOneWave = true:  exactly one whole wave calls it (the rest of the block does other
//                     set-up work meanwhile), and the caller orders its results for the
//                     block with a barrier afterwards. No workgroup barrier is then on the
//                     build's path, which is a chain of short dependent LDS steps.
template <bool kOneWave = false>
__device__ inline void quantizer_finish(Quantizer& q, int L) {
    const int tid = kOneWave ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const int bs = kOneWave ? 64 : (int)blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nw = bs >> 6;
    // kOneWave callers write q.c from the same wave just before: lane i reads c[i + 1] below,
    // another lane's word (the other callers put a workgroup barrier there)
    if constexpr (kOneWave) build_sync<true>();
    bool ok = true;
    float gmin = __builtin_inff(), cmax = 0.0f;
    for (int i = tid; i < L; i += bs) {
        const float ci = q.c[i];
        if (!(fabsf(ci) <= 3.0e38f)) ok = false;
        cmax = fmaxf(cmax, fabsf(ci));
        if (i + 1 < L) {
            const float cn = q.c[i + 1];
            if (!(ci < cn)) ok = false;
            gmin = fminf(gmin, cn - ci);
        }
    }
    gmin = wave_min(gmin);
    cmax = wave_max(cmax);
    const bool wave_ok = __ballot(!ok) == 0;
    if (lane == 0) {
        q.red_f[0][wave] = gmin;
        q.red_f[1][wave] = cmax;
        q.red_i[wave] = wave_ok ? 1 : 0;
    }
    build_sync<kOneWave>();
    if (tid == 0) {
        float g = q.red_f[0][0], m = q.red_f[1][0];
        int k = q.red_i[0];
        for (int w = 1; w < nw; ++w) {
            g = fminf(g, q.red_f[0][w]);
            m = fmaxf(m, q.red_f[1][w]);
            k &= q.red_i[w];
        }
        float yb = -1.0f;
        if (k && L >= 2) {
            yb = ldexpf(g, 20) - m;
            if (!(yb > 0.0f)) yb = -1.0f;
        }
        q.ybound = yb;
        q.L = L;
        int J = 2 * L;
        if (J < 16) J = 16;
        if (J > kMaxBuckets) J = kMaxBuckets;
        q.J = J;
        q.jmax = (float)(J <= kBucketsU8 ? kBucketsU8 - 1 : J - 1);
    }
    build_sync<kOneWave>();
    const bool fast = q.ybound > 0.0f;
    if (fast) {
        for (int i = tid; i < L - 1; i += bs) q.t[i] = threshold_walk4(q.c[i], q.c[i + 1]);
        build_sync<kOneWave>();
        // the pairs the walk left open, one wave each
        for (int i = wave; i < L - 1; i += nw)
            if (q.t[i] != q.t[i]) {
                const float t = exact_threshold_wave(q.c[i], q.c[i + 1]);
                if (lane == 0) q.t[i] = t;
            }
    }
    build_sync<kOneWave>();
    if (tid == 0 && fast) {
        const int J = q.J;
        const float t0 = q.t[0], t1 = q.t[L - 2];
        float s, o;
        if (L > 2 && t1 > t0) {
            s = (float)(J - 2) / (t1 - t0);
            o = 1.0f - t0 * s;
        } else {
            s = 1.0f;
            o = (float)(J / 2) - t0;
        }
        if (!(fabsf(s) <= 3.0e38f) || !(fabsf(o) <= 3.0e38f) || !(s > 0.0f)) {
            q.ybound = -1.0f;
            s = 1.0f;
            o = 0.0f;
        }
        q.scale = s;
        q.offset = o;
    }
    build_sync<kOneWave>();
    int crowded = 0;
    if (q.ybound > 0.0f) {
        for (int i = tid; i < L - 1; i += bs) q.jt[i] = bucket_of(q, q.t[i]);
        build_sync<kOneWave>();
        const int n = L - 1;
        // every entry the bucket map can return: J, or all 256 of the byte map
        const int nent = q.J <= kBucketsU8 ? kBucketsU8 : q.J;
        for (int j = tid; j < nent; j += bs) {
            int lo = 0, hi = n;  // first q with jt[q] >= j
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (q.jt[mid] < j) lo = mid + 1; else hi = mid;
            }
            int lo2 = lo, hi2 = n;  // first q with jt[q] > j
            while (lo2 < hi2) {
                const int mid = (lo2 + hi2) >> 1;
                if (q.jt[mid] <= j) lo2 = mid + 1; else hi2 = mid;
            }
            float2 e;
            const int cnt = lo2 - lo;
            if (cnt == 0) {
                e.x = __builtin_inff();
                e.y = __int_as_float(lo);
            } else if (cnt == 1) {
                e.x = q.t[lo];
                e.y = __int_as_float(lo);
            } else {
                e.x = 0.0f;
                e.y = __int_as_float(-1);
                crowded = 1;
            }
            q.ent[j] = e;
        }
    }
    // workgroup OR of `crowded` (red_i is free again: its last reader passed two barriers)
    const bool wave_crowded = __ballot(crowded) != 0;
    if (lane == 0) q.red_i[wave] = wave_crowded ? 1 : 0;
    build_sync<kOneWave>();
    if (tid == 0) {
        int any = 0;
        for (int w = 0; w < nw; ++w) any |= q.red_i[w];
        q.unit_fast = (q.ybound >= 4.0f && !any) ? 1 : 0;
    }
    build_sync<kOneWave>();
}

// Build the quantizer for L centroids (device memory) in LDS (same contract).
__device__ inline void quantizer_build(Quantizer& q, const float* __restrict__ cent, int L) {
    for (int i = threadIdx.x; i < L; i += blockDim.x) q.c[i] = cent[i];
    __syncthreads();
    quantizer_finish(q, L);
}

// MSB-first bitstream: the 8 codes of group g occupy stream bits [8*b*g, 8*b*(g+1)), code i
// at bits b*(7-i) of the group word, written as b big-endian bytes (for b = 2, 4, 8 these are
// exactly the byte layouts of turboquant_compress.cu:145-185). nbytes < b only for the last,
// partial group of a row.
__device__ __forceinline__ uint64_t group_word(const int (&codes)[8], int bits) {
    uint64_t w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (uint64_t)(uint32_t)codes[i] << (bits * (7 - i));
    return w;
}

__device__ __forceinline__ void store_group(uint8_t* dst, uint64_t w, int bits, int nbytes) {
    if (nbytes == bits) {
        const uintptr_t a = (uintptr_t)dst;
        if (bits == 4 && (a & 3u) == 0) {
            *(uint32_t*)dst = __builtin_bswap32((uint32_t)w);
            return;
        }
        if (bits == 8 && (a & 7u) == 0) {
            *(uint64_t*)dst = __builtin_bswap64(w);
            return;
        }
        if (bits == 2 && (a & 1u) == 0) {
            *(uint16_t*)dst = __builtin_bswap16((uint16_t)w);
            return;
        }
    }
    for (int k = 0; k < nbytes; ++k) dst[k] = (uint8_t)(w >> (8 * (bits - 1 - k)));
}

// Inverse of store_group: the 8 codes of a group (missing trailing bytes read as zero).
__device__ __forceinline__ void load_group(const uint8_t* src, int bits, int nbytes,
                                           int (&codes)[8]) {
    uint64_t w = 0;
    const uintptr_t a = (uintptr_t)src;
    if (nbytes == bits && bits == 4 && (a & 3u) == 0) {
        w = __builtin_bswap32(*(const uint32_t*)src);
    } else if (nbytes == bits && bits == 8 && (a & 7u) == 0) {
        w = __builtin_bswap64(*(const uint64_t*)src);
    } else {
        for (int k = 0; k < bits; ++k)
            w = (w << 8) | (k < nbytes ? (uint64_t)src[k] : 0ull);
    }
    const uint32_t mask = (1u << bits) - 1u;
#pragma unroll
    for (int i = 0; i < 8; ++i) codes[i] = (int)((w >> (bits * (7 - i))) & mask);
}

}  // namespace fhip

// GQA decode attention over a TurboQuant-compressed paged KV cache, for gfx950.
//
// Semantics follow attention_paged_tq.cu:56-257: the query is pre-rotated with Pi_k
// (scores in the rotated K space, dot(q, Pi_k^T y) = dot(Pi_k q, y)), the score of
// position t is (sum_d q_rot[d] * ck[idx_td]) * (norm_k * head_dim^-1/2), causal length
// min(start_pos + t + 1, kv_len), softmax over the positions, V accumulated in the rotated
// V space as sum p * cv[idx] * norm_v, and the output unrotated once with Pi_v^T.
//
// Layout on MI355X: the reference keeps a kv_len-float score row in shared memory
// (attention_paged_tq.cu:287-289), which caps the context; here each workgroup takes one
// (query, kv head, 1024-token split) and all q heads of the kv head's GQA group, so every
// K/V code byte crosses HBM once per group, and keeps an online (max, sum, acc) per head.
// A combine kernel merges the splits and applies Pi_v^T. Three launches in all:
//   1. q_rot = Pi_k q                  (per query head)
//   2. split partials                  (the HBM stream over the pages)
//   3. merge + unrotate -> fp16 output
#include "fhip_internal.h"
#include "tq_attn_index.h"
#include "tq_quant.h"

using namespace fhip;

namespace {

constexpr int kSplit = 1024;   // positions per split workgroup
constexpr int kSub = 256;      // positions per pass (one per lane in the score phase)
constexpr int kMaxG = 8;       // q heads per kv head
constexpr int kMaxHd = 256;
constexpr int kMaxPd = 256;    // packed bytes per head row (hd * bits / 8)

// Page sources: per-page pointer arrays (the reference's interface) or contiguous pools.
struct PtrPages {
    const uint8_t* const* kp;
    const uint8_t* const* kn;
    const uint8_t* const* vp;
    const uint8_t* const* vn;
    int num_pages;  // entries of the pointer arrays
    __device__ bool valid(int p) const { return p >= 0 && p < num_pages; }
    __device__ const uint8_t* kpage(int p) const { return kp[p]; }
    __device__ const uint8_t* knorm(int p) const { return kn[p]; }
    __device__ const uint8_t* vpage(int p) const { return vp[p]; }
    __device__ const uint8_t* vnorm(int p) const { return vn[p]; }
    // The four part addresses of page p (p valid).
    __device__ void addrs(int p, const uint8_t*& k, const uint8_t*& knp, const uint8_t*& v,
                          const uint8_t*& vnp) const {
        k = kp[p];
        knp = kn[p];
        v = vp[p];
        vnp = vn[p];
    }
};
struct PoolPages {
    const uint8_t* kp;
    const uint8_t* kn;
    const uint8_t* vp;
    const uint8_t* vn;
    int64_t skp, skn, svp, svn;
    int num_pages;
    __device__ bool valid(int p) const { return p >= 0 && p < num_pages; }
    __device__ const uint8_t* kpage(int p) const { return kp + p * skp; }
    __device__ const uint8_t* knorm(int p) const { return kn + p * skn; }
    __device__ const uint8_t* vpage(int p) const { return vp + p * svp; }
    __device__ const uint8_t* vnorm(int p) const { return vn + p * svn; }
    __device__ void addrs(int p, const uint8_t*& k, const uint8_t*& knp, const uint8_t*& v,
                          const uint8_t*& vnp) const {
        k = kpage(p);
        knp = knorm(p);
        v = vpage(p);
        vnp = vnorm(p);
    }
};

// Query q_i reads block-table row i (stride 0: one shared table) and attends to
// seq_lens[i] positions, or min(start_pos + i + 1, kv_len) when seq_lens is null.
struct Queries {
    const int32_t* table;
    int64_t table_stride;
    int max_blocks;
    const int32_t* seq_lens;
    int kv_len, start_pos;
    int seq_lens_count;  // number of queries (set by the MFMA launcher)
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

// Byte k of a row held as little-endian 32-bit words.
__device__ __forceinline__ uint32_t row_byte(const uint32_t* w, int k) {
    return (w[k >> 2] >> (8 * (k & 3))) & 0xffu;
}
template <int B>
__device__ __forceinline__ void row_group(const uint32_t* w, int g, int bits_rt, int (&codes)[8]) {
    const int bits = B > 0 ? B : bits_rt;
    uint64_t word;
    if (B == 4) {
        word = __builtin_bswap32(w[g]);
    } else if (B == 8) {
        word = ((uint64_t)__builtin_bswap32(w[2 * g]) << 32) | __builtin_bswap32(w[2 * g + 1]);
    } else {
        word = 0;
        for (int k = 0; k < bits; ++k) word = (word << 8) | row_byte(w, g * bits + k);
    }
    const uint32_t mask = (1u << bits) - 1u;
#pragma unroll
    for (int i = 0; i < 8; ++i) codes[i] = (int)((word >> (bits * (7 - i))) & mask);
}

// 1. q_rot[v, :] = Pi_k q[v, :] (fp32 dots in coordinate order, attention_paged_tq.cu:102-113).
// A workgroup rotates kRotVecs vectors so Pi_k is read once per workgroup: work unit
// (row i, half) computes row i of vectors 4 half .. 4 half + 3.
constexpr int kRotVecs = 8;
constexpr int kMfmaRotVecs = 4096;  // from this many query vectors on, batched MFMA rotations
__global__ __launch_bounds__(256) void tq_attn_prerotate_kernel(const uint16_t* __restrict__ q,
                                                                const float* __restrict__ rot,
                                                                float* __restrict__ qrot, int hd,
                                                                int nvec) {
    __shared__ float qs[kRotVecs][kMaxHd];
    const int v0 = blockIdx.x * kRotVecs;
    {
        // every load is issued before the first is waited for: vectors past nvec read
        // vector 0 (in bounds) and are zeroed
        constexpr int kPer = kRotVecs * kMaxHd / 256;
        uint16_t raw[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = threadIdx.x + k * 256;
            const int v = e / hd, j = e - v * hd;
            const int64_t src = e < kRotVecs * hd && v0 + v < nvec ? (int64_t)(v0 + v) * hd + j : 0;
            raw[k] = q[src];
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = threadIdx.x + k * 256;
            const int v = e / hd, j = e - v * hd;
            if (e < kRotVecs * hd) qs[v][j] = v0 + v < nvec ? h2f(raw[k]) : 0.0f;
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < 2 * hd; r += blockDim.x) {
        const int i = r % hd, vb = 4 * (r / hd);
        const float* pr = rot + (int64_t)i * hd;
        float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j = 0; j < hd; ++j) {
            const float rv = pr[j];
#pragma unroll
            for (int k = 0; k < 4; ++k) dot[k] += rv * qs[vb + k][j];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (v0 + vb + k < nvec) qrot[(int64_t)(v0 + vb + k) * hd + i] = dot[k];
    }
}

// 2. One (split, kv head, query) per workgroup of 256 lanes. Each pass of 256 positions
// stages the positions' packed K and V rows in LDS (row stride padded to an odd number of
// words, so lanes reading different rows hit different banks), scores them one position per
// lane against the group's rotated queries, updates the online softmax, then accumulates V
// with lanes mapped to (8-coordinate code group, position slice).
template <int KB, int VB, class Pages>
__global__ __launch_bounds__(256) void tq_attn_split_kernel(
    const float* __restrict__ qrot, Queries qs, Pages pg, const float* __restrict__ kcent,
    const float* __restrict__ vcent, int kbits_rt, int vbits_rt, int qh, int kvh, int hd,
    float scale, float* __restrict__ part_ml, float* __restrict__ part_acc, int nsplit) {
    int split, kvhead, qi;  // grid (nsplit, kvh, queries), placed on the XCDs by split_grid_item
    fhip_idx::split_grid_item(
        blockIdx.x + (int64_t)gridDim.x * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z),
        (int64_t)gridDim.x * gridDim.y * gridDim.z, nsplit, kvh, split, kvhead, qi);
    const int clen = qs.causal_len(qi);
    const int t0 = split * kSplit;
    if (t0 >= clen) return;
    const int t1 = min(clen, t0 + kSplit);
    const int kbits = KB > 0 ? KB : kbits_rt, vbits = VB > 0 ? VB : vbits_rt;
    const int G = qh / kvh;
    const int pdk = (hd * kbits + 7) / 8, pdv = (hd * vbits + 7) / 8;
    const int kwords = (pdk + 3) / 4, vwords = (pdv + 3) / 4;
    const int ks = kwords | 1, vs = vwords | 1;  // odd LDS row strides
    const int NG = hd / 8;          // code groups per row
    const int NS = 256 / NG;        // position slices in the PV phase
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    __shared__ float kc[kMaxLevels], vc[kMaxLevels];
    __shared__ float qr[kMaxG * kMaxHd];
    __shared__ float w[kSub * kMaxG];            // p * norm_v, [pos][head]
    __shared__ float red[4][kMaxG];
    __shared__ float accbuf[kMaxG * kMaxHd];
    extern __shared__ uint32_t dyn[];
    uint32_t* krows = dyn;                        // [kSub][ks]
    uint32_t* vrows = dyn + kSub * ks;            // [kSub][vs]

    for (int i = tid; i < (1 << kbits); i += 256) kc[i] = kcent[i];
    for (int i = tid; i < (1 << vbits); i += 256) vc[i] = vcent[i];
    const float* qsrc = qrot + ((int64_t)qi * qh + (int64_t)kvhead * G) * hd;
    for (int i = tid; i < G * hd; i += 256) qr[i] = qsrc[i];
    const int32_t* table = qs.table + (int64_t)qi * qs.table_stride;

    float m_run[kMaxG], l_run[kMaxG];
    float acc[kMaxG][8];
#pragma unroll
    for (int h = 0; h < kMaxG; ++h) {
        m_run[h] = -__builtin_inff();
        l_run[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    }
    const int my_group = tid % NG, my_slice = tid / NG;
    __syncthreads();

    for (int sub = t0; sub < t1; sub += kSub) {
        // ---- stage this lane's position: packed K / V rows into LDS
        const int pos = sub + tid;
        bool valid = pos < t1;
        const int page = valid ? table[pos / FHIP_PAGE_TOKENS] : -1;
        valid = valid && pg.valid(page);
        const int slot = pos % FHIP_PAGE_TOKENS;
        const int64_t row = (int64_t)slot * kvh + kvhead;
        float knorm = 0.0f, vnorm = 0.0f;
        uint32_t* kdst = krows + tid * ks;
        uint32_t* vdst = vrows + tid * vs;
        if (valid) {
            const uint8_t* kr = pg.kpage(page) + row * pdk;
            const uint8_t* vr = pg.vpage(page) + row * pdv;
            if ((pdk & 15) == 0 && (((uintptr_t)kr) & 15u) == 0) {
                for (int i = 0; i < kwords; i += 4) {
                    const u32x4 x = ld16(kr + 4 * i);
                    kdst[i] = x[0]; kdst[i + 1] = x[1]; kdst[i + 2] = x[2]; kdst[i + 3] = x[3];
                }
            } else {
                for (int i = 0; i < kwords; ++i) {
                    uint32_t x = 0;
                    for (int b = 0; b < 4; ++b)
                        if (4 * i + b < pdk) x |= (uint32_t)kr[4 * i + b] << (8 * b);
                    kdst[i] = x;
                }
            }
            if ((pdv & 15) == 0 && (((uintptr_t)vr) & 15u) == 0) {
                for (int i = 0; i < vwords; i += 4) {
                    const u32x4 x = ld16(vr + 4 * i);
                    vdst[i] = x[0]; vdst[i + 1] = x[1]; vdst[i + 2] = x[2]; vdst[i + 3] = x[3];
                }
            } else {
                for (int i = 0; i < vwords; ++i) {
                    uint32_t x = 0;
                    for (int b = 0; b < 4; ++b)
                        if (4 * i + b < pdv) x |= (uint32_t)vr[4 * i + b] << (8 * b);
                    vdst[i] = x;
                }
            }
            knorm = h2f(((const uint16_t*)pg.knorm(page))[row]);
            vnorm = h2f(((const uint16_t*)pg.vnorm(page))[row]);
        } else {
            for (int i = 0; i < vwords; ++i) vdst[i] = 0u;
        }

        // ---- scores: lane = position (its own K row, so no barrier needed yet)
        float s[kMaxG];
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) s[h] = -__builtin_inff();
        if (valid) {
            float dot[kMaxG];
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) dot[h] = 0.0f;
            for (int g = 0; g < NG; ++g) {
                int codes[8];
                row_group<KB>(kdst, g, kbits, codes);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float cv = kc[codes[e]];
                    const int d = 8 * g + e;
#pragma unroll
                    for (int h = 0; h < kMaxG; ++h)
                        if (h < G) dot[h] += qr[h * hd + d] * cv;
                }
            }
            const float f = knorm * scale;
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) s[h] = dot[h] * f;
        }

        // ---- online softmax update per head
        float alpha[kMaxG], mnew[kMaxG];
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) {
            if (h >= G) break;
            const float mx = wave_max(s[h]);
            if (lane == 0) red[wave][h] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) {
            if (h >= G) break;
            const float cm = fmaxf(fmaxf(red[0][h], red[1][h]), fmaxf(red[2][h], red[3][h]));
            mnew[h] = fmaxf(m_run[h], cm);
            alpha[h] = m_run[h] == -__builtin_inff() ? 0.0f : expf(m_run[h] - mnew[h]);
        }
        __syncthreads();  // red[] reused below
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) {
            if (h >= G) break;
            const float p = valid ? expf(s[h] - mnew[h]) : 0.0f;
            w[tid * kMaxG + h] = p * vnorm;
            const float ps = wave_sum(p);
            if (lane == 0) red[wave][h] = ps;
        }
        __syncthreads();  // also publishes w[] and vrows[]
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) {
            if (h >= G) break;
            l_run[h] = l_run[h] * alpha[h] + (red[0][h] + red[1][h] + red[2][h] + red[3][h]);
            m_run[h] = mnew[h];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];
        }

        // ---- PV: lane = (code group, position slice)
        const int npos = min(kSub, t1 - sub);
        for (int tk = my_slice; tk < npos; tk += NS) {
            int codes[8];
            row_group<VB>(vrows + tk * vs, my_group, vbits, codes);
            float cv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) cv[e] = vc[codes[e]];
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) {
                if (h >= G) break;
                const float wv = w[tk * kMaxG + h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] += wv * cv[e];
            }
        }
        __syncthreads();  // w / rows / red reused by the next pass
    }

    // ---- merge the position slices in a fixed order, write the split's partials
    for (int i = tid; i < G * hd; i += 256) accbuf[i] = 0.0f;
    __syncthreads();
    for (int sl = 0; sl < NS; ++sl) {
        if (my_slice == sl) {
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) {
                if (h >= G) break;
#pragma unroll
                for (int e = 0; e < 8; ++e) accbuf[h * hd + 8 * my_group + e] += acc[h][e];
            }
        }
        __syncthreads();
    }
    const int64_t head0 = (int64_t)qi * qh + (int64_t)kvhead * G;
    for (int i = tid; i < G * hd; i += 256) {
        const int h = i / hd, d = i - h * hd;
        part_acc[((head0 + h) * nsplit + split) * hd + d] = accbuf[i];
    }
    if (tid < G) {
        part_ml[((head0 + tid) * nsplit + split) * 2 + 0] = m_run[tid];
        part_ml[((head0 + tid) * nsplit + split) * 2 + 1] = l_run[tid];
    }
}

// Merge the splits of kCombHeads consecutive (query, head) vectors per workgroup and apply
// Pi_v^T: out = Pi_v^T (sum_s w_s acc_s) / (sum_s w_s l_s), w_s = exp(m_s - max m). The work
// is a few dependent memory round trips, so each phase issues its loads together:
//   the rotation (hd x hd fp32) is staged in LDS first, overlapping the rest (kRotLds; for
//            head_dim above kRotLdsMaxHd it does not fit LDS and phase 3 reads it from L2);
//   phase 1: a half-wave per vector loads its splits' (m, l) once and folds them into
//            weights (LDS) and 1 / L;
//   phase 2: the weighted split sums, four (vector, coordinate) items per thread, sixteen
//            splits per step, each item summed in split order;
//   phase 3: the matvec, one output coordinate for 4 vectors per thread and step.
// Dynamic LDS: hd * hd rotation floats (kRotLds), then kCombHeads * nsplit weights.
constexpr int kCombHeads = 4;  // two workgroups per CU at the decode workload's 2048 vectors
constexpr int kRotLdsMaxHd = 128;
constexpr int kMaxTokensTq = kSplit * kSplit;  // 1024 splits: 32 KB of combine weights
size_t combine_lds_bytes(int hd, int nsplit, bool merge_only = false) {
    return ((hd <= kRotLdsMaxHd && !merge_only ? (size_t)hd * hd : 0) + (size_t)kCombHeads * nsplit) *
           sizeof(float);
}
// The merge alone with one wave per vector, four vectors per workgroup, when a vector has at
// most 8 splits (contexts up to 8192 positions; causal prefill): lane s holds split s's
// (m, l), the weights reach the dim loop by lane broadcasts, and each merged vector (fp32,
// divided by its sum) goes to merged[vector]. The combine kernel's 16-split load batches
// would be mostly clamped repeats at these sizes.
constexpr int kMergeWaveMaxSplits = 8;
__global__ __launch_bounds__(256) void tq_attn_merge_wave_kernel(
    Queries qs, const float* __restrict__ part_ml, const float* __restrict__ part_acc, int qh,
    int hd, int nsplit, int64_t nvec, float* __restrict__ merged) {
    const int lane = threadIdx.x & 63;
    const int64_t vec = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (vec >= nvec) return;
    const int clen = qs.causal_len((int)(vec / qh));
    const int ns = (clen + kSplit - 1) / kSplit;  // <= nsplit <= kMergeWaveMaxSplits
    const float* ml = part_ml + vec * nsplit * 2;
    const float ms = lane < ns ? ml[2 * lane] : -__builtin_inff();
    const float ls = lane < ns ? ml[2 * lane + 1] : 0.0f;
    const float M = wave_max(ms);
    const float w = lane < ns && ms != -__builtin_inff() ? expf(ms - M) : 0.0f;
    const float L = wave_sum(w * ls);
    const float linv = L > 0.0f ? 1.0f / L : 0.0f;
    float ws[kMergeWaveMaxSplits];
#pragma unroll
    for (int j = 0; j < kMergeWaveMaxSplits; ++j) ws[j] = __shfl(w, j);
    const float* a = part_acc + vec * nsplit * hd;
    for (int d = lane; d < hd; d += 64) {
        float av[kMergeWaveMaxSplits];
#pragma unroll
        for (int j = 0; j < kMergeWaveMaxSplits; ++j) av[j] = j < ns ? a[(int64_t)j * hd + d] : 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kMergeWaveMaxSplits; ++j) sum = fmaf(av[j], ws[j], sum);
        merged[vec * hd + d] = sum * linv;
    }
}

// kMergeOnly: phase 2 writes each merged vector (fp32, already divided by its sum) to
// merged[vector] and the kernel ends; the unrotation then runs as a batched MFMA product.
template <bool kRotLds, bool kMergeOnly = false>
__global__ __launch_bounds__(256) void tq_attn_combine_kernel(
    Queries qs, const float* __restrict__ part_ml, const float* __restrict__ part_acc,
    const float* __restrict__ vrot, uint16_t* __restrict__ out, int qh, int hd, int nsplit,
    int64_t nvec, float* __restrict__ merged = nullptr) {
    __shared__ float o[kCombHeads][kMaxHd];
    __shared__ float linv[kCombHeads];
    __shared__ int nsv[kCombHeads];
    extern __shared__ uint32_t dyn[];
    float* rl = (float*)dyn;                                  // [hd][hd] (kRotLds)
    float* wts = (float*)dyn + (kRotLds && !kMergeOnly ? hd * hd : 0);  // [kCombHeads][nsplit]
    const float* rot = kRotLds ? (const float*)rl : vrot;
    const int tid = threadIdx.x;
    const int64_t h0 = (int64_t)blockIdx.x * kCombHeads;
    if (kRotLds && !kMergeOnly) {   // the rotation into LDS: hd * hd / 4 16-byte chunks, all loads first
        const int n16 = hd * hd / 4;
        for (int c0 = tid; c0 < n16; c0 += 16 * 256) {
            u32x4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = ld16(vrot + 4 * min(c0 + u * 256, n16 - 1));
#pragma unroll
            for (int u = 0; u < 16; ++u) *(u32x4*)&rl[4 * min(c0 + u * 256, n16 - 1)] = v[u];
        }
    }
    {
        // a half-wave per vector (the half-waves past kCombHeads only join the shuffles)
        const int hh = min(tid >> 5, kCombHeads - 1), l32 = tid & 31;
        const bool mine = (tid >> 5) < kCombHeads;
        const int64_t head = h0 + hh;
        int ns = 0;
        if (mine && head < nvec) {
            const int clen = qs.causal_len((int)(head / qh));
            ns = (clen + kSplit - 1) / kSplit;
        }
        const float* ml = part_ml + head * nsplit * 2;
        float M = -__builtin_inff();
        for (int sp = l32; sp < ns; sp += 32) M = fmaxf(M, ml[2 * sp]);
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        float L = 0.0f;
        for (int sp = l32; sp < ns; sp += 32) {
            const float m = ml[2 * sp];
            const float w = (m == -__builtin_inff()) ? 0.0f : expf(m - M);
            wts[hh * nsplit + sp] = w;
            L += ml[2 * sp + 1] * w;
        }
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) L += __shfl_xor(L, off);
        if (mine && l32 == 0) {
            linv[hh] = L > 0.0f ? 1.0f / L : 0.0f;
            nsv[hh] = ns;
        }
    }
    __syncthreads();
    for (int idx0 = tid; idx0 < kCombHeads * hd; idx0 += 4 * 256) {
        const float* a[4];
        int hh[4], ns[4];
        float sum[4];
        int nsmax = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int idx = min(idx0 + k * 256, kCombHeads * hd - 1);
            hh[k] = idx / hd;
            const int d = idx - hh[k] * hd;
            ns[k] = idx0 + k * 256 < kCombHeads * hd ? nsv[hh[k]] : 0;
            nsmax = max(nsmax, ns[k]);
            // vectors past nvec (last workgroup) read vector 0's row: in bounds, unused
            a[k] = part_acc + (h0 + hh[k] < nvec ? (h0 + hh[k]) * nsplit * hd : 0) + d;
            sum[k] = 0.0f;
        }
        for (int sp = 0; sp < nsmax; sp += 16) {
            float v[4][16];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int u = 0; u < 16; ++u)  // clamped: every load is in bounds, unused ones ignored
                    v[k][u] = a[k][(int64_t)min(sp + u, max(ns[k] - 1, 0)) * hd];
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (sp + u < ns[k]) sum[k] = fmaf(v[k][u], wts[hh[k] * nsplit + sp + u], sum[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (idx0 + k * 256 >= kCombHeads * hd) continue;
            const float v = sum[k] * linv[hh[k]];
            if constexpr (kMergeOnly) {
                if (h0 + hh[k] < nvec) merged[(h0 + hh[k]) * hd + idx0 + k * 256 - hh[k] * hd] = v;
            } else {
                o[hh[k]][idx0 + k * 256 - hh[k] * hd] = v;
            }
        }
    }
    if constexpr (kMergeOnly) return;
    __syncthreads();
    for (int idx = tid; idx < 2 * hd; idx += 256) {
        const int hg = idx / hd, i = idx - hg * hd;
        float dot[kCombHeads / 2] = {};
        for (int j = 0; j < hd; ++j) {
            const float v = rot[j * hd + i];
#pragma unroll
            for (int k = 0; k < kCombHeads / 2; ++k) dot[k] += v * o[hg + 2 * k][j];
        }
#pragma unroll
        for (int k = 0; k < kCombHeads / 2; ++k) {
            const int64_t head = h0 + hg + 2 * k;
            if (head < nvec) out[head * hd + i] = (uint16_t)f2h(dot[k]);
        }
    }
}

// ---------------------------------------------------------------------------------------
// 2'. MFMA split kernel: head_dim 128, 4-bit K codes and 4- or 2-bit V codes (kV2: widened to
//     4 bits on their way into LDS), G <= 8 query heads per kv head.
//
// A workgroup owns one (query, kv head, 1024-position block); each of its two waves walks
// one 512-position split of it in 64-position chunks:
//   QK  D[pos][col] = sum_k A[pos][k] B[k][col] on v_mfma_f32_16x16x32_f16. The K slots come
//       in (hi, lo') pairs per coordinate: A = (c_hi, c_lo*2^12) of the position's centroid,
//       B = (q_hi, 0) in column h and (q_lo*2^12, q_hi) in column 8+h, so one MFMA gives
//       D[h] = sum c_hi q_hi and D[8+h] = 2^12 (sum c_hi q_lo + c_lo q_hi), and the score is
//       (D[h] + 2^-12 D[8+h]) * norm_k / sqrt(128): fp16 operands, ~fp32 accuracy, no fp16
//       subnormals. A fragments come from an LDS table indexed by a code byte (two
//       coordinates): byte -> the (c_hi | c_lo' << 16) words of its two codes, one
//       ds_read_b64 and one address op per two codes.
//   PV  out[h][d] accumulates W[h][pos] V[pos][d] the same way: B = (v_hi, v_lo') of the V
//       code, A = (w_hi, 0) in row h and (w_lo*2^12, w_hi) in row 8+h, w = p * norm_v.
//       The B operand needs 4 positions of one coordinate per lane; ds_read_b64_tr_b4 reads
//       them transposed out of the chunk's V code rows staged in LDS in their page layout.
// Chunk position order: QK tile pt (16 rows) holds positions 4i + pt, so the 4 scores a lane
// ends up with for tile pt (rows 4rg..4rg+3) are positions 16rg + 4e + pt, and the PV
// K slots of lane group rg in tile pt are those same positions: no score shuffling.
// Online softmax per head (lanes n = h), lazily rescaling the accumulators.
// ---------------------------------------------------------------------------------------
constexpr int kChunkM = 64;     // positions per chunk
constexpr int kSplitMfma = 512;  // positions per wave item (split)
constexpr int kXcds = 8;         // MI355X: accelerator complex dies, each with its own L2
constexpr int kSplitPages = kSplitMfma / FHIP_PAGE_TOKENS;
constexpr int kWavesM = 2;      // waves per workgroup (independent work items)
static_assert(kChunkM == fhip_idx::kChunk && kSplitMfma == fhip_idx::kSplitPositions &&
                  kWavesM == fhip_idx::kBlockWaves && kXcds == fhip_idx::kXcdCount &&
                  FHIP_PAGE_TOKENS == fhip_idx::kPageTokens,
              "the kernel's shape is the one its index helpers describe");

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t hi_lo_pair(float v, float& hi_f) {
    const _Float16 hi = (_Float16)v;
    hi_f = (float)hi;
    const _Float16 lo = (_Float16)((v - hi_f) * 4096.0f);
    return (uint32_t)__builtin_bit_cast(uint16_t, hi) |
           ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}
__device__ __forceinline__ float ror8(float v) {  // lane n of each 16-lane row gets lane n^8
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}
// Row-local DPP moves (rotations within each 16-lane row: lane n takes lane (n - kRor) mod 16)
// that write only the lanes of the 4-lane banks in kBank; other lanes keep `old`.
template <int kRor, int kBank>
__device__ __forceinline__ float dpp_into(float old, float src) {
    constexpr int kCtrl = kRor == 0 ? 0xE4 : 0x120 + kRor;  // identity quad_perm, or row_ror
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src),
                                                      kCtrl, 0xF, kBank, false));
}
template <int kRor, int kBank>
__device__ __forceinline__ uint32_t dpp_into_u(uint32_t old, uint32_t src) {
    constexpr int kCtrl = kRor == 0 ? 0xE4 : 0x120 + kRor;
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, kCtrl, 0xF, kBank, false);
}
// acc += 2^-12 * (lane (n - kRor) mod 16's src), in the lanes of bank kBank only
// (v_fmac_f32_dpp; `c` holds 2^-12).
template <int kRor, int kBank>
__device__ __forceinline__ void dpp_fmac_lo(float& acc, float src, float c) {
    static_assert(kBank == 1 || kBank == 2 || kBank == 4 || kBank == 8, "one bank");
#define FHIP_FMAC_DPP(CTRL, BANK) \
    asm("v_fmac_f32_dpp %0, %1, %2 " CTRL " row_mask:0xf bank_mask:" BANK : "+v"(acc) : "v"(src), "v"(c))
    if constexpr (kBank == 1) {
        static_assert(kRor == 8, "tile 0");
        FHIP_FMAC_DPP("row_ror:8", "0x1");
    } else if constexpr (kBank == 2) {
        static_assert(kRor == 12, "tile 1");
        FHIP_FMAC_DPP("row_ror:12", "0x2");
    } else if constexpr (kBank == 4) {
        static_assert(kRor == 0, "tile 2");
        FHIP_FMAC_DPP("quad_perm:[0,1,2,3]", "0x4");
    } else {
        static_assert(kRor == 4, "tile 3");
        FHIP_FMAC_DPP("row_ror:4", "0x8");
    }
#undef FHIP_FMAC_DPP
}
// Max / sum over the 4 banks of each row (lanes n, n ^ 4, n ^ 8, n ^ 12 hold one head).
// A DPP read of a VGPR that a VALU instruction has just written needs two wait states, which
// the compiler does not insert for inline asm: each DPP instruction here follows an s_nop 1.
__device__ __forceinline__ float bank_max(float v) {
    asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf" : "+v"(v));
    asm("s_nop 1\n\tv_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf" : "+v"(v));
    return v;
}
__device__ __forceinline__ float bank_sum(float v) {
    asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf" : "+v"(v));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf" : "+v"(v));
    return v;
}

// 8 * (byte kByte of x), the byte offset of a pair-table entry, in one v_lshlrev_b32_sdwa.
// Written as asm: the compiler turns the extract-and-shift into two instructions for most
// byte positions.
template <int kByte>
__device__ __forceinline__ uint32_t byte_x8(uint32_t x) {
    uint32_t r;
    if constexpr (kByte == 0)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "s"(3u), "v"(x));
    else if constexpr (kByte == 1)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "s"(3u), "v"(x));
    else if constexpr (kByte == 2)
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "s"(3u), "v"(x));
    else
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "s"(3u), "v"(x));
    return r;
}
// Pair-table entries of bytes kB and kB + 1 of a code word w: the (c_hi | c_lo' << 16) words
// of those bytes' four codes, in the order the table holds each byte's two.
template <int kB>
__device__ __forceinline__ u32x4 pair2(const u32x2* tab, uint32_t w) {
    const u32x2 e0 = *(const u32x2*)((const char*)tab + byte_x8<kB>(w));
    const u32x2 e1 = *(const u32x2*)((const char*)tab + byte_x8<kB + 1>(w));
    return u32x4{e0[0], e0[1], e1[0], e1[1]};
}

// The split's pages, read once per split into a per-wave LDS table: entry j holds the four
// part addresses (K codes, V codes, K norms, V norms) of the split's page j. Where page j holds
// no position of the split, or its table entry is outside the pool, the entry holds the split's
// first valid page instead, so every chunk load below reads a real page; the positions of such
// pages are masked in the scores (bit j of the returned mask clear) and their norms zeroed.
// With no valid page at all (mask 0) the split reads nothing.
struct PageAddrs {
    const uint8_t *k, *v, *kn, *vn;
};
template <class Pages>
__device__ __forceinline__ uint64_t split_pages(const Pages& pg, const int32_t* table, int t_begin,
                                                int t_end, int lane, PageAddrs* pages) {
    int column;
    const bool in = fhip_idx::split_page_column(t_begin, t_end, lane, column);
    const int id = in ? table[column] : -1;
    const bool ok = in && pg.valid(id);
    const uint64_t vmask = __ballot(ok);
    if (vmask == 0) return 0;
    const int first = __builtin_amdgcn_readlane(id, (int)__builtin_ctzll(vmask));
    PageAddrs a;
    pg.addrs(ok ? id : first, a.k, a.kn, a.v, a.vn);
    if (lane < kSplitPages) pages[lane] = a;
    wave_lds_sync();  // the wave reads other lanes' entries next
    return vmask;
}
// Loads through global-address-space pointers: addresses read back from LDS lose their
// address space, and generic (flat) loads would also count against the LDS counter, so every
// table-read wait would wait for them too.
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const uint16_t g_u16;
__device__ __forceinline__ u32x4 gld16(const uint8_t* p) { return *(g_u32x4*)p; }
__device__ __forceinline__ uint32_t gld2(const uint8_t* p) { return *(g_u16*)p; }

// Lane j's address as a wave-uniform value (v_readlane into SGPRs).
__device__ __forceinline__ const uint8_t* addr_of_lane(const uint8_t* p, int j) {
    const uint64_t u = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, j);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
    return (const uint8_t*)(((uint64_t)hi << 32) | lo);
}

// One 16-byte LDS DMA copy per lane from sbase + voff (sbase wave-uniform, in SGPRs): lane L
// writes lds + 16 L (lds wave-uniform). Issued as asm so that the compiler, which counts
// pending LDS DMA against the LDS counter as well, keeps exact LDS waits for the table lookups
// that run while copies are in flight (the hardware tracks these copies on the vector memory
// counter only). Every read of the DMA buffers waits for them explicitly.
__device__ __forceinline__ void dma16(const uint8_t* sbase, uint32_t voff, uint8_t* lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds);
    // m0 is saved and restored around the copy: the compiler may keep a value in it
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(m)
        : "memory");
}

// Chunk loads. The chunk starts at split page j0 (positions t0 .. t0 + 63 = pages j0 .. j0 + 3);
// every address comes from the split's page lanes, so no load needs a per-position check.
//
// K codes, straight into the registers QK uses (LDS DMA streams markedly slower than vector
// loads, and K needs no LDS stage): tile pt is position 4n + pt, bytes [16rg, 16rg + 16) for
// lane (n, rg); the lane's page is j0 + n / 4 and the four tiles are 4 rows apart.
__device__ __forceinline__ void load_k(const PageAddrs* pages, int j0, int kvh, int g, int lane,
                                       u32x4 (&kc)[4]) {
    const uint8_t* src = pages[j0 + fhip_idx::k_page(lane)].k + fhip_idx::k_offset(lane, kvh, g);
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) kc[pt] = gld16(src + pt * fhip_idx::k_tile_stride(kvh));
}
// V codes by LDS DMA: copy i moves page j0 + i (positions 16i .. 16i + 15); lane L takes
// position p = 16i + L / 4 and stores 16 bytes at 64p + 16(L % 4). The 16-byte segment it
// copies is (L % 4) ^ ((p / 2) % 4): rows are XOR-swizzled so the transposed reads of one
// dim range from 16 rows spread over the banks. `voff` is that segment's offset in the page.
__device__ __forceinline__ void dma_v(const PageAddrs* pages, int j0, uint32_t voff, uint8_t* vb,
                                      int lane) {
    const uint8_t* v4 = pages[j0 + (lane & 3)].v;  // lane i < 4: page j0 + i
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(addr_of_lane(v4, i), voff, vb + 1024 * i);
}
// 2-bit V codes (kV2): the same segments as dma_v, from rows of 32 bytes. Lane L takes 8 bytes of
// position 16i + L / 4 of page j0 + i (v2_offset), and once they have arrived store_v2 widens
// each 2-bit code to a 4-bit one and writes the 16 bytes that dma_v would have copied, so the
// transposed reads and the pair table serve both widths (its V entries map codes 0..3).
typedef __attribute__((address_space(1))) const u32x2 g_u32x2;
__device__ __forceinline__ void load_v2(const PageAddrs* pages, int j0, uint32_t voff,
                                        u32x2 (&r)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = *(g_u32x2*)(pages[j0 + i].v + voff);
}
// Bytes sel of w (two code bytes, four codes each, the first in the top bits) as four bytes
// of 4-bit codes, the first in the high nibble: byte b -> (c0 << 4 | c1), (c2 << 4 | c3).
__device__ __forceinline__ uint32_t widen2(uint32_t w, uint32_t sel) {
    const uint32_t x = __builtin_amdgcn_perm(w, w, sel);  // b0, b0, b1, b1
    return ((x & 0x00C000C0u) >> 2) | ((x & 0x00300030u) >> 4) | ((x & 0x0C000C00u) << 2) |
           (x & 0x03000300u);
}
__device__ __forceinline__ void store_v2(const u32x2 (&r)[4], uint8_t* vb, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *(u32x4*)(vb + 1024 * i + 16 * lane) =
            u32x4{widen2(r[i][0], 0x01010000u), widen2(r[i][0], 0x03030202u),
                  widen2(r[i][1], 0x01010000u), widen2(r[i][1], 0x03030202u)};
}

// Norms of position t0 + lane, loaded raw (fp16 bits): pack() gives (knorm, vnorm) in fp32
// once they are needed (0 where there is none), so each norm is converted once, by the lane
// that loaded it. Packing later keeps the wait for them away from the copies issued after them.
struct NormRegs {
    uint32_t k, v;
    bool ok;
    __device__ float2 pack() const {
        uint32_t a = k, b = v;
        // pins the pack here: the compiler would otherwise pack right after the loads
        asm volatile("" : "+v"(a), "+v"(b));
        const float fk = (float)__builtin_bit_cast(_Float16, (uint16_t)a);
        const float fv = (float)__builtin_bit_cast(_Float16, (uint16_t)b);
        return ok ? float2{fk, fv} : float2{0.0f, 0.0f};
    }
};
__device__ __forceinline__ NormRegs load_norms(const PageAddrs* pages, int j0, uint32_t pm, int t0,
                                               int t_end, int kvh, int g, int lane) {
    const int k = fhip_idx::norm_page(lane);
    const uint32_t row = fhip_idx::norm_offset(lane, kvh, g);
    const bool ok = ((pm >> k) & 1u) && t0 + lane < t_end;
    const PageAddrs& pa = pages[j0 + k];
    return NormRegs{gld2(pa.kn + row), gld2(pa.vn + row), ok};
}

// Loads of chunk i + 1 (V codes by LDS DMA, then norms and K codes into registers) are issued
// together right after chunk i's QK, and chunk i + 1 starts by waiting for all of them
// (vmcnt(0)), so its PV reads the V buffer with no further wait. The transposed V reads are
// asm: the compiler's own wait counting would also hold PV back for the loads issued after QK.
// The "memory" clobber keeps every copy on its side of these reads.
// Transposed V reads of dim tiles 0..7 (tile c at row segment (c / 2) ^ sw, half c % 2):
// seg[s] is the lane's address of its row's segment s ^ sw.
__device__ __forceinline__ void read_v_codes(const uint32_t (&seg)[4], v2i_t (&tv)[8]) {
    asm volatile(
        "ds_read_b64_tr_b4 %0, %8\n"
        "ds_read_b64_tr_b4 %1, %8 offset:8\n"
        "ds_read_b64_tr_b4 %2, %9\n"
        "ds_read_b64_tr_b4 %3, %9 offset:8\n"
        "ds_read_b64_tr_b4 %4, %10\n"
        "ds_read_b64_tr_b4 %5, %10 offset:8\n"
        "ds_read_b64_tr_b4 %6, %11\n"
        "ds_read_b64_tr_b4 %7, %11 offset:8\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(tv[0]), "=&v"(tv[1]), "=&v"(tv[2]), "=&v"(tv[3]), "=&v"(tv[4]), "=&v"(tv[5]),
          "=&v"(tv[6]), "=&v"(tv[7])
        : "v"(seg[0]), "v"(seg[1]), "v"(seg[2]), "v"(seg[3])
        : "memory");
}

// kG4 score compaction: tile kPt's head-h score D[h] + 2^-12 D[8 + h] (MFMA columns h and 8 + h
// of the lane's row) into lane 4 kPt + h, elements e = 0..3; the other banks keep theirs.
template <int kPt>
__device__ __forceinline__ void compact_scores(float (&S)[4], const f32x4_t& d, float c12) {
    constexpr int kBank = 1 << kPt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        S[e] = dpp_into<(4 * kPt) & 15, kBank>(S[e], d[e]);
        dpp_fmac_lo<(4 * kPt + 8) & 15, kBank>(S[e], d[e], c12);
    }
}
// kG4 PV operand of tile kPt: column h (lanes h < 4) takes (w_hi, 0) and column 8 + h takes
// (w_lo', w_hi) of lane 4 kPt + h; banks 1 and 3 are not written (they stay 0).
template <int kPt>
__device__ __forceinline__ void expand_weights(uint32_t (&b)[4], const uint32_t (&x)[4],
                                               const uint32_t (&y)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        b[e] = dpp_into_u<(16 - 4 * kPt) & 15, 0x1>(b[e], x[e]);
        b[e] = dpp_into_u<(24 - 4 * kPt) & 15, 0x4>(b[e], y[e]);
    }
}

template <class Pages, bool kG4, bool kV2>
__global__ __launch_bounds__(64 * kWavesM) __attribute__((amdgpu_waves_per_eu(3))) void
tq_attn_mfma_kernel(const float* __restrict__ qrot, Queries qs, Pages pg,
                    const float* __restrict__ kcent, const float* __restrict__ vcent, int qh,
                    int kvh, float scale, float* __restrict__ part_ml,
                    float* __restrict__ part_acc, int nsplit, int nblk, int tok) {
    constexpr int hd = 128;
    // Code-byte tables: byte b -> the (c_hi | c_lo' << 16) words of its two codes, K as
    // {high nibble, low nibble} (the QK A operand's order), V as {low, high} (the PV B
    // operand's). One ds_read_b64 serves two codes: lookups at random entries of 2 KB tables
    // cost some bank conflicts, but half the LDS instructions and under half the address
    // arithmetic of per-code lookups in a 16-word table. The DMA
    // targets are separate objects: table reads never wait for DMA traffic.
    __shared__ u32x2 pk[256], pv[256];
    __shared__ __attribute__((aligned(16))) uint8_t vbuf[kWavesM][2][kChunkM * 64];  // by chunk parity
    __shared__ __attribute__((aligned(16))) float2 nbuf[kWavesM][kChunkM];  // (knorm, vnorm)
    __shared__ PageAddrs pagebuf[kWavesM][kSplitPages];  // the wave's split pages
    __shared__ int waves_done;  // waves that have left their state for the merge
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, rg = lane >> 4;  // MFMA column / row group
    static_assert(kWavesM * kSplitMfma == kSplit, "a workgroup's splits make one partial's block");

    // Workgroup (query, kv head, block of kWavesM consecutive splits); wave w takes split
    // kWavesM * blk + w. Workgroups go to the 8 XCDs round-robin (workgroup b on XCD b % 8),
    // and the kv heads of one token row share 128-byte lines, so the index puts every kv head
    // of one (query, block) item on the same XCD: item i = (query, block) and kv head g run
    // as workgroup (i / 8) (8 kvh) + 8 g + i % 8, and each line is filled into one L2 only.
    // A workgroup whose block holds no position leaves before the tables are built (the exit
    // is uniform, so no wave misses the barriers below).
    int64_t item;
    int g;
    fhip_idx::wg_item(blockIdx.x, kvh, item, g);
    // Item (token group, block): a group is `tok` consecutive queries of one sequence (causal
    // prefill; 1 in decode), whose G query heads each fill MFMA columns h = G t + head.
    const int qg = (int)(item / nblk);
    const int tq0 = qg * tok;
    if (tq0 >= qs.seq_lens_count) return;
    const int tq_last = min(tq0 + tok, qs.seq_lens_count) - 1;
    const int blk = (int)(item % nblk);
    const int clen = qs.causal_len(tq_last);  // the group's longest causal length
    if (blk * kSplit >= clen) return;
    for (int b = threadIdx.x; b < 256; b += 64 * kWavesM) {
        float hf;
        const uint32_t kh = hi_lo_pair(kcent[b >> 4], hf), kl = hi_lo_pair(kcent[b & 15], hf);
        const int v0 = kV2 ? min(b >> 4, 3) : b >> 4, v1 = kV2 ? min(b & 15, 3) : b & 15;
        const uint32_t vh = hi_lo_pair(vcent[v0], hf), vl = hi_lo_pair(vcent[v1], hf);
        pk[b] = u32x2{kh, kl};
        pv[b] = u32x2{vl, vh};
        if (b == 0) waves_done = 0;
    }
    __syncthreads();

    const int t_begin = fhip_idx::split_begin(blk, wave);
    const int t_end = min(clen, t_begin + kSplitMfma);
    const int G = qh / kvh;
    const int32_t* table = qs.table + (int64_t)tq0 * qs.table_stride;
    uint8_t* vb = vbuf[wave][0];
    float2* nb = nbuf[wave];
    const int ncols = tok * G;  // live head columns (at most 8)
    // this lane's column: token tq0 + ct, head ch; its causal length (0 for a column past the
    // queries, so that every position is masked for it)
    const int ct = (n & 7) / G;
    bool col_ok;  // the column is head (n & 7) % G of a query of the group
    const int64_t qvec = fhip_idx::q_vector(lane, tq0, tok, G, qs.seq_lens_count, qh, g, col_ok);
    const int col_len = col_ok ? qs.causal_len(tq0 + ct) : 0;
    // the shortest length of the group (its first query's): chunks below it need no mask
    const int min_len = tok > 1 ? qs.causal_len(tq0) : clen;

    float m_run = -__builtin_inff(), l_run = 0.0f;  // log2 units; lanes n, n ^ 8: head n & 7
    // PV accumulators out^T, dim tile c: lane (n, rg) holds head slot n (n < 8: head n, hi
    // part; n >= 8: head n - 8, lo' part) at dims 16c + ((4rg + e) ^ 1), e = 0..3
    f32x4_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // The split's pages (at most kSplitPages), read once: the chunk loop then issues no memory
    // instruction besides its loads and copies. A wave with no position to read (its split
    // starts past the end, or no page is in the pool) keeps the empty state.
    PageAddrs* pages = pagebuf[wave];
    const uint64_t vmask = t_begin < clen ? split_pages(pg, table, t_begin, t_end, lane, pages) : 0;
    if (vmask != 0) {
    // first chunk's copies go out before the Q set-up
    const uint32_t v_lane_off = kV2 ? fhip_idx::v2_offset(lane, kvh, g) : fhip_idx::v_offset(lane, kvh, g);
    uint32_t pmask = (uint32_t)vmask & 0xfu;  // pages of the current chunk to read
    u32x2 v2reg[kV2 ? 4 : 1];  // kV2: the next chunk's V codes, widened into LDS when it starts
    if constexpr (kV2)
        load_v2(pages, 0, v_lane_off, v2reg);
    else
        dma_v(pages, 0, v_lane_off, vb, lane);  // chunk 0: buffer 0
    NormRegs nreg = load_norms(pages, 0, pmask, t_begin, t_end, kvh, g, lane);
    u32x4 kreg[4];
    load_k(pages, 0, kvh, g, lane, kreg);

    // Q as the QK B operand, pre-scaled by scale * log2(e) so scores come out in log2 units:
    // step s, lane (n, rg) holds coordinates 32rg + 4s + c4.
    uint32_t bq[8][4];
    {
        // heads past G read head 0 and are zeroed by the multiplier
        // columns past the group's heads read the group's first vector and are zeroed
        const float* qsrc = qrot + qvec * hd;
        const float qmul = col_ok ? scale * 1.4426950408889634f : 0.0f;
        f32x4_t qv[8];
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) qv[s8] = *(const f32x4_t*)(qsrc + fhip_idx::q_lane_offset(lane, s8));
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const float q = qv[s8][c4] * qmul;
                float qhf;
                const uint32_t pr = hi_lo_pair(q, qhf);  // q_hi | q_lo' << 16
                // column h: (q_hi, 0); column 8 + h: (q_lo', q_hi)
                bq[s8][c4] = n < 8 ? (pr & 0xffffu) : ((pr >> 16) | (pr << 16));
            }
        }
    }
    // Score of head n & 7 in both lanes n and n ^ 8: D[h] + 2^-12 D[8 + h].
    const float ca = n < 8 ? 1.0f : 1.0f / 4096.0f, cb = n < 8 ? 1.0f / 4096.0f : 1.0f;
    // PV A operand of weight w: row h (lanes n < 8) takes (w_hi, 0), row 8 + h takes
    // (w_lo', w_hi), w_hi = w rounded toward zero. r = pkrtz(w, w) = (w_hi, w_hi), then
    // r.lo = f16(r.lo * wb + w * wc) in place (lanes n < 8: w_hi; n >= 8: 2^12 (w - w_hi)),
    // then lanes n < 8 clear r.hi.
    const float wb = n < 8 ? 1.0f : -4096.0f, wc = n < 8 ? 0.0f : 4096.0f;
    const uint32_t hmask = n < 8 ? 0xffffu : 0xffffffffu;
    // cross-row exchanges (lane ^ 16, lane ^ 32) as ds_bpermute byte addresses
    const int bp16 = (lane ^ 16) << 2, bp32 = (lane ^ 32) << 2;
    auto xrow = [](int bp, float v) {
        return __int_as_float(__builtin_amdgcn_ds_bpermute(bp, __float_as_int(v)));
    };
    // transposed V reads: source lane m of group rg reads position 16rg + 4(m % 4) + m / 4;
    // segment s of that row sits at vrow[s ^ sw]
    const int srow = 16 * rg + 4 * (n & 3) + (n >> 2);
    const int sw = (srow >> 1) & 3;
    uint32_t vseg[4];
#pragma unroll
    for (int sg = 0; sg < 4; ++sg)
        vseg[sg] = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)(
            vb + 64 * srow + 16 * (sg ^ sw));

    // kG4 (at most 4 query heads per kv head): scores, probabilities and weights are held
    // compactly, lane (n, rg) with n = 4 pt + h holding head h's 4 positions 16rg + 4e + pt of
    // tile pt (one distinct value per lane and element, where the MFMA layout repeats each
    // four times); the tiles' weights are moved back into the PV operand layout per tile.
    // Norm records are stored in that order (nb index 16 rg + 4 pt + e), so a lane's four come
    // in two 16-byte reads.
    const int ptc = n >> 2;  // kG4: the lane's position tile
    const int nb_idx = kG4 ? (lane & 0x30) | ((lane & 3) << 2) | ((lane >> 2) & 3) : lane;
    const float c12 = 1.0f / 4096.0f;
    uint32_t awz[4] = {0u, 0u, 0u, 0u};  // kG4 PV operand: banks 1 and 3 (heads 4-7) stay 0

    for (int t0 = t_begin, par = 0; t0 < t_end; t0 += kChunkM, par ^= 1) {
        const int tn = t0 + kChunkM;  // next chunk
        const int jn = fhip_idx::chunk_first_page(tn, t_begin);  // its first split page
        const uint32_t pmask_n = tn < t_end ? (uint32_t)(vmask >> jn) & 0xfu : 0u;
        const bool full = pmask == 0xfu && tn <= t_end && tn <= min_len;

        // ---- QK: 4 tiles x 8 steps, K codes from this wave's DMA buffer
        float sc[4][4];  // !kG4 [pt][e]: position 16rg + 4e + pt, head n & 7
        float scc[4];    // kG4 [e]: position 16rg + 4e + ptc, head n & 3
        // all loads of this chunk are in (the V copies included)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // the V buffer PV reads below (the sync after the norm records orders these writes
        // before the transposed reads)
        if constexpr (kV2) store_v2(v2reg, vb + par * (kChunkM * 64), lane);
        const u32x4 kcs[4] = {kreg[0], kreg[1], kreg[2], kreg[3]};
        // 32 MFMA steps t = (tile pt, word s2, half): the A operand of step t holds the table
        // entries of bytes 2 half, 2 half + 1 of word s2 (coordinates 8 s2 + 4 half + 0..3).
        // Table reads run kLookAhead steps ahead of their MFMA, so their LDS latency is
        // covered by the MFMAs in between.
        constexpr int kLookAhead = 2;
        auto qk_a = [&](int t) -> u32x4 {
            const uint32_t w = kcs[t >> 3][(t >> 1) & 3];
            return (t & 1) ? pair2<2>(pk, w) : pair2<0>(pk, w);
        };
        {
            u32x4 ahead[kLookAhead + 1];
#pragma unroll
            for (int t = 0; t < kLookAhead; ++t) ahead[t] = qk_a(t);
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                if (t + kLookAhead < 32) ahead[(t + kLookAhead) % (kLookAhead + 1)] = qk_a(t + kLookAhead);
                const int s8 = t & 7;  // Q step 2 s2 + half
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8_t, ahead[t % (kLookAhead + 1)]),
                    __builtin_bit_cast(f16x8_t, u32x4{bq[s8][0], bq[s8][1], bq[s8][2], bq[s8][3]}),
                    d, 0, 0, 0);
                if ((t & 7) == 7) {
                    if constexpr (kG4) {
                        // tile pt's head-h score D[h] + 2^-12 D[8 + h] into lanes 4 pt + h
                        switch (t >> 3) {
                            case 0: compact_scores<0>(scc, d, c12); break;
                            case 1: compact_scores<1>(scc, d, c12); break;
                            case 2: compact_scores<2>(scc, d, c12); break;
                            default: compact_scores<3>(scc, d, c12); break;
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            // fma(ror8(d), cb, d * ca) with the row rotation folded into the
                            // fmac (the multiply reads d first, after the MFMA result is ready)
                            float v = d[e] * ca;
                            asm("v_fmac_f32_dpp %0, %1, %2 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1"
                                : "+v"(v)
                                : "v"(d[e]), "v"(cb));
                            sc[t >> 3][e] = v;
                        }
                    }
                    d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                }
                // keeps the scheduler from sinking the look-ahead reads to their MFMAs
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // ---- K norms; then the K and norm registers are free: all loads of the next chunk,
        // its V codes into the other V buffer. The previous chunk's nb reads are above the
        // transposed V reads' asm (a compiler barrier); the sync after the write keeps the
        // cross-lane reads below it also when no copy asm follows (the last chunk).
        nb[nb_idx] = nreg.pack();
        wave_lds_sync();
        uint8_t* vnext = vb + (par ^ 1) * (kChunkM * 64);
        if (tn < t_end) {
            if constexpr (kV2)
                load_v2(pages, jn, v_lane_off, v2reg);
            else
                dma_v(pages, jn, v_lane_off, vnext, lane);
            nreg = load_norms(pages, jn, pmask_n, tn, t_end, kvh, g, lane);
            load_k(pages, jn, kvh, g, lane, kreg);
        }
        float m_new, alpha;
        uint32_t aw[4][4];  // !kG4 [pt][e]
        uint32_t xw[4], yw[4];  // kG4: (w_hi, 0) and (w_lo', w_hi) of the lane's 4 weights
        if constexpr (kG4) {
            const f32x4_t n0 = *(const f32x4_t*)&nb[16 * rg + 4 * ptc];
            const f32x4_t n1 = *(const f32x4_t*)&nb[16 * rg + 4 * ptc + 2];
            const float kn[4] = {n0[0], n0[2], n1[0], n1[2]};
            const float vn[4] = {n0[1], n0[3], n1[1], n1[3]};
#pragma unroll
            for (int e = 0; e < 4; ++e) scc[e] *= kn[e];
            if (!full) {
                const bool row_ok = (pmask >> rg) & 1u;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (!(row_ok && t0 + 16 * rg + 4 * e + ptc < t_end)) scc[e] = -__builtin_inff();
            }
            float cmax = fmaxf(fmaxf(scc[0], scc[1]), fmaxf(scc[2], scc[3]));
            cmax = bank_max(cmax);
            cmax = fmaxf(cmax, xrow(bp16, cmax));
            cmax = fmaxf(cmax, xrow(bp32, cmax));
            m_new = fmaxf(m_run, cmax);
            alpha = m_run == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            float psum = 0.0f;
            const float mref = m_new == -__builtin_inff() ? 0.0f : m_new;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float pr = __builtin_amdgcn_exp2f(scc[e] - mref);
                psum += pr;
                const float w = pr * vn[e];
                // w_hi = w rounded toward zero; lo' = f16(2^12 (w - w_hi)) in place of r.lo
                uint32_t r = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(w, w));
                xw[e] = r & 0xffffu;
                asm("v_fma_mixlo_f16 %0, %0, %1, %2 op_sel_hi:[1,0,0]"
                    : "+v"(r)
                    : "v"(-4096.0f), "v"(w * 4096.0f));
                yw[e] = r;
            }
            psum = bank_sum(psum);
            psum += xrow(bp16, psum);
            psum += xrow(bp32, psum);
            l_run = l_run * alpha + psum;
        } else {
            float kn[16], vn[16];  // positions 16rg + j
#pragma unroll
            for (int j2 = 0; j2 < 8; ++j2) {
                const f32x4_t v = *(const f32x4_t*)&nb[16 * rg + 2 * j2];
                kn[2 * j2] = v[0];
                vn[2 * j2] = v[1];
                kn[2 * j2 + 1] = v[2];
                vn[2 * j2 + 1] = v[3];
            }
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int e = 0; e < 4; ++e) sc[pt][e] *= kn[4 * e + pt];
            if (!full) {
                const bool row_ok = (pmask >> rg) & 1u;
                const int lim = min(t_end, col_len);
#pragma unroll
                for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (!(row_ok && t0 + 16 * rg + 4 * e + pt < lim)) sc[pt][e] = -__builtin_inff();
            }
            float cmax = -__builtin_inff();
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int e = 0; e < 4; ++e) cmax = fmaxf(cmax, sc[pt][e]);
            cmax = fmaxf(cmax, xrow(bp16, cmax));
            cmax = fmaxf(cmax, xrow(bp32, cmax));
            m_new = fmaxf(m_run, cmax);
            alpha = m_run == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            // ---- probabilities, weights, B operands of PV
            float psum = 0.0f;
            const float mref = m_new == -__builtin_inff() ? 0.0f : m_new;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float pr = __builtin_amdgcn_exp2f(sc[pt][e] - mref);
                    psum += pr;
                    const float w = pr * vn[4 * e + pt];
                    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(w, w));
                    // in place: written in C, the compiler merges the halves with an extra v_bfi
                    asm("v_fma_mixlo_f16 %0, %0, %1, %2 op_sel_hi:[1,0,0]"
                        : "+v"(r)
                        : "v"(wb), "v"(w * wc));
                    aw[pt][e] = r & hmask;
                }
            }
            psum += xrow(bp16, psum);
            psum += xrow(bp32, psum);
            l_run = l_run * alpha + psum;
        }
        // rescale the accumulators when some head's max moved (each lane's alpha is that of
        // its accumulator slot's head)
        const bool moved_any =
            __ballot((n < ncols) && (!kG4 || n < 4) && (rg == 0) && (m_new > m_run)) != 0;
        if (moved_any) {
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[c][e] *= alpha;
        }
        m_run = m_new;

        // ---- PV: 8 dim tiles x 4 position tiles
        v2i_t tvs[8];
        {
            const uint32_t vo = (uint32_t)par * (kChunkM * 64);
            const uint32_t seg[4] = {vseg[0] + vo, vseg[1] + vo, vseg[2] + vo, vseg[3] + vo};
            read_v_codes(seg, tvs);
        }
        // out^T = V^T W^T: the V entries are the A operand (row m: dim 16c + (m ^ 1)), the
        // weights the B operand (column n: head slot n). 32 MFMA steps t = (position tile pt,
        // dim tile c): nibble 4pt + c4 of dim tile c's transposed read is the code of position
        // (pt, c4) at dim 16c + (n ^ 1); tile pt sits in word pt / 2, bytes 2 (pt % 2),
        // 2 (pt % 2) + 1. Table reads run kLookAhead steps ahead as in QK.
        auto pv_b = [&](int t) -> u32x4 {
            const int pt = t >> 3, c = t & 7;
            const uint32_t w = (uint32_t)tvs[c][pt >> 1];
            return (pt & 1) ? pair2<2>(pv, w) : pair2<0>(pv, w);
        };
        {
            constexpr int kAheadPv = kLookAhead;
            u32x4 ahead[kAheadPv + 1];
#pragma unroll
            for (int t = 0; t < kAheadPv; ++t) ahead[t] = pv_b(t);
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                if (t + kAheadPv < 32) ahead[(t + kAheadPv) % (kAheadPv + 1)] = pv_b(t + kAheadPv);
                const int pt = t >> 3, c = t & 7;
                if constexpr (kG4) {
                    if (c == 0) {  // tile pt's weights into the operand layout
                        switch (pt) {
                            case 0: expand_weights<0>(awz, xw, yw); break;
                            case 1: expand_weights<1>(awz, xw, yw); break;
                            case 2: expand_weights<2>(awz, xw, yw); break;
                            default: expand_weights<3>(awz, xw, yw); break;
                        }
                    }
                }
                const u32x4 bw = kG4 ? u32x4{awz[0], awz[1], awz[2], awz[3]}
                                     : u32x4{aw[pt][0], aw[pt][1], aw[pt][2], aw[pt][3]};
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8_t, ahead[t % (kAheadPv + 1)]),
                    __builtin_bit_cast(f16x8_t, bw), acc[c], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        pmask = pmask_n;
    }

    }  // vmask != 0

    // no copy may land in LDS after this point: the V buffers hold the merge state next
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- merge the workgroup's splits into the block's partial. Each wave leaves its state
    // in its own V buffer: acc[h][d] = slot h (hi) + 2^-12 slot 8 + h (lo'), lanes n and n ^ 8,
    // then m (log2 units) and l per head, and counts itself done; the last wave to finish
    // merges (no barrier: the others leave at once and free their slots). Each output (h, d)
    // sums the waves in wave order, weighted by exp2(m_w - max m) (0 for a wave with
    // m = -inf), whichever wave merges.
    // Head rows are kStRow floats apart (144: the 16 writing lanes of a 16-byte store, 4 heads
    // x 4 row groups, land in distinct banks); a lane's 4 values of dim tile c are dims
    // 16c + 4rg + 0..3 (element e holds dim e ^ 1), one 16-byte store.
    constexpr int kStRow = hd + 16;
    constexpr int kStM = kMaxG * kStRow, kStL = kStM + kMaxG;
    float* st = (float*)vbuf[wave][0];
    static_assert(sizeof(vbuf[0]) >= (kStL + kMaxG) * sizeof(float), "merge state");
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        f32x4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e ^ 1] = fmaf(ror8(acc[c][e]), 1.0f / 4096.0f, acc[c][e]);
        if (n < ncols) *(f32x4_t*)&st[n * kStRow + 16 * c + 4 * rg] = v;
    }
    if (n < ncols && rg == 0) {
        st[kStM + n] = m_run;
        st[kStL + n] = l_run;
    }
    // the state writes complete before the count (workgroup-scope release), and the merging
    // wave reads the others' states after it (acquire)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    int arrived = 0;
    if (lane == 0) arrived = atomicAdd(&waves_done, 1);
    arrived = __builtin_amdgcn_readfirstlane(arrived);
    if (arrived != kWavesM - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // one (head, 8-coordinate group) per lane and step: the head's wave weights once, then two
    // 16-byte reads per wave state and two 16-byte stores
    for (int it = lane; it < ncols * (hd / 8); it += 64) {
        const int h = it / (hd / 8), d0 = 8 * (it % (hd / 8));
        if (tq0 + h / G >= qs.seq_lens_count) continue;  // a column past the queries
        const int64_t vec = fhip_idx::partial_vector(h, tq0, G, qh, g);
        const int64_t prow = fhip_idx::partial_row(vec, nsplit, blk);
        float mw[kWavesM], M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < kWavesM; ++w) {
            mw[w] = ((const float*)vbuf[w][0])[kStM + h];
            M = fmaxf(M, mw[w]);
        }
        float L = 0.0f;
        f32x4_t A0 = {0.0f, 0.0f, 0.0f, 0.0f}, A1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < kWavesM; ++w) {
            const float* sw = (const float*)vbuf[w][0];
            if (mw[w] != -__builtin_inff()) {
                const float wt = __builtin_amdgcn_exp2f(mw[w] - M);
                L = fmaf(wt, sw[kStL + h], L);
                const f32x4_t a0 = *(const f32x4_t*)&sw[h * kStRow + d0];
                const f32x4_t a1 = *(const f32x4_t*)&sw[h * kStRow + d0 + 4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    A0[k] = fmaf(wt, a0[k], A0[k]);
                    A1[k] = fmaf(wt, a1[k], A1[k]);
                }
            }
        }
        float* pa = part_acc + prow * hd + d0;
        *(f32x4_t*)pa = A0;
        *(f32x4_t*)(pa + 4) = A1;
        if (d0 == 0) {  // m back in natural units
            part_ml[prow * 2 + 0] = M == -__builtin_inff() ? M : M * 0.6931471805599453f;
            part_ml[prow * 2 + 1] = L;
        }
    }
}

template <class Pages>
void launch_mfma_split(const float* qrot, const Queries& qsv, const Pages& pg,
                       const float* kcent, const float* vcent, int nq, int qh, int kvh,
                       int nsplit, bool v2, float* ml, float* acc, hipStream_t s) {
    // Causal prefill (queries at consecutive positions of one sequence: one shared block table,
    // lengths from start_pos) groups 8 / G consecutive queries per item so that they share the
    // MFMA columns and every code lookup; decode keeps one query per item.
    const int G = qh / kvh;
    const int tok = (!qsv.seq_lens && qsv.table_stride == 0 && nq > 1 && G < 8) ? 8 / G : 1;
    const int64_t items = ceil_div((int64_t)nq, tok);
    // one workgroup per (item, kv head, kSplit-position block): the block count is the
    // partial layout's split count; the (item, block) pairs are padded to a multiple of the
    // XCD count (the kernel's index spreads them, not heads, over the XCDs)
    const int64_t wgs = ceil_div(items * nsplit, kXcds) * kXcds * kvh;
    Queries q2 = qsv;
    q2.seq_lens_count = nq;
    const bool g4 = G <= 4 && tok == 1;
    auto kern = v2 ? (g4 ? tq_attn_mfma_kernel<Pages, true, true> : tq_attn_mfma_kernel<Pages, false, true>)
                   : (g4 ? tq_attn_mfma_kernel<Pages, true, false> : tq_attn_mfma_kernel<Pages, false, false>);
    hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(64 * kWavesM), 0, s, qrot, q2, pg, kcent,
                       vcent, qh, kvh, 1.0f / sqrtf(128.0f), ml, acc, nsplit, nsplit, tok);
}

struct AttnArgs {
    void* out;
    const void* q;
    Queries qs;
    int nq;
    const float *krot, *vrot, *kcent, *vcent;
    int qh, kvh, hd, kbits, vbits;
    void* ws;
};

size_t ws_layout(int nq, int qh, int hd, int max_tokens, size_t* off_ml, size_t* off_acc,
                 int* nsplit) {
    const int ns = max_tokens > 0 ? (max_tokens + kSplit - 1) / kSplit : 1;
    const size_t qrot = (size_t)nq * qh * hd * sizeof(float);
    const size_t ml = (size_t)nq * qh * ns * 2 * sizeof(float);
    const size_t acc = (size_t)nq * qh * ns * hd * sizeof(float);
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    if (off_ml) *off_ml = al(qrot);
    if (off_acc) *off_acc = al(qrot) + al(ml);
    if (nsplit) *nsplit = ns;
    return al(qrot) + al(ml) + al(acc);
}

template <int KB, int VB, class Pages>
void launch_split(const AttnArgs& a, const Pages& pg, int nsplit, float* ml, float* acc,
                  hipStream_t s) {
    dim3 grid(nsplit, a.kvh, a.nq);
    const int kwords = ((a.hd * a.kbits + 7) / 8 + 3) / 4, vwords = ((a.hd * a.vbits + 7) / 8 + 3) / 4;
    const size_t lds = (size_t)kSub * ((kwords | 1) + (vwords | 1)) * sizeof(uint32_t);
    hipLaunchKernelGGL((tq_attn_split_kernel<KB, VB, Pages>), grid, dim3(256), lds, s,
                       (const float*)a.ws, a.qs, pg, a.kcent, a.vcent, a.kbits, a.vbits, a.qh,
                       a.kvh, a.hd, 1.0f / sqrtf((float)a.hd), ml, acc, nsplit);
}

template <class Pages>
int launch_attention(const AttnArgs& a, const Pages& pg, hipStream_t s) {
    if (a.nq == 0) return hipSuccess;
    size_t off_ml, off_acc;
    int nsplit;
    ws_layout(a.nq, a.qh, a.hd, a.qs.max_blocks * FHIP_PAGE_TOKENS, &off_ml, &off_acc, &nsplit);
    float* qrot = (float*)a.ws;
    float* ml = (float*)((char*)a.ws + off_ml);
    float* acc = (float*)((char*)a.ws + off_acc);
    const int nvec = a.nq * a.qh;
    // Many vectors (prefill): both rotations as batched MFMA products (the VALU kernels'
    // per-workgroup copies of Pi would cross L2 once per 8 vectors); the merged outputs reuse
    // the q_rot buffer, which the split kernel has finished with.
    const bool batched_rot = nvec >= kMfmaRotVecs && a.hd == 128 &&
                             fhip_host::aligned16(a.q) && fhip_host::aligned16(a.out);
    if (batched_rot) {
        const int e = fhip_internal::tq_rotate_rows(a.q, a.krot, qrot, nvec, s);
        if (e != hipSuccess) return e;
    } else {
        const unsigned rot_groups = (unsigned)ceil_div(nvec, kRotVecs);
        hipLaunchKernelGGL(tq_attn_prerotate_kernel, dim3(rot_groups), dim3(256), 0, s,
                           (const uint16_t*)a.q, a.krot, qrot, a.hd, nvec);
    }
    if (a.kbits == 4 && (a.vbits == 4 || a.vbits == 2) && a.hd == 128 && a.qh / a.kvh <= 8)
        launch_mfma_split(qrot, a.qs, pg, a.kcent, a.vcent, a.nq, a.qh, a.kvh, nsplit,
                          a.vbits == 2, ml, acc, s);
    else if (a.kbits == 4 && a.vbits == 4)
        launch_split<4, 4>(a, pg, nsplit, ml, acc, s);
    else if (a.kbits == 4 && a.vbits == 2)
        launch_split<4, 2>(a, pg, nsplit, ml, acc, s);
    else
        launch_split<0, 0>(a, pg, nsplit, ml, acc, s);
    if (batched_rot) {
        if (nsplit <= kMergeWaveMaxSplits)
            hipLaunchKernelGGL(tq_attn_merge_wave_kernel, dim3((unsigned)ceil_div(nvec, 4)),
                               dim3(256), 0, s, a.qs, ml, acc, a.qh, a.hd, nsplit, (int64_t)nvec,
                               qrot);
        else
            hipLaunchKernelGGL((tq_attn_combine_kernel<true, true>),
                               dim3((unsigned)ceil_div(nvec, kCombHeads)), dim3(256),
                               combine_lds_bytes(a.hd, nsplit, true), s, a.qs, ml, acc, a.vrot,
                               (uint16_t*)a.out, a.qh, a.hd, nsplit, (int64_t)nvec, qrot);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return fhip_internal::tq_rotate_back_rows(qrot, a.vrot, a.out, nvec, s);
    }
    auto comb = a.hd <= kRotLdsMaxHd ? tq_attn_combine_kernel<true> : tq_attn_combine_kernel<false>;
    hipLaunchKernelGGL(comb, dim3((unsigned)ceil_div(nvec, kCombHeads)), dim3(256),
                       combine_lds_bytes(a.hd, nsplit), s, a.qs, ml, acc, a.vrot,
                       (uint16_t*)a.out, a.qh, a.hd, nsplit, (int64_t)nvec, nullptr);
    return hipGetLastError();
}

// Split-partial scratch of fhip_launch_attention_paged_tq_noalloc: one copy per device, held
// until the process ends. Host code never passes the name `scratch` to a kernel (on the host
// it is a stand-in, not a device address); it resolves each device's address once with
// hipGetSymbolAddress and passes that.
constexpr size_t kNoAllocScratchBytes = FHIP_TQ_ATTN_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The scratch address on `dev`, looked up on the first call for that device (made current for
// the lookup, then restored).
hipError_t scratch_on_device(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) {
            hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess) return e;
        if (!ptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

bool attn_shape_ok(int qh, int kvh, int hd, int kbits, int vbits) {
    return kvh > 0 && qh > 0 && qh % kvh == 0 && qh / kvh <= kMaxG && hd % 8 == 0 && hd > 0 &&
           hd <= kMaxHd && kbits >= 1 && kbits <= 8 && vbits >= 1 && vbits <= 8 &&
           (hd * kbits + 7) / 8 <= kMaxPd && (hd * vbits + 7) / 8 <= kMaxPd && 256 % (hd / 8) == 0;
}

}  // namespace

extern "C" {

size_t fhip_attention_tq_workspace_bytes(int batch, int num_q_heads, int head_dim,
                                         int max_blocks) {
    if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_blocks <= 0) return 0;
    return ws_layout(batch, num_q_heads, head_dim, max_blocks * FHIP_PAGE_TOKENS, nullptr, nullptr,
                     nullptr);
}

int fhip_launch_attention_tq_decode(void* output, const void* q, const int32_t* block_table,
                                    const int32_t* seq_lens, int batch, int max_blocks,
                                    int num_pages, const void* k_packed_pool,
                                    const void* k_norms_pool, const void* v_packed_pool,
                                    const void* v_norms_pool, int64_t page_k_packed_bytes,
                                    int64_t page_k_norm_bytes, int64_t page_v_packed_bytes,
                                    int64_t page_v_norm_bytes, const float* k_rotation,
                                    const float* v_rotation, const float* k_centroids,
                                    const float* v_centroids, int num_q_heads, int num_kv_heads,
                                    int head_dim, int key_bits, int value_bits, void* workspace,
                                    fhip_stream_t stream) {
    if (batch < 0 || max_blocks <= 0 || num_pages < 0 ||
        !attn_shape_ok(num_q_heads, num_kv_heads, head_dim, key_bits, value_bits))
        return hipErrorInvalidValue;
    if ((int64_t)batch * num_q_heads > (int64_t)1 << 30 || batch > 65535 ||
        max_blocks * (int64_t)FHIP_PAGE_TOKENS > kMaxTokensTq)
        return hipErrorInvalidValue;
    // each page stride must cover a page: the kernels read rows [0, 16) of every page
    const int64_t pdk = (head_dim * key_bits + 7) / 8, pdv = (head_dim * value_bits + 7) / 8;
    if (page_k_packed_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * pdk ||
        page_v_packed_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * pdv ||
        page_k_norm_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * 2 ||
        page_v_norm_bytes < (int64_t)FHIP_PAGE_TOKENS * num_kv_heads * 2)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (!output || !q || !block_table || !seq_lens || !k_packed_pool || !k_norms_pool ||
        !v_packed_pool || !v_norms_pool || !k_rotation || !v_rotation || !k_centroids ||
        !v_centroids || !workspace)
        return hipErrorInvalidValue;
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{block_table, max_blocks, max_blocks, seq_lens, 0, 0, batch};
    a.nq = batch;
    a.krot = k_rotation;
    a.vrot = v_rotation;
    a.kcent = k_centroids;
    a.vcent = v_centroids;
    a.qh = num_q_heads;
    a.kvh = num_kv_heads;
    a.hd = head_dim;
    a.kbits = key_bits;
    a.vbits = value_bits;
    a.ws = workspace;
    PoolPages pg{(const uint8_t*)k_packed_pool, (const uint8_t*)k_norms_pool,
                 (const uint8_t*)v_packed_pool, (const uint8_t*)v_norms_pool,
                 page_k_packed_bytes, page_k_norm_bytes, page_v_packed_bytes, page_v_norm_bytes,
                 num_pages};
    return launch_attention(a, pg, fhip_host::as_stream(stream));
}

int fhip_launch_attention_tq_decode_ptrs(void* output, const void* q, const int32_t* block_table,
                                         const int32_t* seq_lens, int batch, int max_blocks,
                                         int num_pages, const void** k_packed_ptrs,
                                         const void** k_norms_ptrs, const void** v_packed_ptrs,
                                         const void** v_norms_ptrs, const float* k_rotation,
                                         const float* v_rotation, const float* k_centroids,
                                         const float* v_centroids, int num_q_heads,
                                         int num_kv_heads, int head_dim, int key_bits,
                                         int value_bits, void* workspace,
                                         fhip_stream_t stream) {
    if (batch < 0 || max_blocks <= 0 || num_pages < 0 ||
        !attn_shape_ok(num_q_heads, num_kv_heads, head_dim, key_bits, value_bits))
        return hipErrorInvalidValue;
    if ((int64_t)batch * num_q_heads > (int64_t)1 << 30 || batch > 65535 ||
        max_blocks * (int64_t)FHIP_PAGE_TOKENS > kMaxTokensTq)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (!output || !q || !block_table || !seq_lens || (num_pages > 0 && (!k_packed_ptrs ||
        !k_norms_ptrs || !v_packed_ptrs || !v_norms_ptrs)) || !k_rotation || !v_rotation ||
        !k_centroids || !v_centroids || !workspace)
        return hipErrorInvalidValue;
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{block_table, max_blocks, max_blocks, seq_lens, 0, 0, batch};
    a.nq = batch;
    a.krot = k_rotation;
    a.vrot = v_rotation;
    a.kcent = k_centroids;
    a.vcent = v_centroids;
    a.qh = num_q_heads;
    a.kvh = num_kv_heads;
    a.hd = head_dim;
    a.kbits = key_bits;
    a.vbits = value_bits;
    a.ws = workspace;
    PtrPages pg{(const uint8_t* const*)k_packed_ptrs, (const uint8_t* const*)k_norms_ptrs,
                (const uint8_t* const*)v_packed_ptrs, (const uint8_t* const*)v_norms_ptrs,
                num_pages};
    return launch_attention(a, pg, fhip_host::as_stream(stream));
}

}  // extern "C"

namespace fhip_internal {

int attention_tq_decode_ptrs_staged(void* output, const void* q, const int32_t* block_table,
                                    const int32_t* seq_lens, int batch, int max_blocks,
                                    int table_stride, int num_pages, const void** k_packed_ptrs,
                                    const void** k_norms_ptrs, const void** v_packed_ptrs,
                                    const void** v_norms_ptrs, const float* k_rotation,
                                    const float* v_rotation, const float* k_centroids,
                                    const float* v_centroids, int num_q_heads, int num_kv_heads,
                                    int head_dim, int key_bits, int value_bits, void* workspace,
                                    hipStream_t stream) {
    if (batch < 0 || max_blocks <= 0 || num_pages < 0 || table_stride < max_blocks ||
        !attn_shape_ok(num_q_heads, num_kv_heads, head_dim, key_bits, value_bits))
        return hipErrorInvalidValue;
    if ((int64_t)batch * num_q_heads > (int64_t)1 << 30 || batch > 65535 ||
        max_blocks * (int64_t)FHIP_PAGE_TOKENS > kMaxTokensTq)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (!output || !q || !block_table || !seq_lens || (num_pages > 0 && (!k_packed_ptrs ||
        !k_norms_ptrs || !v_packed_ptrs || !v_norms_ptrs)) || !k_rotation || !v_rotation ||
        !k_centroids || !v_centroids || !workspace)
        return hipErrorInvalidValue;
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{block_table, table_stride, max_blocks, seq_lens, 0, 0, batch};
    a.nq = batch;
    a.krot = k_rotation;
    a.vrot = v_rotation;
    a.kcent = k_centroids;
    a.vcent = v_centroids;
    a.qh = num_q_heads;
    a.kvh = num_kv_heads;
    a.hd = head_dim;
    a.kbits = key_bits;
    a.vbits = value_bits;
    a.ws = workspace;
    PtrPages pg{(const uint8_t* const*)k_packed_ptrs, (const uint8_t* const*)k_norms_ptrs,
                (const uint8_t* const*)v_packed_ptrs, (const uint8_t* const*)v_norms_ptrs,
                num_pages};
    return launch_attention(a, pg, stream);
}

}  // namespace fhip_internal

extern "C" {

// The reference interface: one sequence, num_tokens queries at positions
// start_pos .. start_pos + num_tokens - 1, per-block pointer arrays. `ws` holds the split
// partials (fhip_attention_tq_workspace_bytes(num_tokens, qh, hd, ceil(kv_len / 16)) bytes);
// null asks for a stream-ordered allocation freed on the same stream.
static int attention_paged_tq_ref(void* output, const void* q, const int* block_table,
                                  const void** k_packed_ptrs, const void** k_norms_ptrs,
                                  const void** v_packed_ptrs, const void** v_norms_ptrs,
                                  const float* k_rotation, const float* v_rotation,
                                  const float* k_centroids, const float* v_centroids,
                                  int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                                  int kv_len, int start_pos, int key_bits, int value_bits,
                                  int k_packed_dim_per_head, int v_packed_dim_per_head,
                                  void* ws, size_t ws_bytes, hipStream_t s) {
    if (num_tokens < 0 || kv_len < 0 || start_pos < 0 || kv_len > kMaxTokensTq ||
        !attn_shape_ok(num_q_heads, num_kv_heads, head_dim, key_bits, value_bits) ||
        k_packed_dim_per_head != (head_dim * key_bits + 7) / 8 ||
        v_packed_dim_per_head != (head_dim * value_bits + 7) / 8 || num_tokens > 65535)
        return hipErrorInvalidValue;
    if (num_tokens == 0) return hipSuccess;
    if (!output || !q || !k_rotation || !v_rotation || !k_centroids || !v_centroids)
        return hipErrorInvalidValue;
    const int nblocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    if (nblocks > 0 && (!block_table || !k_packed_ptrs || !k_norms_ptrs || !v_packed_ptrs ||
                        !v_norms_ptrs))
        return hipErrorInvalidValue;
    const int mb = nblocks > 0 ? nblocks : 1;
    const size_t bytes = ws_layout(num_tokens, num_q_heads, head_dim, mb * FHIP_PAGE_TOKENS,
                                   nullptr, nullptr, nullptr);
    const bool own = ws == nullptr;
    if (!own && ws_bytes < bytes) return hipErrorInvalidValue;
    if (own) {
        hipError_t e = hipMallocAsync(&ws, bytes, s);
        if (e != hipSuccess) return e;
    }
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{(const int32_t*)block_table, 0, mb, nullptr, kv_len, start_pos, num_tokens};
    a.nq = num_tokens;
    a.krot = k_rotation;
    a.vrot = v_rotation;
    a.kcent = k_centroids;
    a.vcent = v_centroids;
    a.qh = num_q_heads;
    a.kvh = num_kv_heads;
    a.hd = head_dim;
    a.kbits = key_bits;
    a.vbits = value_bits;
    a.ws = ws;
    PtrPages pg{(const uint8_t* const*)k_packed_ptrs, (const uint8_t* const*)k_norms_ptrs,
                (const uint8_t* const*)v_packed_ptrs, (const uint8_t* const*)v_norms_ptrs,
                0x7fffffff};
    int r = launch_attention(a, pg, s);
    if (own) {
        hipError_t e2 = hipFreeAsync(ws, s);
        if (r == hipSuccess) r = e2;
    }
    return r;
}

int fhip_launch_attention_paged_tq(void* output, const void* q, const int* block_table,
                                   const void** k_packed_ptrs, const void** k_norms_ptrs,
                                   const void** v_packed_ptrs, const void** v_norms_ptrs,
                                   const float* k_rotation, const float* v_rotation,
                                   const float* k_centroids, const float* v_centroids,
                                   int num_tokens, int num_q_heads, int num_kv_heads,
                                   int head_dim, int kv_len, int start_pos, int key_bits,
                                   int value_bits, int k_packed_dim_per_head,
                                   int v_packed_dim_per_head, fhip_stream_t stream) {
    return attention_paged_tq_ref(output, q, block_table, k_packed_ptrs, k_norms_ptrs,
                                  v_packed_ptrs, v_norms_ptrs, k_rotation, v_rotation,
                                  k_centroids, v_centroids, num_tokens, num_q_heads,
                                  num_kv_heads, head_dim, kv_len, start_pos, key_bits,
                                  value_bits, k_packed_dim_per_head, v_packed_dim_per_head,
                                  nullptr, 0, fhip_host::as_stream(stream));
}

int fhip_launch_attention_paged_tq_noalloc(void* output, const void* q, const int* block_table,
                                           const void** k_packed_ptrs, const void** k_norms_ptrs,
                                           const void** v_packed_ptrs, const void** v_norms_ptrs,
                                           const float* k_rotation, const float* v_rotation,
                                           const float* k_centroids, const float* v_centroids,
                                           int num_tokens, int num_q_heads, int num_kv_heads,
                                           int head_dim, int kv_len, int start_pos, int key_bits,
                                           int value_bits, int k_packed_dim_per_head,
                                           int v_packed_dim_per_head, fhip_stream_t stream) {
    if (num_tokens < 0 || kv_len < 0 || num_q_heads <= 0 || head_dim <= 0)
        return hipErrorInvalidValue;
    if (num_tokens == 0) return hipSuccess;
    const int nblocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    const size_t need = ws_layout(num_tokens, num_q_heads, head_dim,
                                  (nblocks > 0 ? nblocks : 1) * FHIP_PAGE_TOKENS, nullptr,
                                  nullptr, nullptr);
    if (need > kNoAllocScratchBytes) return hipErrorOutOfMemory;
    hipStream_t s = fhip_host::as_stream(stream);
    int dev = -1;
    hipError_t e = hipStreamGetDevice(s, &dev);
    if (e != hipSuccess) return e;
    void* ws = nullptr;
    if ((e = scratch_on_device(dev, &ws)) != hipSuccess) return e;
    return attention_paged_tq_ref(output, q, block_table, k_packed_ptrs, k_norms_ptrs,
                                  v_packed_ptrs, v_norms_ptrs, k_rotation, v_rotation,
                                  k_centroids, v_centroids, num_tokens, num_q_heads,
                                  num_kv_heads, head_dim, kv_len, start_pos, key_bits,
                                  value_bits, k_packed_dim_per_head, v_packed_dim_per_head, ws,
                                  kNoAllocScratchBytes, s);
}

int fhip_launch_attention_paged_tq_ws(void* output, const void* q, const int* block_table,
                                      const void** k_packed_ptrs, const void** k_norms_ptrs,
                                      const void** v_packed_ptrs, const void** v_norms_ptrs,
                                      const float* k_rotation, const float* v_rotation,
                                      const float* k_centroids, const float* v_centroids,
                                      int num_tokens, int num_q_heads, int num_kv_heads,
                                      int head_dim, int kv_len, int start_pos, int key_bits,
                                      int value_bits, int k_packed_dim_per_head,
                                      int v_packed_dim_per_head, void* workspace,
                                      size_t workspace_bytes, fhip_stream_t stream) {
    if (!workspace) return hipErrorInvalidValue;
    return attention_paged_tq_ref(output, q, block_table, k_packed_ptrs, k_norms_ptrs,
                                  v_packed_ptrs, v_norms_ptrs, k_rotation, v_rotation,
                                  k_centroids, v_centroids, num_tokens, num_q_heads,
                                  num_kv_heads, head_dim, kv_len, start_pos, key_bits,
                                  value_bits, k_packed_dim_per_head, v_packed_dim_per_head,
                                  workspace, workspace_bytes, fhip_host::as_stream(stream));
}

}  // extern "C"

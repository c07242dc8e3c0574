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
};

// Query q_i reads block-table row i (stride 0: one shared table) and attends to
// seq_lens[i] positions, or min(start_pos + i + 1, kv_len) when seq_lens is null.
struct Queries {
    const int32_t* table;
    int64_t table_stride;
    int max_blocks;
    const int32_t* seq_lens;
    int kv_len, start_pos;
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

// 1. q_rot[qi, h, :] = Pi_k q[qi, h, :] (sequential fp32 dot, attention_paged_tq.cu:102-113).
__global__ __launch_bounds__(256) void tq_attn_prerotate_kernel(const uint16_t* __restrict__ q,
                                                                const float* __restrict__ rot,
                                                                float* __restrict__ qrot,
                                                                int hd) {
    __shared__ float qs[kMaxHd];
    const int64_t v = blockIdx.x;
    for (int j = threadIdx.x; j < hd; j += blockDim.x) qs[j] = h2f(q[v * hd + j]);
    __syncthreads();
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        const float* pr = rot + (int64_t)i * hd;
        float dot = 0.0f;
        for (int j = 0; j < hd; ++j) dot += pr[j] * qs[j];
        qrot[v * hd + i] = dot;
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
    const int split = blockIdx.x, kvhead = blockIdx.y, qi = blockIdx.z;
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

// 3. Merge the splits of one (query, q head) and unrotate: out = fp16(Pi_v^T (acc / l)).
__global__ __launch_bounds__(256) void tq_attn_combine_kernel(
    Queries qs, const float* __restrict__ part_ml, const float* __restrict__ part_acc,
    const float* __restrict__ vrot, uint16_t* __restrict__ out, int qh, int hd, int nsplit) {
    __shared__ float o[kMaxHd];
    __shared__ float wts[kSplit];  // per split weights (nsplit <= kSplit)
    __shared__ float Lsum;
    const int64_t head = blockIdx.x;  // qi * qh + h
    const int qi = (int)(head / qh);
    const int clen = qs.causal_len(qi);
    const int ns = (clen + kSplit - 1) / kSplit;
    if (threadIdx.x == 0) {
        float M = -__builtin_inff();
        for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, part_ml[(head * nsplit + sp) * 2]);
        float L = 0.0f;
        for (int sp = 0; sp < ns; ++sp) {
            const float m = part_ml[(head * nsplit + sp) * 2];
            const float wgt = (m == -__builtin_inff()) ? 0.0f : expf(m - M);
            wts[sp] = wgt;
            L += part_ml[(head * nsplit + sp) * 2 + 1] * wgt;
        }
        Lsum = L;
    }
    __syncthreads();
    const float inv = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float a = 0.0f;
        for (int sp = 0; sp < ns; ++sp) a += part_acc[(head * nsplit + sp) * hd + d] * wts[sp];
        o[d] = a * inv;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        float dot = 0.0f;
        for (int j = 0; j < hd; ++j) dot += vrot[(int64_t)j * hd + i] * o[j];
        out[head * hd + i] = (uint16_t)f2h(dot);
    }
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
    hipLaunchKernelGGL(tq_attn_prerotate_kernel, dim3(a.nq * a.qh), dim3(128), 0, s,
                       (const uint16_t*)a.q, a.krot, qrot, a.hd);
    if (a.kbits == 4 && a.vbits == 4)
        launch_split<4, 4>(a, pg, nsplit, ml, acc, s);
    else if (a.kbits == 4 && a.vbits == 2)
        launch_split<4, 2>(a, pg, nsplit, ml, acc, s);
    else
        launch_split<0, 0>(a, pg, nsplit, ml, acc, s);
    hipLaunchKernelGGL(tq_attn_combine_kernel, dim3(a.nq * a.qh), dim3(128), 0, s, a.qs, ml, acc,
                       a.vrot, (uint16_t*)a.out, a.qh, a.hd, nsplit);
    return hipGetLastError();
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
        max_blocks * (int64_t)FHIP_PAGE_TOKENS > (int64_t)kSplit * kSplit)
        return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    if (!output || !q || !block_table || !seq_lens || !k_packed_pool || !k_norms_pool ||
        !v_packed_pool || !v_norms_pool || !k_rotation || !v_rotation || !k_centroids ||
        !v_centroids || !workspace)
        return hipErrorInvalidValue;
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{block_table, max_blocks, max_blocks, seq_lens, 0, 0};
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

// The reference interface: one sequence, num_tokens queries at positions
// start_pos .. start_pos + num_tokens - 1, per-block pointer arrays. The split partials
// live in a stream-ordered allocation freed on the same stream.
int fhip_launch_attention_paged_tq(void* output, const void* q, const int* block_table,
                                   const void** k_packed_ptrs, const void** k_norms_ptrs,
                                   const void** v_packed_ptrs, const void** v_norms_ptrs,
                                   const float* k_rotation, const float* v_rotation,
                                   const float* k_centroids, const float* v_centroids,
                                   int num_tokens, int num_q_heads, int num_kv_heads,
                                   int head_dim, int kv_len, int start_pos, int key_bits,
                                   int value_bits, int k_packed_dim_per_head,
                                   int v_packed_dim_per_head, fhip_stream_t stream) {
    if (num_tokens < 0 || kv_len < 0 || start_pos < 0 ||
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
    hipStream_t s = fhip_host::as_stream(stream);
    const int mb = nblocks > 0 ? nblocks : 1;
    const size_t bytes = ws_layout(num_tokens, num_q_heads, head_dim, mb * FHIP_PAGE_TOKENS,
                                   nullptr, nullptr, nullptr);
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, bytes, s);
    if (e != hipSuccess) return e;
    AttnArgs a;
    a.out = output;
    a.q = q;
    a.qs = Queries{(const int32_t*)block_table, 0, mb, nullptr, kv_len, start_pos};
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
    hipError_t e2 = hipFreeAsync(ws, s);
    if (r != hipSuccess) return r;
    return e2;
}

}  // extern "C"

// Elementwise and row-normalisation kernels for gfx950: add, SwiGLU (silu_mul), RMSNorm,
// fused residual-add + RMSNorm, RoPE and embedding gather.
//
// All of these are HBM-bound streams. Every kernel moves 16 bytes per lane per access
// (global_load/store_dwordx4), keeps each row in registers so that it crosses HBM once,
// and reduces with wave64 DPP steps, using LDS only to combine the per-wave partials.
#include "fhip_common.h"

using namespace fhip;

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 2;  // 16-byte vectors per lane per streaming pass

// ---------------------------------------------------------------------------------------
// add: out = a + b (add.cu:5-14). The fp32 sum of two fp16 (or bf16) values rounded once to
// the storage type equals the directly rounded sum, so this is bit-exact with __hadd.
// ---------------------------------------------------------------------------------------
template <class Tr>
__global__ __launch_bounds__(kBlock) void add_vec_kernel(void* __restrict__ out,
                                                         const void* __restrict__ a,
                                                         const void* __restrict__ b,
                                                         int64_t n) {
    constexpr int V = Tr::kVec;
    const int64_t nvec = n / V;
    const int64_t v0 = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    u32x4 va[kUnroll], vb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kBlock;
        if (v < nvec) {
            va[u] = ld16((const char*)a + v * 16);
            vb[u] = ld16((const char*)b + v * 16);
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kBlock;
        if (v < nvec) {
            float x[V], y[V];
            unpack16<Tr>(va[u], x);
            unpack16<Tr>(vb[u], y);
#pragma unroll
            for (int i = 0; i < V; ++i) x[i] += y[i];
            st16((char*)out + v * 16, pack16<Tr>(x));
        }
    }
    if (blockIdx.x == 0) {
        const int64_t i = nvec * V + threadIdx.x;
        if (i < n) st1<Tr>(out, i, ld1<Tr>(a, i) + ld1<Tr>(b, i));
    }
}

template <class Tr>
__global__ __launch_bounds__(kBlock) void add_scalar_kernel(void* __restrict__ out,
                                                            const void* __restrict__ a,
                                                            const void* __restrict__ b,
                                                            int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock)
        st1<Tr>(out, i, ld1<Tr>(a, i) + ld1<Tr>(b, i));
}

// ---------------------------------------------------------------------------------------
// silu_mul: out = silu(gate) * up, silu(g) = g / (1 + exp(-g)) in fp32 (silu_mul.cu:17-22).
// exp(-g) is the hardware exp2 of -g*log2(e) and the quotient a hardware reciprocal, each
// within ~1 ulp of fp32, so the fp32 result is within a few 1e-7 relative of the IEEE
// expression (the special values agree too: g = -inf gives NaN, large negative g gives -0),
// and the IEEE divide and libm exp would otherwise make this stream VALU-bound.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float silu_f32(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

template <class Tr>
__global__ __launch_bounds__(kBlock) void silu_mul_vec_kernel(void* __restrict__ out,
                                                              const void* __restrict__ gate,
                                                              const void* __restrict__ up,
                                                              int64_t n) {
    constexpr int V = Tr::kVec;
    const int64_t nvec = n / V;
    const int64_t v0 = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    u32x4 vg[kUnroll], vu[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kBlock;
        if (v < nvec) {
            vg[u] = ld16_stream((const char*)gate + v * 16);
            vu[u] = ld16_stream((const char*)up + v * 16);
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = v0 + (int64_t)u * kBlock;
        if (v < nvec) {
            float g[V], x[V];
            unpack16<Tr>(vg[u], g);
            unpack16<Tr>(vu[u], x);
#pragma unroll
            for (int i = 0; i < V; ++i) g[i] = silu_f32(g[i]) * x[i];
            st16_stream((char*)out + v * 16, pack16<Tr>(g));
        }
    }
    if (blockIdx.x == 0) {
        const int64_t i = nvec * V + threadIdx.x;
        if (i < n) st1<Tr>(out, i, silu_f32(ld1<Tr>(gate, i)) * ld1<Tr>(up, i));
    }
}

template <class Tr>
__global__ __launch_bounds__(kBlock) void silu_mul_scalar_kernel(void* __restrict__ out,
                                                                 const void* __restrict__ gate,
                                                                 const void* __restrict__ up,
                                                                 int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kBlock)
        st1<Tr>(out, i, silu_f32(ld1<Tr>(gate, i)) * ld1<Tr>(up, i));
}

// ---------------------------------------------------------------------------------------
// RMSNorm (rmsnorm.cu:10-67), optionally fused with the residual add that precedes it in
// the engine (engine.rs:692-697): one workgroup per row, the row held in registers
// (kVpt 16-byte vectors per lane), so x (and the residual) cross HBM once.
//   kResid = false: out = x * inv * w,                       x = in
//   kResid = true : h = round(h + delta) stored back to h;  out = h * inv * w
// inv = 1 / sqrt(sum(x^2) / cols + eps), products evaluated as (x * inv) * w.
// ---------------------------------------------------------------------------------------
template <class Tr, bool kResid, int kVpt>
__global__ __launch_bounds__(1024) void rmsnorm_vec_kernel(void* __restrict__ out,
                                                           void* __restrict__ resid,
                                                           const void* __restrict__ in,
                                                           const void* __restrict__ weight,
                                                           float eps, int cols) {
    constexpr int V = Tr::kVec;
    __shared__ float red[16];
    const int bs = blockDim.x;
    const int nvec = cols / V;
    const int64_t rowoff = (int64_t)blockIdx.x * cols * (int64_t)sizeof(typename Tr::S);
    const char* xin = (const char*)in + rowoff;
    char* hres = (char*)resid + rowoff;
    char* yout = (char*)out + rowoff;

    // Every load (row, residual, weight) goes out at once with clamped indices (lanes past
    // the row end reload its last vector and store nothing): a guarded load, or the weight
    // loaded after the reduction, would each add a memory round trip to this short kernel.
    float x[kVpt][V];
    u32x4 raw[kVpt], rres[kVpt], wraw[kVpt];
#pragma unroll
    for (int k = 0; k < kVpt; ++k) {
        const int64_t vc = min(k * bs + (int)threadIdx.x, nvec - 1);
        raw[k] = ld16(xin + vc * 16);
        if constexpr (kResid) rres[k] = ld16(hres + vc * 16);
        wraw[k] = ld16((const char*)weight + vc * 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first use
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kVpt; ++k) {
        const int vi = k * bs + threadIdx.x;
        unpack16<Tr>(raw[k], x[k]);
        if constexpr (kResid) {
            float h[V];
            unpack16<Tr>(rres[k], h);
#pragma unroll
            for (int i = 0; i < V; ++i) x[k][i] = round_to<Tr>(h[i] + x[k][i]);
            if (vi < nvec) st16(hres + (int64_t)vi * 16, pack16<Tr>(x[k]));
        }
        if (vi < nvec) {
#pragma unroll
            for (int i = 0; i < V; ++i) ss += x[k][i] * x[k][i];
        }
    }
    // workgroup sum (waves in order) behind an LDS-only barrier: __syncthreads would also
    // wait for the residual stores above
    {
        const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        lds_barrier();
        float t = 0.0f;
        for (int w = 0; w < (bs + kWave - 1) / kWave; ++w) t += red[w];
        ss = t;
    }
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int k = 0; k < kVpt; ++k) {
        const int vi = k * bs + threadIdx.x;
        if (vi < nvec) {
            float w[V];
            unpack16<Tr>(wraw[k], w);
#pragma unroll
            for (int i = 0; i < V; ++i) x[k][i] = x[k][i] * inv * w[i];
            st16(yout + (int64_t)vi * 16, pack16<Tr>(x[k]));
        }
    }
}

// Any cols / alignment: two passes over the row (the second mostly from L2).
template <class Tr, bool kResid>
__global__ __launch_bounds__(256) void rmsnorm_generic_kernel(void* __restrict__ out,
                                                              void* __restrict__ resid,
                                                              const void* __restrict__ in,
                                                              const void* __restrict__ weight,
                                                              float eps, int cols) {
    __shared__ float red[16];
    const int64_t base = (int64_t)blockIdx.x * cols;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        float x = ld1<Tr>(in, base + i);
        if constexpr (kResid) {
            x = round_to<Tr>(ld1<Tr>(resid, base + i) + x);
            st1<Tr>(resid, base + i, x);
        }
        ss += x * x;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        const float x = kResid ? ld1<Tr>(resid, base + i) : ld1<Tr>(in, base + i);
        st1<Tr>(out, base + i, x * inv * ld1<Tr>(weight, i));
    }
}

// ---------------------------------------------------------------------------------------
// RoPE (rope.cu:20-49), split-half pairs (d, d + hd/2), applied in place to Q and K in one
// launch. One workgroup per token: the hd/2 (cos, sin) pairs of the token's angles
// angle = float(pos) * freq[d] are computed once into LDS with accurate sincosf and shared
// by all of the token's Q and K heads; each lane then rotates 8 pairs with two 16-byte
// loads (x0 block and x1 block) and two 16-byte stores.
// ---------------------------------------------------------------------------------------
template <class Tr, bool kVecPath>
__global__ __launch_bounds__(256) void rope_kernel(void* __restrict__ q, void* __restrict__ k,
                                                   const uint32_t* __restrict__ positions,
                                                   const float* __restrict__ freq, int qh,
                                                   int kvh, int hd) {
    extern __shared__ float cs[];  // [hd/2][2] = (cos, sin)
    const int t = blockIdx.x;
    const int half = hd / 2;
    const int tid = threadIdx.x;
    // The position and this lane's first frequency are loaded before any row: loads return
    // in order, so waiting for them after the row prefetch would also wait for the rows.
    const float p = (float)positions[t];
    const float fr0 = freq[min(tid, half - 1)];
    auto angles = [&]() {
        if (tid < half) {
            float s, c;
            sincosf(p * fr0, &s, &c);
            cs[2 * tid] = c;
            cs[2 * tid + 1] = s;
        }
        for (int d = tid + blockDim.x; d < half; d += blockDim.x) {
            float s, c;
            sincosf(p * freq[d], &s, &c);
            cs[2 * d] = c;
            cs[2 * d + 1] = s;
        }
    };
    using S = typename Tr::S;
    if constexpr (kVecPath) {
        constexpr int V = Tr::kVec;
        const int chunks = half / V;
        const int items = (qh + kvh) * chunks;
        auto item_row = [&](int it) -> S* {
            const int head = it / chunks;
            const int ch = it - head * chunks;
            S* row = head < qh ? (S*)q + ((int64_t)t * qh + head) * hd
                               : (S*)k + ((int64_t)t * kvh + (head - qh)) * hd;
            return row + ch * V;
        };
        auto rotate = [&](int it, u32x4 r0, u32x4 r1) {
            const int ch = it % chunks;
            S* p0 = item_row(it);
            float x0[V], x1[V];
            unpack16<Tr>(r0, x0);
            unpack16<Tr>(r1, x1);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const int d = ch * V + e;
                const float c = cs[2 * d], s = cs[2 * d + 1];
                const float a = x0[e], b = x1[e];
                x0[e] = a * c - b * s;
                x1[e] = a * s + b * c;
            }
            st16(p0, pack16<Tr>(x0));
            st16(p0 + half, pack16<Tr>(x1));
        };
        // The lane's first kPre items are read while the angles are computed. A lane with
        // fewer items reloads item 0 in place of the missing ones and stores nothing there.
        constexpr int kPre = 2;
        u32x4 pre0[kPre], pre1[kPre];
#pragma unroll
        for (int j = 0; j < kPre; ++j) {
            const int it = tid + j * (int)blockDim.x;
            const S* p0 = item_row(it < items ? it : 0);
            pre0[j] = ld16(p0);
            pre1[j] = ld16(p0 + half);
        }
        angles();
        lds_barrier();
#pragma unroll
        for (int j = 0; j < kPre; ++j) {
            const int it = tid + j * (int)blockDim.x;
            if (it < items) rotate(it, pre0[j], pre1[j]);
        }
        for (int it = tid + kPre * (int)blockDim.x; it < items; it += blockDim.x) {
            const S* p0 = item_row(it);
            rotate(it, ld16(p0), ld16(p0 + half));
        }
    } else {
        angles();
        __syncthreads();
        const int items = (qh + kvh) * half;
        for (int it = threadIdx.x; it < items; it += blockDim.x) {
            const int head = it / half;
            const int d = it - head * half;
            void* row = head < qh ? (void*)((S*)q + ((int64_t)t * qh + head) * hd)
                                  : (void*)((S*)k + ((int64_t)t * kvh + (head - qh)) * hd);
            const float a = ld1<Tr>(row, d), b = ld1<Tr>(row, d + half);
            const float c = cs[2 * d], s = cs[2 * d + 1];
            st1<Tr>(row, d, a * c - b * s);
            st1<Tr>(row, d + half, a * s + b * c);
        }
    }
}

// RoPE at head_dim 128 for 16-bit types: one wave per (token, group of 8 heads), so a
// decode batch of 64 tokens x 40 heads spreads over 320 workgroups instead of 64. Lane l
// rotates the 8 pairs (8c + e, 64 + 8c + e), c = l % 8, of head 8 group + l / 8, and computes
// the angle of dim l itself (one accurate sincosf per lane, the same call as rope_kernel);
// the 8 angles a lane needs come from lanes 8c .. 8c + 7 by shuffles: no LDS, no barrier.
template <class Tr>
__global__ __launch_bounds__(64) void rope_wave_kernel(void* __restrict__ q, void* __restrict__ k,
                                                      const uint32_t* __restrict__ positions,
                                                      const float* __restrict__ freq, int qh,
                                                      int kvh) {
    constexpr int kHalf = 64;
    using S = typename Tr::S;
    const int t = blockIdx.x, lane = threadIdx.x;
    const int head = blockIdx.y * 8 + (lane >> 3), ch = lane & 7;
    const bool ok = head < qh + kvh;
    const int hh = ok ? head : 0;  // lanes past the last head reload head 0 and store nothing
    S* row = hh < qh ? (S*)q + ((int64_t)t * qh + hh) * (2 * kHalf)
                     : (S*)k + ((int64_t)t * kvh + (hh - qh)) * (2 * kHalf);
    S* p0 = row + ch * 8;
    const u32x4 r0 = ld16(p0), r1 = ld16(p0 + kHalf);
    float sn, cs;
    sincosf((float)positions[t] * freq[lane], &sn, &cs);
    float x0[8], x1[8];
    unpack16<Tr>(r0, x0);
    unpack16<Tr>(r1, x1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float c = __shfl(cs, 8 * ch + e), s = __shfl(sn, 8 * ch + e);
        const float a = x0[e], b = x1[e];
        x0[e] = a * c - b * s;
        x1[e] = a * s + b * c;
    }
    if (ok) {
        st16(p0, pack16<Tr>(x0));
        st16(p0 + kHalf, pack16<Tr>(x1));
    }
}

// ---------------------------------------------------------------------------------------
// Embedding gather (embedding.cu:7-28): out[t,:] = table[id,:], zeros when id >= vocab.
// Grid (row chunks, tokens); each lane copies 16 bytes.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void embedding_vec_kernel(char* __restrict__ out,
                                                               const char* __restrict__ table,
                                                               const uint32_t* __restrict__ ids,
                                                               int64_t row_bytes, int vocab,
                                                               int num_tokens) {
    const int64_t nv = row_bytes / 16;
    const int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (v >= nv) return;
    for (int t = blockIdx.y; t < num_tokens; t += gridDim.y) {
        const uint32_t id = ids[t];
        u32x4 val = {0u, 0u, 0u, 0u};
        if (id < (uint32_t)vocab) val = ld16(table + (int64_t)id * row_bytes + v * 16);
        st16(out + (int64_t)t * row_bytes + v * 16, val);
    }
}

__global__ __launch_bounds__(kBlock) void embedding_scalar_kernel(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ table,
    const uint32_t* __restrict__ ids, int64_t row_elems, int vocab, int num_tokens) {
    for (int t = blockIdx.y; t < num_tokens; t += gridDim.y) {
        const uint32_t id = ids[t];
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < row_elems;
             i += (int64_t)gridDim.x * kBlock)
            out[(int64_t)t * row_elems + i] =
                id < (uint32_t)vocab ? table[(int64_t)id * row_elems + i] : (uint16_t)0;
    }
}

// ---------------------------------------------------------------------------------------
// Host launch helpers
// ---------------------------------------------------------------------------------------
template <class Tr>
int launch_add_t(void* out, const void* a, const void* b, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (fhip_host::aligned16(out) && fhip_host::aligned16(a) && fhip_host::aligned16(b)) {
        const int64_t nvec = n / Tr::kVec;
        const int64_t grid = nvec > 0 ? ceil_div(nvec, kBlock * kUnroll) : 1;
        hipLaunchKernelGGL(add_vec_kernel<Tr>, dim3((unsigned)grid), dim3(kBlock), 0, s, out, a,
                           b, n);
    } else {
        const int64_t grid = std::min<int64_t>(ceil_div(n, kBlock), fhip_host::kStreamGroups);
        hipLaunchKernelGGL(add_scalar_kernel<Tr>, dim3((unsigned)grid), dim3(kBlock), 0, s, out,
                           a, b, n);
    }
    return hipGetLastError();
}

template <class Tr>
int launch_silu_t(void* out, const void* g, const void* u, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (fhip_host::aligned16(out) && fhip_host::aligned16(g) && fhip_host::aligned16(u)) {
        const int64_t nvec = n / Tr::kVec;
        const int64_t grid = nvec > 0 ? ceil_div(nvec, kBlock * kUnroll) : 1;
        hipLaunchKernelGGL(silu_mul_vec_kernel<Tr>, dim3((unsigned)grid), dim3(kBlock), 0, s,
                           out, g, u, n);
    } else {
        const int64_t grid = std::min<int64_t>(ceil_div(n, kBlock), fhip_host::kStreamGroups);
        hipLaunchKernelGGL(silu_mul_scalar_kernel<Tr>, dim3((unsigned)grid), dim3(kBlock), 0, s,
                           out, g, u, n);
    }
    return hipGetLastError();
}

template <class Tr, bool kResid, int kVpt>
void launch_rms_vec(int bs, void* out, void* resid, const void* in, const void* w, float eps,
                    int rows, int cols, hipStream_t s) {
    hipLaunchKernelGGL((rmsnorm_vec_kernel<Tr, kResid, kVpt>), dim3(rows), dim3(bs), 0, s, out,
                       resid, in, w, eps, cols);
}

template <class Tr, bool kResid>
int launch_rms_t(void* out, void* resid, const void* in, const void* w, float eps, int rows,
                 int cols, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    constexpr int V = Tr::kVec;
    const bool vec_ok = cols % V == 0 && fhip_host::aligned16(out) &&
                        fhip_host::aligned16(in) && fhip_host::aligned16(w) &&
                        (!kResid || fhip_host::aligned16(resid));
    const int nvec = cols / V;
    if (vec_ok && nvec > 0 && nvec <= 1024 * 8) {
        // Smallest vectors-per-lane (1, 2, 4, 8) that fits in a <=1024-lane workgroup of at
        // most 256 lanes when possible (512 when there are too few rows to fill the chip:
        // a decode batch of 64 rows then has fewer loads in flight per lane); the block is a
        // multiple of the wave.
        const int64_t lanes = rows < 512 ? 512 : 256;
        int vpt = 1;
        while (vpt < 8 && (int64_t)vpt * lanes < nvec) vpt *= 2;
        int bs = (int)ceil_div(ceil_div(nvec, vpt), kWave) * kWave;
        if (bs > 1024) return hipErrorInvalidValue;
        switch (vpt) {
            case 1: launch_rms_vec<Tr, kResid, 1>(bs, out, resid, in, w, eps, rows, cols, s); break;
            case 2: launch_rms_vec<Tr, kResid, 2>(bs, out, resid, in, w, eps, rows, cols, s); break;
            case 4: launch_rms_vec<Tr, kResid, 4>(bs, out, resid, in, w, eps, rows, cols, s); break;
            default: launch_rms_vec<Tr, kResid, 8>(bs, out, resid, in, w, eps, rows, cols, s); break;
        }
    } else {
        hipLaunchKernelGGL((rmsnorm_generic_kernel<Tr, kResid>), dim3(rows), dim3(256), 0, s, out,
                           resid, in, w, eps, cols);
    }
    return hipGetLastError();
}

template <class Tr>
int launch_rope_t(void* q, void* k, const uint32_t* pos, const float* freq, int T, int qh, int kvh,
                  int hd, hipStream_t s) {
    if (T == 0 || qh + kvh == 0) return hipSuccess;
    const int half = hd / 2;
    const size_t lds = (size_t)half * 2 * sizeof(float);
    const bool vec_ok = half % Tr::kVec == 0 && fhip_host::aligned16(q) &&
                        (kvh == 0 || fhip_host::aligned16(k));
    const int work = (qh + kvh) * (vec_ok ? half / Tr::kVec : half);
    int bs = (int)std::min<int64_t>(256, std::max<int64_t>(kWave, ceil_div(work, kWave) * kWave));
    if (vec_ok && Tr::kVec == 8 && hd == 128 && ceil_div(qh + kvh, 8) <= 65535) {
        const dim3 grid((unsigned)T, (unsigned)ceil_div(qh + kvh, 8));
        hipLaunchKernelGGL((rope_wave_kernel<Tr>), grid, dim3(64), 0, s, q, k, pos, freq, qh, kvh);
    } else if (vec_ok)
        hipLaunchKernelGGL((rope_kernel<Tr, true>), dim3(T), dim3(bs), lds, s, q, k, pos, freq, qh,
                           kvh, hd);
    else
        hipLaunchKernelGGL((rope_kernel<Tr, false>), dim3(T), dim3(bs), lds, s, q, k, pos, freq,
                           qh, kvh, hd);
    return hipGetLastError();
}

}  // namespace

// =========================================================================================
// C ABI
// =========================================================================================
extern "C" {

int fhip_launch_add_ex(void* out, const void* a, const void* b, int64_t n, int dtype,
                       fhip_stream_t stream) {
    if (n < 0 || (n > 0 && (!out || !a || !b))) return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    switch (dtype) {
        case FHIP_FP16: return launch_add_t<TrF16>(out, a, b, n, s);
        case FHIP_BF16: return launch_add_t<TrBF16>(out, a, b, n, s);
        case FHIP_FP32: return launch_add_t<TrF32>(out, a, b, n, s);
        default: return hipErrorInvalidValue;
    }
}

int fhip_launch_add(void* out, const void* a, const void* b, int n, fhip_stream_t stream) {
    return fhip_launch_add_ex(out, a, b, n, FHIP_FP16, stream);
}

int fhip_launch_silu_mul_ex(void* out, const void* gate, const void* up, int64_t n, int dtype,
                            fhip_stream_t stream) {
    if (n < 0 || (n > 0 && (!out || !gate || !up))) return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    switch (dtype) {
        case FHIP_FP16: return launch_silu_t<TrF16>(out, gate, up, n, s);
        case FHIP_BF16: return launch_silu_t<TrBF16>(out, gate, up, n, s);
        case FHIP_FP32: return launch_silu_t<TrF32>(out, gate, up, n, s);
        default: return hipErrorInvalidValue;
    }
}

int fhip_launch_silu_mul(void* out, const void* gate, const void* up, int n,
                         fhip_stream_t stream) {
    return fhip_launch_silu_mul_ex(out, gate, up, n, FHIP_FP16, stream);
}

int fhip_launch_rmsnorm_ex(void* out, const void* in, const void* w, float eps, int rows,
                           int cols, int dtype, fhip_stream_t stream) {
    if (rows < 0 || cols <= 0 || (rows > 0 && (!out || !in || !w))) return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    switch (dtype) {
        case FHIP_FP16: return launch_rms_t<TrF16, false>(out, nullptr, in, w, eps, rows, cols, s);
        case FHIP_BF16: return launch_rms_t<TrBF16, false>(out, nullptr, in, w, eps, rows, cols, s);
        case FHIP_FP32: return launch_rms_t<TrF32, false>(out, nullptr, in, w, eps, rows, cols, s);
        default: return hipErrorInvalidValue;
    }
}

int fhip_launch_rmsnorm(void* out, const void* in, const void* w, float eps, int rows, int cols,
                        fhip_stream_t stream) {
    return fhip_launch_rmsnorm_ex(out, in, w, eps, rows, cols, FHIP_FP16, stream);
}

int fhip_launch_add_rmsnorm(void* residual, const void* delta, const void* weight, float eps,
                            void* normed_out, int rows, int cols, int dtype,
                            fhip_stream_t stream) {
    if (rows < 0 || cols <= 0 || (rows > 0 && (!residual || !delta || !weight || !normed_out)))
        return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    switch (dtype) {
        case FHIP_FP16:
            return launch_rms_t<TrF16, true>(normed_out, residual, delta, weight, eps, rows, cols, s);
        case FHIP_BF16:
            return launch_rms_t<TrBF16, true>(normed_out, residual, delta, weight, eps, rows, cols, s);
        case FHIP_FP32:
            return launch_rms_t<TrF32, true>(normed_out, residual, delta, weight, eps, rows, cols, s);
        default: return hipErrorInvalidValue;
    }
}

int fhip_launch_rope_ex(void* q, void* k, const uint32_t* positions, const float* freq_table,
                        int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                        int dtype, fhip_stream_t stream) {
    if (num_tokens < 0 || num_q_heads < 0 || num_kv_heads < 0 || head_dim <= 0 ||
        head_dim % 2 != 0 || head_dim > 4096)
        return hipErrorInvalidValue;
    if (num_tokens > 0 && (!positions || !freq_table || (num_q_heads > 0 && !q) ||
                           (num_kv_heads > 0 && !k)))
        return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    switch (dtype) {
        case FHIP_FP16:
            return launch_rope_t<TrF16>(q, k, positions, freq_table, num_tokens, num_q_heads,
                                        num_kv_heads, head_dim, s);
        case FHIP_BF16:
            return launch_rope_t<TrBF16>(q, k, positions, freq_table, num_tokens, num_q_heads,
                                         num_kv_heads, head_dim, s);
        case FHIP_FP32:
            return launch_rope_t<TrF32>(q, k, positions, freq_table, num_tokens, num_q_heads,
                                        num_kv_heads, head_dim, s);
        default: return hipErrorInvalidValue;
    }
}

int fhip_launch_rope(void* q, void* k, const uint32_t* positions, const float* freq_table,
                     int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                     fhip_stream_t stream) {
    return fhip_launch_rope_ex(q, k, positions, freq_table, num_tokens, num_q_heads, num_kv_heads,
                               head_dim, FHIP_FP16, stream);
}

int fhip_launch_embedding_ex(void* out, const void* table, const uint32_t* ids, int num_tokens,
                             int hidden_dim, int vocab_size, int elem_bytes,
                             fhip_stream_t stream) {
    if (num_tokens < 0 || hidden_dim < 0 || vocab_size < 0 || (elem_bytes != 2 && elem_bytes != 4))
        return hipErrorInvalidValue;
    if (num_tokens == 0 || hidden_dim == 0) return hipSuccess;
    if (!out || !ids || (vocab_size > 0 && !table)) return hipErrorInvalidValue;
    hipStream_t s = fhip_host::as_stream(stream);
    const int64_t row_bytes = (int64_t)hidden_dim * elem_bytes;
    if (row_bytes % 16 == 0 && fhip_host::aligned16(out) && fhip_host::aligned16(table)) {
        const int64_t nv = row_bytes / 16;
        dim3 grid((unsigned)ceil_div(nv, kBlock), (unsigned)std::min(num_tokens, 65535));
        hipLaunchKernelGGL(embedding_vec_kernel, grid, dim3(kBlock), 0, s, (char*)out,
                           (const char*)table, ids, row_bytes, vocab_size, num_tokens);
    } else {
        const int64_t elems = row_bytes / 2;  // copied as 16-bit units
        dim3 grid((unsigned)std::min<int64_t>(ceil_div(elems, kBlock), 64),
                  (unsigned)std::min(num_tokens, 65535));
        hipLaunchKernelGGL(embedding_scalar_kernel, grid, dim3(kBlock), 0, s, (uint16_t*)out,
                           (const uint16_t*)table, ids, elems, vocab_size, num_tokens);
    }
    return hipGetLastError();
}

int fhip_launch_embedding(void* out, const void* table, const uint32_t* ids, int num_tokens,
                          int hidden_dim, int vocab_size, fhip_stream_t stream) {
    return fhip_launch_embedding_ex(out, table, ids, num_tokens, hidden_dim, vocab_size, 2, stream);
}

}  // extern "C"

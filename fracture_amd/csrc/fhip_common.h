// Shared device helpers for the gfx950 kernels: element traits, 128-bit vector access,
// wave64 DPP reductions and workgroup combines.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <vector>

#include "fracture_hip.h"

namespace fhip {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------
// Scalar conversions. fp16 uses the hardware RNE conversion; bf16 is rounded to nearest
// even by hand (NaN stays a quiet NaN), the rounding `half::bf16::from_f32` performs.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t f2h(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float b2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t f2b(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Element traits: storage type, values per 16-byte vector, conversions.
struct TrF16 {
    using S = uint16_t;
    static constexpr int kVec = 8;
    static constexpr int kDtype = FHIP_FP16;
    __device__ static float ld(uint32_t b) { return h2f(b); }
    __device__ static uint32_t st(float f) { return f2h(f); }
};
struct TrBF16 {
    using S = uint16_t;
    static constexpr int kVec = 8;
    static constexpr int kDtype = FHIP_BF16;
    __device__ static float ld(uint32_t b) { return b2f(b); }
    __device__ static uint32_t st(float f) { return f2b(f); }
};
struct TrF32 {
    using S = float;
    static constexpr int kVec = 4;
    static constexpr int kDtype = FHIP_FP32;
};

// Unpack one 16-byte vector into kVec floats / pack kVec floats back.
template <class Tr>
__device__ __forceinline__ void unpack16(const u32x4& v, float* out) {
    if constexpr (Tr::kVec == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = Tr::ld(v[i] & 0xffffu);
            out[2 * i + 1] = Tr::ld(v[i] >> 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(v[i]);
    }
}
template <class Tr>
__device__ __forceinline__ u32x4 pack16(const float* in) {
    u32x4 v;
    if constexpr (Tr::kVec == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = Tr::st(in[2 * i]) | (Tr::st(in[2 * i + 1]) << 16);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(in[i]);
    }
    return v;
}
// Scalar element access for tails / unaligned fallbacks.
template <class Tr>
__device__ __forceinline__ float ld1(const void* p, int64_t i) {
    if constexpr (Tr::kVec == 8)
        return Tr::ld(((const uint16_t*)p)[i]);
    else
        return ((const float*)p)[i];
}
template <class Tr>
__device__ __forceinline__ void st1(void* p, int64_t i, float f) {
    if constexpr (Tr::kVec == 8)
        ((uint16_t*)p)[i] = (uint16_t)Tr::st(f);
    else
        ((float*)p)[i] = f;
}
// Round a float through the storage type (the value a reader of the stored element sees).
template <class Tr>
__device__ __forceinline__ float round_to(float f) {
    if constexpr (Tr::kVec == 8)
        return Tr::ld(Tr::st(f));
    else
        return f;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *(u32x4*)p = v; }
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
    return __builtin_nontemporal_load((const u32x4*)p);
}
__device__ __forceinline__ void st16_stream(void* p, const u32x4& v) {
    __builtin_nontemporal_store(v, (u32x4*)p);
}

// The readlane builtin moves 32-bit integers: floats cross it as their bit patterns.
__device__ __forceinline__ float lane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---------------------------------------------------------------------------------------
// Wave64 reductions with DPP: quad swaps, half-row and row mirrors, then row_bcast:15 /
// row_bcast:31 carry the row totals up to lane 63, which is read back as a scalar.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x140, 0xF, 0xF, true);  // row_mirror
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x142, 0xA, 0xF, false); // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0.0f, v, 0x143, 0xC, 0xF, false); // row_bcast:31
    return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
    const float ninf = -__builtin_inff();
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0xB1, 0xF, 0xF, true));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0x4E, 0xF, 0xF, true));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0x141, 0xF, 0xF, true));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0x140, 0xF, 0xF, true));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0x142, 0xA, 0xF, false));
    v = fmaxf(v, __builtin_amdgcn_update_dpp(ninf, v, 0x143, 0xC, 0xF, false));
    return lane63(v);
}
__device__ __forceinline__ int wave_max_int(int v) {
    const int lo = INT32_MIN;
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0xB1, 0xF, 0xF, true));
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0x4E, 0xF, 0xF, true));
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0x141, 0xF, 0xF, true));
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0x140, 0xF, 0xF, true));
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0x142, 0xA, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(lo, v, 0x143, 0xC, 0xF, false));
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float wave_min(float v) {
    const float pinf = __builtin_inff();
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0xB1, 0xF, 0xF, true));
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0x4E, 0xF, 0xF, true));
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0x141, 0xF, 0xF, true));
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0x140, 0xF, 0xF, true));
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0x142, 0xA, 0xF, false));
    v = fminf(v, __builtin_amdgcn_update_dpp(pinf, v, 0x143, 0xC, 0xF, false));
    return lane63(v);
}

// Workgroup barrier that orders LDS only. __syncthreads() also fences global memory, which
// on gfx9 makes every wave drain its outstanding global loads and stores (vmcnt(0)) before
// the barrier; kernels that keep prefetches in flight across a barrier use this instead.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Ordering point for an LDS exchange between the lanes of one wave (no other wave involved).
// The hardware performs one wave's LDS instructions in program order, so no wait is needed;
// the fences and the barrier stop the compiler from moving a lane's LDS accesses across this
// point, which it may otherwise do whenever it can show that the lane's own addresses differ
// (it reasons per lane, not per wave). Place one between the writes and the cross-lane
// reads, and one between those reads and the next overwrite of the same words.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup sum of one float per thread. `scratch` holds one float per wave; the result is
// returned to every thread. Contains two barriers.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nwaves = (blockDim.x + kWave - 1) / kWave;
    v = wave_sum(v);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nwaves; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) {
    return (a + b - 1) / b;
}

}  // namespace fhip

// Host-side helpers shared by the launch wrappers.
namespace fhip_host {
inline bool aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
inline hipStream_t as_stream(fhip_stream_t s) { return (hipStream_t)s; }
// Workgroups that fill the chip for a streaming kernel: 256 CUs, a few groups each.
constexpr int kStreamGroups = 256 * 8;

// Compute units of the current device (cached per device; 256 on MI355X).
inline int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Grid of a persistent kernel: as many workgroups as are resident at once on the device
// (occupancy of `kernel` at `block` lanes and `lds` dynamic bytes), capped by the work.
// The occupancy is looked up once per (kernel, block, lds) and cached.
template <class K>
inline int resident_grid(K kernel, int block, size_t lds, int64_t work_units) {
    struct Entry {
        const void* fn;
        int block;
        size_t lds;
        int per_cu;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int per_cu = 0;
    {
        std::lock_guard<std::mutex> g(mu);
        for (const Entry& e : cache)
            if (e.fn == (const void*)kernel && e.block == block && e.lds == lds) per_cu = e.per_cu;
        if (per_cu == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) !=
                    hipSuccess ||
                per_cu <= 0)
                per_cu = 1;
            cache.push_back(Entry{(const void*)kernel, block, lds, per_cu});
        }
    }
    const int64_t g = (int64_t)per_cu * cu_count();
    return (int)(work_units < g ? (work_units > 0 ? work_units : 1) : g);
}
}  // namespace fhip_host

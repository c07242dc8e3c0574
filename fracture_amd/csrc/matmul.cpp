// Dense fp16 GEMM for the Backend::matmul surface: C[M, N] = A[M, K] · B[N, K]ᵀ, row-major,
// fp16 in and out with fp32 accumulation — the contract of CudaBackend::matmul
// (cuda/src/backend.rs:75-128: weights stored [out_features, in_features], y = x Wᵀ,
// cublasGemmEx with CUBLAS_COMPUTE_32F). A plain library GEMM: rocBLAS gemm_ex on the
// caller's stream, which dispatches to the library's tuned gfx950 MFMA kernels.
//
// Row-major operands are column-major transposes, so the call computes Cᵀ (N × M,
// column-major, ld N) = op(B) · Aᵀ with B read transposed (ld K) and A as is (ld K).
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <mutex>
#include <vector>

#include "fracture_hip.h"

namespace {

struct Handles {
    std::mutex mu;  // a handle carries its stream: set_stream + gemm run under the lock
    std::vector<rocblas_handle> per_device;
};
Handles& handles() {
    static Handles h;
    return h;
}

// The calling thread's current device's handle (created on first use, kept for the
// process's lifetime). Called with the lock held.
int device_handle(rocblas_handle* out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    Handles& h = handles();
    if ((int)h.per_device.size() <= dev) h.per_device.resize(dev + 1, nullptr);
    if (!h.per_device[dev]) {
        rocblas_handle r = nullptr;
        if (rocblas_create_handle(&r) != rocblas_status_success) return hipErrorOutOfMemory;
        h.per_device[dev] = r;
    }
    *out = h.per_device[dev];
    return hipSuccess;
}

}  // namespace

extern "C" {

int fhip_launch_matmul(void* c, const void* a, const void* b, int m, int n, int k,
                       fhip_stream_t stream) {
    if (m < 0 || n < 0 || k < 0) return hipErrorInvalidValue;
    if (m == 0 || n == 0) return hipSuccess;
    if (!c || (k > 0 && (!a || !b))) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> g(handles().mu);
    rocblas_handle h;
    int e = device_handle(&h);
    if (e != hipSuccess) return e;
    if (rocblas_set_stream(h, (hipStream_t)stream) != rocblas_status_success)
        return hipErrorInvalidValue;
    const float alpha = 1.0f, beta = 0.0f;
    const rocblas_status st = rocblas_gemm_ex(
        h, rocblas_operation_transpose, rocblas_operation_none, n, m, k, &alpha, b,
        rocblas_datatype_f16_r, k, a, rocblas_datatype_f16_r, k, &beta, c, rocblas_datatype_f16_r,
        n, c, rocblas_datatype_f16_r, n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success) return hipErrorLaunchFailure;
    return hipGetLastError();
}

}  // extern "C"

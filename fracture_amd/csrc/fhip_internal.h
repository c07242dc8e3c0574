// Entry points shared between the kernel sources and the handle runtime that are not part of
// the C ABI (include/fracture_hip.h).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace fhip_internal {

// fhip_launch_attention_tq_decode_ptrs over a block table of row stride table_stride
// (>= max_blocks) in device memory; the workspace is fhip_attention_tq_workspace_bytes.
int attention_tq_decode_ptrs_staged(void* output, const void* q, const int32_t* block_table,
                                    const int32_t* seq_lens, int batch, int max_blocks,
                                    int table_stride, int num_pages, const void** k_packed_ptrs,
                                    const void** k_norms_ptrs, const void** v_packed_ptrs,
                                    const void** v_norms_ptrs, const float* k_rotation,
                                    const float* v_rotation, const float* k_centroids,
                                    const float* v_centroids, int num_q_heads, int num_kv_heads,
                                    int head_dim, int key_bits, int value_bits, void* workspace,
                                    hipStream_t stream);

// Rows of 128: out[r] = Pi x[r] in fp32 from fp16 x (the compress kernel's MFMA rotation,
// fp16 operands split hi / lo for fp32 accuracy, without normalisation).
int tq_rotate_rows(const void* input, const float* rotation, float* out, int64_t rows,
                   hipStream_t stream);

// Rows of 128: out[r] = fp16(Pi^T y[r]) from fp32 y (the dequantize kernel's MFMA products,
// y split into fp16 hi / lo operands).
int tq_rotate_back_rows(const float* input, const float* rotation, void* out, int64_t rows,
                        hipStream_t stream);

}  // namespace fhip_internal

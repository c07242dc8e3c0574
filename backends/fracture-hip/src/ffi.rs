//! The C ABI of libfracture_hip.so (include/fracture_hip.h).
//!
//! * Section 1, the raw launchers: `fhip_launch_*`, one for one with the `launch_*` block of
//!   backends/fracture-cuda/src/ffi.rs:141-274 (device pointers, `c_int` dims, a stream; they
//!   return a HIP error code, 0 on success). Each is also re-exported under the reference's
//!   name (`launch_rmsnorm` ..), so code that calls `fracture_cuda::ffi::launch_*` with
//!   `backend.stream()` (bins/fracture-server-cuda/tests/turboquant_gpu.rs:127-143) compiles
//!   against `fracture_hip::ffi::*` unchanged.
//! * Section 2, the handle runtime: the C mirror of the Backend trait that `HipBackend` wraps.
//!   Status codes are `FHIP_*`; the message of a thread's last failing call is
//!   `fhip_last_error()`.

use std::ffi::{c_char, c_int, c_void};

/// The stream every launch of a backend goes to (`cudaStream_t` in the CUDA backend).
#[allow(non_camel_case_types)]
pub type hipStream_t = *mut c_void;
/// A HIP runtime status code (`cudaError_t` in the CUDA backend); 0 is success.
#[allow(non_camel_case_types)]
pub type hipError_t = c_int;
pub const HIP_SUCCESS: hipError_t = 0;

pub const FHIP_OK: c_int = 0;
pub const FHIP_ERR_BACKEND: c_int = 1;
pub const FHIP_ERR_INVALID_SHAPE: c_int = 2;
pub const FHIP_ERR_TENSOR_NOT_FOUND: c_int = 3;
pub const FHIP_ERR_OUT_OF_MEMORY: c_int = 4;
pub const FHIP_ERR_UNSUPPORTED_DTYPE: c_int = 5;
pub const FHIP_ERR_GENERATION: c_int = 6;

/// Element type codes, in the order of fracture_core::DType.
pub const FHIP_FP16: i32 = 0;
pub const FHIP_FP32: i32 = 1;
pub const FHIP_BF16: i32 = 2;
pub const FHIP_INT8: i32 = 3;
pub const FHIP_INT4: i32 = 4;

pub const FHIP_MAX_DIMS: usize = 8;

/// fracture_core::DeviceTensor by value: id, dtype code, rank and row-major shape.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct FhipTensor {
    pub id: u64,
    pub dtype: i32,
    pub ndim: i32,
    pub shape: [u64; FHIP_MAX_DIMS],
}

/// Opaque `fhip_backend*`.
#[repr(C)]
pub struct FhipBackend {
    _private: [u8; 0],
}

unsafe extern "C" {
    pub fn fhip_last_error() -> *const c_char;
    pub fn fhip_version() -> *const c_char;

    // construction, device info, streams (CudaBackend::new / Drop / get_ptr / stream)
    pub fn fhip_backend_create(device_id: c_int, out: *mut *mut FhipBackend) -> c_int;
    pub fn fhip_backend_destroy(b: *mut FhipBackend);
    pub fn fhip_get_ptr(b: *mut FhipBackend, id: u64, out: *mut *mut c_void) -> c_int;
    pub fn fhip_stream(b: *mut FhipBackend) -> *mut c_void;
    pub fn fhip_device_name(b: *mut FhipBackend) -> *const c_char;
    pub fn fhip_total_memory(b: *mut FhipBackend) -> usize;
    pub fn fhip_available_memory(b: *mut FhipBackend) -> usize;
    pub fn fhip_synchronize(b: *mut FhipBackend) -> c_int;
    pub fn fhip_precompute_rope_freqs(b: *mut FhipBackend, head_dim: usize, theta: f64) -> c_int;

    // memory (Backend::alloc / free / copy_to_device / copy_to_host)
    pub fn fhip_alloc(b: *mut FhipBackend, shape: *const u64, ndim: c_int, dtype: c_int,
                      out: *mut FhipTensor) -> c_int;
    pub fn fhip_free(b: *mut FhipBackend, t: *const FhipTensor) -> c_int;
    pub fn fhip_copy_to_device(b: *mut FhipBackend, dst: *const FhipTensor, src: *const c_void,
                               src_len: usize) -> c_int;
    pub fn fhip_copy_to_host(b: *mut FhipBackend, src: *const FhipTensor, dst: *mut c_void,
                             dst_len: usize) -> c_int;

    // compute (Backend::matmul .. copy_rows)
    pub fn fhip_matmul(b: *mut FhipBackend, a: *const FhipTensor, bm: *const FhipTensor,
                       out: *const FhipTensor) -> c_int;
    pub fn fhip_rmsnorm(b: *mut FhipBackend, input: *const FhipTensor, weight: *const FhipTensor,
                        eps: f64, out: *const FhipTensor) -> c_int;
    pub fn fhip_rope(b: *mut FhipBackend, q: *const FhipTensor, k: *const FhipTensor,
                     positions: *const u32, num_positions: usize, theta: f64,
                     head_dim: usize) -> c_int;
    pub fn fhip_attention(b: *mut FhipBackend, q: *const FhipTensor, k_cache: *const FhipTensor,
                          v_cache: *const FhipTensor, num_kv_heads: usize, start_pos: usize,
                          out: *const FhipTensor) -> c_int;
    pub fn fhip_attention_paged(b: *mut FhipBackend, q: *const FhipTensor,
                                block_table: *const i32, num_blocks: usize,
                                k_blocks: *const FhipTensor, v_blocks: *const FhipTensor,
                                pool_len: usize, num_kv_heads: usize, kv_len: usize,
                                start_pos: usize, out: *const FhipTensor) -> c_int;
    pub fn fhip_silu_mul(b: *mut FhipBackend, gate: *const FhipTensor, up: *const FhipTensor,
                         out: *const FhipTensor) -> c_int;
    pub fn fhip_embedding(b: *mut FhipBackend, token_ids: *const u32, num_tokens: usize,
                          table: *const FhipTensor, out: *const FhipTensor) -> c_int;
    pub fn fhip_add(b: *mut FhipBackend, a: *const FhipTensor, bt: *const FhipTensor,
                    out: *const FhipTensor) -> c_int;
    pub fn fhip_copy_rows(b: *mut FhipBackend, src: *const FhipTensor, dst: *const FhipTensor,
                          src_offset: usize, dst_offset: usize, count: usize) -> c_int;

    // profiling
    pub fn fhip_create_timer(b: *mut FhipBackend, timer_id: *mut u64) -> c_int;
    pub fn fhip_start_timer(b: *mut FhipBackend, timer_id: u64) -> c_int;
    pub fn fhip_stop_timer(b: *mut FhipBackend, timer_id: u64, ms_out: *mut f32) -> c_int;
    pub fn fhip_destroy_timer(b: *mut FhipBackend, timer_id: u64) -> c_int;
    pub fn fhip_marker_push(b: *mut FhipBackend, name: *const c_char);
    pub fn fhip_marker_pop(b: *mut FhipBackend);

    // TurboQuant (Backend::turboquant_compress / attention_paged_tq)
    pub fn fhip_turboquant_compress(b: *mut FhipBackend, input: *const FhipTensor,
                                    rotation: *const FhipTensor, centroids: *const FhipTensor,
                                    bits: u8, packed_out: *const FhipTensor,
                                    norms_out: *const FhipTensor) -> c_int;
    pub fn fhip_attention_paged_tq(b: *mut FhipBackend, q: *const FhipTensor,
                                   block_table: *const i32, num_blocks: usize,
                                   k_packed: *const FhipTensor, k_norms: *const FhipTensor,
                                   v_packed: *const FhipTensor, v_norms: *const FhipTensor,
                                   pool_len: usize, k_rotation: *const FhipTensor,
                                   v_rotation: *const FhipTensor, k_centroids: *const FhipTensor,
                                   v_centroids: *const FhipTensor, key_bits: u8, value_bits: u8,
                                   num_kv_heads: usize, kv_len: usize, start_pos: usize,
                                   out: *const FhipTensor) -> c_int;

    // additive: registered page pools, the engine's KV-cache write and batched decode paths
    pub fn fhip_page_pool_create(b: *mut FhipBackend, blocks: *const FhipTensor, nlists: usize,
                                 pool_len: usize, pool_out: *mut u64) -> c_int;
    pub fn fhip_page_pool_destroy(b: *mut FhipBackend, pool: u64) -> c_int;
    pub fn fhip_attention_paged_tq_pool(b: *mut FhipBackend, q: *const FhipTensor,
                                        block_table: *const i32, num_blocks: usize, pool: u64,
                                        k_rotation: *const FhipTensor,
                                        v_rotation: *const FhipTensor,
                                        k_centroids: *const FhipTensor,
                                        v_centroids: *const FhipTensor, key_bits: u8,
                                        value_bits: u8, num_kv_heads: usize, kv_len: usize,
                                        start_pos: usize, out: *const FhipTensor) -> c_int;
    pub fn fhip_tq_append_kv(b: *mut FhipBackend, pool: u64, keys: *const FhipTensor,
                             values: *const FhipTensor, k_rotation: *const FhipTensor,
                             v_rotation: *const FhipTensor, k_centroids: *const FhipTensor,
                             v_centroids: *const FhipTensor, key_bits: u8, value_bits: u8,
                             block_table: *const i32, num_blocks: usize,
                             start_pos: usize) -> c_int;
    pub fn fhip_attention_paged_tq_batched(b: *mut FhipBackend, q: *const FhipTensor,
                                           block_tables: *const i32, num_seqs: usize,
                                           max_blocks: usize, seq_lens: *const u32, pool: u64,
                                           k_rotation: *const FhipTensor,
                                           v_rotation: *const FhipTensor,
                                           k_centroids: *const FhipTensor,
                                           v_centroids: *const FhipTensor, key_bits: u8,
                                           value_bits: u8, num_kv_heads: usize,
                                           out: *const FhipTensor) -> c_int;
    pub fn fhip_add_rmsnorm(b: *mut FhipBackend, residual: *const FhipTensor,
                            delta: *const FhipTensor, weight: *const FhipTensor, eps: f64,
                            normed_out: *const FhipTensor) -> c_int;
    pub fn fhip_argmax_rows(b: *mut FhipBackend, logits: *const FhipTensor,
                            tokens_out: *mut u32, rows: usize) -> c_int;
    pub fn fhip_softmax_rows(b: *mut FhipBackend, logits: *const FhipTensor, temperature: f32,
                             probs: *const FhipTensor) -> c_int;
    pub fn fhip_tq_dequantize(b: *mut FhipBackend, packed: *const FhipTensor,
                              norms: *const FhipTensor, rotation: *const FhipTensor,
                              centroids: *const FhipTensor, bits: u8,
                              out: *const FhipTensor) -> c_int;
    pub fn fhip_tq_quantize_pack(b: *mut FhipBackend, y: *const FhipTensor,
                                 centroids: *const FhipTensor, bits: u8,
                                 packed_out: *const FhipTensor) -> c_int;

    // graph capture of a decode step's device-resident launches
    pub fn fhip_rope_dev(b: *mut FhipBackend, q: *const FhipTensor, k: *const FhipTensor,
                         positions: *const FhipTensor, num_positions: usize,
                         head_dim: usize) -> c_int;
    pub fn fhip_embedding_dev(b: *mut FhipBackend, token_ids: *const FhipTensor,
                              num_tokens: usize, table: *const FhipTensor,
                              out: *const FhipTensor) -> c_int;
    pub fn fhip_graph_begin(b: *mut FhipBackend) -> c_int;
    pub fn fhip_graph_end(b: *mut FhipBackend, graph_out: *mut u64) -> c_int;
    pub fn fhip_graph_launch(b: *mut FhipBackend, graph: u64) -> c_int;
    pub fn fhip_graph_destroy(b: *mut FhipBackend, graph: u64) -> c_int;
}

// ── Section 1: raw launchers (ffi.rs:141-274 and the additive ones) ────────────────────

unsafe extern "C" {
    pub fn fhip_launch_rmsnorm(output: *mut c_void, input: *const c_void, weight: *const c_void,
                               eps: f32, rows: c_int, cols: c_int,
                               stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_rope(q: *mut c_void, k: *mut c_void, positions: *const u32,
                            freq_table: *const f32, num_tokens: c_int, num_q_heads: c_int,
                            num_kv_heads: c_int, head_dim: c_int,
                            stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_silu_mul(output: *mut c_void, gate: *const c_void, up: *const c_void,
                                n: c_int, stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_attention(output: *mut c_void, q: *const c_void, k_cache: *const c_void,
                                 v_cache: *const c_void, num_tokens: c_int, num_q_heads: c_int,
                                 num_kv_heads: c_int, head_dim: c_int, kv_len: c_int,
                                 start_pos: c_int, stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_paged_attention(output: *mut c_void, q: *const c_void,
                                       block_table: *const c_int,
                                       k_block_ptrs: *const *const c_void,
                                       v_block_ptrs: *const *const c_void, num_tokens: c_int,
                                       num_q_heads: c_int, num_kv_heads: c_int,
                                       head_dim: c_int, kv_len: c_int, start_pos: c_int,
                                       num_blocks_in_seq: c_int,
                                       stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_embedding(output: *mut c_void, table: *const c_void,
                                 token_ids: *const u32, num_tokens: c_int, hidden_dim: c_int,
                                 vocab_size: c_int, stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_add(output: *mut c_void, a: *const c_void, b: *const c_void, n: c_int,
                           stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_turboquant_compress(input: *const c_void, rotation: *const f32,
                                           centroids: *const f32, packed_out: *mut c_void,
                                           norms_out: *mut c_void, num_tokens: c_int,
                                           num_kv_heads: c_int, head_dim: c_int,
                                           n_levels: c_int, bits: c_int,
                                           packed_dim_per_head: c_int,
                                           stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_turboquant_decompress(packed_in: *const c_void, norms_in: *const c_void,
                                             rotation: *const f32, centroids: *const f32,
                                             output: *mut c_void, num_tokens: c_int,
                                             num_kv_heads: c_int, head_dim: c_int, bits: c_int,
                                             packed_dim_per_head: c_int,
                                             stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_attention_paged_tq(output: *mut c_void, q: *const c_void,
                                          block_table: *const c_int,
                                          k_packed_ptrs: *const *const c_void,
                                          k_norms_ptrs: *const *const c_void,
                                          v_packed_ptrs: *const *const c_void,
                                          v_norms_ptrs: *const *const c_void,
                                          k_rotation: *const f32, v_rotation: *const f32,
                                          k_centroids: *const f32, v_centroids: *const f32,
                                          num_tokens: c_int, num_q_heads: c_int,
                                          num_kv_heads: c_int, head_dim: c_int, kv_len: c_int,
                                          start_pos: c_int, key_bits: c_int,
                                          value_bits: c_int, k_packed_dim_per_head: c_int,
                                          v_packed_dim_per_head: c_int,
                                          stream: hipStream_t) -> hipError_t;
    /// CudaBackend::matmul's GEMM (cuda/src/backend.rs:75-128 calls cuBLAS directly).
    pub fn fhip_launch_matmul(c: *mut c_void, a: *const c_void, b: *const c_void, m: c_int,
                              n: c_int, k: c_int, stream: hipStream_t) -> hipError_t;

    // additive raw launchers
    pub fn fhip_launch_attention_paged_tq_ws(output: *mut c_void, q: *const c_void,
                                             block_table: *const c_int,
                                             k_packed_ptrs: *const *const c_void,
                                             k_norms_ptrs: *const *const c_void,
                                             v_packed_ptrs: *const *const c_void,
                                             v_norms_ptrs: *const *const c_void,
                                             k_rotation: *const f32, v_rotation: *const f32,
                                             k_centroids: *const f32, v_centroids: *const f32,
                                             num_tokens: c_int, num_q_heads: c_int,
                                             num_kv_heads: c_int, head_dim: c_int,
                                             kv_len: c_int, start_pos: c_int, key_bits: c_int,
                                             value_bits: c_int, k_packed_dim_per_head: c_int,
                                             v_packed_dim_per_head: c_int,
                                             workspace: *mut c_void, workspace_bytes: usize,
                                             stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_attention_paged_tq_noalloc(output: *mut c_void, q: *const c_void,
                                                  block_table: *const c_int,
                                                  k_packed_ptrs: *const *const c_void,
                                                  k_norms_ptrs: *const *const c_void,
                                                  v_packed_ptrs: *const *const c_void,
                                                  v_norms_ptrs: *const *const c_void,
                                                  k_rotation: *const f32,
                                                  v_rotation: *const f32,
                                                  k_centroids: *const f32,
                                                  v_centroids: *const f32, num_tokens: c_int,
                                                  num_q_heads: c_int, num_kv_heads: c_int,
                                                  head_dim: c_int, kv_len: c_int,
                                                  start_pos: c_int, key_bits: c_int,
                                                  value_bits: c_int,
                                                  k_packed_dim_per_head: c_int,
                                                  v_packed_dim_per_head: c_int,
                                                  stream: hipStream_t) -> hipError_t;
    pub fn fhip_attention_tq_workspace_bytes(batch: c_int, num_q_heads: c_int, head_dim: c_int,
                                             max_blocks: c_int) -> usize;
    pub fn fhip_launch_add_rmsnorm(residual: *mut c_void, delta: *const c_void,
                                   weight: *const c_void, eps: f32, normed_out: *mut c_void,
                                   rows: c_int, cols: c_int, dtype: c_int,
                                   stream: hipStream_t) -> hipError_t;
    pub fn fhip_rows_workspace_bytes(rows: c_int, cols: c_int) -> usize;
    pub fn fhip_launch_softmax_rows(logits: *const f32, probs: *mut f32, rows: c_int,
                                    cols: c_int, temperature: f32, workspace: *mut c_void,
                                    stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_argmax_rows(logits: *const f32, index_out: *mut i32,
                                   flags_out: *mut u32, rows: c_int, cols: c_int,
                                   workspace: *mut c_void, stream: hipStream_t) -> hipError_t;
    pub fn fhip_launch_tq_quantize_pack(y: *const f32, centroids: *const f32, n_levels: c_int,
                                        bits: c_int, packed_out: *mut c_void, rows: c_int,
                                        head_dim: c_int, packed_dim_per_head: c_int,
                                        stream: hipStream_t) -> hipError_t;
}

// The reference's launcher names (ffi.rs:141-274), for callers written against
// `fracture_cuda::ffi::*`.
pub use self::fhip_launch_add as launch_add;
pub use self::fhip_launch_attention as launch_attention;
pub use self::fhip_launch_attention_paged_tq as launch_attention_paged_tq;
pub use self::fhip_launch_embedding as launch_embedding;
pub use self::fhip_launch_paged_attention as launch_paged_attention;
pub use self::fhip_launch_rmsnorm as launch_rmsnorm;
pub use self::fhip_launch_rope as launch_rope;
pub use self::fhip_launch_silu_mul as launch_silu_mul;
pub use self::fhip_launch_turboquant_compress as launch_turboquant_compress;
pub use self::fhip_launch_turboquant_decompress as launch_turboquant_decompress;

//! The handle runtime of libfracture_hip.so (include/fracture_hip.h, section 2): the C mirror
//! of the Backend trait that `HipBackend` wraps. Status codes are `FHIP_*`; the message of a
//! thread's last failing call is `fhip_last_error()`.

use std::ffi::{c_char, c_int, c_void};

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
                                           block_tables: *const i32, max_blocks: usize,
                                           seq_lens: *const u32, pool: u64,
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

//! `impl Backend for HipBackend` (backends/fracture-cuda/src/backend.rs:7-710 is the CUDA
//! counterpart): each method converts its tensors to `FhipTensor` descriptors and makes one
//! handle-runtime call; shape rules, error messages and staging live in the library.

use crate::ext::BackendExt;
use crate::ffi::*;
use fracture_core::{Backend, DType, DeviceTensor, DeviceTimer, FractureError, Result, TensorId};
use std::ffi::{c_int, c_void, CStr, CString};

/// One GPU: a handle-runtime backend (its own stream, tensor registry, staging slots,
/// workspace and small-tensor arena).
pub struct HipBackend {
    h: *mut FhipBackend,
    name: String,
}

// The runtime guards its registry, staging ring and launches with its own mutexes.
unsafe impl Send for HipBackend {}
unsafe impl Sync for HipBackend {}

fn last_error() -> String {
    let p = unsafe { fhip_last_error() };
    if p.is_null() {
        return String::new();
    }
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

/// Status code -> FractureError, with the message of the failing call.
fn check(code: c_int) -> Result<()> {
    match code {
        FHIP_OK => Ok(()),
        FHIP_ERR_INVALID_SHAPE => Err(FractureError::InvalidShape(last_error())),
        FHIP_ERR_TENSOR_NOT_FOUND => Err(FractureError::TensorNotFound(last_error())),
        FHIP_ERR_UNSUPPORTED_DTYPE => Err(FractureError::UnsupportedDType(last_error())),
        FHIP_ERR_GENERATION => Err(FractureError::Generation(last_error())),
        _ => Err(FractureError::Backend(last_error())),
    }
}

fn dtype_code(d: DType) -> i32 {
    match d {
        DType::FP16 => FHIP_FP16,
        DType::FP32 => FHIP_FP32,
        DType::BF16 => FHIP_BF16,
        DType::INT8 => FHIP_INT8,
        DType::INT4 => FHIP_INT4,
    }
}

fn desc(t: &DeviceTensor) -> Result<FhipTensor> {
    if t.shape.len() > FHIP_MAX_DIMS {
        return Err(FractureError::InvalidShape(format!(
            "rank {} exceeds {FHIP_MAX_DIMS}",
            t.shape.len()
        )));
    }
    let mut shape = [0u64; FHIP_MAX_DIMS];
    for (d, &n) in shape.iter_mut().zip(&t.shape) {
        *d = n as u64;
    }
    Ok(FhipTensor { id: t.id.0, dtype: dtype_code(t.dtype), ndim: t.shape.len() as i32, shape })
}

fn descs(ts: &[&DeviceTensor]) -> Result<Vec<FhipTensor>> {
    ts.iter().map(|t| desc(t)).collect()
}

impl HipBackend {
    /// CudaBackend::new (lib.rs:76-114): the backend of device `device_id`.
    pub fn new(device_id: i32) -> Result<Self> {
        let mut h = std::ptr::null_mut();
        check(unsafe { fhip_backend_create(device_id as c_int, &mut h) })?;
        let p = unsafe { fhip_device_name(h) };
        let name = if p.is_null() {
            String::new()
        } else {
            unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
        };
        Ok(Self { h, name })
    }

    /// CudaBackend::get_ptr (lib.rs:117-125).
    pub fn get_ptr(&self, id: TensorId) -> Result<*mut c_void> {
        let mut p = std::ptr::null_mut();
        check(unsafe { fhip_get_ptr(self.h, id.0, &mut p) })?;
        Ok(p)
    }

    /// CudaBackend::stream (lib.rs:127-129): the stream every launch goes to, for direct
    /// calls of the raw launchers in `ffi`.
    pub fn stream(&self) -> hipStream_t {
        unsafe { fhip_stream(self.h) }
    }

    /// CudaBackend::precompute_rope_freqs (lib.rs:133-155): the frequency table `rope` reads
    /// (`&mut self` as in the reference; the table lives in the runtime).
    pub fn precompute_rope_freqs(&mut self, head_dim: usize, theta: f64) -> Result<()> {
        check(unsafe { fhip_precompute_rope_freqs(self.h, head_dim, theta) })
    }

    // ── additive API ──────────────────────────────────────────────

    /// Register a KV page pool once: (K, V) lists, or (K packed, K norms, V packed, V norms),
    /// each of pool_len block tensors indexed by physical block id.
    pub fn page_pool_create(&self, lists: &[&[&DeviceTensor]]) -> Result<u64> {
        let n = lists.first().map_or(0, |l| l.len());
        if lists.iter().any(|l| l.len() != n) {
            return Err(FractureError::InvalidShape("block lists differ in length".into()));
        }
        let mut flat = Vec::with_capacity(n * lists.len());
        for l in lists {
            flat.extend(descs(l)?);
        }
        let mut pool = 0u64;
        check(unsafe {
            fhip_page_pool_create(self.h, flat.as_ptr(), lists.len(), n, &mut pool)
        })?;
        Ok(pool)
    }

    pub fn page_pool_destroy(&self, pool: u64) -> Result<()> {
        check(unsafe { fhip_page_pool_destroy(self.h, pool) })
    }

    /// QuantizedKvCacheManager::append_kv for one layer (quantized_paged_kv_cache.rs:404-500)
    /// straight into a registered TurboQuant pool, keys and values in one launch.
    #[allow(clippy::too_many_arguments)]
    pub fn tq_append_kv(&self, pool: u64, keys: &DeviceTensor, values: &DeviceTensor,
                        k_rotation: &DeviceTensor, v_rotation: &DeviceTensor,
                        k_centroids: &DeviceTensor, v_centroids: &DeviceTensor, key_bits: u8,
                        value_bits: u8, block_table: &[i32], start_pos: usize) -> Result<()> {
        check(unsafe {
            fhip_tq_append_kv(self.h, pool, &desc(keys)?, &desc(values)?, &desc(k_rotation)?,
                              &desc(v_rotation)?, &desc(k_centroids)?, &desc(v_centroids)?,
                              key_bits, value_bits, block_table.as_ptr(), block_table.len(),
                              start_pos)
        })
    }

    /// The engine's per-sequence attention_paged_tq calls of a decode step (batched.rs:145-194)
    /// as one call over a registered pool: block_tables is [B, max_blocks] row-major and
    /// seq_lens has B entries, B being q's first dimension (checked here and in the library,
    /// which reads the two host arrays only that far).
    #[allow(clippy::too_many_arguments)]
    pub fn attention_paged_tq_batched_pool(&self, q: &DeviceTensor, block_tables: &[i32],
                                           max_blocks: usize, seq_lens: &[u32], pool: u64,
                                           k_rotation: &DeviceTensor, v_rotation: &DeviceTensor,
                                           k_centroids: &DeviceTensor,
                                           v_centroids: &DeviceTensor, key_bits: u8,
                                           value_bits: u8, num_kv_heads: usize,
                                           out: &DeviceTensor) -> Result<()> {
        let b = q.shape.first().copied().unwrap_or(0);
        if seq_lens.len() != b || block_tables.len() != b * max_blocks {
            return Err(FractureError::InvalidShape(format!(
                "attention_paged_tq_batched: {} lengths and {} block-table entries ({} per \
                 sequence) for {} queries",
                seq_lens.len(),
                block_tables.len(),
                max_blocks,
                b
            )));
        }
        check(unsafe {
            fhip_attention_paged_tq_batched(self.h, &desc(q)?, block_tables.as_ptr(),
                                            seq_lens.len(), max_blocks, seq_lens.as_ptr(), pool,
                                            &desc(k_rotation)?, &desc(v_rotation)?,
                                            &desc(k_centroids)?, &desc(v_centroids)?, key_bits,
                                            value_bits, num_kv_heads, &desc(out)?)
        })
    }

    /// Capture the launches issued between graph_begin and graph_end into a replayable graph
    /// (only device-resident ops are accepted while capturing: rope_dev / embedding_dev for
    /// positions and token ids).
    pub fn graph_begin(&self) -> Result<()> {
        check(unsafe { fhip_graph_begin(self.h) })
    }
    pub fn graph_end(&self) -> Result<u64> {
        let mut g = 0u64;
        check(unsafe { fhip_graph_end(self.h, &mut g) })?;
        Ok(g)
    }
    pub fn graph_launch(&self, graph: u64) -> Result<()> {
        check(unsafe { fhip_graph_launch(self.h, graph) })
    }
    pub fn graph_destroy(&self, graph: u64) -> Result<()> {
        check(unsafe { fhip_graph_destroy(self.h, graph) })
    }
    pub fn rope_dev(&self, q: &DeviceTensor, k: &DeviceTensor, positions: &DeviceTensor,
                    num_positions: usize, head_dim: usize) -> Result<()> {
        check(unsafe {
            fhip_rope_dev(self.h, &desc(q)?, &desc(k)?, &desc(positions)?, num_positions, head_dim)
        })
    }
    pub fn embedding_dev(&self, token_ids: &DeviceTensor, num_tokens: usize,
                         table: &DeviceTensor, out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_embedding_dev(self.h, &desc(token_ids)?, num_tokens, &desc(table)?, &desc(out)?)
        })
    }
}

impl Drop for HipBackend {
    fn drop(&mut self) {
        unsafe { fhip_backend_destroy(self.h) }
    }
}

impl Backend for HipBackend {
    fn alloc(&self, shape: &[usize], dtype: DType) -> Result<DeviceTensor> {
        let dims: Vec<u64> = shape.iter().map(|&n| n as u64).collect();
        let mut t = FhipTensor { id: 0, dtype: 0, ndim: 0, shape: [0; FHIP_MAX_DIMS] };
        check(unsafe {
            fhip_alloc(self.h, dims.as_ptr(), dims.len() as c_int, dtype_code(dtype), &mut t)
        })?;
        Ok(DeviceTensor::new(TensorId(t.id), shape.to_vec(), dtype))
    }

    fn free(&self, tensor: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_free(self.h, &desc(tensor)?) })
    }

    fn copy_to_device(&self, dst: &DeviceTensor, src: &[u8]) -> Result<()> {
        check(unsafe {
            fhip_copy_to_device(self.h, &desc(dst)?, src.as_ptr() as *const c_void, src.len())
        })
    }

    fn copy_to_host(&self, src: &DeviceTensor, dst: &mut [u8]) -> Result<()> {
        check(unsafe {
            fhip_copy_to_host(self.h, &desc(src)?, dst.as_mut_ptr() as *mut c_void, dst.len())
        })
    }

    fn matmul(&self, a: &DeviceTensor, b: &DeviceTensor, out: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_matmul(self.h, &desc(a)?, &desc(b)?, &desc(out)?) })
    }

    fn rmsnorm(&self, input: &DeviceTensor, weight: &DeviceTensor, eps: f64,
               out: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_rmsnorm(self.h, &desc(input)?, &desc(weight)?, eps, &desc(out)?) })
    }

    fn rope(&self, q: &DeviceTensor, k: &DeviceTensor, positions: &[u32], theta: f64,
            head_dim: usize) -> Result<()> {
        check(unsafe {
            fhip_rope(self.h, &desc(q)?, &desc(k)?, positions.as_ptr(), positions.len(), theta,
                      head_dim)
        })
    }

    fn attention(&self, q: &DeviceTensor, k_cache: &DeviceTensor, v_cache: &DeviceTensor,
                 num_kv_heads: usize, start_pos: usize, out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_attention(self.h, &desc(q)?, &desc(k_cache)?, &desc(v_cache)?, num_kv_heads,
                           start_pos, &desc(out)?)
        })
    }

    fn attention_paged(&self, q: &DeviceTensor, block_table: &[i32], k_blocks: &[&DeviceTensor],
                       v_blocks: &[&DeviceTensor], num_kv_heads: usize, kv_len: usize,
                       start_pos: usize, out: &DeviceTensor) -> Result<()> {
        if k_blocks.len() != v_blocks.len() {
            return Err(FractureError::InvalidShape("k_blocks and v_blocks differ in length".into()));
        }
        let (k, v) = (descs(k_blocks)?, descs(v_blocks)?);
        check(unsafe {
            fhip_attention_paged(self.h, &desc(q)?, block_table.as_ptr(), block_table.len(),
                                 k.as_ptr(), v.as_ptr(), k.len(), num_kv_heads, kv_len,
                                 start_pos, &desc(out)?)
        })
    }

    fn silu_mul(&self, gate: &DeviceTensor, up: &DeviceTensor, out: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_silu_mul(self.h, &desc(gate)?, &desc(up)?, &desc(out)?) })
    }

    fn embedding(&self, token_ids: &[u32], embedding_table: &DeviceTensor,
                 out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_embedding(self.h, token_ids.as_ptr(), token_ids.len(), &desc(embedding_table)?,
                           &desc(out)?)
        })
    }

    fn add(&self, a: &DeviceTensor, b: &DeviceTensor, out: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_add(self.h, &desc(a)?, &desc(b)?, &desc(out)?) })
    }

    fn copy_rows(&self, src: &DeviceTensor, dst: &DeviceTensor, src_offset: usize,
                 dst_offset: usize, count: usize) -> Result<()> {
        check(unsafe {
            fhip_copy_rows(self.h, &desc(src)?, &desc(dst)?, src_offset, dst_offset, count)
        })
    }

    fn device_name(&self) -> &str {
        &self.name
    }

    fn total_memory(&self) -> usize {
        unsafe { fhip_total_memory(self.h) }
    }

    fn available_memory(&self) -> usize {
        unsafe { fhip_available_memory(self.h) }
    }

    fn synchronize(&self) -> Result<()> {
        check(unsafe { fhip_synchronize(self.h) })
    }

    fn create_timer(&self) -> Result<DeviceTimer> {
        let mut id = 0u64;
        check(unsafe { fhip_create_timer(self.h, &mut id) })?;
        Ok(DeviceTimer(id))
    }

    fn start_timer(&self, timer: &DeviceTimer) -> Result<()> {
        check(unsafe { fhip_start_timer(self.h, timer.0) })
    }

    fn stop_timer(&self, timer: &DeviceTimer) -> Result<f32> {
        let mut ms = 0f32;
        check(unsafe { fhip_stop_timer(self.h, timer.0, &mut ms) })?;
        Ok(ms)
    }

    fn destroy_timer(&self, timer: &DeviceTimer) -> Result<()> {
        check(unsafe { fhip_destroy_timer(self.h, timer.0) })
    }

    fn marker_push(&self, name: &str) {
        if let Ok(c) = CString::new(name) {
            unsafe { fhip_marker_push(self.h, c.as_ptr()) }
        }
    }

    fn marker_pop(&self) {
        unsafe { fhip_marker_pop(self.h) }
    }

    fn turboquant_compress(&self, input: &DeviceTensor, rotation_matrix: &DeviceTensor,
                           centroids: &DeviceTensor, bits: u8, packed_out: &DeviceTensor,
                           norms_out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_turboquant_compress(self.h, &desc(input)?, &desc(rotation_matrix)?,
                                     &desc(centroids)?, bits, &desc(packed_out)?,
                                     &desc(norms_out)?)
        })
    }

    fn attention_paged_tq(&self, q: &DeviceTensor, block_table: &[i32],
                          k_packed: &[&DeviceTensor], k_norms: &[&DeviceTensor],
                          v_packed: &[&DeviceTensor], v_norms: &[&DeviceTensor],
                          k_rotation: &DeviceTensor, v_rotation: &DeviceTensor,
                          k_centroids: &DeviceTensor, v_centroids: &DeviceTensor, key_bits: u8,
                          value_bits: u8, num_kv_heads: usize, kv_len: usize, start_pos: usize,
                          out: &DeviceTensor) -> Result<()> {
        let n = k_packed.len();
        if k_norms.len() != n || v_packed.len() != n || v_norms.len() != n {
            return Err(FractureError::InvalidShape("block lists differ in length".into()));
        }
        let (kp, kn, vp, vn) = (descs(k_packed)?, descs(k_norms)?, descs(v_packed)?, descs(v_norms)?);
        check(unsafe {
            fhip_attention_paged_tq(self.h, &desc(q)?, block_table.as_ptr(), block_table.len(),
                                    kp.as_ptr(), kn.as_ptr(), vp.as_ptr(), vn.as_ptr(), n,
                                    &desc(k_rotation)?, &desc(v_rotation)?,
                                    &desc(k_centroids)?, &desc(v_centroids)?, key_bits,
                                    value_bits, num_kv_heads, kv_len, start_pos, &desc(out)?)
        })
    }
}

/// The additive ops on this backend's fused kernels.
impl BackendExt for HipBackend {
    /// One pass: residual += delta (rounded), normed = rmsnorm(residual).
    fn add_rmsnorm(&self, residual: &DeviceTensor, delta: &DeviceTensor,
                   weight: &DeviceTensor, eps: f64, normed: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_add_rmsnorm(self.h, &desc(residual)?, &desc(delta)?, &desc(weight)?, eps,
                             &desc(normed)?)
        })
    }

    fn softmax_rows(&self, logits: &DeviceTensor, temperature: f32,
                    probs: &DeviceTensor) -> Result<()> {
        check(unsafe { fhip_softmax_rows(self.h, &desc(logits)?, temperature, &desc(probs)?) })
    }

    fn argmax_rows(&self, logits: &DeviceTensor) -> Result<Vec<u32>> {
        let cols = logits.shape.last().copied().unwrap_or(0);
        let rows = if cols == 0 { 0 } else { logits.numel() / cols };
        let mut out = vec![0u32; rows];
        check(unsafe { fhip_argmax_rows(self.h, &desc(logits)?, out.as_mut_ptr(), rows) })?;
        Ok(out)
    }

    fn tq_dequantize(&self, packed: &DeviceTensor, norms: &DeviceTensor,
                     rotation: &DeviceTensor, centroids: &DeviceTensor, bits: u8,
                     out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_tq_dequantize(self.h, &desc(packed)?, &desc(norms)?, &desc(rotation)?,
                               &desc(centroids)?, bits, &desc(out)?)
        })
    }

    fn tq_quantize_pack(&self, y: &DeviceTensor, centroids: &DeviceTensor, bits: u8,
                        packed_out: &DeviceTensor) -> Result<()> {
        check(unsafe {
            fhip_tq_quantize_pack(self.h, &desc(y)?, &desc(centroids)?, bits, &desc(packed_out)?)
        })
    }

    /// The whole batch in one launch sequence: the block lists are registered as a pool for
    /// the call (their device address arrays built once), then released. Callers that keep
    /// a pool across steps use `page_pool_create` and `attention_paged_tq_batched_pool`.
    fn attention_paged_tq_batched(&self, q: &DeviceTensor, block_tables: &[i32],
                                  max_blocks: usize, seq_lens: &[u32],
                                  k_packed: &[&DeviceTensor], k_norms: &[&DeviceTensor],
                                  v_packed: &[&DeviceTensor], v_norms: &[&DeviceTensor],
                                  k_rotation: &DeviceTensor, v_rotation: &DeviceTensor,
                                  k_centroids: &DeviceTensor, v_centroids: &DeviceTensor,
                                  key_bits: u8, value_bits: u8, num_kv_heads: usize,
                                  out: &DeviceTensor) -> Result<()> {
        let pool = self.page_pool_create(&[k_packed, k_norms, v_packed, v_norms])?;
        let run = self.attention_paged_tq_batched_pool(q, block_tables, max_blocks, seq_lens,
                                                       pool, k_rotation, v_rotation,
                                                       k_centroids, v_centroids, key_bits,
                                                       value_bits, num_kv_heads, out);
        let done = self.page_pool_destroy(pool);
        run.and(done)
    }
}

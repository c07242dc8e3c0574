//! `BackendExt`: the ops this backend adds to `fracture_core::Backend`, as an extension trait.
//!
//! Every method has a default built from `Backend` methods only, so any backend (the CUDA
//! one included) gets them with an empty `impl BackendExt for CudaBackend {}` and the engine
//! needs no change to call them; `HipBackend` overrides each with its fused kernels. The
//! defaults reproduce what the reference does today:
//!
//! * `add_rmsnorm`: `add` then `rmsnorm`, as the engine issues them (engine.rs:692-697);
//! * `softmax_rows` / `argmax_rows`: the sampler on the host after a copy of the logits
//!   (sampling.rs:45-82, engine.rs:728-738);
//! * `attention_paged_tq_batched`: one `attention_paged_tq` per sequence at its last
//!   position, as `dispatch_attention` does (batched.rs:145-194);
//! * `tq_dequantize` / `tq_quantize_pack`: no trait method composes them, so the default is
//!   the trait's own "not supported" error, as for its optional TurboQuant methods
//!   (backend.rs:166-222).

use fracture_core::{Backend, DType, DeviceTensor, FractureError, Result};

fn f32_rows<B: Backend + ?Sized>(b: &B, t: &DeviceTensor) -> Result<(usize, usize, Vec<f32>)> {
    if t.dtype != DType::FP32 || t.shape.is_empty() {
        return Err(FractureError::InvalidShape(format!(
            "logits must be fp32 [rows, vocab], got {:?} {:?}",
            t.shape, t.dtype
        )));
    }
    let cols = t.shape[t.shape.len() - 1];
    let rows = if cols == 0 { 0 } else { t.numel() / cols };
    let mut bytes = vec![0u8; t.size_bytes()];
    b.copy_to_host(t, &mut bytes)?;
    let vals = bytes
        .chunks_exact(4)
        .map(|c| f32::from_le_bytes([c[0], c[1], c[2], c[3]]))
        .collect();
    Ok((rows, cols, vals))
}

pub trait BackendExt: Backend {
    /// residual += delta (in place, rounded to the dtype); normed = rmsnorm(residual).
    fn add_rmsnorm(&self, residual: &DeviceTensor, delta: &DeviceTensor,
                   weight: &DeviceTensor, eps: f64, normed: &DeviceTensor) -> Result<()> {
        self.add(residual, delta, residual)?;
        self.rmsnorm(residual, weight, eps, normed)
    }

    /// probs [rows, vocab] fp32 = exp(logits / T - max) / sum per row (sampling.rs:69-82).
    fn softmax_rows(&self, logits: &DeviceTensor, temperature: f32,
                    probs: &DeviceTensor) -> Result<()> {
        let (rows, cols, l) = f32_rows(self, logits)?;
        if probs.dtype != DType::FP32 || probs.numel() != rows * cols {
            return Err(FractureError::InvalidShape("probs must match logits, fp32".into()));
        }
        let mut out = Vec::with_capacity(rows * cols * 4);
        for r in 0..rows {
            let row = &l[r * cols..(r + 1) * cols];
            let scaled: Vec<f32> = row.iter().map(|&x| x / temperature).collect();
            let max = scaled.iter().copied().fold(f32::NEG_INFINITY, f32::max);
            let exps: Vec<f32> = scaled.iter().map(|&x| (x - max).exp()).collect();
            let sum: f32 = exps.iter().sum();
            for e in exps {
                out.extend_from_slice(&(e / sum).to_le_bytes());
            }
        }
        self.copy_to_device(probs, &out)
    }

    /// The greedy token of each row of logits [rows, vocab] fp32 (sampling.rs:45-66): the
    /// largest value, ties to the last index; empty, NaN or Inf rows are errors.
    fn argmax_rows(&self, logits: &DeviceTensor) -> Result<Vec<u32>> {
        let (rows, cols, l) = f32_rows(self, logits)?;
        if cols == 0 {
            return Err(FractureError::Generation("empty logits".into()));
        }
        let mut out = Vec::with_capacity(rows);
        for r in 0..rows {
            let row = &l[r * cols..(r + 1) * cols];
            if row.iter().any(|x| x.is_nan()) {
                return Err(FractureError::Generation("NaN in logits".into()));
            }
            if row.iter().any(|x| x.is_infinite()) {
                return Err(FractureError::Generation("Inf in logits".into()));
            }
            let mut best = 0usize;
            for (i, &x) in row.iter().enumerate() {
                if x >= row[best] {
                    best = i;
                }
            }
            out.push(best as u32);
        }
        Ok(out)
    }

    /// launch_turboquant_decompress through tensors: packed [N, kvh * pd] and norms [N, kvh]
    /// back to out [N, kvh, hd] fp16.
    #[allow(clippy::too_many_arguments)]
    fn tq_dequantize(&self, _packed: &DeviceTensor, _norms: &DeviceTensor,
                     _rotation: &DeviceTensor, _centroids: &DeviceTensor, _bits: u8,
                     _out: &DeviceTensor) -> Result<()> {
        Err(FractureError::Backend("TurboQuant dequantize not supported by this backend".into()))
    }

    /// Quantize + pack of given fp32 rotated vectors y [N, kvh, hd] into packed
    /// [N, kvh * pd] (first nearest centroid, MSB-first bit order).
    fn tq_quantize_pack(&self, _y: &DeviceTensor, _centroids: &DeviceTensor, _bits: u8,
                        _packed_out: &DeviceTensor) -> Result<()> {
        Err(FractureError::Backend(
            "TurboQuant quantize-pack not supported by this backend".into(),
        ))
    }

    /// Decode attention of a batch: q [B, qh, hd] fp16, one query per sequence at its last
    /// position; sequence i attends seq_lens[i] positions through row i of block_tables
    /// [B, max_blocks]; out [B, qh, hd] fp16.
    #[allow(clippy::too_many_arguments)]
    fn attention_paged_tq_batched(&self, q: &DeviceTensor, block_tables: &[i32],
                                  max_blocks: usize, seq_lens: &[u32],
                                  k_packed: &[&DeviceTensor], k_norms: &[&DeviceTensor],
                                  v_packed: &[&DeviceTensor], v_norms: &[&DeviceTensor],
                                  k_rotation: &DeviceTensor, v_rotation: &DeviceTensor,
                                  k_centroids: &DeviceTensor, v_centroids: &DeviceTensor,
                                  key_bits: u8, value_bits: u8, num_kv_heads: usize,
                                  out: &DeviceTensor) -> Result<()> {
        let b = q.shape.first().copied().unwrap_or(0);
        if q.shape.len() != 3 || seq_lens.len() != b || block_tables.len() != b * max_blocks {
            return Err(FractureError::InvalidShape(format!(
                "attention_paged_tq_batched: q {:?}, {} lengths, {} block-table entries for {} \
                 blocks per sequence",
                q.shape,
                seq_lens.len(),
                block_tables.len(),
                max_blocks
            )));
        }
        let row_shape = [1, q.shape[1], q.shape[2]];
        let q1 = self.alloc(&row_shape, q.dtype)?;
        let o1 = self.alloc(&row_shape, out.dtype)?;
        let run = (|| -> Result<()> {
            for (i, &len) in seq_lens.iter().enumerate() {
                let len = len as usize;
                let used = len.div_ceil(16).min(max_blocks);
                self.copy_rows(q, &q1, i, 0, 1)?;
                self.attention_paged_tq(&q1, &block_tables[i * max_blocks..i * max_blocks + used],
                                        k_packed, k_norms, v_packed, v_norms, k_rotation,
                                        v_rotation, k_centroids, v_centroids, key_bits,
                                        value_bits, num_kv_heads, len, len.saturating_sub(1),
                                        &o1)?;
                self.copy_rows(&o1, out, 0, i, 1)?;
            }
            Ok(())
        })();
        let f1 = self.free(&q1);
        let f2 = self.free(&o1);
        run.and(f1).and(f2)
    }
}

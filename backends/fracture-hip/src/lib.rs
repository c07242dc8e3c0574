//! AMD MI355X backend for Fracture: `HipBackend` implements `fracture_core::Backend` over the
//! handle runtime of libfracture_hip.so (include/fracture_hip.h), the way
//! backends/fracture-cuda implements it over its CUDA kernels.
//!
//! Every trait method is one call into the library, which resolves tensor ids to device
//! memory, checks shapes with the same rules and messages as the CUDA backend, stages
//! host-side arguments (positions, token ids, block tables) through pinned buffers and
//! launches on the backend's stream. Status codes map to `FractureError` variants with the
//! library's message.

//!
//! `BackendExt` carries the ops this backend adds (fused add + RMSNorm, row softmax and
//! argmax, TurboQuant dequantize and quantize-pack, batched decode attention), each with a
//! default composed from `Backend` methods, so other backends and the engine take it
//! unchanged. `ffi` also binds the raw launchers under the reference's `launch_*` names.
//! The crate's inherent API matches `CudaBackend`'s for its callers: `new(i32)`,
//! `get_ptr(TensorId)`, `stream()`, `precompute_rope_freqs(&mut self, usize, f64)`.

pub mod ffi;
mod backend;
mod ext;

pub use backend::HipBackend;
pub use ext::BackendExt;

//! AMD MI355X backend for Fracture: `HipBackend` implements `fracture_core::Backend` over the
//! handle runtime of libfracture_hip.so (include/fracture_hip.h), the way
//! backends/fracture-cuda implements it over its CUDA kernels.
//!
//! Every trait method is one call into the library, which resolves tensor ids to device
//! memory, checks shapes with the same rules and messages as the CUDA backend, stages
//! host-side arguments (positions, token ids, block tables) through pinned buffers and
//! launches on the backend's stream. Status codes map to `FractureError` variants with the
//! library's message.

pub mod ffi;
mod backend;

pub use backend::HipBackend;

"""fracture_amd: an MI355X (gfx950) backend for Fracture's elementwise, reduction and
TurboQuant KV-cache hot path.

* ``fracture_amd.backend.HipBackend`` — the `Backend` trait over opaque tensor ids;
* ``fracture_amd.kernels`` — raw launchers on torch device tensors;
* ``fracture_amd.turboquant`` — TurboQuant configuration and host tables;
* ``include/fracture_hip.h`` — the C ABI of ``libfracture_hip.so`` behind all of them.
"""
from .backend import (BackendError, DeviceTensor, DeviceTimer, DType, FractureError,
                      GenerationError, HipBackend, InvalidShape, OutOfMemory, TensorId,
                      TensorNotFound, UnsupportedDType)

__all__ = ["HipBackend", "DeviceTensor", "DeviceTimer", "DType", "TensorId", "FractureError",
           "BackendError", "InvalidShape", "TensorNotFound", "OutOfMemory", "UnsupportedDType",
           "GenerationError"]
__version__ = "0.1.0"

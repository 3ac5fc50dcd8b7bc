"""MI355X (gfx950) fused attention for the Supra2-Img Web attention hot path.

The operator itself is HIP code behind the C ABI in include/supra_attn.h
(lib/libsupra_attn.so); this package is its Python binding:

- `_lib`      ctypes declarations of every exported symbol, AttnArgs, status codes
- `device`    device buffers / stream / events over the C ABI helpers
- `workloads` seeded inputs for the DiT, T5 and VAE call shapes
- `runner`    stage a workload on the device and launch it
"""

from ._lib import AttnArgs, LinearArgs, SaError, attention, bucket_lut, kernel_name, linear, load, workspace_bytes  # noqa: F401

__all__ = ["AttnArgs", "LinearArgs", "SaError", "attention", "bucket_lut", "kernel_name", "linear", "load", "workspace_bytes"]

"""flashmap_amd: the FlashMap drafter's attention hot path on MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (include/flashmap_amd.h), bound with ctypes
(flashmap_amd._native) and exposed as torch functions (flashmap_amd.ops).
"""

__version__ = "0.1.0"

"""woodcock_amd -- MI355X-native (gfx950) speculative-decoding round for Woodcock.

Hand-written HIP kernels behind a C ABI (``include/woodcock_hip.h``,
``woodcock_amd/csrc``), driven from Python through ctypes on PyTorch-ROCm
device memory.  The host modules mirror the reference's drafter / verify /
KV-compaction API (python/woodcock/{drafter,sampling,target,spec}.py).
Importing this package does not load the HIP library; the first call that
needs it does, and raises if it is missing.
"""

__version__ = "0.1.0"

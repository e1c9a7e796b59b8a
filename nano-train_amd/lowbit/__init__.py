"""MI355X-native low-bit linear hot path of nano-train (gfx950 HIP kernels behind a C-ABI).

Public surface:
  lowbit.backend.HipLowBitBackend   - the LowBitBackend drop-in ("hip")
  lowbit.ops                        - tensor-level kernel wrappers
  lowbit.contracts                  - the reference's precision value types
"""

__all__ = ["backend", "ops", "contracts"]

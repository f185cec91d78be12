"""flash_lab for MI355X (gfx950): FlashAttention-2 prefill and split-KV decode as hand-written
HIP kernels behind the reference's flash_lab API (reference flash_lab/__init__.py:1-5).

The reference also exports its fp64 test oracle as flash_lab.reference; in this build the oracle
is test infrastructure and lives outside the package (oracle/reference.py at the repository root).
"""

from flash_lab.ops import attention, available_impls, decode

__version__ = "0.1.0"
__all__ = ["attention", "available_impls", "decode"]

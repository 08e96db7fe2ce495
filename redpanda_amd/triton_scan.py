"""Module with the reference's `triton_scan` interface, backed by the HIP kernels.

The reference's callers import exactly these names:
  engine/mamba.py:344   from triton_scan import HAS_TRITON, triton_trapezoidal_scan
  engine/train.py:711   from triton_scan import HAS_TRITON, verify as verify_triton
Putting `engine/triton_scan.py` = `from redpanda_amd.triton_scan import *`
(or `sys.modules["triton_scan"] = redpanda_amd.triton_scan`) routes both to
the HIP path with no other change to the reference.
"""

from redpanda_amd.scan import HAS_TRITON, hip_scan_with_state, triton_trapezoidal_scan
from redpanda_amd.verify import verify

__all__ = ["HAS_TRITON", "triton_trapezoidal_scan", "verify", "hip_scan_with_state"]

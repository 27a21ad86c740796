"""flarellm_amd -- MI355X-native decode backend for flarellm.

The compute path is libflare_hip.so (hand-written HIP for gfx950) behind the
C-ABI in include/flare_hip.h; this package is the Python host binding used by
tests and the benchmark.
"""
from ._lib import FL_F32, FL_KV_F16, FL_KV_F32, FL_KV_KIVI2, FL_KV_Q8, FL_Q4K, FL_Q6K, FL_Q8_0, FlareError, load  # noqa: F401

__all__ = ["FL_F32", "FL_Q8_0", "FL_Q4K", "FL_Q6K", "FL_KV_F32", "FL_KV_F16", "FL_KV_Q8", "FL_KV_KIVI2", "FlareError", "load"]

"""lal_amd: MI355X (gfx950) token-sampling path of LAL.

The product is the C ABI in include/lal_gpu_sample.h, implemented by
lal_amd/liblal_gpu.so (built from lal_amd/csrc/lal_gpu_sample.hip).  This
package only loads that library for Python callers (tests, benchmarks); it has
no compute of its own and raises when the library is missing.
"""
from .abi import (LIB_PATH, load, GpuError, Device, SampleParams, SampleIO,  # noqa: F401
                  VARIANT_BASIC, VARIANT_FILTERED, F_WRITEBACK, F_DRAW_GPT2,
                  MAX_K, MAX_HISTORY, MAX_BAN_IDS)

"""MI355X (gfx950) quantized-K pruned decode attention: host side of libffa_mi355x.so.

Compute runs only in the HIP kernels of libffa_mi355x.so (csrc/); this
package validates arguments, owns scratch through torch allocations and
calls the C ABI (include/ffa_mi355x.h) on the current HIP stream.
"""
from .decode import DecodeWorkspace, decode_nparts, decode_ntbs, run_decode, skip_ratio_of  # noqa: F401
from .paged import PAGE, PagedQ2Cache  # noqa: F401

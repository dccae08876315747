"""aegaeon_amd: MI355X-native KV-cache movement (swap-out, swap-in, in-HBM copy).

The data plane is libaegkv.so (hand-written HIP for gfx950, C ABI in
include/aegkv.h); this package is the host-side mirror of the reference's
operator API for that path.
"""

__all__ = ["ops"]

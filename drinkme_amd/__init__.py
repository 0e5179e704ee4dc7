"""drinkme_amd — drinkme's fused radix decode + matmul, native to MI355X (gfx950).

The kernels and the host codec live in libdmx_radix.so (include/dmx_radix.h);
radix_ops mirrors drinkme's radix_ops launcher surface over it, swap the
runtime dict and the compressed Linear, radix_pack the producer side
(profiles, encoder, raw fallback, descriptor gate).
"""

__all__ = ["radix_ops", "radix_pack", "swap", "synth"]

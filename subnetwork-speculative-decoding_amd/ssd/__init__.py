"""Subnetwork speculative decoding on MI355X (gfx950): the reference ``ssd`` API over
hand-written HIP kernels (libssd_mi355x.so, include/ssd_mi355x.h)."""

__version__ = "0.1.0"

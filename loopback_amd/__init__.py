"""loopback_amd -- the Loopback depth-attention read on MI355X (gfx950): HIP kernels behind a C ABI
(include/loopback_read.h, built by `loopback_amd.build`) and the reference module's autograd interface
(`loopback_amd.fused_dattn`), its caller cell (`loopback_amd.cell`) and the synthetic chain (`loopback_amd.chain`).

Importing the package does not load the library; importing `loopback_amd.fused_dattn` does, and fails if it is not
built.
"""
__version__ = "0.1.0"

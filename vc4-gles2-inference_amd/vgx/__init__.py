"""vgx: the MI355X (gfx950) quantized decode path over MMCF weights.

`vgx.lib` binds libvgx's C-ABI (include/vgx.h); `vgx.gpu` mirrors the
reference engine's GPU object over it; `vgx.mmcf` reads and writes the
container the kernels consume; `vgx.synth` makes the seeded synthetic models
the tests and the benchmark use.
"""

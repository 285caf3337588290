"""hf_kernels_helion_amd: MI355X (gfx950) block-FP8 linear path.

Subpackage ``finegrained_fp8_helion`` is the drop-in for the reference package
of the same name; its ops run hand-written HIP kernels from
``_lib/libfp8_blockwise.so`` through the C ABI in include/fp8_blockwise.h.
"""
__version__ = "0.1.0"

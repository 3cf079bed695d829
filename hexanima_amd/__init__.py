"""hexanima_amd -- MI355X (gfx950) DiT block runner behind the HexAnima block-execution C-ABI.

The compute path is libhexanima_hip.so (hand-written HIP kernels; see include/hexanima_hip.h), loaded through
hexanima_amd.hip. Importing this package does not touch the GPU.
"""
__version__ = "0.1.0"

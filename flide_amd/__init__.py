"""flide_amd: Flide's mixture-of-experts layer, built for AMD Instinct MI355X (gfx950).

flide_amd.kernels.moe / fp8 / pointwise keep the Python signatures of flide/kernels/moe.py, fp8.py and
pointwise.py; the arithmetic runs in hand-written HIP kernels behind the C ABI of include/flide_moe.h
(libflide_moe.so, built in-tree by flide_amd.build).
"""
__version__ = "0.1.0"

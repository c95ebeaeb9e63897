"""HIP-backed replacements for flide.kernels.moe, flide.kernels.fp8 and the MoE-path pieces of
flide.kernels.pointwise (same function names and signatures)."""
from . import fp8, moe, pointwise  # noqa: F401

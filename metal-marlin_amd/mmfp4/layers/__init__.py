"""Module-level layers over the FP4 kernels (the reference's
`metal_marlin.layers` surface for this path)."""

from .mmfp4_linear import MMFP4Linear, mmfp4_gemm, rowpacked_to_marlin

__all__ = ["MMFP4Linear", "mmfp4_gemm", "rowpacked_to_marlin"]

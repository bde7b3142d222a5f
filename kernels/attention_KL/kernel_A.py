"""Drop-in for the reference module kernel_A.py: same entry point name, HIP implementation."""

from linearard_amd.attention_KL.kernel_A import SUPPORTED_HEAD_DIMS, lse_stats

lse_stats_triton = lse_stats  # the reference's wrapper name, kept so existing imports resolve

__all__ = ["SUPPORTED_HEAD_DIMS", "lse_stats", "lse_stats_triton"]

"""Drop-in for the reference module kernel_B.py: same entry point name, HIP implementation."""

from linearard_amd.attention_KL.kernel_B import SUPPORTED_HEAD_DIMS, kl_forward

kl_forward_triton = kl_forward  # the reference's wrapper name, kept so existing imports resolve

__all__ = ["SUPPORTED_HEAD_DIMS", "kl_forward", "kl_forward_triton"]

"""Drop-in for the reference module kernel_C.py: same entry point name, HIP implementation."""

from linearard_amd.attention_KL.kernel_C import SUPPORTED_HEAD_DIMS, kl_backward

kl_backward_triton = kl_backward  # the reference's wrapper name, kept so existing imports resolve

__all__ = ["SUPPORTED_HEAD_DIMS", "kl_backward", "kl_backward_triton"]

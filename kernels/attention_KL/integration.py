"""Drop-in for the reference module integration.py (train.py imports ``attn_kl_align`` from here)."""

from linearard_amd.attention_KL.integration import AttnKLAlignFn, attn_kl_align

__all__ = ["AttnKLAlignFn", "attn_kl_align"]

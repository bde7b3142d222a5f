"""Mirror of the reference package ``kernels/attention_KL``."""

from .batched import AttnKLBatchedFn, attn_kl_align_batched, relation_kl_loss
from .integration import AttnKLAlignFn, attn_kl_align
from .kernel_A import SUPPORTED_HEAD_DIMS, lse_stats
from .kernel_B import kl_forward
from .kernel_C import kl_backward

__all__ = ["AttnKLAlignFn", "attn_kl_align", "lse_stats", "kl_forward", "kl_backward", "SUPPORTED_HEAD_DIMS",
           "AttnKLBatchedFn", "attn_kl_align_batched", "relation_kl_loss"]

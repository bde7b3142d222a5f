"""Drop-in for the reference package ``kernels/attention_KL``.

``from kernels.attention_KL.integration import attn_kl_align`` (train.py)
keeps working; everything resolves to ``linearard_amd.attention_KL``.
"""

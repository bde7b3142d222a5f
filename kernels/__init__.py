"""Drop-in import path of the reference (``kernels/attention_KL``); see linearard_amd."""

"""MI355X-native (gfx950 HIP) attention-relation KL for LinearARD.

``linearard_amd.attention_KL`` mirrors the reference package
``kernels/attention_KL`` (integration.py, kernel_A/B/C.py); the compute runs
in ``liblinearard_amd.so`` (hand-written HIP kernels behind a C ABI).
"""

__version__ = "0.1.0"

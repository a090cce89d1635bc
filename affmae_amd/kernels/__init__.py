"""Kernel-level entry points mirroring src/layers/kernels/ of the reference."""
from .knn import knn, knn_forward, knn_hip, KNNFunction  # noqa: F401
from .local_attn import (  # noqa: F401
    FlashLocalAttentionFunction,
    launch_flash_nbhood_attn_fwd,
    nbhd_attn_fwd,
)

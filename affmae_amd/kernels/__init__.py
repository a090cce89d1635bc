"""Kernel-level entry points mirroring src/layers/kernels/ of the reference."""
from .knn import knn, knn_forward, knn_hip, KNNFunction  # noqa: F401
from .local_attn import (  # noqa: F401
    FlashLocalAttentionFunction,
    launch_flash_nbhood_attn_fwd,
    nbhd_attn_fwd,
)
from .weighted_features import weighted_features, WeightedFeaturesFunction  # noqa: F401
from .weighted_gather import (  # noqa: F401
    launch_weighted_gather_fwd_kernel,
    softmax_merge,
    weighted_gather,
    WeightedGatherFunction,
)
from .fused_deform_attn import (  # noqa: F401
    FusedDeformAttnFunction,
    FusedKNNDeformCrossAttnFunction,
    FusedKNNDeformSelfAttnFunction,
    fused_deformable_attention,
    fused_knn_deformable_cross_attention,
    fused_knn_deformable_self_attention,
    ms_deformable_attention,
)
from .msdetrpc import MSDETRPCFunction, launch_msdetrpc_forward  # noqa: F401
from .mssample import mssample, MSSampleFunction  # noqa: F401
from .nbhd_index import cluster_members  # noqa: F401

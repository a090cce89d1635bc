"""nn.Modules with the reference's constructor/forward signatures and parameter names."""
from .attention import ClusterAttention, DeformableCrossAttention, DeformableSelfAttention  # noqa: F401
from .aff import ClusterMerging, neighbourhood_index  # noqa: F401

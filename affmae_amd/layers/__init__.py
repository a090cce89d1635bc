"""nn.Modules with the reference's constructor/forward signatures and parameter names."""
from .attention import ClusterAttention, DeformableCrossAttention, DeformableSelfAttention  # noqa: F401
from .aff import (  # noqa: F401
    AFFEncoder, AFFPatchEmbed, BasicLayer, ClusterMerging, ClusterTransformerBlock, DropPath, L2NormMerging,
    LayerNorm2dImages, Mlp, neighbourhood_index,
)
from .decoder import (  # noqa: F401
    CrossAttentionPixelDecoder, GlobalSelfAttention, MSDecoderBlock, PositionEmbeddingSine, ShapeSpec,
)

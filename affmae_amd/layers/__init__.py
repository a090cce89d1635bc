"""nn.Modules with the reference's constructor/forward signatures and parameter names."""
from .attention import ClusterAttention  # noqa: F401

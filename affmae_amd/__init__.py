"""affmae_amd: the AFFMAE point-token hot path as hand-written HIP kernels for MI355X (gfx950).

Kernels live in libaffmae.so (sources in affmae_amd/csrc, C ABI in
include/affmae.h) and are reached through ctypes wrappers that keep the
reference's Python signatures:

* ``affmae_amd.kernels.knn``          - knn, knn_forward, KNNFunction
* ``affmae_amd.kernels.local_attn``   - launch_flash_nbhood_attn_fwd,
                                        FlashLocalAttentionFunction, nbhd_attn_fwd
* ``affmae_amd.layers.attention``     - ClusterAttention

The shared library is loaded on first use; build it with
``python -m affmae_amd.build_lib``.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]

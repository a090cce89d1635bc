"""Distance-softmax sampling weights (HIP, gfx950).

Drop-in for src/layers/kernels/mssample.py of the reference (``mssample``
:452, ``MSSampleFunction`` :402-449, ``mssample_forward`` :300-342):

    weights[b, n, k, 0] = softmax_k(-max(power, 1e-6) * sqrt(d2 + 1e-6))   (denominator + 1e-8)
"""
from __future__ import annotations

from torch.autograd import Function
from torch.amp import custom_fwd, custom_bwd

from .fused_deform_attn import deform_sample_launch


def mssample_forward(sampling_locs, kv_pos, nb_idx, power, D=2):
    """[B,N,K,1] weights in sampling_locs.dtype."""
    assert sampling_locs.shape[-1] == D
    _, w = deform_sample_launch(1, sampling_locs, kv_pos, nb_idx, power, want_weights=True,
                                weights_dtype=sampling_locs.dtype)
    return w.unsqueeze(-1)


class MSSampleFunction(Function):
    """Autograd entry (forward only: the backward kernel is not built yet)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, sampling_locs, kv_pos, nb_idx, power, D=2):
        return mssample_forward(sampling_locs, kv_pos, nb_idx, power, D)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        raise NotImplementedError("mssample backward is not implemented in affmae_amd yet")


def mssample(sampling_locs, kv_pos, nb_idx, power, D=2):
    return MSSampleFunction.apply(sampling_locs, kv_pos, nb_idx, power, D)

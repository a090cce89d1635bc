"""Distance-softmax sampling weights (HIP, gfx950).

Drop-in for src/layers/kernels/mssample.py of the reference (``mssample``
:452, ``MSSampleFunction`` :402-449, ``mssample_forward`` :300-342):

    weights[b, n, k, 0] = softmax_k(-max(power, 1e-6) * sqrt(d2 + 1e-6))   (denominator + 1e-8)
"""
from __future__ import annotations

from torch.autograd import Function
from torch.amp import custom_fwd, custom_bwd

from .. import _lib
from .fused_deform_attn import _power_grad, _save_power, deform_backward_launch, deform_sample_launch


def mssample_forward(sampling_locs, kv_pos, nb_idx, power, D=2):
    """[B,N,K,1] weights in sampling_locs.dtype."""
    assert sampling_locs.shape[-1] == D
    _, w = deform_sample_launch(1, sampling_locs, kv_pos, nb_idx, power, want_weights=True,
                                weights_dtype=sampling_locs.dtype)
    return w.unsqueeze(-1)


class MSSampleFunction(Function):
    """Autograd entry (reference mssample.py:402-449): backward returns
    (d_sampling_locs, d_kv_pos, None, d_power, None) through aff_deform_bwd."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, sampling_locs, kv_pos, nb_idx, power, D=2):
        ctx.save_for_backward(sampling_locs, kv_pos, nb_idx, _save_power(ctx, power))
        return mssample_forward(sampling_locs, kv_pos, nb_idx, power, D)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        sl, kv, nb_idx, power = ctx.saved_tensors
        n = ctx.needs_input_grad
        d_sl, d_kv, d_pow = mssample_backward(dout, sl, kv, nb_idx, power if power is not None else ctx.power_num,
                                              want=(n[0], n[1], n[3] and power is not None))
        return d_sl, d_kv, None, d_pow, None


def mssample_backward(dout, sampling_locs, kv_pos, nb_idx, power, want=(True, True, True)):
    """(d_sampling_locs, d_kv_pos, d_power) from dL/dweights [B,N,K(,1)] (reference mssample.py:345-399)."""
    B, N, K = nb_idx.shape
    g = deform_backward_launch(_lib.DEFORM_BWD_SAMPLE_SQ, None, idx=nb_idx.reshape(B, N, 1, 1, K),
                               loc=sampling_locs, kv_pos=kv_pos, d_w_in=dout.reshape(B, N, 1, 1, K), power=power,
                               want_loc=want[0], want_kv=want[1], want_power=want[2])
    d_sl = g["d_loc"].reshape(B, N, -1).to(sampling_locs.dtype) if want[0] else None
    d_kv = g["d_kv_pos"].to(kv_pos.dtype) if want[1] else None
    d_pow = _power_grad(g["d_power"], power) if want[2] else None
    return d_sl, d_kv, d_pow


def mssample(sampling_locs, kv_pos, nb_idx, power, D=2):
    return MSSampleFunction.apply(sampling_locs, kv_pos, nb_idx, power, D)

"""The reference's backward of the deformable gathers, restated in torch fp64.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: tests/ compare the
HIP backward (aff_deform_bwd) with :func:`deform_backward`; the product
package ``affmae_amd`` never imports this module.

Rows r = (b, q, h) hold S samples of K neighbours; ``rows`` gives each
neighbour's row in kv_pos / values (-1 for none).  With w the forward weights,
g_j = dL/dw_j = attn * <dout, v_j> (or the given dL/dw), the reference's
chain rule is:

* softmax modes (fused_deform_attn.py:2014-2186 for the fused K-NN kernels,
  :253-500 for given indices, mssample.py:142-298): dlg_j = w_j (g_j - sum_i
  w_i g_i) with w taken from the forward (its 1e-8 in the denominator kept
  in w, absent from the Jacobian), d_dist_j = -p dlg_j, d_power = sum dlg_j
  (-dist_j), d(loc) = sum_j d_dist_j diff_j / den_j with den_j =
  sqrt(d2) + 1e-6 ("shepard", :2128-2140), max(dist - 1e-6, 1e-8) ("sample",
  :470-480) or sqrt(d2 + 1e-6) + 1e-8 ("sample_sq", mssample.py:270-281);
  d(kv_pos[row_j]) = -(the pair's term).
* "idw" (the multi-level composition's inverse_distance_weighting,
  src/utils/geometry.py:40-53, which the reference differentiates with
  autograd): u_j = 1 / (d2^p + 1e-10), w = u / (sum u + 1e-12), exact
  derivatives in d2 and p.
* "given" (msdetrpc.py:133-300): d_w = attn * <dout, v>, d_attn = sum_j w_j
  <dout, v_j>, d_val[row] += attn * w * dout.

Pinning: tests/test_oracle.py checks every mode against torch.autograd of the
fp64 forward composition on well-separated points, where the eps terms above
change the result by less than 1e-7 relative; the den_j choices themselves
only matter within ~1e-6 of a neighbour and are restated from the reference
text (parity unpinned below that distance).
"""
from __future__ import annotations

import torch


def forward_weights(mode, d2, valid, power, weights=None):
    """Forward weights [.., K] of each mode (fp64), zero for invalid neighbours."""
    if mode == "given":
        return torch.where(valid, weights, torch.zeros_like(weights))
    if mode == "idw":
        u = torch.where(valid, 1.0 / (d2 ** power + 1e-10), torch.zeros_like(d2))
        return u / (u.sum(-1, keepdim=True) + 1e-12)
    p = power.clamp(min=1e-6) if torch.is_tensor(power) else max(float(power), 1e-6)
    dist = torch.sqrt(d2 + 1e-6) if mode == "sample_sq" else torch.sqrt(d2) + 1e-6
    lg = torch.where(valid, -p * dist, torch.full_like(dist, -float("inf")))
    e = torch.where(valid, torch.exp(lg - lg.max(-1, keepdim=True).values), torch.zeros_like(lg))
    return e / (e.sum(-1, keepdim=True) + 1e-8)


def forward(mode, loc, kv_pos, rows, power, attn=None, weights=None, values=None):
    """out [B,Q,H,C] (values given) or the weights [B,Q,H,S,K] (values None); fp64.
    loc [B,Q,H,S,D] sample locations, kv_pos [B,Nkv,D], rows [B,Q,H,S,K],
    values [B,Nkv,H,C]."""
    B, Q, H, S, K = rows.shape
    valid = rows >= 0
    r = rows.clamp(min=0)
    if mode != "given":
        kp = kv_pos[torch.arange(B)[:, None, None, None, None], r]            # [B,Q,H,S,K,D]
        d2 = ((loc.unsqueeze(-2) - kp) ** 2).sum(-1)
    else:
        d2 = None
    w = forward_weights(mode, d2, valid, power, weights)
    if values is None:
        return w
    a = attn if attn is not None else torch.ones(B, Q, H, S, dtype=w.dtype)
    hh = torch.arange(H)[None, None, :, None, None]
    v = values[torch.arange(B)[:, None, None, None, None], r, hh]              # [B,Q,H,S,K,C]
    return ((a.unsqueeze(-1) * w).unsqueeze(-1) * v).sum(dim=(3, 4))


def deform_backward(mode, dout, loc, kv_pos, rows, power, attn=None, weights=None, values=None, d_w_in=None):
    """The reference's gradients (fp64): dict of d_loc [B,Q,H,S,D], d_attn [B,Q,H,S],
    d_weights [B,Q,H,S,K], d_kv_pos [B,Nkv,D], d_values [B,Nkv,H,C], d_power."""
    B, Q, H, S, K = rows.shape
    valid = rows >= 0
    r = rows.clamp(min=0)
    bi = torch.arange(B)[:, None, None, None, None]
    out = {}
    a = attn if attn is not None else torch.ones(B, Q, H, S, dtype=torch.float64)
    if mode != "given":
        kp = kv_pos[bi, r]
        diff = loc.unsqueeze(-2) - kp                                          # [B,Q,H,S,K,D]
        d2 = (diff ** 2).sum(-1)
    w = forward_weights(mode, d2 if mode != "given" else None, valid, power, weights)
    if values is not None:
        hh = torch.arange(H)[None, None, :, None, None]
        v = values[bi, r, hh]                                                  # [B,Q,H,S,K,C]
        dot = (v * dout[:, :, :, None, None, :]).sum(-1)
        dot = torch.where(valid, dot, torch.zeros_like(dot))
        out["d_attn"] = (w * dot).sum(-1)
        g = a.unsqueeze(-1) * dot
        coef = (a.unsqueeze(-1) * w).unsqueeze(-1) * dout[:, :, :, None, None, :]
        dv = torch.zeros_like(values)
        idx = (bi * values.shape[1] + r).expand(B, Q, H, S, K)
        hix = torch.arange(H)[None, None, :, None, None].expand(B, Q, H, S, K)
        flat = dv.view(-1, values.shape[-1])
        lin = (idx * H + hix)[valid]
        flat.index_add_(0, lin, coef[valid])
        out["d_values"] = dv
    else:
        g = torch.where(valid, d_w_in, torch.zeros_like(d_w_in))
    if mode == "given":
        out["d_weights"] = torch.where(valid, g, torch.zeros_like(g))
        return out
    gw = (w * g).sum(-1, keepdim=True)
    if mode == "idw":
        u = torch.where(valid, 1.0 / (d2 ** power + 1e-10), torch.zeros_like(d2))
        su = u.sum(-1, keepdim=True) + 1e-12
        dldu = (g - gw) / su
        dudd2 = -power * d2 ** (power - 1) * u * u
        term = 2.0 * dldu * dudd2
        logd2 = torch.where(d2 > 0, torch.log(torch.where(d2 > 0, d2, torch.ones_like(d2))), torch.zeros_like(d2))
        dpow = torch.where(valid & (d2 > 0), dldu * (-logd2 * d2 ** power * u * u), torch.zeros_like(d2))
    else:
        p = max(float(power), 1e-6)
        dlg = w * (g - gw)
        if mode == "sample_sq":
            dist = torch.sqrt(d2 + 1e-6)
            den = dist + 1e-8
        else:
            dist = torch.sqrt(d2) + 1e-6
            den = dist if mode == "shepard" else torch.clamp(dist - 1e-6, min=1e-8)
        term = -p * dlg / den
        dpow = torch.where(valid, dlg * (-dist), torch.zeros_like(dlg))
    term = torch.where(valid, term, torch.zeros_like(term))
    pair = term.unsqueeze(-1) * diff                                           # [B,Q,H,S,K,D]
    out["d_loc"] = pair.sum(-2)
    dkv = torch.zeros_like(kv_pos)
    flatk = dkv.view(-1, kv_pos.shape[-1])
    flatk.index_add_(0, (bi * kv_pos.shape[1] + r).expand(B, Q, H, S, K)[valid], -pair[valid])
    out["d_kv_pos"] = dkv
    out["d_power"] = dpow.sum()
    return out

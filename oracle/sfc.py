"""The reference's space-filling-curve orderings, restated in torch.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: tests/ compare the
HIP keys and argsort (aff_sfc_*) with these functions evaluated by torch on
the same device, so the float semantics of the reference's own torch ops on
that device are what the kernels are held to.  The product package
``affmae_amd`` never imports this module.

* :func:`peano_keys` / :func:`hilbert_keys` follow calculate_peano_order /
  calculate_hilbert_order (src/utils/geometry.py:322-460) up to the
  ``final_order`` they sort: digit levels by repeated division of the canvas
  height, per-level orders from the flip / rotation tables, summed with
  powers of 9 / 4.
* :func:`scanline_keys` follows the non-anchor scanline branch
  (geometry.py:276-287).
* :func:`anchor_keys` follows the anchor branch (geometry.py:199-268) up to
  the key it sorts.

Pinning (tests/test_oracle.py): the Peano order visits every cell of a 3^L
grid (and of the wide 3 x 6, 9 x 18 grids) exactly once with every step to
a 4-neighbour; the Hilbert order does so up to 8 x 8 (the reference keeps
the orientation as a rotation mod 3, geometry.py:429-440, which takes 8
jumps on a 16 x 16 grid; restated as is); the 3 x 3 Peano and 2 x 2 / 4 x 4
Hilbert orders equal their textbook first steps; the scanline anchor key
ranks tokens as the product's independent CPU ordering does.
"""
from __future__ import annotations

import math

import torch


def _levels(pos, h, base):
    n_levels = math.ceil(math.log(h, base))
    assert n_levels >= 1, "h too short"
    digits, rem, last = [], pos, h
    for _ in range(n_levels):
        cur = last / base
        digits.append((rem / cur).floor())
        rem = rem % cur
        last = cur
    return n_levels, digits


def peano_keys(h, w, pos):
    """fp32 [b,n] Peano final_order of pos [b,n,2] on an h x w canvas (geometry.py:322-384)."""
    b, n, _ = pos.shape
    dev = pos.device
    L, digits = _levels(pos, h, 3)
    fw = None
    if h != w:
        fw = round(3 * (w / h))
        if fw == 3:
            fw = None
    order = torch.tensor([[2, 3, 8], [1, 4, 7], [0, 5, 6]], dtype=torch.float32, device=dev)
    flip = torch.tensor([[[1, 1], [1, -1], [1, 1]], [[-1, 1], [-1, -1], [-1, 1]], [[1, 1], [1, -1], [1, 1]]],
                        dtype=torch.float32, device=dev)
    if fw is not None:
        order_w = torch.cat([order, order.flip(dims=[0])], dim=1).repeat(1, math.ceil(fw / 6))[:, :fw]
        order_w = order_w + torch.arange(math.ceil(fw / 3), device=dev).repeat_interleave(3)[:fw] * 9
        flip_w = flip[:, :2].repeat(1, math.ceil(fw / 2), 1)[:, :fw]
    orders = []
    for i in range(L):
        sign = torch.ones_like(pos)
        for j in range(i):
            lv = digits[i - j - 1]
            if i - j - 1 == 0 and fw is not None:
                f = flip_w[lv[..., 1].long(), lv[..., 0].long()]
            else:
                f = flip[lv[..., 1].long(), lv[..., 0].long()]
            sign = f * sign
        q = torch.where(sign > 0, digits[i], 2 - digits[i])
        tab = order_w if (i == 0 and fw is not None) else order
        orders.append(tab[q[..., 1].long(), q[..., 0].long()])
    final = orders[-1]
    for i in range(L - 1):
        final = final + orders[i] * (9 ** (L - i - 1))
    return final


def hilbert_keys(h, w, pos):
    """fp32 [b,n] Hilbert final_order of pos on a square h x h canvas (geometry.py:387-460)."""
    assert h == w or round(2 * (w / h)) == 2, "the reference's Hilbert order covers square canvases"
    dev = pos.device
    L, digits = _levels(pos, h, 2)
    rot_tab = torch.tensor([[[-1, 1], [0, 0]], [[0, -1], [0, 1]], [[1, 0], [-1, 0]]], dtype=torch.float32,
                           device=dev)
    res_tab = torch.tensor([[0, 3, 1, 2], [2, 3, 1, 0], [2, 1, 3, 0], [0, 1, 3, 2]], dtype=torch.float32, device=dev)
    orders = []
    for i in range(L):
        rot = torch.zeros_like(pos[..., 0])
        for j in range(i):
            lv = digits[j]
            cur = rot_tab[(rot % 3).long(), lv[..., 1].long(), lv[..., 0].long()]
            rot = cur + rot
        rot = rot % 4
        idx = (digits[i][..., 0] + digits[i][..., 1] * 2).long()
        orders.append(res_tab[rot.long(), idx])
    final = orders[-1]
    for i in range(L - 1):
        final = final + orders[i] * (4 ** (L - i - 1))
    return final


def scanline_keys(h, w, pos):
    """[b,n] alternating-scanline index of each token (geometry.py:276-287)."""
    ys, xs = torch.meshgrid(torch.arange(h, device=pos.device), torch.arange(w, device=pos.device), indexing="ij")
    om = torch.where(ys % 2 == 1, (w - 1) - xs, xs) + ys * w
    pid = (pos[..., 0] + pos[..., 1] * w).long()
    return om.reshape(-1)[pid]


def anchor_keys(pos, m, h, w, sf_type=""):
    """fp32 [b,n] sort keys of the anchor branch (geometry.py:199-268)."""
    b, n, d = pos.shape
    dev = pos.device
    k = int(math.ceil(n / m))
    patch_len = (h * w / k) ** 0.5
    nph, npw = int(round(h / patch_len)), int(round(w / patch_len))
    plh, plw = h / nph, w / npw
    if sf_type in ("peano", "hilbert"):
        base = 3 if sf_type == "peano" else 2
        nph = max(base, int(base ** round(math.log(nph, base))))
        plh = h / nph
        npw = int(round(w / h * base) * (nph / base))
        plw = w / npw
    ys, xs = torch.meshgrid(torch.arange(nph, device=dev), torch.arange(npw, device=dev), indexing="ij")
    grid = torch.stack([xs, ys], dim=2).reshape(-1, 2)
    if sf_type == "peano":
        key = peano_keys(nph, npw, grid.unsqueeze(0))[0]
    elif sf_type == "hilbert":
        key = hilbert_keys(nph, npw, grid.unsqueeze(0))[0]
    else:
        key = torch.where(ys % 2 == 1, -xs + (w - 1), xs).reshape(-1) + ys.reshape(-1) * w
    order = key.sort()[1]
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel(), device=dev)
    plhw = torch.tensor([plw, plh], dtype=torch.float32, device=dev)
    c = grid[order] * plhw + plhw / 2 - 0.5
    prev = torch.cat([(c[0] - (c[1] - c[0])).unsqueeze(0), c[:-1]])
    nxt = torch.cat([c[1:], (c[-1] + (c[-1] - c[-2])).unsqueeze(0)])
    cell = (pos / plhw).floor()
    cell = (cell[..., 0] + cell[..., 1] * npw).long()
    r = rank[cell]
    ratio = (pos - prev[r]).pow(2).sum(-1) / ((pos - nxt[r]).pow(2).sum(-1) + 1e-5)
    return r * (ratio.max() + 1) + ratio

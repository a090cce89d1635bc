"""Inference precision helpers for the encoder and decoder modules."""
from __future__ import annotations

import torch
from torch import nn


def cast_matmul_weights(module: nn.Module, dtype=torch.bfloat16) -> nn.Module:
    """Store the weights and biases of every nn.Linear / nn.Conv2d under `module` in
    `dtype`, once, in place; normalisation layers, every other parameter and the
    layers a module lists in `fp32_submodules` (products it runs in fp32 under
    autocast too) keep their dtype.

    Under torch.autocast(dtype) a Linear or convolution casts its fp32 weight and
    bias to `dtype` (round to nearest even) on every call before the product; the
    stored copy holds exactly those values, so an autocast forward computes the
    same products without the per-call cast kernels.  For inference: the fp32
    master weights are gone from the module afterwards.
    """
    keep = set()
    for m in module.modules():
        for name in getattr(m, "fp32_submodules", ()):
            keep.add(id(getattr(m, name)))
    for m in module.modules():
        if isinstance(m, (nn.Linear, nn.Conv2d)) and id(m) not in keep:
            m.weight.data = m.weight.data.to(dtype)
            if m.bias is not None:
                m.bias.data = m.bias.data.to(dtype)
    for m in module.modules():
        for name in ("clear_weights_cache", "clear_pe_table_cache"):   # tables built from the old weights
            clear = getattr(m, name, None)
            if callable(clear):
                clear()
    return module

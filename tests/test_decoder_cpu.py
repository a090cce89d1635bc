"""CPU checks of the decoder's host-side pieces (no GPU): the sine position
embedding against its closed form (reference decoder.py:34-58), the module
tree / parameter names of the reference's decoder (state_dict compatibility,
decoder.py:73-276) and the construction rules of CrossAttentionPixelDecoder."""
import math

import numpy as np
import pytest
import torch

from affmae_amd.layers import CrossAttentionPixelDecoder, MSDecoderBlock, PositionEmbeddingSine, ShapeSpec


def test_position_embedding_closed_form():
    pe = PositionEmbeddingSine(num_pos_feats=4, temperature=10000, normalize=False)
    pos = torch.tensor([[[3.0, 5.0], [0.5, 7.25]]])
    out = pe(pos).numpy()[0]
    for n, (x, y) in enumerate(pos[0].tolist()):
        # frequencies 1, 1, 100, 100: sin of the even ones, then cos of the odd ones
        ex = [math.sin(x), math.sin(x / 100), math.cos(x), math.cos(x / 100)]
        ey = [math.sin(y), math.sin(y / 100), math.cos(y), math.cos(y / 100)]
        np.testing.assert_allclose(out[n], ex + ey, rtol=1e-6, atol=1e-6)


def test_position_embedding_normalize_uses_batch_max():
    pe = PositionEmbeddingSine(num_pos_feats=2, temperature=10000, normalize=True)
    pos = torch.tensor([[[1.0, 2.0]], [[4.0, 8.0]]])
    out = pe(pos)
    x = 4.0 / (4.0 + 1e-6) * 2 * math.pi          # the second image's x is the batch maximum
    assert abs(float(out[1, 0, 0]) - math.sin(x)) < 1e-5
    x0 = 1.0 / (4.0 + 1e-6) * 2 * math.pi
    assert abs(float(out[0, 0, 0]) - math.sin(x0)) < 1e-5
    with pytest.raises(ValueError):
        PositionEmbeddingSine(8, scale=1.0, normalize=False)


def test_block_parameter_names():
    names = {k for k, _ in MSDecoderBlock(d_model=32, n_heads=4, d_ffn=64).named_parameters()}
    attn = ["sampling_offsets.weight", "sampling_offsets.bias", "attention_weights.weight", "attention_weights.bias",
            "value_proj.weight", "value_proj.bias", "output_proj.weight", "output_proj.bias", "shepard_power"]
    want = {f"{m}.{a}" for m in ("self_attn", "cross_attn") for a in attn}
    want |= {f"norm{i}.{p}" for i in (1, 2, 3) for p in ("weight", "bias")}
    want |= {f"linear{i}.{p}" for i in (1, 2) for p in ("weight", "bias")}
    assert names == want


def test_pixel_decoder_levels_and_projections():
    shapes = {"res2": ShapeSpec(64, 4), "res3": ShapeSpec(128, 8), "res4": ShapeSpec(256, 16),
              "res5": ShapeSpec(512, 32)}
    dec = CrossAttentionPixelDecoder(shapes, transformer_dropout=0.0, transformer_nheads=8,
                                     transformer_dim_feedforward=64, transformer_dec_layers=3, conv_dim=64,
                                     mask_dim=64, transformer_in_features=["res5", "res3", "res4"], common_stride=4,
                                     shepard_power=1.5, shepard_power_learnable=True)
    assert dec.in_features == ["res2", "res3", "res4", "res5"]
    assert dec.transformer_in_features == ["res3", "res4", "res5"]
    # projections run coarsest first: res5 (512), res4 (256), res3 (128)
    assert [p[0].in_features for p in dec.input_proj] == [512, 256, 128]
    assert all(float(p[0].bias.abs().max()) == 0.0 for p in dec.input_proj)
    assert len(dec.decoder_blocks) == 3 and all(len(s) == 3 for s in dec.decoder_blocks)
    assert dec.pe_layer.num_pos_feats == 32 and dec.pe_layer.normalize

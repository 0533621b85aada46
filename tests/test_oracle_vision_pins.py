"""Pins of the vision-tower oracle (oracle/vision.py) against independent
computations: transformers' own Qwen3-VL vision modules and geometry helpers
(the modules the reference's NativeNormVision.core calls), the PIL image
processor of Qwen2-VL (the processor whose pixel values the reference checks
its packing against), torch's LayerNorm, and fp64 closed forms. CPU only.
"""
import warnings

import numpy as np
import pytest
import torch

from oracle import vision as OV
from tests.helpers import bf16_ulps

BF16 = torch.bfloat16


def _hf_tower(seed=0, depth=3, hidden=64, heads=4, inter=96, out=48, deep=(0, 2), pos_side=6):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel
    torch.manual_seed(seed)
    cfg = Qwen3VLVisionConfig(depth=depth, hidden_size=hidden, hidden_act="gelu_pytorch_tanh", intermediate_size=inter,
                              num_heads=heads, in_channels=3, patch_size=16, spatial_merge_size=2,
                              temporal_patch_size=2, out_hidden_size=out, num_position_embeddings=pos_side ** 2,
                              deepstack_visual_indexes=list(deep))
    cfg._attn_implementation = "sdpa"
    m = Qwen3VLVisionModel(cfg).eval()
    for p in m.parameters():
        torch.nn.init.normal_(p, 0, 0.1)
        p.data = p.data.to(BF16)   # parameters in bf16; the rotary inv_freq buffer stays fp32
    shape = OV.VisionShape(depth=depth, hidden=hidden, heads=heads, inter=inter, out_hidden=out, deepstack=tuple(deep),
                           pos_side=pos_side)
    return m, shape


@pytest.mark.parametrize("gh,gw", [(4, 8), (6, 6), (2, 4)])
def test_vision_geometry_matches_hf(gh, gw):
    from transformers.vision_utils import get_vision_interpolation_indices_and_weights
    m, shape = _hf_tower()
    grid = torch.tensor([[1, gh, gw]])
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        assert torch.equal(m.rot_pos_emb(grid).float(), OV.rot_pos_freqs(shape, gh, gw))
        pe = m.fast_pos_embed_interpolate(grid).to(BF16)
    idx, wt = get_vision_interpolation_indices_and_weights(grid, shape.pos_side, mode="bilinear", align_corners=True,
                                                           spatial_merge_size=2)
    oi, ow = OV.pos_interp(shape, gh, gw)
    assert torch.equal(idx, oi) and torch.equal(wt, ow)
    assert torch.equal(pe, OV.pos_embeds(shape, m.pos_embed.weight.detach(), gh, gw))


def test_product_geometry_equals_oracle():
    """The product's host-side geometry tables (fastforward_amd.vision) equal the
    oracle's, which equal transformers' (test above)."""
    from fastforward_amd.vision import VisionConfig, interp_taps, rope_tables
    cfg = VisionConfig("t", 1, 1152, 16, 4304, 4096, (), pos_side=48)
    shape = OV.VisionShape(depth=1, hidden=1152, heads=16, inter=4304, out_hidden=4096, deepstack=(), pos_side=48)
    for gh, gw in ((16, 32), (32, 64), (30, 32)):
        c, s = rope_tables(cfg, gh, gw)
        oc, os_ = OV.rope_cos_sin(shape, gh, gw)
        assert torch.equal(c, oc) and torch.equal(s, os_)
        i, w = interp_taps(cfg, gh, gw)
        oi, ow = OV.pos_interp(shape, gh, gw)
        assert torch.equal(i, oi) and torch.equal(w, ow)


def test_pack_pixels_matches_hf_image_processor():
    from transformers.models.qwen2_vl.image_processing_pil_qwen2_vl import Qwen2VLImageProcessorPil
    proc = Qwen2VLImageProcessorPil(do_resize=False, patch_size=16, temporal_patch_size=2, merge_size=2,
                                    image_mean=[0.5, 0.5, 0.5], image_std=[0.5, 0.5, 0.5])
    rng = np.random.default_rng(0)
    for h, w in ((64, 96), (32, 32), (96, 64)):
        rgb = rng.integers(0, 256, size=(h, w, 3), dtype=np.uint8)
        out = proc(images=[rgb], return_tensors="pt")
        assert out["image_grid_thw"].tolist() == [[1, h // 16, w // 16]]
        assert torch.equal(out["pixel_values"].to(BF16), OV.pack_pixels(rgb))


def test_pixel_values_do_not_depend_on_the_division_rounding():
    """(u - 127.5) / 127.5 for all 256 codes: the bf16 result is the same for the
    correctly rounded fp32 quotient and for its fp32 neighbours, so any fp32
    division within one ulp (the Triton kernel's, the processor's, the HIP
    kernel's) packs the same bits."""
    u = np.arange(256, dtype=np.float32)
    q = (u - np.float32(127.5)) / np.float32(127.5)
    for d in (-1, 1):
        nb = np.nextafter(q, q + d * np.float32(1.0)).astype(np.float32)
        assert torch.equal(torch.from_numpy(q).to(BF16), torch.from_numpy(nb).to(BF16))


def test_vision_rope_matches_hf():
    from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb_vision
    shape = OV.VisionShape(depth=1, hidden=1152, heads=16, inter=4304, out_hidden=4096, deepstack=())
    cos, sin = OV.rope_cos_sin(shape, 8, 12)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(96, 16, 72, generator=g).to(BF16)
    k = torch.randn(96, 16, 72, generator=g).to(BF16)
    hq, hk = apply_rotary_pos_emb_vision(q, k, cos, sin)
    oq, ok = OV.vision_rope(q, k, cos, sin)
    assert torch.equal(hq, oq) and torch.equal(hk, ok)


def test_layer_norm_matches_torch_and_fp64():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(64, 1152, generator=g) * 2 + 0.3).to(BF16)
    w = (1 + 0.1 * torch.randn(1152, generator=g)).to(BF16)
    b = (0.1 * torch.randn(1152, generator=g)).to(BF16)
    got = OV.layer_norm(x, w, b, 1e-6)
    ref = torch.nn.functional.layer_norm(x, (1152,), w, b, 1e-6)
    assert int(bf16_ulps(got, ref).max()) <= 1
    xd = x.double()
    mean = xd.mean(-1, keepdim=True)
    exact = (xd - mean) / torch.sqrt(((xd - mean) ** 2).mean(-1, keepdim=True) + 1e-6) * w.double() + b.double()
    assert int(bf16_ulps(got, exact.to(BF16)).max()) <= 1


def test_gelu_forms_match_closed_forms():
    x = torch.linspace(-8, 8, 4001).to(BF16)
    xd = x.double()
    tanh_form = 0.5 * xd * (1 + torch.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    erf_form = 0.5 * xd * (1 + torch.erf(xd / np.sqrt(2)))
    # within one bf16 ulp of the fp64 form, plus the fp32 cancellation of
    # 1 + tanh / 1 + erf for negative x (a few fp32 ulps of 1, times x / 2)
    for got, want in ((OV.gelu_tanh(x), tanh_form), (OV.gelu_erf(x), erf_form)):
        d = (got.double() - want).abs()
        assert bool((d <= want.abs() * 2.0 ** -8 + xd.abs() * 2.0 ** -21).all())


def test_attention_matches_bruteforce():
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(9, 2, 8, generator=g).to(BF16) for _ in range(3))
    got = OV.attention(q, k, v, 8 ** -0.5).float()
    qd, kd, vd = q.double(), k.double(), v.double()
    out = torch.zeros(9, 2, 8, dtype=torch.float64)
    for h in range(2):
        for i in range(9):
            s = [float((qd[i, h] * kd[j, h]).sum()) * 8 ** -0.5 for j in range(9)]
            mx = max(s)
            e = [np.exp(x - mx) for x in s]
            out[i, h] = sum(e[j] * vd[j, h] for j in range(9)) / sum(e)
    assert torch.equal(got.reshape(9, 2, 8), out.to(torch.float32).to(BF16).float())


def test_vision_oracle_matches_hf_tower():
    """The whole tower (patch embed, 3 blocks, 2 DeepStack mergers, merger) against
    transformers' Qwen3VLVisionModel in bf16 on the CPU: same module sequence,
    different matmul accumulation (fp64 here), so within bf16 noise."""
    m, shape = _hf_tower()
    gh, gw = 4, 8
    pix = torch.randn(gh * gw, 1536, generator=torch.Generator().manual_seed(4)).to(BF16)
    with torch.no_grad():
        out = m(pix, grid_thw=torch.tensor([[1, gh, gw]]))
    merged, deep = OV.tower(shape, OV.from_hf(m), pix, gh, gw)
    def rel(a, b):
        return float((a.float() - b.float()).norm() / b.float().norm())
    assert rel(merged, out.pooler_output) <= 1e-2
    assert len(deep) == len(out.deepstack_features) == 2
    for a, b in zip(deep, out.deepstack_features):
        assert rel(a, b) <= 1e-2

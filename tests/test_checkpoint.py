"""Checkpoint loading (fastforward_amd.checkpoint) against transformers'
own Qwen3-VL model: a tiny random-init Qwen3VLForConditionalGeneration is
saved with save_pretrained (safetensors) and read back.

CPU: the config mapping and tensor access. GPU: the loaded FP8 linears equal
the quantisation of the concatenated HF weights bit for bit, the vision
weights equal HF's (MLP zero-padded), and the image + prompt step on the
loaded weights agrees with transformers' bf16 forward of the same model on
the same pixels and token ids (relative L2 of the option logits <= 0.15: the
LM linears are FP8 here, bf16 there).
"""
import numpy as np
import pytest
import torch

DEV = "cuda"
IMAGE_ID = 999


def _tiny_hf(tmp_path, seed=0, save=True, layers=2):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLForConditionalGeneration
    torch.manual_seed(seed)
    cfg = Qwen3VLConfig(
        text_config=dict(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=128, rms_norm_eps=1e-6,
                         rope_parameters={"rope_type": "default", "rope_theta": 5e6, "mrope_section": [24, 20, 20],
                                          "mrope_interleaved": True}),
        vision_config=dict(depth=2, hidden_size=576, intermediate_size=200, num_heads=8, out_hidden_size=512,
                           num_position_embeddings=36, deepstack_visual_indexes=[0, 1]),
        image_token_id=IMAGE_ID, vision_start_token_id=998, video_token_id=997, tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    m = Qwen3VLForConditionalGeneration(cfg).eval()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name and name.endswith("weight"):
                p.copy_(1 + 0.1 * torch.randn_like(p))
            elif "norm" in name and name.endswith("bias"):
                p.copy_(0.1 * torch.randn_like(p))
            p.data = p.data.to(torch.bfloat16)     # parameters bf16, rotary buffers fp32
    path = tmp_path / "tiny-qwen3vl"
    if save:
        m.save_pretrained(path)
    return m, str(path)


def test_read_config_and_tensors(tmp_path):
    from fastforward_amd.checkpoint import Tensors, read_config
    m, path = _tiny_hf(tmp_path)
    lm, vis, meta = read_config(path)
    assert (lm.layers, lm.hidden, lm.heads, lm.kv_heads, lm.head_dim, lm.inter, lm.vocab) == (2, 512, 4, 2, 128, 1024,
                                                                                              1000)
    assert lm.theta == 5e6 and lm.sections == (24, 20, 20) and not lm.tie_embed
    assert (vis.depth, vis.hidden, vis.heads, vis.inter, vis.out_hidden, vis.deepstack, vis.pos_side) == \
        (2, 576, 8, 200, 512, (0, 1), 6)
    assert meta["image_token_id"] == IMAGE_ID
    ts = Tensors(path)
    w = ts.get("model.language_model.layers.1.mlp.down_proj.weight", "cpu")
    assert torch.equal(w, m.model.language_model.layers[1].mlp.down_proj.weight.detach())


@pytest.mark.gpu
def test_loaded_weights_equal_hf(gpu, tmp_path):
    from fastforward_amd.checkpoint import load_pretrained
    from fastforward_amd.linear import FP8Linear
    m, path = _tiny_hf(tmp_path, seed=1)
    lm, lw, vis, vw, meta = load_pretrained(path, option_ids=list(range(10, 18)))
    L = m.model.language_model.layers[1]
    qkv = torch.cat([L.self_attn.q_proj.weight, L.self_attn.k_proj.weight, L.self_attn.v_proj.weight]).detach()
    ref = FP8Linear(qkv.to(DEV))
    assert torch.equal(lw.layers[1].qkv.weight.view(torch.uint8), ref.weight.view(torch.uint8))
    assert torch.equal(lw.layers[1].qkv.scale, ref.scale)
    gu = torch.cat([L.mlp.gate_proj.weight, L.mlp.up_proj.weight]).detach()
    assert torch.equal(lw.layers[1].gateup.weight.view(torch.uint8), FP8Linear(gu.to(DEV)).weight.view(torch.uint8))
    assert torch.equal(lw.head.cpu(), m.lm_head.weight.detach()[10:18])
    vb = m.model.visual.blocks[0]
    assert torch.equal(vw.blocks[0].fc1.w[:200].cpu(), vb.mlp.linear_fc1.weight.detach())
    assert not bool(vw.blocks[0].fc1.w[200:].float().abs().sum())
    assert torch.equal(vw.patch.w.cpu(), m.model.visual.patch_embed.proj.weight.detach().reshape(576, -1))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["int4_half", "int4_ffn"])
def test_loaded_mixed_banks(gpu, tmp_path, mode):
    """A 10-layer checkpoint loaded in a mixed execution mode: the interior
    linears that the mode takes from the int4 bank hold the reference's
    asymmetric group-32 codes and (scale, zero) table of the HF weight (the
    oracle's int4_quantize_asym, bit for bit), the others the static-FP8 codes
    and per-tensor scale."""
    from oracle import ops as O
    from fastforward_amd.checkpoint import load_pretrained
    from fastforward_amd.linear import Int4, StaticFP8Linear, bank_of
    m, path = _tiny_hf(tmp_path, seed=3, layers=10)
    lm, lw, _, _, _ = load_pretrained(path, option_ids=list(range(10, 18)), mode=mode, fp8_bank="fp8_static")
    hl = m.model.language_model.layers
    for j in (2, 3, 4, 5, 6):
        a, mlp = hl[j].self_attn, hl[j].mlp
        full = {"qkv": torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]), "o": a.o_proj.weight,
                "gateup": torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight]), "down": mlp.down_proj.weight}
        for role, wt in full.items():
            op = getattr(lw.layers[j], role)
            wt = wt.detach()
            if bank_of(mode, j, lm.layers, role) == "int4":
                assert isinstance(op, Int4) and op.group == 32 and not op.symmetric
                _, packed, scales = O.int4_quantize_asym(wt.float(), 32)
                assert torch.equal(op.packed.cpu(), packed) and torch.equal(op.scales.cpu(), scales), (j, role)
            else:
                assert isinstance(op, StaticFP8Linear)
                q, sc = O.fp8_weight_quant(wt, per_channel=False)
                assert torch.equal(op.weight.cpu().view(torch.uint8), q.view(torch.uint8)), (j, role)
                assert torch.equal(op.weight_scale.cpu(), sc), (j, role)


@pytest.mark.gpu
def test_loaded_int4_operator_check(gpu, tmp_path):
    """Loaded in the int4 mode, the middle layer's QKV (and only it) keeps the
    fp32 dequantised weight, as pack_release builds it; the step's first call
    runs the operator check on the loaded weights and passes."""
    from fastforward_amd.checkpoint import load_pretrained
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_request
    m, path = _tiny_hf(tmp_path, seed=4, layers=4)
    lm, lw, _, _, _ = load_pretrained(path, option_ids=list(range(10, 18)), mode="int4")
    mid = lm.layers // 2
    assert lw.layers[mid].qkv.oracle is not None
    assert all(getattr(L, r).oracle is None for j, L in enumerate(lw.layers) for r in ("qkv", "o", "gateup", "down")
               if (j, r) != (mid, "qkv"))
    rt = Runtime(lm, lw, 64)
    rt.set_inputs(*make_request(lm, 64, 2, 2, seed=1))
    rt.step()
    torch.cuda.synchronize()
    chk = lw.layers[mid].qkv.operator_check
    assert chk is not None and chk["passed"] and chk["relative_rms"] <= 0.01, chk


@pytest.mark.gpu
def test_image_step_on_loaded_weights_matches_transformers(gpu, tmp_path):
    from fastforward_amd.checkpoint import load_pretrained
    from fastforward_amd.pipeline import ImageStep
    from fastforward_amd.runtime import mrope_positions
    from oracle import vision as OV
    m, path = _tiny_hf(tmp_path, seed=2)
    options = list(range(10, 18))
    lm, lw, vis, vw, meta = load_pretrained(path, option_ids=options)
    gh, gw, start, tail = 8, 12, 5, 20
    nm = gh * gw // 4
    g = torch.Generator().manual_seed(3)
    ids = torch.cat([torch.randint(0, 990, (start,), generator=g), torch.full((nm,), IMAGE_ID),
                     torch.randint(0, 990, (tail,), generator=g)])
    n = ids.numel()
    rgb = np.random.default_rng(4).integers(0, 256, size=(16 * gh, 16 * gw, 3), dtype=np.uint8)
    pix = OV.pack_pixels(rgb)
    grid = torch.tensor([[1, gh, gw]])
    with torch.no_grad():
        out = m(input_ids=ids[None], pixel_values=pix.float(), image_grid_thw=grid,
                mm_token_type_ids=(ids[None] == IMAGE_ID).int())
    want = out.logits[0, -1, options].float()
    tokens = 64
    st = ImageStep(lm, lw, vis, vw, gh, gw, tokens, start)
    st.set_inputs(torch.from_numpy(rgb), ids, mrope_positions(start, gh // 2, gw // 2, tokens), n - 1)
    got = st.step().clone().cpu()
    torch.cuda.synchronize()
    rel = float((got - want).norm() / want.norm())
    print(f"loaded checkpoint, image step vs transformers bf16: rel L2 {rel:.4f}", flush=True)
    print("ours", got.tolist(), "\nhf  ", want.tolist(), flush=True)
    assert rel <= 0.15

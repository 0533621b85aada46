"""Load a Qwen3-VL checkpoint (transformers layout, safetensors) into the
step's formats.

Restates the setup half of the reference's runtime: the model comes from
``Qwen3VLForConditionalGeneration.from_pretrained(...)`` (scaled_qwen_runtime.py:62-69)
and ``pack_release`` (_family/depth_runtime.py:99-117) turns each decoder layer
into four FP8 linears -- q/k/v and gate/up concatenated row-wise -- and
releases the bf16 copies. Here the tensors are read one at a time from the
safetensors files (one file or an index of shards), moved to the GPU in bf16
and quantised there by the linear ops (``FP8Linear`` / ``RuntimeScaleLinear``
/ ``Int4``); no bf16 copy of a linear outlives its quantisation. The vision
tower keeps bf16 weights (its MLP intermediate zero-padded to a multiple of
64). The choice head is the rows of ``lm_head`` (or of the tied embedding)
at the option token ids, as the reference slices it
(scaled_qwen_runtime.py:70-72).
"""
import json
import os

import torch

from .linear import MIXED_MODES, FP8Linear, Int4, RuntimeScaleLinear, bank_of
from .ops import RMSNorm
from .runtime import LayerWeights, LMConfig, ModelWeights
from .vision import Lin, Norm, VBlock, VisionConfig, VisionWeights, VMerger, pad_mlp

BF16 = torch.bfloat16


class Tensors:
    """Lazy name -> tensor access over model.safetensors or a sharded index."""

    def __init__(self, path):
        from safetensors import safe_open
        self._open = safe_open
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                wmap = json.load(f)["weight_map"]
            self.where = {k: os.path.join(path, v) for k, v in wmap.items()}
        else:
            single = os.path.join(path, "model.safetensors")
            if not os.path.exists(single):
                raise FileNotFoundError(f"no model.safetensors or index in {path}")
            with safe_open(single, "pt") as f:
                self.where = {k: single for k in f.keys()}
        self._files = {}

    def __contains__(self, name):
        return name in self.where

    def get(self, name, device="cuda"):
        if name not in self.where:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        fn = self.where[name]
        if fn not in self._files:
            self._files[fn] = self._open(fn, "pt")
        return self._files[fn].get_tensor(name).to(device=device, dtype=BF16).contiguous()


def read_config(path):
    """(LMConfig, VisionConfig, meta) from the checkpoint's config.json; meta holds
    the image / vision-start token ids and whether the embedding is tied."""
    with open(os.path.join(path, "config.json")) as f:
        c = json.load(f)
    t, v = c["text_config"], c["vision_config"]
    rope = t.get("rope_parameters") or t.get("rope_scaling") or {}
    theta = rope.get("rope_theta", t.get("rope_theta", 5e6))
    sections = tuple(rope.get("mrope_section", (24, 20, 20)))
    tie = bool(c.get("tie_word_embeddings", t.get("tie_word_embeddings", False)))
    name = os.path.basename(os.path.normpath(path))
    lm = LMConfig(name, t["num_hidden_layers"], t["hidden_size"], t["num_attention_heads"],
                  t["num_key_value_heads"], t.get("head_dim", t["hidden_size"] // t["num_attention_heads"]),
                  t["intermediate_size"], t["vocab_size"], eps=t.get("rms_norm_eps", 1e-6), theta=float(theta),
                  sections=sections, tie_embed=tie)
    side = int(round(v.get("num_position_embeddings", 2304) ** 0.5))
    vis = VisionConfig(name, v["depth"], v["hidden_size"], v["num_heads"], v["intermediate_size"],
                       v["out_hidden_size"], tuple(v.get("deepstack_visual_indexes", ())), pos_side=side,
                       merge=v.get("spatial_merge_size", 2))
    if v.get("patch_size", 16) != 16 or v.get("temporal_patch_size", 2) != 2 or v.get("in_channels", 3) != 3:
        raise ValueError("only 16 x 16 patches, 2 frames, 3 channels are supported")
    meta = dict(image_token_id=c.get("image_token_id"), vision_start_token_id=c.get("vision_start_token_id"),
                tie_word_embeddings=tie)
    return lm, vis, meta


def option_ids_from_tokenizer(path, n=8):
    """First token id of ' A' ... for the n options, from the checkpoint's
    tokenizer.json (the reference's option_token_ids)."""
    from tokenizers import Tokenizer
    tok = Tokenizer.from_file(os.path.join(path, "tokenizer.json"))
    return [tok.encode(" " + chr(ord("A") + i), add_special_tokens=False).ids[0] for i in range(n)]


def _linear(w, mode, static_bound, oracle=False):
    """One linear of the ``mode`` bank; ``oracle`` (int4 banks) keeps the fp32
    dequantised weight for the first-call operator check (``Int4``)."""
    if mode == "fp8":
        return FP8Linear(w)
    if mode == "fp8_static":
        return RuntimeScaleLinear(w, 448.0 / static_bound)
    if mode == "w4a16":
        return Int4(w, oracle=oracle)
    if mode == "int4":      # the reference's asymmetric group-32 quantizer
        return Int4(w, group=32, symmetric=False, oracle=oracle)
    raise ValueError(f"unknown linear mode {mode!r}")


def load_lm(path, cfg, option_ids, mode="fp8", device="cuda", static_bound=8.0, tensors=None, fp8_bank="fp8"):
    """ModelWeights of the language model, one decoder layer at a time.
    ``mode`` "int4_half" / "int4_ffn" mixes the int4 bank (the reference's
    asymmetric group-32 Int4) into the interior layers (``bank_of``) and
    takes the other linears in the ``fp8_bank`` format ("fp8" or
    "fp8_static")."""
    ts = tensors or Tensors(path)
    p = "model.language_model."
    embed = ts.get(p + "embed_tokens.weight", device)
    layers = []

    def lin(w, j, role):
        # the middle layer's int4 QKV carries the operator check, as pack_release
        # builds it (_family/night_runtime.py:77)
        oracle = j == cfg.layers // 2 and role == "qkv"
        if mode in MIXED_MODES:
            bank = "int4" if bank_of(mode, j, cfg.layers, role) == "int4" else fp8_bank
            return _linear(w, bank, static_bound, oracle)
        return _linear(w, mode, static_bound, oracle)
    for j in range(cfg.layers):
        q = f"{p}layers.{j}."
        ops = {}
        w = torch.cat([ts.get(q + f"self_attn.{x}_proj.weight", device) for x in "qkv"])
        ops["qkv"] = lin(w, j, "qkv")
        del w
        ops["o"] = lin(ts.get(q + "self_attn.o_proj.weight", device), j, "o")
        w = torch.cat([ts.get(q + f"mlp.{x}_proj.weight", device) for x in ("gate", "up")])
        ops["gateup"] = lin(w, j, "gateup")
        del w
        ops["down"] = lin(ts.get(q + "mlp.down_proj.weight", device), j, "down")
        layers.append(LayerWeights(
            input_norm=RMSNorm(ts.get(q + "input_layernorm.weight", device), cfg.eps),
            post_norm=RMSNorm(ts.get(q + "post_attention_layernorm.weight", device), cfg.eps),
            q_norm=RMSNorm(ts.get(q + "self_attn.q_norm.weight", device), cfg.eps),
            k_norm=RMSNorm(ts.get(q + "self_attn.k_norm.weight", device), cfg.eps), **ops))
    ids = torch.tensor(list(option_ids), device=device)
    if cfg.tie_embed or "lm_head.weight" not in ts:
        head = embed.index_select(0, ids).contiguous()
    else:
        head = ts.get("lm_head.weight", device).index_select(0, ids).contiguous()
    return ModelWeights(embed=embed, layers=layers, norm=RMSNorm(ts.get(p + "norm.weight", device), cfg.eps),
                        head=head)


def load_vision(path, vcfg, device="cuda", tensors=None):
    """VisionWeights of the vision tower (bf16, MLP intermediate padded)."""
    ts = tensors or Tensors(path)
    p = "model.visual."
    g = lambda n: ts.get(p + n, device)  # noqa: E731
    blocks = []
    for j in range(vcfg.depth):
        b = f"blocks.{j}."
        w1, b1, w2 = pad_mlp(vcfg, g(b + "mlp.linear_fc1.weight"), g(b + "mlp.linear_fc1.bias"),
                             g(b + "mlp.linear_fc2.weight"))
        blocks.append(VBlock(Norm(g(b + "norm1.weight"), g(b + "norm1.bias")),
                             Lin(g(b + "attn.qkv.weight"), g(b + "attn.qkv.bias")),
                             Lin(g(b + "attn.proj.weight"), g(b + "attn.proj.bias")),
                             Norm(g(b + "norm2.weight"), g(b + "norm2.bias")), Lin(w1, b1),
                             Lin(w2, g(b + "mlp.linear_fc2.bias"))))
    def merger(pre, post):
        return VMerger(Norm(g(pre + "norm.weight"), g(pre + "norm.bias")),
                       Lin(g(pre + "linear_fc1.weight"), g(pre + "linear_fc1.bias")),
                       Lin(g(pre + "linear_fc2.weight"), g(pre + "linear_fc2.bias")), post)
    pw = g("patch_embed.proj.weight")
    return VisionWeights(Lin(pw.reshape(pw.shape[0], -1).contiguous(), g("patch_embed.proj.bias")),
                         g("pos_embed.weight"), blocks, merger("merger.", False),
                         [merger(f"deepstack_merger_list.{i}.", True) for i in range(len(vcfg.deepstack))])


def load_pretrained(path, option_ids=None, mode="fp8", device="cuda", n_options=8, fp8_bank="fp8"):
    """(lm_cfg, lm_weights, vis_cfg, vis_weights, meta) of a local Qwen3-VL
    checkpoint directory. ``option_ids`` default to the first tokens of
    ' A' ... from the checkpoint's tokenizer."""
    lm, vis, meta = read_config(path)
    if option_ids is None:
        option_ids = option_ids_from_tokenizer(path, n_options)
    ts = Tensors(path)
    lw = load_lm(path, lm, option_ids, mode=mode, device=device, tensors=ts, fp8_bank=fp8_bank)
    vw = load_vision(path, vis, device=device, tensors=ts)
    meta["option_ids"] = list(option_ids)
    return lm, lw, vis, vw, meta

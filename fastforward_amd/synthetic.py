"""Seeded synthetic models and requests of the Qwen3-VL LM shapes.

No checkpoint can be loaded here, so weights are random-init N(0, 0.02) bf16
(RMSNorm weights 1 unless ``norm_jitter`` is set) generated on the device from
per-tensor seeds -- any layer can be regenerated alone -- and quantized on the
GPU at setup, as ``pack_release`` does for real weights
(_family/depth_runtime.py:99-117). The Q/K/V and gate/up weights are
concatenated row-wise as the reference packs them.
"""
import torch

from .linear import MIXED_MODES, FP8Linear, Int4, RuntimeScaleLinear, bank_of
from .ops import RMSNorm
from .runtime import LayerWeights, ModelWeights, mrope_positions

BF16 = torch.bfloat16
ROLES = ("qkv", "o", "gateup", "down")
# Stand-ins for the tokenizer ids of " A" ... " H" (the option rows of lm_head).
OPTION_IDS = (362, 425, 356, 422, 468, 434, 479, 472)


def _seed(seed, *parts):
    s = seed * 1000003 + 7
    for p in parts:
        s = (s * 1000033 + p) % (2 ** 62)
    return s


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def linear_shapes(cfg):
    d = cfg.head_dim
    return {"qkv": (cfg.qkv_out, cfg.hidden), "o": (cfg.hidden, cfg.heads * d),
            "gateup": (2 * cfg.inter, cfg.hidden), "down": (cfg.hidden, cfg.inter)}


def linear_weight(cfg, layer, role, seed=0, device="cuda"):
    """The bf16 weight (N, K) of one linear, regenerated from its seed."""
    n, k = linear_shapes(cfg)[role]
    g = _gen(device, _seed(seed, layer, ROLES.index(role)))
    return (torch.randn((n, k), generator=g, device=device) * 0.02).to(BF16)


def _norm(n, jitter, device, seed):
    if not jitter:
        return torch.ones(n, device=device, dtype=BF16)
    g = _gen(device, seed)
    return (1 + jitter * torch.randn(n, generator=g, device=device)).to(BF16)


def make_model(cfg, mode="fp8", seed=0, device="cuda", n_options=8, norm_jitter=0.0,
               static_bound=8.0, int4_group=128, int4_symmetric=True, keep_bf16=None, fp8_bank="fp8_static"):
    """Build ModelWeights for ``cfg``.

    mode: "fp8" (FP8Linear: per-token / per-channel), "fp8_static"
    (RuntimeScaleLinear with activation bound ``static_bound``), "w4a16" (Int4,
    ``int4_group`` / ``int4_symmetric``), "int4" (Int4, asymmetric group 32),
    "int4_half" / "int4_ffn" (the reference's mixed execution modes: the
    asymmetric group-32 int4 bank in the interior layers by ``bank_of``, the
    ``fp8_bank`` format elsewhere).
    ``keep_bf16`` (a dict) receives the bf16 weights by (layer, role) on the CPU.
    """
    H, D = cfg.hidden, cfg.head_dim
    g = _gen(device, _seed(seed, 10 ** 6))
    embed = (torch.randn((cfg.vocab, H), generator=g, device=device) * 0.02).to(BF16)
    layers = []
    for j in range(cfg.layers):
        ops = {}
        for role in ROLES:
            w = linear_weight(cfg, j, role, seed, device)
            if keep_bf16 is not None:
                keep_bf16[(j, role)] = w.cpu()
            m = mode
            if mode in MIXED_MODES:
                m = "int4" if bank_of(mode, j, cfg.layers, role) == "int4" else fp8_bank
            if m == "fp8":
                ops[role] = FP8Linear(w)
            elif m == "fp8_static":
                ops[role] = RuntimeScaleLinear(w, 448.0 / static_bound)
            elif m == "w4a16":
                ops[role] = Int4(w, group=int4_group, symmetric=int4_symmetric)
            elif m == "int4":       # the reference's asymmetric group-32 quantizer
                ops[role] = Int4(w, group=32, symmetric=False)
            else:
                raise ValueError(mode)
            del w
        ns = lambda k: _seed(seed, j, 100 + k)  # noqa: E731
        layers.append(LayerWeights(
            input_norm=RMSNorm(_norm(H, norm_jitter, device, ns(0)), cfg.eps),
            post_norm=RMSNorm(_norm(H, norm_jitter, device, ns(1)), cfg.eps),
            q_norm=RMSNorm(_norm(D, norm_jitter, device, ns(2)), cfg.eps),
            k_norm=RMSNorm(_norm(D, norm_jitter, device, ns(3)), cfg.eps),
            **ops))
    norm = RMSNorm(_norm(H, norm_jitter, device, _seed(seed, 10 ** 6 + 1)), cfg.eps)
    ids = torch.tensor(OPTION_IDS[:n_options], device=device)
    if cfg.tie_embed:
        head = embed.index_select(0, ids).contiguous()
    else:
        gh = _gen(device, _seed(seed, 10 ** 6 + 2))
        head = (torch.randn((n_options, H), generator=gh, device=device) * 0.02).to(BF16)
    return ModelWeights(embed=embed, layers=layers, norm=norm, head=head)


def make_request(cfg, tokens, grid_h, grid_w, prefix_tokens=4, seed=0, real_tokens=None):
    """Seeded synthetic request: token ids uniform in the vocabulary, M-RoPE
    positions for one image of merged grid (grid_h, grid_w) after
    ``prefix_tokens`` text tokens, and the picked (last real) row.
    Returns (ids (n,), pos (3, tokens), pick)."""
    n = tokens if real_tokens is None else real_tokens
    g = torch.Generator().manual_seed(_seed(seed, 42))
    ids = torch.randint(0, cfg.vocab, (n,), generator=g, dtype=torch.int64)
    pos = torch.from_numpy(mrope_positions(prefix_tokens, grid_h, grid_w, tokens))
    return ids, pos, n - 1

"""Whole-step parity of the gfx950 LM step against the CPU oracle.

Bar (stated in the task): final choice logits within 1e-2 relative
(max_c |dz_c| <= 1e-2 * max_c |z_c|) with the identical argmax (ties -> lowest
index). Internal consistency is bit-exact: the fused FP8 path equals the
reference op sequence (generic path), every hipGraph replay equals the eager
step, and padding tokens after the picked row cannot change the logits.
"""
import os
import sys

import pytest
import torch

from oracle import model as omodel
from oracle import ops as O
from tests.helpers import rel_err, to_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"

torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))


def _tiny(layers=3):
    from fastforward_amd.runtime import LMConfig
    return LMConfig("tiny", layers, 512, 4, 2, 128, 1024, 1000)


def _run(cfg, w, tokens, ids, pos, pick, path=None, **kw):
    from fastforward_amd.runtime import Runtime
    rt = Runtime(cfg, w, tokens, path=path, **kw)
    rt.set_inputs(ids, pos, pick)
    z = rt.step().clone()
    torch.cuda.synchronize()
    return rt, z.cpu()


def _check_vs_oracle(z, want, what):
    print(f"{what}: gpu={z.tolist()} oracle={want.tolist()}", flush=True)
    assert rel_err(z, want) <= 1e-2, (what, rel_err(z, want))
    assert O.choose(z.tolist()) == O.choose(want.tolist()), what


@pytest.mark.parametrize("mode", ["fp8", "fp8_static", "w4a16"])
def test_tiny_model_vs_oracle(gpu, mode):
    from fastforward_amd.synthetic import make_model, make_request
    cfg = _tiny()
    w = make_model(cfg, mode=mode, seed=1, norm_jitter=0.2, n_options=4)
    ids, pos, pick = make_request(cfg, 96, 4, 6, seed=1)
    _, z = _run(cfg, w, 96, ids, pos, pick)
    shape, ow = to_oracle(cfg, w)
    want = omodel.step(shape, ow, ids, pos, pick)
    _check_vs_oracle(z, want, f"tiny {mode}")


def test_fused_path_equals_reference_op_sequence(gpu):
    from fastforward_amd.synthetic import make_model, make_request
    cfg = _tiny(4)
    w = make_model(cfg, mode="fp8", seed=2, norm_jitter=0.2)
    ids, pos, pick = make_request(cfg, 130, 5, 5, seed=2)
    _, z1 = _run(cfg, w, 130, ids, pos, pick, path="fused")
    _, z2 = _run(cfg, w, 130, ids, pos, pick, path="generic")
    assert torch.equal(z1, z2), (z1, z2)


@pytest.mark.parametrize("path", ["fused", "generic"])
def test_graph_replays_equal_eager(gpu, path):
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_model, make_request
    cfg = _tiny()
    w = make_model(cfg, mode="fp8", seed=3, norm_jitter=0.2)
    rt = Runtime(cfg, w, 128, path=path)
    reqs = [make_request(cfg, 128, 4, 4, seed=s, real_tokens=n) for s, n in ((10, 128), (11, 100), (12, 77))]
    eager = []
    for ids, pos, pick in reqs:
        rt.set_inputs(ids, pos, pick)
        eager.append(rt.step().clone())
    rt.set_inputs(*reqs[0])
    rt.capture()
    for rep in range(2):
        for (ids, pos, pick), ze in zip(reqs, eager):
            rt.set_inputs(ids, pos, pick)
            z = rt.replay().clone()
            torch.cuda.synchronize()
            _ = torch.ones(1000, device=DEV).sum().item()       # eager work between replays
            assert torch.equal(z, ze), (rep, z, ze)


def test_padding_isolation(gpu):
    """Changing pad tokens after the picked row leaves the logits bit-identical
    (_legacy/sub10_runtime.py:166-167)."""
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_model, make_request
    cfg = _tiny()
    w = make_model(cfg, mode="fp8", seed=4, norm_jitter=0.2)
    ids, pos, pick = make_request(cfg, 128, 4, 4, seed=4, real_tokens=90)
    rt = Runtime(cfg, w, 128)
    rt.set_inputs(ids, pos, pick)
    z0 = rt.step().clone()
    full = torch.cat([ids, torch.randint(0, cfg.vocab, (38,))])
    rt.set_inputs(full, pos, pick)
    z1 = rt.step().clone()
    assert torch.equal(z0, z1)


def test_visual_rows_and_deepstack_vs_oracle(gpu):
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_model, make_request
    cfg = _tiny()
    w = make_model(cfg, mode="fp8", seed=5, norm_jitter=0.2)
    ids, pos, pick = make_request(cfg, 96, 4, 6, seed=5)
    g = torch.Generator().manual_seed(5)
    visual = torch.randn(24, cfg.hidden, generator=g).to(torch.bfloat16)
    deep = [(torch.randn(24, cfg.hidden, generator=g) * 0.5).to(torch.bfloat16) for _ in range(2)]
    rt = Runtime(cfg, w, 96, visual_rows=24, image_start=4, deep_layers=2)
    rt.set_inputs(ids, pos, pick, visual=visual.to(DEV), deep=[d.to(DEV) for d in deep])
    z = rt.step().clone().cpu()
    shape, ow = to_oracle(cfg, w)
    want = omodel.step(shape, ow, ids, pos, pick, visual=visual, image_start=4, deep=deep)
    _check_vs_oracle(z, want, "visual+deepstack")
    rt2 = Runtime(cfg, w, 96, path="generic", visual_rows=24, image_start=4, deep_layers=2)
    rt2.set_inputs(ids, pos, pick, visual=visual.to(DEV), deep=[d.to(DEV) for d in deep])
    assert torch.equal(rt2.step().cpu(), z)


@pytest.mark.parametrize("preset,tokens,grid,choices,mode", [
    ("qwen3vl-2b", 320, (16, 16), 4, "fp8"),
    ("qwen3vl-8b", 576, (16, 32), 8, "fp8"),
    ("qwen3vl-8b", 576, (16, 32), 8, "w4a16"),
])
def test_full_model_vs_oracle(gpu, preset, tokens, grid, choices, mode):
    """The full-depth BASELINE shapes, hipGraph-replayed, against the oracle run on
    the same quantized weights (bf16 embeddings, random-init N(0, 0.02))."""
    from fastforward_amd.runtime import PRESETS, Runtime
    from fastforward_amd.synthetic import make_model, make_request
    cfg = PRESETS[preset]
    print(f"building {preset} {mode}", flush=True)
    w = make_model(cfg, mode=mode, seed=7, n_options=choices)
    ids, pos, pick = make_request(cfg, tokens, *grid, seed=7)
    rt = Runtime(cfg, w, tokens)
    rt.set_inputs(ids, pos, pick)
    z_eager = rt.step().clone()
    rt.capture()
    z = rt.replay().clone()
    torch.cuda.synchronize()
    assert torch.equal(z, z_eager)
    z = z.cpu()
    print("running the oracle", flush=True)
    shape, ow = to_oracle(cfg, w)
    del w, rt
    torch.cuda.empty_cache()
    want = omodel.step(shape, ow, ids, pos, pick)
    _check_vs_oracle(z, want, f"{preset} {mode}")
    sys.stdout.flush()

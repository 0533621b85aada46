"""Image + prompt step (vision tower -> LM step) on the GPU.

Bit-exact internal consistency: the fused pipeline (the vision step writing
into the LM runtime's visual / DeepStack buffers) equals the two steps run
separately with the vision outputs handed over, and hipGraph replays of the
whole pipeline equal its eager runs for different images. Each half is checked
against the oracle in test_gpu_vision.py and test_gpu_model.py.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(seed=0):
    from fastforward_amd.runtime import LMConfig, mrope_positions
    from fastforward_amd.synthetic import make_model
    from fastforward_amd.vision import VisionConfig, make_vision
    cfg = LMConfig("tiny", 3, 512, 4, 2, 128, 1024, 1000)
    vis = VisionConfig("small", 2, 576, 8, 200, 512, (0, 1), pos_side=6)
    w = make_model(cfg, mode="fp8", seed=seed, norm_jitter=0.2)
    vw = make_vision(vis, seed=seed, std=0.05)
    gh, gw, tokens, start = 8, 12, 96, 4
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, cfg.vocab, (tokens,), generator=g)
    pos = torch.from_numpy(mrope_positions(start, gh // 2, gw // 2, tokens))
    return cfg, vis, w, vw, gh, gw, tokens, start, ids, pos, tokens - 1


def test_image_step_equals_the_two_steps_composed(gpu):
    from fastforward_amd.pipeline import ImageStep
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.vision import VisionRuntime
    cfg, vis, w, vw, gh, gw, tokens, start, ids, pos, pick = _setup()
    rgb = torch.from_numpy(np.random.default_rng(1).integers(0, 256, size=(16 * gh, 16 * gw, 3), dtype=np.uint8))
    st = ImageStep(cfg, w, vis, vw, gh, gw, tokens, start)
    st.set_inputs(rgb, ids, pos, pick)
    z = st.step().clone()
    v = VisionRuntime(vis, vw, gh, gw)
    v.set_image(rgb)
    merged, deep = v.step()
    rt = Runtime(cfg, w, tokens, visual_rows=merged.shape[0], image_start=start, deep_layers=len(deep))
    rt.set_inputs(ids, pos, pick, visual=merged, deep=deep)
    z2 = rt.step().clone()
    torch.cuda.synchronize()
    assert torch.isfinite(z).all()
    assert torch.equal(z, z2)


def test_image_step_graph_replays_equal_eager(gpu):
    from fastforward_amd.pipeline import ImageStep
    cfg, vis, w, vw, gh, gw, tokens, start, ids, pos, pick = _setup(seed=2)
    st = ImageStep(cfg, w, vis, vw, gh, gw, tokens, start)
    rng = np.random.default_rng(3)
    images = [torch.from_numpy(rng.integers(0, 256, size=(16 * gh, 16 * gw, 3), dtype=np.uint8)) for _ in range(2)]
    eager = []
    for img in images:
        st.set_inputs(img, ids, pos, pick)
        eager.append(st.step().clone())
    assert not torch.equal(eager[0], eager[1])  # the image reaches the logits
    st.capture()
    for _ in range(2):
        for img, want in zip(images, eager):
            st.set_inputs(img, ids, pos, pick)
            torch.cuda.synchronize()
            got = st.replay().clone()
            torch.cuda.synchronize()
            assert torch.equal(got, want)

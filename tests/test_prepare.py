"""Host request preparation (fastforward_amd.prepare), CPU only.

Pinned by brute force over the candidate block grids (canvas), by the fit's
geometric invariants, by exact pixel placement (letterbox), and by the prompt
structure the readout relies on (the image placeholder once, in the prefix;
the suffix ends at 'Answer:'; options lettered in order).
"""
import math

import numpy as np
import pytest

from fastforward_amd import prepare as P


@pytest.mark.parametrize("variant", P.VARIANTS)
def test_canvas_brute_force(variant):
    rng = np.random.default_rng(0)
    side = 256 if variant.endswith("256") else 320
    blocks = side // 32
    for _ in range(300):
        h, w = (int(x) for x in rng.integers(1, 4000, size=2))
        ch, cw = P.canvas(h, w, variant)
        assert ch % 32 == 0 and cw % 32 == 0
        if variant.startswith("square"):
            assert (ch, cw) == (side, side)
            continue
        # every candidate grid: about the canvas side's area, both orientations
        cands = set()
        for a in range(1, 64):
            for b in range(1, 64):
                if (a, b) in P._PAIRS[side] or (b, a) in P._PAIRS[side]:
                    cands.add((a, b))
        assert all(a * b <= blocks * blocks * 1.05 for a, b in cands)
        d = lambda p: abs(math.log((p[0] / p[1]) / (h / w)))  # noqa: E731
        best = min(d(p) for p in cands)
        assert abs(d((ch // 32, cw // 32)) - best) < 1e-12
        tied = [p for p in cands if abs(d(p) - best) < 1e-12]
        assert (ch // 32) * (cw // 32) == max(a * b for a, b in tied)


def test_canvas_orientation_follows_the_image():
    assert P.canvas(100, 1000, "aspect256") == (64, 1024)      # wide -> 2 x 32 blocks
    assert P.canvas(1000, 100, "aspect256") == (1024, 64)
    assert P.canvas(500, 500, "aspect320") == (320, 320)
    with pytest.raises(ValueError):
        P.canvas(10, 10, "square512")


def test_fit_invariants():
    rng = np.random.default_rng(1)
    for _ in range(500):
        h, w = (int(x) for x in rng.integers(1, 3000, size=2))
        th, tw = (int(x) for x in rng.integers(1, 60, size=2) * 32)
        nh, nw, top, left = P.fit(h, w, (th, tw))
        assert 1 <= nh <= th and 1 <= nw <= tw
        assert nh == th or nw == tw                           # touches the canvas on one axis
        assert abs(nh / nw - h / w) <= (h / w) * (1.0 / min(nh, nw)) + 1e-9 or min(nh, nw) == 1
        assert top == (th - nh) // 2 and left == (tw - nw) // 2


def test_letterbox_places_pixels_exactly():
    img = np.arange(5 * 7 * 3, dtype=np.uint8).reshape(5, 7, 3)
    out = P.letterbox(img, (16, 12), 3, 2)
    assert out.shape == (16, 12, 3) and out.dtype == np.uint8
    assert np.array_equal(out[3:8, 2:9], img)
    mask = np.ones((16, 12), bool)
    mask[3:8, 2:9] = False
    assert (out[mask] == 128).all()
    with pytest.raises(ValueError):
        P.letterbox(img, (4, 4), 0, 0)


def test_prepare_image_uses_canvas_and_fit():
    calls = []
    def resize(img, size):
        calls.append(size)
        return np.zeros((*size, 3), np.uint8)
    out = P.prepare_image(np.zeros((300, 900, 3), np.uint8), "aspect256", resize)
    shape = P.canvas(300, 900, "aspect256")
    nh, nw, top, left = P.fit(300, 900, shape)
    assert out.shape == (*shape, 3) and calls == [(nh, nw)]
    out = P.prepare_image(np.zeros((300, 900, 3), np.uint8), "square320", resize)
    assert out.shape == (320, 320, 3) and calls[-1] == (320, 320)


@pytest.mark.parametrize("style", ["short", "minimal", "standard"])
def test_prompt_structure(style):
    row = dict(instruction="  Which one?  ", candidates=["cat", "dog", "bird"])
    prefix, suffix = P.text_parts(row, style)
    full = prefix + suffix
    assert full.count("<|image_pad|>") == 1 and prefix.endswith(P.IMAGE if style != "standard" else P.IMAGE)
    assert "<|image_pad|>" not in suffix
    assert suffix.endswith("<|im_start|>assistant\nAnswer:")
    assert "A. cat\nB. dog\nC. bird" in suffix
    assert "Which one?" in suffix and "  Which one?  " not in suffix
    assert ("Reply with one letter." in suffix) == (style == "short")
    if style == "standard":
        assert prefix.startswith("<|im_start|>system\n") and "Question: Which one?" in suffix
    else:
        assert prefix == "<|im_start|>user\n" + P.IMAGE


def test_option_strings():
    assert P.option_strings(3) == [" A", " B", " C"]
    with pytest.raises(ValueError):
        P.option_strings(27)

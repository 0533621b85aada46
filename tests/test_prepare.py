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


def _fine_area(img, nh, nw):
    """Area resampling by exact supersampling: every source pixel replicated
    onto a grid of lcm resolution, then each output's block averaged."""
    h, w = img.shape[:2]
    ly, lx = math.lcm(h, nh), math.lcm(w, nw)
    fine = np.repeat(np.repeat(img.astype(np.float64), ly // h, 0), lx // w, 1)
    return fine.reshape(nh, ly // nh, nw, lx // nw, 3).mean(axis=(1, 3))


def test_area_resize_identity_and_constant():
    rng = np.random.default_rng(1)
    img = rng.integers(0, 256, size=(13, 17, 3), dtype=np.uint8)
    assert np.array_equal(P.area_resize(img, (13, 17)), img)
    flat = np.full((40, 30, 3), 77, dtype=np.uint8)
    for size in [(7, 11), (40, 60), (90, 13)]:
        assert np.array_equal(P.area_resize(flat, size), np.full(size + (3,), 77, dtype=np.uint8))


@pytest.mark.parametrize("src,dst", [((64, 48), (16, 12)), ((21, 14), (7, 7)), ((37, 53), (10, 16)),
                                     ((60, 90), (25, 36))])
def test_area_resize_downscale_is_the_area_integral(src, dst):
    rng = np.random.default_rng(2)
    img = rng.integers(0, 256, size=src + (3,), dtype=np.uint8)
    got = P.area_resize(img, dst).astype(np.float64)
    want = _fine_area(img, *dst)
    assert np.abs(got - want).max() <= 0.5 + 1e-9        # the integral, rounded
    if src[0] % dst[0] == 0 and src[1] % dst[1] == 0:  # integer factors: block means
        fy, fx = src[0] // dst[0], src[1] // dst[1]
        block = img.astype(np.float64).reshape(dst[0], fy, dst[1], fx, 3).mean(axis=(1, 3))
        clear = np.abs(block - np.floor(block) - 0.5) > 1e-6    # ties may round either way
        assert np.array_equal(got[clear], np.rint(block)[clear])


def test_area_resize_integer_upscale_replicates():
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, size=(5, 7, 3), dtype=np.uint8)
    assert np.array_equal(P.area_resize(img, (15, 14)), np.repeat(np.repeat(img, 3, 0), 2, 1))
    up = P.area_resize(img, (12, 17)).astype(int)          # non-integer growth stays within source range
    assert up.min() >= img.min() and up.max() <= img.max()


def test_decode_image_roundtrip(tmp_path):
    from PIL import Image
    rng = np.random.default_rng(4)
    img = rng.integers(0, 256, size=(9, 23, 3), dtype=np.uint8)
    Image.fromarray(img).save(tmp_path / "x.png")
    assert np.array_equal(P.decode_image(tmp_path / "x.png"), img)
    Image.fromarray(img[..., 0]).convert("L").save(tmp_path / "g.png")   # gray -> RGB
    g = P.decode_image(tmp_path / "g.png")
    assert g.shape == (9, 23, 3) and np.array_equal(g[..., 1], img[..., 0])


@pytest.mark.parametrize("variant", P.VARIANTS)
def test_canvases_cover_every_canvas(variant):
    cs = set(P.canvases(variant))
    rng = np.random.default_rng(5)
    seen = set()
    for _ in range(3000):
        h, w = (int(x) for x in rng.integers(1, 5000, size=2))
        c = P.canvas(h, w, variant)
        assert c in cs
        seen.add(c)
    assert seen == cs      # and each listed canvas is reachable

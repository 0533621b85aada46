"""Image requests over a local checkpoint (fastforward_amd.family, the
qwen3_vl_family bundle of fastforward_amd.api, the CLI).

CPU: bundle checks, the identity repair-adapter check, the prompt prefix with
its image placeholder expanded per canvas, request preparation (canvas,
tokens, readout row, no truncation), CLI argument handling.

GPU: ``Accelerator.predict(image, question, candidates)`` on a tiny
random-init transformers Qwen3-VL checkpoint with an offline word-level
tokenizer agrees with transformers' own bf16 forward of the same model on the
same canvas pixels and token ids, its LM linears given the same per-token /
per-channel e4m3 rounding: relative L2 of the 8 option logits <= 0.08 (0.04
measured) and under a quarter of the two test images' own difference; a
second request on the captured graph reproduces a fresh eager step of the
same inputs bit for bit.
"""
import hashlib
import json

import numpy as np
import pytest
import torch

from tests.test_checkpoint import IMAGE_ID, _tiny_hf

SPECIALS = {"<|image_pad|>": IMAGE_ID, "<|vision_start|>": 998, "<|vision_end|>": 996, "<|im_start|>": 995,
            "<|im_end|>": 994}


def _tiny_tokenizer(path):
    """Word-level tokenizer.json with the Qwen chat / vision special tokens at
    the tiny config's ids; unknown words map to [UNK] (id 0)."""
    from tokenizers import AddedToken, Tokenizer, models, pre_tokenizers
    words = (["[UNK]"] + [chr(c) for c in range(65, 91)] + [chr(c) for c in range(97, 123)] + list(".,:?!") +
             "user assistant system Answer Options Reply with one letter of the What color is shown".split())
    vocab = {w: i for i, w in enumerate(dict.fromkeys(words))}
    vocab.update(SPECIALS)
    tok = Tokenizer(models.WordLevel(vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    tok.add_special_tokens([AddedToken(s, special=True, normalized=False) for s in SPECIALS])
    tok.save(str(path / "tokenizer.json"))
    return tok


def _repair(tmp_path, nonzero=False):
    p = tmp_path / "repair.pt"
    up = torch.zeros(4, 8)
    if nonzero:
        up[1, 2] = 1.0
    torch.save({"state_dict": {"up": up, "bias": torch.zeros(8), "down": torch.randn(8, 4)}}, p)
    return p, hashlib.sha256(p.read_bytes()).hexdigest()


def _bundle(tmp_path, model, **kw):
    c = dict(schema_version=1, task="visual_choice", architecture="qwen3_vl_family", model=str(model),
             buckets=[64, 96, 128, 192], variant="aspect256", prompt_style="short")
    c.update(kw)
    p = tmp_path / "bundle.json"
    p.write_text(json.dumps(c))
    return p


def test_family_bundle_checks(tmp_path):
    from fastforward_amd.api import check_identity_repair, read_bundle
    with pytest.raises(FileNotFoundError):
        read_bundle(_bundle(tmp_path, tmp_path / "absent"))
    for bad in ([], [0, 64], "64", None):
        with pytest.raises(ValueError):
            read_bundle(_bundle(tmp_path, tmp_path, buckets=bad))
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, tmp_path, linear="fp16"))
    ck, digest = _repair(tmp_path)
    assert read_bundle(_bundle(tmp_path, tmp_path, checkpoint=str(ck), checkpoint_sha256=digest))["model"]
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, tmp_path, checkpoint=str(ck), checkpoint_sha256="0" * 64))
    check_identity_repair(ck)
    bad, _ = _repair(tmp_path, nonzero=True)
    with pytest.raises(ValueError):
        check_identity_repair(bad)


def _cpu_runtime(tmp_path, variant="aspect256", buckets=(64, 96, 128, 192)):
    """A FamilyRuntime with its tokenizer and request state but no weights
    (the request-preparation half needs no GPU)."""
    from fastforward_amd.family import FamilyRuntime
    rt = FamilyRuntime.__new__(FamilyRuntime)
    rt.tokenizer = _tiny_tokenizer(tmp_path)
    rt.image_token = IMAGE_ID
    rt.buckets = sorted(buckets)
    rt.max_tokens = rt.buckets[-1]
    rt.style = "short"
    rt.variant = variant
    rt.geometry, rt.cache, rt.profiles = {}, {}, {}
    return rt


def test_prefix_expansion_and_prepare(tmp_path):
    rt = _cpu_runtime(tmp_path)
    g = rt.setup_side((192, 320))
    # <|im_start|> user <|vision_start|> then 6 x 10 image tokens, then <|vision_end|>
    assert g["image_start"] == 3 and g["grid"] == (6, 10)
    pre = g["prefix"].tolist()
    assert pre[:3] == [995, rt.tokenizer.token_to_id("user"), 998]
    assert pre[3:63] == [IMAGE_ID] * 60 and pre[63:] == [996]
    rgb = np.random.default_rng(0).integers(0, 256, size=(200, 300, 3), dtype=np.uint8)
    row = dict(rgb=rgb, instruction="What color is shown?", candidates=["red", "green", "blue"])
    p = rt.prepare(row)
    assert p["side"] == (192, 320) and p["rgb"].shape == (192, 320, 3)
    assert p["k"] == 3 and p["pick"] == len(p["ids"]) - 1
    assert p["ids"][:64].tolist() == pre
    tail = [rt.tokenizer.id_to_token(int(i)) for i in p["ids"][-4:]]
    assert tail == ["<|im_start|>", "assistant", "Answer", ":"]
    assert rt.bucket_for(len(p["ids"])) == 96
    # square variants: the whole 256 x 256 canvas, 64 image tokens
    sq = _cpu_runtime(tmp_path, variant="square256")
    q = sq.prepare(row)
    assert q["side"] == (256, 256) and int((q["ids"] == IMAGE_ID).sum()) == 64
    # text is never truncated
    small = _cpu_runtime(tmp_path, buckets=(64,))
    with pytest.raises(ValueError):
        small.prepare(row)


def test_cli_arguments(tmp_path):
    from fastforward_amd.cli import main
    with pytest.raises(SystemExit):
        main(["--bundle", "b.json"])
    with pytest.raises(FileNotFoundError):
        main(["--bundle", str(tmp_path / "absent.json"), "--image", "x.png", "--question", "q", "--choices", "a",
              "b"])


def _fp8_reference(m):
    """Give transformers' LM linears the step's FP8 rounding: weights replaced
    by their per-output-channel e4m3 round trip (s = amax/448), inputs by
    their per-token e4m3 round trip (forward pre-hooks). What remains between
    the two paths is bf16 rounding of the dequantised operands and
    accumulation order."""
    def rt(x, dim):
        x = x.float()
        s = x.abs().amax(dim=dim, keepdim=True).clamp_min(1e-12) / 448.0
        return ((x / s).clamp(-448, 448).to(torch.float8_e4m3fn).float() * s).to(torch.bfloat16)

    def hook(mod, args):
        return (rt(args[0], -1),) + tuple(args[1:])

    for layer in m.model.language_model.layers:
        for lin in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj, layer.self_attn.o_proj,
                    layer.mlp.gate_proj, layer.mlp.up_proj, layer.mlp.down_proj):
            with torch.no_grad():
                lin.weight.copy_(rt(lin.weight, 1))
            lin.register_forward_pre_hook(hook)
    return m


def _hf_option_logits(m, g, option_ids):
    from oracle import vision as OV
    ids = torch.from_numpy(np.asarray(g["ids"], dtype=np.int64))[None]
    h, w = g["side"]
    pix = OV.pack_pixels(g["rgb"])
    with torch.no_grad():
        out = m(input_ids=ids, pixel_values=pix.float(), image_grid_thw=torch.tensor([[1, h // 16, w // 16]]),
                mm_token_type_ids=(ids == IMAGE_ID).int())
    return out.logits[0, -1, option_ids[:g["k"]]].float()


@pytest.mark.gpu
def test_predict_matches_transformers(gpu, tmp_path):
    from PIL import Image

    from fastforward_amd.api import Accelerator
    from fastforward_amd.pipeline import ImageStep
    m, path = _tiny_hf(tmp_path, seed=5)
    from pathlib import Path
    _tiny_tokenizer(Path(path))
    ck, digest = _repair(tmp_path)
    bundle = _bundle(tmp_path, path, checkpoint=str(ck), checkpoint_sha256=digest, expected_dimensions=[2, 512, 2])
    rng = np.random.default_rng(6)
    imgs = []
    for j, shape in enumerate([(200, 300, 3), (210, 290, 3)]):
        f = tmp_path / f"img{j}.png"
        Image.fromarray(rng.integers(0, 256, size=shape, dtype=np.uint8)).save(f)
        imgs.append(f)
    acc = Accelerator(bundle)      # loads (and quantises) the saved bf16 weights first
    rt = acc.runtime
    _fp8_reference(m)
    cands = ["red", "green", "blue", "black", "white", "gray", "pink", "brown"]
    q = "What color is shown?"
    print("family predict: tiny checkpoint, aspect256, 2 images, 8 options", flush=True)
    r0 = acc.predict(imgs[0], q, cands, item_id="a")
    assert r0["id"] == "a" and len(r0["probabilities"]) == 8
    # second request, same canvas and bucket: the refilled graph equals a fresh eager step
    r1 = acc.predict(imgs[1], q, cands, item_id="b")
    assert len(rt.cache) == 1
    g = [rt.prepare(dict(image_path=str(f), instruction=q, candidates=cands)) for f in imgs]
    geo = rt.setup_side(g[1]["side"])
    bucket = rt.bucket_for(len(g[1]["ids"]))
    st = ImageStep(rt.lm_cfg, rt.lm_w, rt.vis_cfg, rt.vis_w, g[1]["side"][0] // 16, g[1]["side"][1] // 16, bucket,
                   geo["image_start"])
    st.set_inputs(torch.from_numpy(g[1]["rgb"]), torch.from_numpy(g[1]["ids"]), rt.positions(g[1]["side"], bucket),
                  g[1]["pick"])
    eager = st.step()[:8].float().cpu()
    torch.cuda.synchronize()
    assert torch.equal(eager, torch.tensor(r1["logits"])), (eager.tolist(), r1["logits"])
    # both requests against transformers; the two images' own difference is the scale a wiring
    # mistake (image rows, positions, pixels) would show
    want = [_hf_option_logits(m, gi, rt.meta["option_ids"]) for gi in g]
    got = [torch.tensor(r["logits"]) for r in (r0, r1)]
    rel = [float((a - b).norm() / b.norm()) for a, b in zip(got, want)]
    between = float((want[0] - want[1]).norm() / want[0].norm())
    for j in range(2):
        print(f"request {j}: ours {got[j].tolist()}\n           hf   {want[j].tolist()}", flush=True)
    print(f"vs transformers (FP8-rounded linears): rel L2 {rel[0]:.4f}, {rel[1]:.4f}; "
          f"between the two images {between:.4f}", flush=True)
    assert max(rel) <= 0.08 and max(rel) < between / 4


def _fp8_static_reference(m, bounds):
    """transformers' LM linears with the static-FP8 rounding of a calibration
    profile: weights round-tripped through e4m3 with one scale per packed
    weight (amax/448 over q/k/v together, over gate/up together, o, down),
    inputs through e4m3(clamp(x * 448/bound, +-448)) * bound/448 with the
    layer's bound for that role. Returns the hook handles."""
    def wq(ws):
        s = max(float(w.detach().float().abs().max()) for w in ws) / 448.0
        with torch.no_grad():
            for w in ws:
                w.copy_(((w.float() / s).to(torch.float8_e4m3fn).float() * s).to(torch.bfloat16))

    def act(bound):
        inv = 448.0 / bound

        def hook(mod, args):
            x = args[0].float()
            q = (x * inv).clamp(-448, 448).to(torch.float8_e4m3fn).float() * (bound / 448.0)
            return (q.to(torch.bfloat16),) + tuple(args[1:])
        return hook

    handles = []
    for j, layer in enumerate(m.model.language_model.layers):
        a, mlp = layer.self_attn, layer.mlp
        groups = {"qkv": [a.q_proj, a.k_proj, a.v_proj], "output": [a.o_proj], "gateup": [mlp.gate_proj, mlp.up_proj],
                  "down": [mlp.down_proj]}
        for role, lins in groups.items():
            wq([lin.weight for lin in lins])
            for lin in lins:
                handles.append(lin.register_forward_pre_hook(act(bounds[f"{j}:{role}"])))
    return handles


@pytest.mark.gpu
def test_predict_with_calibration_profile_and_select(gpu, tmp_path):
    """A bundle with a calibration profile: static FP8 linears (one weight scale
    per packed weight, the profile's activation bounds), the variant's canvas;
    ``select`` switches bounds and canvas and re-captures. Each variant's answer
    logits agree with transformers given the same static e4m3 rounding: relative
    L2 <= 0.10 (0.046 and 0.072 measured; the static bounds quantise more
    coarsely than per-token scales, so rounding flips weigh more)."""
    from pathlib import Path

    from PIL import Image

    from fastforward_amd.api import Accelerator
    m0, path = _tiny_hf(tmp_path, seed=7)
    _tiny_tokenizer(Path(path))
    roles = ("qkv", "output", "gateup", "down")
    profiles = {"aspect256": {f"{j}:{r}": b for j in range(2) for r, b in zip(roles, (6.0, 4.0, 8.0, 2.0))},
                "square256": {f"{j}:{r}": b for j in range(2) for r, b in zip(roles, (5.0, 3.0, 6.0, 1.5))}}
    prof = tmp_path / "profiles.json"
    prof.write_text(json.dumps({"profiles": profiles}))
    digest = hashlib.sha256(prof.read_bytes()).hexdigest()
    bundle = _bundle(tmp_path, path, profile_path=str(prof), profile_sha256=digest, variant="aspect256")
    f = tmp_path / "img.png"
    Image.fromarray(np.random.default_rng(8).integers(0, 256, size=(200, 300, 3), dtype=np.uint8)).save(f)
    acc = Accelerator(bundle)
    rt = acc.runtime
    assert rt.linear == "fp8_static"
    cands = ["red", "green", "blue", "black", "white", "gray", "pink", "brown"]
    q = "What color is shown?"
    for variant, side in (("aspect256", (192, 320)), ("square256", (256, 256))):
        if variant != acc.variant:
            acc.select(variant)
        print(f"calibrated predict: variant {variant}", flush=True)
        r = acc.predict(f, q, cands)
        g = rt.prepare(dict(image_path=str(f), instruction=q, candidates=cands))
        assert g["side"] == side
        m, _ = _tiny_hf(tmp_path, seed=7, save=False)      # a fresh bf16 copy of the same model
        handles = _fp8_static_reference(m, profiles[variant])
        want = _hf_option_logits(m, g, rt.meta["option_ids"])
        for h in handles:
            h.remove()
        got = torch.tensor(r["logits"])
        rel = float((got - want).norm() / want.norm())
        print(f"{variant}: ours {got.tolist()}\n           hf   {want.tolist()}\n  rel L2 {rel:.4f}", flush=True)
        assert rel <= 0.10


def _int4_reference(m):
    """transformers' LM linear weights replaced by the reference's asymmetric
    group-32 int4 round trip (_family/night_runtime.py:18-23): per group
    s = max((max - min)/15, 1e-6), q = clamp(round((w - min)/s), 0, 15),
    z = min + 8 s, stored as bf16 (s, z); w = (q - 8) s + z."""
    for layer in m.model.language_model.layers:
        a, mlp = layer.self_attn, layer.mlp
        for lin in (a.q_proj, a.k_proj, a.v_proj, a.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            w = lin.weight.detach().float()
            n, k = w.shape
            x = w.reshape(n, k // 32, 32)
            low, high = x.amin(-1, keepdim=True), x.amax(-1, keepdim=True)
            s = ((high - low) / 15).clamp_min(1e-6)
            q = ((x - low) / s).round().clamp(0, 15)
            z = low + s * 8
            sb, zb = s.to(torch.bfloat16).float(), z.to(torch.bfloat16).float()
            with torch.no_grad():
                lin.weight.copy_(((q - 8) * sb + zb).reshape(n, k).to(torch.bfloat16))
    return m


@pytest.mark.gpu
def test_predict_int4_execution_mode(gpu, tmp_path):
    """execution_mode 'int4' loads the reference's asymmetric group-32 W4A16
    linears; the answer logits agree with transformers whose weights took the
    same int4 round trip (bf16 activations on both sides): relative L2 <= 0.05,
    0.014 measured."""
    from pathlib import Path

    from PIL import Image

    from fastforward_amd.api import Accelerator
    m, path = _tiny_hf(tmp_path, seed=9)
    _tiny_tokenizer(Path(path))
    bundle = _bundle(tmp_path, path, execution_mode="int4")
    f = tmp_path / "img.png"
    Image.fromarray(np.random.default_rng(10).integers(0, 256, size=(200, 300, 3), dtype=np.uint8)).save(f)
    acc = Accelerator(bundle)
    rt = acc.runtime
    assert rt.linear == "int4"
    cands = ["red", "green", "blue", "black", "white", "gray", "pink", "brown"]
    q = "What color is shown?"
    print("int4 predict", flush=True)
    r = acc.predict(f, q, cands)
    g = rt.prepare(dict(image_path=str(f), instruction=q, candidates=cands))
    want = _hf_option_logits(_int4_reference(m), g, rt.meta["option_ids"])
    got = torch.tensor(r["logits"])
    rel = float((got - want).norm() / want.norm())
    print(f"int4: ours {got.tolist()}\n      hf   {want.tolist()}\n  rel L2 {rel:.4f}", flush=True)
    assert rel <= 0.05


@pytest.mark.gpu
def test_two_canvases_alternate_over_shared_arenas(gpu, tmp_path):
    """Requests that alternate between two canvases (a landscape and a portrait
    image under aspect256) run two captured image steps whose LM activations
    alias one arena and whose vision activations alias another: both steps'
    buffers start at the arenas' bases, and every replay, over two rounds,
    equals an eager ImageStep of the same inputs on private buffers bit for bit."""
    from pathlib import Path

    from PIL import Image

    from fastforward_amd.api import Accelerator
    from fastforward_amd.pipeline import ImageStep
    m, path = _tiny_hf(tmp_path, seed=11)
    _tiny_tokenizer(Path(path))
    acc = Accelerator(_bundle(tmp_path, path))
    rt = acc.runtime
    rng = np.random.default_rng(12)
    files = []
    for j, shape in enumerate([(200, 300, 3), (300, 200, 3)]):
        f = tmp_path / f"alt{j}.png"
        Image.fromarray(rng.integers(0, 256, size=shape, dtype=np.uint8)).save(f)
        files.append(f)
    cands = ["red", "green", "blue", "black"]
    q = "What color is shown?"
    g = [rt.prepare(dict(image_path=str(f), instruction=q, candidates=cands)) for f in files]
    assert g[0]["side"] != g[1]["side"], "the two images must land on different canvases"
    eager = []
    for gi in g:
        geo = rt.setup_side(gi["side"])
        bucket = rt.bucket_for(len(gi["ids"]))
        st = ImageStep(rt.lm_cfg, rt.lm_w, rt.vis_cfg, rt.vis_w, gi["side"][0] // 16, gi["side"][1] // 16, bucket,
                       geo["image_start"])
        st.set_inputs(torch.from_numpy(gi["rgb"]), torch.from_numpy(gi["ids"]), rt.positions(gi["side"], bucket),
                      gi["pick"])
        eager.append(st.step()[:len(cands)].float().cpu())
        del st
    print("two canvases alternating over the shared arenas", flush=True)
    for rnd in range(2):
        for j, f in enumerate(files):
            r = acc.predict(f, q, cands)
            assert torch.equal(torch.tensor(r["logits"]), eager[j]), (rnd, j, r["logits"], eager[j].tolist())
    assert len(rt.cache) == 2
    for st, *_ in rt.cache.values():
        assert st.lm.cos.data_ptr() == rt.arena.buf.data_ptr()
        assert st.vision.pixels.data_ptr() == rt.vision_arena.buf.data_ptr()
    assert not torch.equal(eager[0], eager[1])

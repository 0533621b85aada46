"""Request-API contract: the reference's tests/test_contract.py cases
(test_request, test_response) on this build's api module, plus bundle
validation and, on the GPU, predict_tokens against an eager step."""
import json

import pytest

from fastforward_amd.api import Accelerator, read_bundle, response, validate_request


def test_request(tmp_path):
    image = tmp_path / "input.png"
    image.touch()
    validate_request(image, "Question", ["A", "B"])
    for choices in (["A"], ["A", ""], ["A"] * 9, "AB", ["A", 3]):
        with pytest.raises(ValueError):
            validate_request(image, "Question", choices)
    with pytest.raises(ValueError):
        validate_request(image, "  ", ["A", "B"])
    with pytest.raises(FileNotFoundError):
        validate_request(tmp_path / "missing.png", "Question", ["A", "B"])


def test_response():
    r = response([1.0, 1.0], ["a", "b"], "x")
    assert r["answer"] == {"letter": "A", "text": "a"} and r["id"] == "x"
    assert abs(sum(r["probabilities"]) - 1.0) < 1e-12
    with pytest.raises(RuntimeError):
        response([float("nan"), 0.0], ["a", "b"], "x")
    with pytest.raises(RuntimeError):
        response([0.0], ["a", "b"], "x")
    r = response([0.5, 2.0, 2.0, -1.0], ["a", "b", "c", "d"], "y")   # ties -> first index
    assert r["answer"]["letter"] == "B" and r["probabilities"][1] == r["probabilities"][2]


def _bundle(tmp_path, **kw):
    c = dict(schema_version=1, task="visual_choice", architecture="qwen3_vl_lm", preset="qwen3vl-2b",
             linear="fp8", seed=3, tokens=320, image_grid=[16, 16], prefix_tokens=4)
    c.update(kw)
    p = tmp_path / "bundle.json"
    p.write_text(json.dumps(c))
    return p


@pytest.mark.parametrize("bad", [dict(schema_version=2), dict(task="caption"), dict(architecture="llama"),
                                 dict(preset="qwen3vl-70b"), dict(linear="int8"), dict(tokens=100),
                                 dict(buckets=[200, 320]), dict(buckets=[]), dict(buckets="320")])
def test_bundle_rejected(tmp_path, bad):
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, **bad))


def test_bundle_checkpoint_and_backend(tmp_path):
    with pytest.raises(FileNotFoundError):
        read_bundle(_bundle(tmp_path, checkpoint=str(tmp_path / "absent.pt")))
    ck = tmp_path / "ck.pt"
    ck.write_bytes(b"weights")
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, checkpoint=str(ck), checkpoint_sha256="0" * 64))
    assert read_bundle(_bundle(tmp_path))["preset"] == "qwen3vl-2b"
    with pytest.raises(ValueError):
        Accelerator(_bundle(tmp_path), backend="turbo")
    with pytest.raises(RuntimeError):
        Accelerator(_bundle(tmp_path), backend="native")


@pytest.mark.gpu
def test_predict_tokens_matches_eager_step(gpu, tmp_path):
    import torch
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_request
    acc = Accelerator(_bundle(tmp_path))
    image = tmp_path / "input.png"
    image.touch()
    with pytest.raises(RuntimeError):
        acc.predict(image, "Which?", ["yes", "no"])
    eager = Runtime(acc.cfg, acc.weights, acc.tokens)
    for seed, n_choices in ((1, 4), (2, 2)):
        ids, pos, pick = make_request(acc.cfg, 320, 16, 16, seed=seed, real_tokens=300)
        cands = [f"c{i}" for i in range(n_choices)]
        r = acc.predict_tokens(ids, cands, item_id=f"r{seed}")
        eager.set_inputs(ids, pos, pick)
        z = eager.step().cpu().tolist()[:n_choices]
        assert r["logits"] == z and r["id"] == f"r{seed}"
        assert r["answer"] == response(z, cands, "r")["answer"]
    with pytest.raises(ValueError):
        acc.predict_tokens(torch.zeros(10, dtype=torch.int64), ["a", "b"])


def test_step_graphs_buckets_and_position_templates():
    """Bucket choice (smallest bucket that holds the request) and the
    per-bucket M-RoPE template: on a prompt's real tokens it equals the
    positions of the prompt alone (the reference's template check)."""
    import numpy as np
    from fastforward_amd.graphs import StepGraphs
    from fastforward_amd.runtime import PRESETS, mrope_positions
    g = StepGraphs(PRESETS["qwen3vl-2b"], None, [320, 288], (16, 16), 4)
    assert g.buckets == [288, 320]
    assert g.bucket_for(260) == 288 and g.bucket_for(288) == 288 and g.bucket_for(289) == 320
    with pytest.raises(ValueError):
        g.bucket_for(321)
    for n in (260, 275, 288):
        t = g.positions(g.bucket_for(n)).numpy()
        assert np.array_equal(t[:, :n], mrope_positions(4, 16, 16, n))
    with pytest.raises(ValueError):
        StepGraphs(PRESETS["qwen3vl-2b"], None, [200], (16, 16), 4)


@pytest.mark.gpu
def test_bucketed_graphs_match_eager_and_isolate_padding(gpu, tmp_path):
    """Requests of 270, 300 and 280 tokens over buckets (288, 320): each bucket
    captures on its first request only, every replay equals an eager step of
    its bucket bit for bit (the buckets' activations alias one arena; the eager
    steps have their own), and the gate (position template, graph == eager,
    padding ids set to 42 leave the answer's bits unchanged) passes."""
    import torch
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_request
    acc = Accelerator(_bundle(tmp_path, buckets=[288, 320]))
    seen = []
    for seed, n in ((1, 270), (2, 300), (3, 280)):
        ids, _, _ = make_request(acc.cfg, n, 16, 16, seed=seed, real_tokens=n)
        ids = torch.as_tensor(ids)[:n]
        z, captured = acc.graphs.run(ids, n - 1, 4)
        b = acc.graphs.bucket_for(n)
        assert captured == (b not in seen)
        seen.append(b)
        eager = Runtime(acc.cfg, acc.weights, b)
        eager.set_inputs(ids, acc.graphs.positions(b), n - 1)
        assert torch.equal(z.cpu(), eager.step()[:4].cpu())
        report = acc.graphs.gate(ids, n - 1, 4)
        assert report["passed"] and report["bucket"] == b
        r = acc.predict_tokens(ids, ["a", "b", "c", "d"], item_id=f"r{seed}")
        assert r["logits"] == z.cpu().tolist()
    src, pin, _ = acc.graphs.staging[288]
    assert src.is_pinned() and pin.is_pinned()
    # the two buckets' activations alias one arena (each bucket's replays above
    # ran after the other bucket had overwritten it, and still equalled eager steps)
    r288, r320 = acc.graphs.cache[288], acc.graphs.cache[320]
    base, size = acc.graphs.arena.buf.data_ptr(), acc.graphs.arena.nbytes
    assert r288.cos.data_ptr() == r320.cos.data_ptr() == base   # both laid out from offset 0
    for rt in (r288, r320):
        assert base <= rt.gws.data_ptr() and rt.gws.data_ptr() + rt.gws.numel() <= base + size


def _profile(tmp_path, variants, layers=28):
    roles = ("qkv", "output", "gateup", "down")
    p = tmp_path / "profile.json"
    p.write_text(json.dumps({"profiles": {v: {f"{j}:{r}": b for j in range(layers) for r in roles}
                                          for v, b in variants.items()}}))
    from fastforward_amd.api import sha256
    return p, sha256(p)


def test_calibration_profiles_read_and_bundle_checks(tmp_path):
    """Profile files as activate_fast reads them (digest checked), and the
    bundle rules: a profile needs static FP8 linears and a known variant."""
    from fastforward_amd.profiles import read_profiles
    p, digest = _profile(tmp_path, {"square256": 8.0, "tall": 12.0})
    assert set(read_profiles(p, digest)) == {"square256", "tall"}
    with pytest.raises(ValueError):
        read_profiles(p, "0" * 64)
    with pytest.raises(FileNotFoundError):
        read_profiles(tmp_path / "none.json")
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps({"profiles": {"v": {"0:qkv": -1}}}))
    with pytest.raises(ValueError):
        read_profiles(bad)
    kw = dict(profile_path=str(p), profile_sha256=digest, variant="tall")
    assert read_bundle(_bundle(tmp_path, linear="fp8_static", **kw))["variant"] == "tall"
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, linear="fp8", **kw))
    with pytest.raises(ValueError):
        read_bundle(_bundle(tmp_path, linear="fp8_static", **dict(kw, variant="wide")))


def test_set_bound_matches_reference_select():
    """select's per-op update (_family/night_runtime.py:52-54) on a host-side
    op: inverse_scale = 448/bound, input_scale refilled in place with bound/448;
    apply_profile names the first missing entry."""
    import types
    import torch
    from fastforward_amd.linear import StaticFP8Linear
    from fastforward_amd.profiles import apply_profile
    op = object.__new__(StaticFP8Linear)
    op.input_scale = torch.zeros(1)
    buf = op.input_scale
    op.set_bound(7.0)
    assert op.inverse_scale == 448.0 / 7.0 and op.input_scale is buf
    assert float(op.input_scale[0]) == float(torch.tensor(7.0 / 448.0))
    layer = types.SimpleNamespace(qkv=op, o=op, gateup=op, down=op)
    w = types.SimpleNamespace(layers=[layer])
    assert apply_profile(w, {"0:qkv": 2.0, "0:output": 3.0, "0:gateup": 4.0, "0:down": 5.0}) == 4
    assert op.inverse_scale == 448.0 / 5.0
    with pytest.raises(KeyError):
        apply_profile(w, {"0:qkv": 2.0})


@pytest.mark.gpu
def test_select_switches_static_fp8_variants(gpu, tmp_path):
    """A static-FP8 bundle with two calibration variants: each select gives the
    eager step of that calibration bit for bit through a re-captured graph,
    and selecting the first variant again restores its logits exactly."""
    import torch
    from fastforward_amd.profiles import apply_profile
    from fastforward_amd.runtime import Runtime
    from fastforward_amd.synthetic import make_request
    p, digest = _profile(tmp_path, {"a": 6.0, "b": 14.0})
    acc = Accelerator(_bundle(tmp_path, linear="fp8_static", profile_path=str(p), profile_sha256=digest,
                              variant="a"))
    ids, _, _ = make_request(acc.cfg, 300, 16, 16, seed=5, real_tokens=300)
    ids = torch.as_tensor(ids)[:300]
    za, cap = acc.graphs.run(ids, 299, 4)
    za = za.cpu()
    assert cap
    acc.select("b")
    zb, cap = acc.graphs.run(ids, 299, 4)
    zb = zb.cpu()
    assert cap and not torch.equal(za, zb)
    eager = Runtime(acc.cfg, acc.weights, 320)
    eager.set_inputs(ids, acc.graphs.positions(320), 299)
    assert torch.equal(eager.step()[:4].cpu(), zb)
    acc.select("a")
    assert torch.equal(acc.graphs.run(ids, 299, 4)[0].cpu(), za)
    with pytest.raises(ValueError):
        acc.select("c")


def test_arena_holds_every_bucket_layout():
    """The shared activation arena is sized by the largest layout over all
    buckets, not the largest bucket's: the k-split workspace of the packed FP8
    GEMMs is needed only where a shape's tiles do not fill the GPU unsplit, so
    mid-sized buckets can need more bytes than the largest one. Walks the 8B
    shape over the reference's 8B bucket list (64..2048 in steps of 16,
    configs/8B.json:10-141) on the host: every bucket's layout fits, and at
    least one bucket needs more than the largest bucket (the case the sizing
    must cover)."""
    from fastforward_amd.runtime import PRESETS, Arena
    cfg = PRESETS["qwen3vl-8b"]
    buckets = list(range(64, 2049, 16))
    sizes = {b: Arena.size_for(cfg, b) for b in buckets}
    need = Arena.size_for_buckets(cfg, buckets)
    assert need == max(sizes.values())
    assert all(s <= need for s in sizes.values())
    assert any(s > sizes[2048] for s in sizes.values()), "no bucket exceeds the largest one's layout"
    # the generic path (non-FP8Linear weights) lays out only the shared buffers
    assert Arena.size_for(cfg, 2048, "generic") < Arena.size_for(cfg, 2048)


def test_mixed_execution_mode_banks():
    """int4_half / int4_ffn pick banks as the reference's set_mode does
    (_family/night_runtime.py:60-64): interior = 3 <= j < final - 3; int4_half
    takes all four roles of the even interior layers from the int4 bank,
    int4_ffn the gate/up and down projections of every interior layer."""
    from fastforward_amd.linear import bank_of
    layers = 36
    final = layers - 1
    roles = ("qkv", "o", "gateup", "down")
    for j in range(layers):
        interior = 3 <= j < final - 3
        for r in roles:
            assert bank_of("int4_half", j, layers, r) == ("int4" if interior and j % 2 == 0 else "fp8")
            assert bank_of("int4_ffn", j, layers, r) == ("int4" if interior and r in ("gateup", "down") else "fp8")
            assert bank_of("int4", j, layers, r) == "int4"
            assert bank_of("precise", j, layers, r) == "fp8"
    half = sum(bank_of("int4_half", j, layers, r) == "int4" for j in range(layers) for r in roles)
    ffn = sum(bank_of("int4_ffn", j, layers, r) == "int4" for j in range(layers) for r in roles)
    assert (half, ffn) == (14 * 4, 29 * 2)

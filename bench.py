"""Benchmark: Qwen3-VL-8B-shaped FP8 prefill + choice-score step on one MI355X.

Workload (the headline metric): 36 decoder layers, hidden 4096, GQA 32/8,
head_dim 128, MLP 12288, vocab 151936; FP8 e4m3 linears (per-token activation /
per-channel weight scales), bf16 elsewhere; 576 tokens (4 text + 16x32 image
grid + 60 text), pick-only final layer, 8 answer choices; the whole step is one
hipGraph. Weights are random-init N(0, 0.02) and token ids uniform (seeded):
there is no checkpoint. A step = one graph replay with inputs resident in HBM.

Prints ONE JSON line. ``roofline`` covers the dominant kernel, the gate/up FP8
GEMM with its SwiGLU epilogue, timed live with HIP events on the step's own
shape and weights; ``roofline.all_fp8_gemm`` the same for all of the step's FP8
GEMM launches (the metric's "FP8 GEMM % MFMA peak"); ``cpu_baseline`` times the
CPU oracle on a bounded sample of the same step (a few layers + the tail),
scaled to the full step.
"""
import argparse
import json
import os
import sys
import time
import types

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "ms per prefill+choice-score step (8B-shape FP8, 576 tok); FP8 GEMM % MFMA peak"
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense fp8 MFMA
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
GEMM_KERNELS = ("FP8 GEMM launches of the step: gemm_fp8_swiglu_packed_kernel (gate/up), "
                "gemm_fp8_split_packed_kernel (down, timed with split_reduce_kernel adding its partials, which "
                "the step's next add_rms launch does; 80 x 128 tiles unsplit for o), "
                "gemm_fp8_qkv_packed_kernel (qkv, 128 x 128 tiles, with its epilogue), gemv_fp8 kernels (the tail's "
                "single row)")
MICRO_SHAPES = [(320, 2048, 6144), (320, 6144, 2048), (576, 4096, 12288), (576, 12288, 4096),
                (1024, 5120, 25600)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_graph(rt, steps, warmup):
    for _ in range(warmup):
        rt.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        rt.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def gemm_launches(cfg, T):
    """(role, m, count) of every FP8 GEMM launch in one step: full layers run all
    four linears on T rows; the pick-only final layer runs qkv on T rows and
    o / gateup / down on one row."""
    full = cfg.layers - 1
    return [("qkv", T, full + 1), ("o", T, full), ("gateup", T, full), ("down", T, full),
            ("o", 1, 1), ("gateup", 1, 1), ("down", 1, 1)]


def gemm_buffers(cfg, role, n, m, T):
    """Output buffers of one launch of ``role`` as the step allocates them."""
    dev, bf = "cuda", torch.bfloat16
    if role == "qkv":
        D, Tp = cfg.head_dim, (T + 63) // 64 * 64
        b = dict(yq=torch.empty(cfg.heads, T, D, device=dev, dtype=bf),
                 yk=torch.empty(cfg.kv_heads, T, D, device=dev, dtype=bf),
                 vt=torch.empty(cfg.kv_heads, D, Tp, device=dev, dtype=bf),
                 cos=torch.ones(T, D, device=dev, dtype=bf), sin=torch.zeros(T, D, device=dev, dtype=bf),
                 Tp=Tp)
        return b
    if role == "gateup":
        return dict(out=torch.empty((m, n // 2), device=dev, dtype=bf),
                    pmax=torch.empty((m, max(1, n // 128)), device=dev, dtype=torch.float32))
    return dict(out=torch.empty((m, n), device=dev, dtype=bf))


def launch_gemm(cfg, role, lw, q, s, m, b):
    """One FP8 GEMM launch as the step issues it: the QKV projection with its
    q/k norm + rotary + V^T epilogue (ff_gemm_fp8_qkv_pk: packed weights), the
    gate/up projection with its SwiGLU epilogue (ff_gemm_fp8_swiglu_pk), o and down
    through ``FP8Linear.gemm`` (ff_gemm_fp8_pk: the k-split packed kernel and its
    reduction for down -- in the step the next add_rms launch adds the partials
    -- the small packed tiles for o, the GEMV kernels for the tail's single
    row)."""
    from fastforward_amd._lib import call, ptr, stream
    op = getattr(lw, role)
    n, k = op.weight.shape
    if role == "qkv":
        call("ff_gemm_fp8_qkv_pk", ptr(q), ptr(s), 1, ptr(op.weight), ptr(op.packed), ptr(op.scale), 1, m, k,
             cfg.heads, cfg.kv_heads, ptr(lw.q_norm.weight), ptr(lw.k_norm.weight),
             float(lw.q_norm.variance_epsilon), float(lw.k_norm.variance_epsilon), ptr(b["cos"]), ptr(b["sin"]),
             ptr(b["yq"]), ptr(b["yk"]), ptr(b["vt"]), b["Tp"], stream())
    elif role == "gateup":
        call("ff_gemm_fp8_swiglu_pk", ptr(q), ptr(s), ptr(op.weight), ptr(op.packed), ptr(op.scale), ptr(b["out"]),
             n // 2, ptr(b["pmax"]), m, n // 2, k, stream())
    else:
        op.gemm(q[:m], s[:m], b["out"])


def time_gemm(cfg, role, q, s, layers, m, T, reps=3):
    """Average duration (ms) of one launch of ``role``: the launch sequence walks
    every layer's weights in turn, as the step does, so weights come from HBM
    rather than from a cache warmed by the previous launch. HIP events on the
    launch stream bracket reps x len(layers) launches."""
    n = getattr(layers[0], role).weight.shape[0]
    b = gemm_buffers(cfg, role, n, m, T)
    # two untimed passes: the first launches after an idle GPU (buffer set-up) run slow
    for _ in range(2):
        for lw in layers:
            launch_gemm(cfg, role, lw, q, s, m, b)
    torch.cuda.synchronize()
    a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        for lw in layers:
            launch_gemm(cfg, role, lw, q, s, m, b)
    e.record()
    torch.cuda.synchronize()
    return a.elapsed_time(e) / (reps * len(layers))


def gemm_roofline(cfg, w, T):
    """Live FP8 GEMM timing on the step's shapes over all layers' weights. The
    line's roofline is the dominant kernel's, the gate/up GEMM with its SwiGLU
    epilogue (the largest share of the step): its algorithmic FLOPs per launch
    over its average launch duration, and its HBM bytes per launch from the
    committed counter profile. Beside it (``all_fp8_gemm``) the same for all of
    the step's FP8 GEMM launches, weighted by their launch counts."""
    total_flop = total_ms = 0.0
    launches = 0
    per_shape = {}
    first = True
    for role, m, count in gemm_launches(cfg, T):
        op0 = getattr(w.layers[0], role)
        n, k = op0.weight.shape
        x = torch.randn(T, k, device="cuda").to(torch.bfloat16)
        q, s = op0.quantize(x)
        if first:
            # the first shape timed after the GPU idled (model and buffer set-up) runs several us slower
            # per launch until the clocks are back up: one untimed pass of it first
            time_gemm(cfg, role, q, s, w.layers, m, T)
            first = False
        ms = time_gemm(cfg, role, q, s, w.layers, m, T)
        flop = 2.0 * m * n * k
        per_shape[f"{role} {m}x{k}x{n}"] = dict(us=round(ms * 1e3, 2), tflops=round(flop / ms / 1e9, 1))
        total_flop += flop * count
        total_ms += ms * count
        launches += count
    avg_ms = total_ms / launches
    achieved = total_flop / launches / (avg_ms * 1e-3) / 1e12
    gu_key = f"gateup {T}x{cfg.hidden}x{2 * cfg.inter}"
    gu = per_shape[gu_key]
    traffic = _traffic()
    return dict(bound="mfma", achieved=gu["tflops"], peak=PEAK_FP8_TFLOPS, unit="TFLOP/s",
                frac=round(gu["tflops"] / PEAK_FP8_TFLOPS, 4),
                traffic=traffic["by_shape"].get(gu_key) if traffic else None,
                kernel="gemm_fp8_swiglu_packed_kernel (gate/up + SwiGLU epilogue, 144 x 384 tiles)",
                avg_launch_us=gu["us"], flop_per_launch=2.0 * T * cfg.hidden * 2 * cfg.inter,
                all_fp8_gemm=dict(achieved=round(achieved, 1), frac=round(achieved / PEAK_FP8_TFLOPS, 4),
                                  traffic=traffic["per_launch"] if traffic else None, kernel=GEMM_KERNELS,
                                  avg_launch_us=round(avg_ms * 1e3, 2), launches_per_step=launches,
                                  gemm_ms_per_step=round(total_ms, 3), by_shape=per_shape))


def _traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 PMC summary, if
    any: the step-weighted mean and each shape's."""
    path = os.path.join(HERE, "profiles", "gemm_fp8_traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            t = json.load(f)
        return dict(per_launch=t.get("bytes_per_launch"),
                    by_shape={b["shape"]: b["hbm_bytes"] for b in t.get("by_shape", [])})
    return None


def algorithmic_bytes(cfg, role, m, n, k, T):
    """Bytes one launch must move at least: the e4m3 operands and fp32 scales,
    plus what its epilogue reads and writes (QKV: q/k norm weights and cos/sin
    in, head-major q/k and V^T out; gate/up: the SwiGLU product (m, n/2) and
    the fp32 row maxima per 64 channels; o/down: the bf16 (m, n) output)."""
    base = m * k + n * k + 4 * (m + n)
    if role == "qkv":
        D = cfg.head_dim
        return base + 2 * 2 * D + 2 * 2 * T * D + 2 * m * n
    if role == "gateup":
        return base + 2 * m * (n // 2) + 4 * m * (n // 128)
    return base + 2 * m * n


def kernel_pass(cfg, w, T, reps=5):
    """Counter-collection workload: each FP8 GEMM launch of the step (layer 0's
    weights) ``reps`` times, then a 256 MiB bf16 scale-by-one (read 256 MiB,
    write 256 MiB) as the copy kernel that calibrates FETCH_SIZE / WRITE_SIZE.
    Prints the launch manifest (shape, launches per step, algorithmic bytes,
    reps) as one JSON line for ``rocprof_summary traffic``."""
    lw = w.layers[0]
    manifest = []
    for role, m, count in gemm_launches(cfg, T):
        n, k = getattr(lw, role).weight.shape
        manifest.append(dict(shape=f"{role} {m}x{k}x{n}", launches_per_step=count,
                             algorithmic_bytes=algorithmic_bytes(cfg, role, m, n, k, T), reps=reps))
    for role, m, _ in gemm_launches(cfg, T):
        op = getattr(lw, role)
        n, k = op.weight.shape
        q, s = op.quantize(torch.randn(T, k, device="cuda").to(torch.bfloat16))
        b = gemm_buffers(cfg, role, n, m, T)
        for _ in range(reps):
            launch_gemm(cfg, role, lw, q, s, m, b)
        torch.cuda.synchronize()
        log(f"gemm {role} {m}x{k}x{n} x{reps}")
    x = torch.ones(128 << 20, device="cuda", dtype=torch.bfloat16)
    for _ in range(reps):
        y = x * 1.0
    torch.cuda.synchronize()
    del x, y
    log("copy 256 MiB done")
    print(json.dumps(dict(gemm_launches=manifest, copy_bytes=256 << 20, copy_reps=reps)))


def micro_gemms():
    """The FP8 linear microbench shapes (M,K,N) through ``FP8Linear.gemm``, the
    path of every caller (the packed tile kernels, k split where the tiles do not
    fill the GPU): TFLOP/s of one launch with weights streamed from HBM (eight
    weights in rotation, 2 x the 256 MB last-level cache at the largest shape),
    and the fraction of the roofline min(fp8 peak, AI x HBM bandwidth), AI = FLOP
    over the algorithmic bytes (bf16 activations in, e4m3 weights, fp32 scales,
    bf16 out)."""
    from fastforward_amd.linear import FP8Linear
    out = {}
    for m, k, n in MICRO_SHAPES:
        rot = max(8, -(-2 * 256 * 2 ** 20 // (n * k)))
        ops = []
        for j in range(rot):
            w = (torch.randn(n, k, device="cuda") * 0.02).to(torch.bfloat16)
            ops.append(types.SimpleNamespace(micro=FP8Linear(w)))
            del w
        x = torch.randn(m, k, device="cuda")
        x[torch.rand(m, k, device="cuda") < 0.001] *= 20          # 0.1 % outliers at x20
        x = x.to(torch.bfloat16)
        q, s = ops[0].micro.quantize(x)
        ms = time_gemm(None, "micro", q, s, ops, m, m, reps=5)
        # the whole linear call (per-token quantisation launch + GEMM), bf16 in / out
        for o in ops:
            o.micro(x)
        torch.cuda.synchronize()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            for o in ops:
                o.micro(x)
        e.record()
        torch.cuda.synchronize()
        ms_call = a.elapsed_time(e) / (5 * len(ops))
        flop = 2.0 * m * n * k
        byt = 2 * m * k + n * k + 4 * (m + n) + 2 * m * n
        roof = min(PEAK_FP8_TFLOPS, flop / byt * PEAK_HBM_GBS / 1e3)   # TFLOP/s
        tf = flop / ms / 1e9
        out[f"{m}x{k}x{n}"] = dict(us=round(ms * 1e3, 2), tflops=round(tf, 1),
                                   frac_fp8_peak=round(tf / PEAK_FP8_TFLOPS, 4),
                                   roofline_tflops=round(roof, 1), frac_roofline=round(tf / roof, 4),
                                   gbs=round(byt / ms / 1e6, 1), weights_rotated=rot,
                                   us_linear_call=round(ms_call * 1e3, 2))
        del ops
    torch.cuda.empty_cache()
    return out


def vision_flop(vc, n):
    """Algorithmic FLOPs of one vision step over n patches (unpadded widths)."""
    H, I, W4 = vc.hidden, vc.inter, vc.hidden * vc.merge ** 2
    nm = n // vc.merge ** 2
    block = 2 * n * H * (3 * H + H + 2 * I) + 4 * n * n * H
    merger = 2 * nm * W4 * (W4 + vc.out_hidden)
    return 2 * n * 1536 * H + vc.depth * block + (len(vc.deepstack) + 1) * merger


def vision_extras(cfg, w, T, grid, args):
    """The vision tower of the same model size on the step's image (merged grid
    16 x 32 = 2048 patches of 16 x 16 pixels), one hipGraph replay per step,
    and the image + prompt step (vision tower, then the LM step with the image
    tokens scattered in and DeepStack in the first layers) as one graph."""
    from fastforward_amd.pipeline import ImageStep
    from fastforward_amd.synthetic import make_request
    from fastforward_amd.vision import VISION_PRESETS, VisionRuntime, make_vision
    vc = VISION_PRESETS[cfg.name]
    gh, gw = 2 * grid[0], 2 * grid[1]
    vw = make_vision(vc, seed=0)
    rgb = torch.randint(0, 256, (16 * gh, 16 * gw, 3), generator=torch.Generator().manual_seed(0),
                        dtype=torch.uint8)
    vr = VisionRuntime(vc, vw, gh, gw)
    vr.set_image(rgb)
    vr.capture()
    ms = time_graph(vr, args.steps, args.warmup)
    flop = vision_flop(vc, gh * gw)
    tag = f"vision_{cfg.name.split('-')[-1]}_{gh * gw}patch"
    out = {f"{tag}_step_ms": round(ms, 4), f"{tag}_tflops": round(flop / ms / 1e9, 1)}
    log(f"vision step {ms:.3f} ms ({out[tag + '_tflops']} TFLOP/s algorithmic)")
    del vr
    ids, pos, pick = make_request(cfg, T, *grid, seed=0)
    st = ImageStep(cfg, w, vc, vw, gh, gw, T, image_start=4)
    st.set_inputs(rgb, ids, pos, pick)
    st.capture()
    key = f"image_step_{cfg.name.split('-')[-1]}_{T}_ms"
    out[key] = round(time_graph(st, args.steps, args.warmup), 4)
    log(f"image + prompt step {out[key]} ms")
    del st, vw
    torch.cuda.empty_cache()
    return out


def production_extras(cfg, mode, args):
    """The reference's deployed request geometry, as context for its published
    end-to-end latencies (which add image decode and host work): an aspect320
    canvas of 320 x 320 pixels (20 x 20 patches -> 100 image tokens), the
    minimal prompt with a four-option question (the prefix puts the image at
    token 4; about 70 suffix tokens), in the smallest 16-token bucket that holds
    it, 176 tokens (configs/8B.json buckets, variant aspect320, prompt_style
    minimal). One hipGraph replay of the vision tower + the LM step per step."""
    from fastforward_amd.pipeline import ImageStep
    from fastforward_amd.runtime import mrope_positions
    from fastforward_amd.synthetic import make_model
    from fastforward_amd.vision import VISION_PRESETS, make_vision
    vc = VISION_PRESETS[cfg.name]
    gh = gw = 20
    tokens, start, real = 176, 4, 175
    w = make_model(cfg, mode=mode, seed=0, n_options=4)
    vw = make_vision(vc, seed=0)
    g = torch.Generator().manual_seed(0)
    rgb = torch.randint(0, 256, (16 * gh, 16 * gw, 3), generator=g, dtype=torch.uint8)
    ids = torch.randint(0, cfg.vocab, (real,), generator=g, dtype=torch.int64)
    pos = torch.from_numpy(mrope_positions(start, gh // 2, gw // 2, tokens))
    st = ImageStep(cfg, w, vc, vw, gh, gw, tokens, image_start=start)
    st.set_inputs(rgb, ids, pos, real - 1)
    st.capture()
    ms = time_graph(st, args.steps, args.warmup)
    del st, w, vw
    torch.cuda.empty_cache()
    return round(ms, 4)


def cpu_baseline(cfg, w, ids, pos, pick, T, layers_sample):
    """The CPU oracle on ``layers_sample`` decoder layers + the pick-only tail of the
    same step, on this host's cores; scaled to the full depth."""
    from oracle import model as omodel
    from oracle import ops as O
    from tests.helpers import linear_to_oracle
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    shape = omodel.Shape(layers=cfg.layers, hidden=cfg.hidden, heads=cfg.heads, kv_heads=cfg.kv_heads,
                         head_dim=cfg.head_dim, inter=cfg.inter, vocab=cfg.vocab)
    keep = list(range(layers_sample)) + [cfg.layers - 1]
    L = {}
    for j in keep:
        lw = w.layers[j]
        L[j] = omodel.Layer(input_norm=lw.input_norm.weight.cpu(), post_norm=lw.post_norm.weight.cpu(),
                            q_norm=lw.q_norm.weight.cpu(), k_norm=lw.k_norm.weight.cpu(),
                            qkv=linear_to_oracle(lw.qkv), o=linear_to_oracle(lw.o),
                            gateup=linear_to_oracle(lw.gateup), down=linear_to_oracle(lw.down))
    ow = omodel.Weights(embed=None, layers=[], norm=w.norm.weight.cpu(), head=w.head.cpu())
    h = w.embed[torch.as_tensor(ids).cuda()].cpu()[None]
    t0 = time.perf_counter()
    cos, sin = O.mrope_cos_sin(pos, shape.theta, shape.head_dim, shape.sections)
    x = O.fast_norm(h, L[0].input_norm, shape.eps)
    for j in range(layers_sample):
        attn = omodel.attention_block(shape, L[j], x, cos, sin)
        res, post = O.add_rms(h, attn, None, L[j].post_norm, shape.eps)
        val = omodel.mlp(L[j], post)
        nxt = L[j + 1] if j + 1 < layers_sample else L[cfg.layers - 1]
        h, x = O.add_rms(res, val, None, nxt.input_norm, shape.eps)
    t1 = time.perf_counter()
    omodel.tail(shape, L[cfg.layers - 1], ow, h, cos, sin, pick)
    t2 = time.perf_counter()
    per_layer = (t1 - t0) / layers_sample
    full_ms = (per_layer * (cfg.layers - 1) + (t2 - t1)) * 1e3
    return dict(value=round(full_ms, 1), unit="ms per step (scaled)", cores=torch.get_num_threads(),
                kind="port",
                sample=f"{layers_sample} of {cfg.layers - 1} full decoder layers + the pick-only tail of the "
                       f"same 8B-shape FP8 {T}-token step, timed on the host with the oracle "
                       f"(torch CPU, fp32 with e4m3/bf16 rounding points), scaled to the full depth; "
                       f"sample wall time {t2 - t0:.1f} s")


def cpu_layer_2b(reps=5, warmup=2):
    """The CPU reference configuration: one Qwen3-VL-2B-shaped decoder layer
    (hidden 2048, 16/8 heads, head_dim 128, MLP 6144, q/k eps 1e-6, rope theta
    5e6, M-RoPE [24, 20, 20]) over 320 tokens (4 text + 16 x 16 image grid + 60
    text), causal, batch 1, through the oracle's restatement of the reference's
    op sequence with unquantised linears: fp32 arithmetic with the reference's
    bf16 rounding points, weights N(0, 0.02) and hidden states N(0, 1) (seeded).
    Median of ``reps`` runs after ``warmup``, on every core of this host."""
    from oracle import model as omodel
    from oracle import ops as O
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    H, HQ, HK, D, I, T = 2048, 16, 8, 128, 6144, 320
    g = torch.Generator().manual_seed(0)
    lin = lambda rows, cols: dict(kind="bf16", w=(torch.randn(rows, cols, generator=g) * 0.02).to(torch.bfloat16))  # noqa: E731
    shape = omodel.Shape(layers=2, hidden=H, heads=HQ, kv_heads=HK, head_dim=D, inter=I, vocab=151936)
    one = torch.ones(H, dtype=torch.bfloat16)
    layer = omodel.Layer(input_norm=one, post_norm=one, q_norm=torch.ones(D, dtype=torch.bfloat16),
                         k_norm=torch.ones(D, dtype=torch.bfloat16), qkv=lin((HQ + 2 * HK) * D, H),
                         o=lin(H, HQ * D), gateup=lin(2 * I, H), down=lin(H, I))
    h = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    pos = O.mrope_positions(4, 16, 16, T)
    times = []
    for i in range(warmup + reps):
        t0 = time.perf_counter()
        cos, sin = O.mrope_cos_sin(pos, shape.theta, D, shape.sections)
        x = O.fast_norm(h, layer.input_norm, shape.eps)
        attn = omodel.attention_block(shape, layer, x, cos, sin)
        res, post = O.add_rms(h, attn, None, layer.post_norm, shape.eps)
        out = O.add_rms(res, omodel.mlp(layer, post), None, layer.input_norm, shape.eps)
        times.append(time.perf_counter() - t0)
        del out
    ms = sorted(times[warmup:])[reps // 2] * 1e3
    flop = 2.0 * T * H * ((HQ + 2 * HK) * D + HQ * D + 3 * I) + 4.0 * HQ * D * T * (T + 1) / 2
    return dict(value=round(ms, 2), unit="ms per decoder layer", gflops=round(flop / ms / 1e6, 1), cores=n,
                kind="port", workload="one Qwen3-VL-2B-shaped decoder layer, 320 tokens (16x16 image grid + "
                                      "64 text), causal, oracle op formulation in fp32 with bf16 rounding points, "
                                      f"median of {reps} after {warmup} warm-ups")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--preset", default="qwen3vl-8b")
    ap.add_argument("--tokens", type=int, default=576)
    ap.add_argument("--cpu-layers", type=int, default=35, help="decoder layers in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the GEMM microbench and the W4A16 / 2B / 32B steps")
    ap.add_argument("--profile", action="store_true", help="only replay the graph (for rocprofv3 runs)")
    ap.add_argument("--linear", default="fp8", choices=("fp8", "fp8_static", "w4a16"),
                    help="linear format of the --profile step (the benchmark line is always FP8)")
    ap.add_argument("--vision", action="store_true",
                    help="with --profile: replay the vision tower's graph instead of the LM step")
    ap.add_argument("--kernels", action="store_true",
                    help="only run the step's GEMM shapes and a calibration copy (rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the step runs on a single MI355X and has no multi-GPU "
              "path (independent request-level replicas would scale it)", file=sys.stderr)
        sys.exit(2)

    from fastforward_amd import _lib
    from fastforward_amd.runtime import PRESETS, Runtime
    from fastforward_amd.synthetic import make_model, make_request
    _lib.check_device()
    cfg = PRESETS[args.preset]
    T = args.tokens
    # the image's merged grid: 16 x 32 at 576 tokens, 16 x 16 from 320, else the aspect320
    # canvas's 10 x 10 (the 176-token bucket of the deployed geometry)
    grid = (16, 32) if T >= 576 else (16, 16) if T >= 320 else (10, 10)
    if args.profile and args.vision:
        from fastforward_amd.vision import VISION_PRESETS, VisionRuntime, make_vision
        vc = VISION_PRESETS[cfg.name]
        gh, gw = 2 * grid[0], 2 * grid[1]
        vr = VisionRuntime(vc, make_vision(vc, seed=0), gh, gw)
        vr.set_image(torch.randint(0, 256, (16 * gh, 16 * gw, 3), generator=torch.Generator().manual_seed(0),
                                   dtype=torch.uint8))
        vr.capture()
        ms = time_graph(vr, args.steps, args.warmup)
        log(f"vision step {ms:.3f} ms")
        print(json.dumps(dict(metric=f"ms per vision step ({vc.name} tower, {gh * gw} patches)", value=round(ms, 4),
                              unit="ms", profile_run=True)))
        return
    log(f"building {cfg.name} fp8 (random init, seed 0)")
    w = make_model(cfg, mode=args.linear if args.profile else "fp8", seed=0, n_options=8)
    for L in w.layers:  # as Runtime does: the packed tile kernels read these copies
        for op in (L.qkv, L.o, L.gateup, L.down):
            if hasattr(op, "pack"):
                op.pack()
    ids, pos, pick = make_request(cfg, T, *grid, seed=0)
    if args.kernels:
        kernel_pass(cfg, w, T)
        return
    rt = Runtime(cfg, w, T)
    rt.set_inputs(ids, pos, pick)
    rt.capture()
    torch.cuda.synchronize()
    log("graph captured")
    ms = time_graph(rt, args.steps, args.warmup)
    log(f"step {ms:.3f} ms")
    if args.profile:
        print(json.dumps(dict(metric=METRIC, value=round(ms, 4), unit="ms", profile_run=True)))
        return
    roof = gemm_roofline(cfg, w, T)
    log(f"gate/up gemm {roof['achieved']} TFLOP/s ({roof['frac']:.3f} of fp8 peak); all fp8 gemms "
        f"{roof['all_fp8_gemm']['achieved']} TFLOP/s ({roof['all_fp8_gemm']['frac']:.3f})")
    extras = {}
    if not args.no_extras:
        extras["gemm_fp8_microbench"] = micro_gemms()
        log("microbench done")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline(cfg, w, ids, pos, pick, T, args.cpu_layers)
        cpu["layer_2b_320_fp32"] = cpu_layer_2b()
        log(f"cpu 2B layer {cpu['layer_2b_320_fp32']['value']} ms")
    del rt
    if not args.no_extras:
        extras.update(vision_extras(cfg, w, T, grid, args))
        del w
        torch.cuda.empty_cache()
        # the other LM configurations, each one hipGraph replay per step
        for mode in ("fp8_static", "fp8"):
            key = f"image_step_8b_aspect320_100img_176tok_{mode}_ms"
            extras[key] = production_extras(cfg, mode, args)
            log(f"{key} {extras[key]}")
        for key, preset, mode, tokens, gx, n_opt in (
                ("fp8_8b_176_lm_step_ms", args.preset, "fp8", 176, (10, 10), 8),
                ("fp8_static_8b_576_step_ms", args.preset, "fp8_static", T, grid, 8),
                ("w4a16_g128_8b_576_step_ms", args.preset, "w4a16", T, grid, 8),
                ("fp8_2b_320_step_ms", "qwen3vl-2b", "fp8", 320, (16, 16), 4),
                ("fp8_32b_1024_step_ms", "qwen3vl-32b", "fp8", 1024, (30, 32), 2)):
            c = PRESETS[preset]
            wx = make_model(c, mode=mode, seed=0, n_options=n_opt)
            ix, px, kx = make_request(c, tokens, *gx, seed=0)
            rx = Runtime(c, wx, tokens)
            rx.set_inputs(ix, px, kx)
            rx.capture()
            extras[key] = round(time_graph(rx, args.steps, args.warmup), 4)
            log(f"{key} {extras[key]}")
            del rx, wx
            torch.cuda.empty_cache()
    line = dict(
        metric=METRIC, value=round(ms, 4), unit="ms", n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 4), higher_is_better=False, scaling="weak", vs_baseline=None,
        dtype="fp8_e4m3 GEMM (MFMA: ~13-bit sums per 32-product block, fp32 across blocks) / bf16",
        data="synthetic: random-init N(0,0.02) weights, seeded uniform token ids, no checkpoint",
        config=dict(workload=f"{cfg.name} FP8 prefill + choice-score step, hipGraph replay",
                    layers=cfg.layers, hidden=cfg.hidden, heads=f"{cfg.heads}/{cfg.kv_heads}",
                    mlp=cfg.inter, vocab=cfg.vocab, tokens=T, image_grid=f"{grid[0]}x{grid[1]}", choices=8,
                    linear="e4m3 per-token activation / per-channel weight scales"),
        roofline=roof, cpu_baseline=cpu, **extras)
    print(json.dumps(line))


if __name__ == "__main__":
    main()

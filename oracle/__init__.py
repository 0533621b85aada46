"""CPU oracle for the Qwen3-VL language-model prefill + choice-score step.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU with PyTorch, the
arithmetic of FastForward's quantized LM step (the reference's Triton kernels
and its PyTorch formulation of them), with every bf16 / e4m3 rounding point
kept. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg
of ``bench.py`` may import it, and only as the checker (or the timed CPU
baseline): the product package ``fastforward_amd`` never imports it and has no
CPU fallback.

Every function cites the reference file:line it restates (paths relative to
``src/fastforward_accel/`` of the reference). How each function is pinned
(independent numpy / brute-force / closed-form / third-party checks) is listed
in ``oracle.PINNING``; ``tests/test_oracle_pins.py`` runs those checks.
"""
from . import ops, model, vision  # noqa: F401

# function -> the independent checks in tests/test_oracle_pins.py that pin it.
PINNING = {
    "bf16": "numpy RNE bit arithmetic on all exponents (test_bf16_rounding_matches_bit_rne)",
    "e4m3": "exhaustive nearest-of-256-codes search, ties to even (test_e4m3_cast_exhaustive)",
    "fast_norm": "fp64 numpy closed form + HF Qwen3VLTextRMSNorm (test_rms_*)",
    "add_rms": "fp64 numpy closed form incl. DeepStack rows (test_add_rms_*)",
    "qk_pair": "HF apply_rotary_pos_emb + per-head RMSNorm; rotation isometry (test_qk_pair_*)",
    "swiglu": "fp64 numpy silu*u (test_swiglu_matches_fp64)",
    "attention_direct": "fp64 brute-force softmax loops, GQA + causal + selected (test_attention_*)",
    "lm_readout": "fp64 numpy norm + dot (test_lm_readout_matches_fp64)",
    "quant_rows_dynamic": "numpy per-row amax + exhaustive e4m3 (test_fp8_dynamic_*)",
    "quant_static": "numpy multiply + exhaustive e4m3 (test_fp8_static_*)",
    "fp8_weight_quant": "numpy per-channel / per-tensor amax (test_fp8_weight_*)",
    "fp8_linear": "fp64 numpy GEMM of decoded codes x scales (test_fp8_linear_matches_fp64)",
    "fp8_gemm_exact": "pure-Python integer sums of the decoded codes (test_fp8_gemm_exact_and_blocks_brute_force)",
    "fp8_gemm_blocks / round_sig_": "pure-Python brute force of the block model on small GEMMs (exact block sums as "
                                    "Fractions, math.frexp rounding, float32 accumulation); rounding of ties, "
                                    "signs and binade carries against math.frexp (test_round_sig_*)",
    "int4_quantize": "pure-Python loops on tiny matrices: nibble order, [K/g,N,2] indexing (test_int4_*)",
    "w4a16_linear": "fp64 numpy dequant GEMM (test_w4a16_linear_matches_fp64)",
    "mrope_positions": "transformers Qwen3-VL get_rope_index (test_mrope_positions_match_hf)",
    "mrope_cos_sin": "transformers Qwen3VLTextRotaryEmbedding (test_mrope_cos_sin_match_hf)",
    "choice": "reference contract tests: ties -> lowest index, probabilities sum to 1",
    "model.step": "unquantized layer stack vs transformers Qwen3VLTextModel (test_model_matches_hf_text_model)",
    "vision.pack_pixels": "transformers Qwen2-VL PIL image processor, bit-exact; division-rounding stability "
                          "(tests/test_oracle_vision_pins.py)",
    "vision.rot_pos_freqs / pos_interp / pos_embeds": "transformers rot_pos_emb, "
                          "get_vision_interpolation_indices_and_weights, fast_pos_embed_interpolate, bit-exact",
    "vision.vision_rope": "transformers apply_rotary_pos_emb_vision, bit-exact",
    "vision.layer_norm": "torch layer_norm (bf16) and fp64 closed form, <= 1 ulp",
    "vision.gelu_tanh / gelu_erf": "fp64 closed forms within 1 ulp + fp32 cancellation",
    "vision.attention": "pure-Python softmax loops (fp64)",
    "vision.tower": "transformers Qwen3VLVisionModel (bf16, CPU) end to end, rel L2 <= 1%",
}

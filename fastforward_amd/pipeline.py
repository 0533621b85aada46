"""Image + prompt step: the vision tower followed by the LM prefill +
choice-score step, as one hipGraph.

Restates the request path of the reference's runtime with its image branch
(``core_joint``: vision(rgb) -> ``h[0].index_copy_(0, vi, visual)`` -> the
layer loop with DeepStack, _family/depth_runtime.py; the vision graph and the
LM graph of ``VisionGraph.build`` and ``Runtime.graph``). The vision step
writes its merged image tokens and DeepStack features straight into the LM
runtime's static ``visual`` / ``deep`` buffers, so nothing is copied between
the two.
"""
import torch

from .runtime import Runtime
from .vision import VisionRuntime


class ImageStep:
    """One image geometry (a (gh, gw) patch grid) and one token bucket.

    The image occupies rows [image_start, image_start + gh*gw/4) of the
    prompt; DeepStack features go to the first len(deepstack) LM layers.
    ``arena`` / ``vision_arena``: ``runtime.Arena`` regions shared with the
    model's other steps for the LM / vision tower activations (steps that
    share them must not overlap in time).
    """

    def __init__(self, lm_cfg, lm_weights, vis_cfg, vis_weights, gh, gw, tokens, image_start, path=None, arena=None,
                 vision_arena=None):
        nm = gh * gw // vis_cfg.merge ** 2
        if vis_cfg.out_hidden != lm_cfg.hidden:
            raise ValueError("the vision tower's output width must be the LM's hidden size")
        self.lm = Runtime(lm_cfg, lm_weights, tokens, path=path, visual_rows=nm, image_start=image_start,
                          deep_layers=len(vis_cfg.deepstack), arena=arena)
        self.vision = VisionRuntime(vis_cfg, vis_weights, gh, gw, merged=self.lm.visual, deep=self.lm.deep,
                                    arena=vision_arena)
        self.graph = None
        self.graph_out = None

    def set_inputs(self, rgb, ids, pos, pick):
        self.vision.set_image(rgb)
        self.lm.set_inputs(ids, pos, pick)

    def step(self):
        """Vision tower, then the LM step, eagerly on the current stream; returns the logits."""
        self.vision.step()
        return self.lm.step()

    def capture(self, warmup=2):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self.step()
        self.graph, self.graph_out = g, out
        return g

    def replay(self):
        if self.graph is None:
            self.capture()
        self.graph.replay()
        return self.graph_out

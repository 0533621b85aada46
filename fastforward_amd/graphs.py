"""Bucketed hipGraph execution with the reference's graph-input contract.

Reference: ``Runtime.graph`` (_family/night_runtime.py:106-125) and the
per-bucket position templates of ``setup_side`` (_family/depth_runtime.py:
35-52); the request gate of _legacy/sub10_runtime.py:154-167.

* A request of n tokens runs in the smallest configured bucket >= n; ids are
  zero-padded to the bucket.
* Each bucket is one ``Runtime`` whose step is captured once (after warm-up
  runs) on its first request; later requests only refill the static inputs.
  The buckets' activation buffers alias one ``Arena`` that holds the largest
  of their layouts (requests run one at a time).
* The M-RoPE positions of a bucket are a template computed once for the
  bundle's layout (prefix text, one image grid, text after it) and stay
  resident; only token ids and the scored row change per request.
* Inputs go host -> pinned staging -> device with an asynchronous copy on the
  step's stream; an event recorded after the copy guards the reuse of the
  pinned buffers by the next request (only the preceding copy must finish
  before the host writes them again).
"""
import threading

import numpy as np
import torch

from .runtime import Arena, Runtime, mrope_positions


class StepGraphs:
    """Token buckets of one model and one image layout, each a captured step."""

    def __init__(self, cfg, weights, buckets, grid, prefix_tokens, warmup=3):
        self.cfg, self.w = cfg, weights
        self.buckets = sorted({int(b) for b in buckets})
        self.grid = (int(grid[0]), int(grid[1]))
        self.prefix_tokens = int(prefix_tokens)
        self.min_tokens = self.prefix_tokens + self.grid[0] * self.grid[1]
        if not self.buckets or self.buckets[0] < self.min_tokens:
            raise ValueError(f"every bucket must hold the {self.min_tokens}-token prompt prefix and image")
        self.warmup = warmup
        self.arena = None   # one activation region for every bucket's runtime (made at the first capture)
        self.cache = {}     # bucket -> captured Runtime
        self.staging = {}   # bucket -> (pinned ids (bucket,), pinned pick (1,), event)
        # the buckets share one arena and one set of static inputs per bucket, so
        # requests are serialised; callers reading the returned logits view hold it
        self.lock = threading.RLock()

    def select(self, bounds):
        """Apply a calibration profile ({"j:role": bound}) to the static FP8
        linears and drop the captured graphs: the activation multiplier is a
        kernel argument recorded at capture, so each bucket re-captures on its
        next request (the reference selects before it captures)."""
        from .profiles import apply_profile
        with self.lock:
            torch.cuda.synchronize()
            apply_profile(self.w, bounds)
            self.cache.clear()
            self.staging.clear()

    def bucket_for(self, n):
        b = next((b for b in self.buckets if b >= n), None)
        if b is None:
            raise ValueError(f"{n} tokens exceed the largest bucket ({self.buckets[-1]})")
        return b

    def positions(self, bucket):
        """(3, bucket) int64 position template of a bucket (host tensor)."""
        return torch.from_numpy(mrope_positions(self.prefix_tokens, *self.grid, bucket))

    def _check(self, ids, pick, k):
        ids = torch.as_tensor(ids, dtype=torch.int64).reshape(-1)
        n = ids.numel()
        if n < self.min_tokens:
            raise ValueError(f"expected at least {self.min_tokens} token ids, got {n}")
        if int(ids.min()) < 0 or int(ids.max()) >= self.cfg.vocab:
            raise ValueError("token id outside the vocabulary")
        if not 0 <= int(pick) < n:
            raise ValueError("pick must index a real token")
        if not 1 <= int(k) <= self.w.head.shape[0]:
            raise ValueError(f"k must be 1..{self.w.head.shape[0]}")
        return ids, n

    def run(self, ids, pick, k):
        """Logits of the first ``k`` options (fp32 device tensor, a view of the
        bucket's static output: valid until the next request, so a caller on
        another thread reads it under ``lock``) and whether this call captured
        the bucket's graph."""
        with self.lock:
            return self._run(ids, pick, k)

    def _run(self, ids, pick, k):
        ids, n = self._check(ids, pick, k)
        b = self.bucket_for(n)
        captured = b not in self.cache
        if captured:
            if self.arena is None:     # sized so that every bucket's layout fits
                self.arena = Arena(Arena.size_for_buckets(self.cfg, self.buckets, Runtime.path_for(self.w)),
                                   self.w.embed.device)
            rt = Runtime(self.cfg, self.w, b, arena=self.arena)
            rt.set_inputs(ids, self.positions(b), int(pick))
            rt.capture(warmup=self.warmup)
            self.cache[b] = rt
            ev = torch.cuda.Event()
            ev.record()
            self.staging[b] = (torch.zeros(b, dtype=torch.int64, pin_memory=True),
                               torch.zeros(1, dtype=torch.int64, pin_memory=True), ev)
        rt = self.cache[b]
        sid, spick, ev = self.staging[b]
        ev.synchronize()  # the previous copy out of these pinned buffers has finished
        sid.zero_()
        sid[:n].copy_(ids)
        spick[0] = int(pick)
        rt.ids.copy_(sid, non_blocking=True)
        rt.pick.copy_(spick, non_blocking=True)
        ev.record()
        z = rt.replay()
        return z[:k], captured

    def gate(self, ids, pick, k, pad_id=42):
        """The reference's request gate for this layout: the bucket's position
        template equals the prompt's own positions on its real tokens; the graph
        replay equals an eager step of the same bucket (here bit for bit, since
        both run the same kernels); and padding ids cannot reach the answer (an
        eager step with every padding id set to ``pad_id`` gives the same bits).
        Raises AssertionError on a violation."""
        ids, n = self._check(ids, pick, k)
        b = self.bucket_for(n)
        template = self.positions(b).numpy()
        own = mrope_positions(self.prefix_tokens, *self.grid, n)
        assert np.array_equal(own, template[:, :n]), "Position template differs from actual prompt"
        actual = self.run(ids, pick, k)[0].float().cpu()
        eager = Runtime(self.cfg, self.w, b)
        eager.set_inputs(ids, self.positions(b), int(pick))
        native = eager.step()[:k].float().cpu()
        assert torch.equal(native, actual), ("native_graph", native.tolist(), actual.tolist())
        padded = torch.full((b,), pad_id, dtype=torch.int64)
        padded[:n] = ids
        eager.ids.copy_(padded.to(eager.ids.device))
        perturbed = eager.step()[:k].float().cpu()
        assert torch.equal(perturbed, actual), "Padding tokens leak into real answer"
        return dict(passed=True, positions_exact=True, padding_isolated=True, bucket=b,
                    native=native.tolist(), actual=actual.tolist())

"""Recording one fixed training step into a HIP graph and replaying it
(numrs_hip_graph_*; numrs has no counterpart: its training loop,
autograd/train.rs:159-183, runs every op of every step one by one).

    g = StepGraph(ctx, step)   # step() is recorded, not run
    for batch in batches:
        x_dev.upload(batch)      # new data into the recorded input buffers
        g.replay()               # one launch: the whole step
        loss = g.outputs.item()

Run `step()` once eagerly before recording it, so that every buffer it needs
already exists.  Replays reuse the kernel arguments of the recording, so
host-side values that change per step (a scheduler's learning rate, Adam's
step count) stay as recorded; the engine refuses to record optimizers whose
step depends on a host-side step count.  The graph keeps `step` and what it
returned alive, and with them every tensor the recorded kernels address.
"""
from __future__ import annotations

import ctypes

from . import _lib as L


class StepGraph:
    def __init__(self, ctx, step):
        lib = L.load()
        ctx._check(lib.numrs_hip_graph_begin(ctx.handle))
        try:
            outputs = step()
        except BaseException:
            lib.numrs_hip_graph_abort(ctx.handle)
            raise
        handle = ctypes.c_void_p()
        ctx._check(lib.numrs_hip_graph_end(ctx.handle, ctypes.byref(handle)))
        self.ctx = ctx
        self.outputs = outputs
        self._step = step
        self._handle = handle

    def replay(self) -> None:
        """Queues one replay of the recorded step on the context's stream."""
        if not self._handle:
            raise RuntimeError("graph already closed")
        self.ctx._check(L.load().numrs_hip_graph_launch(self._handle))

    def close(self) -> None:
        if self._handle:
            self.ctx._check(L.load().numrs_hip_graph_destroy(self._handle))
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

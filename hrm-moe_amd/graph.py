"""HIP-graph replay of the MoE FFN forward for a fixed token count.

At decode sizes (a few to a few hundred tokens per step) the layer's GPU work
is a few microseconds of weight streaming, while the host spends far longer
checking arguments, allocating outputs and enqueuing eight kernels.  Capturing
the no-autograd forward once and replaying it takes all of that host work out
of the step.  This is the serving counterpart of the reference's batched decode
loop (inference/simple_inference_engine.py), which calls the module eagerly.

Every kernel of the forward takes its sizes from arguments fixed at capture
and reads tokens_per_expert on the device, so a replay recomputes routing,
dispatch and the expert GEMMs for whatever the static input holds.  None of
them records a memset.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .layers import SparseMoESwiGLU


class GraphedMoEForward:
    """Replays ``layer(x)`` (no autograd) from a HIP graph captured for ``example``'s shape and dtype.

    The call copies ``x`` into the captured input buffer ``static_in``,
    replays the graph and returns the captured output buffer: the next call
    overwrites it, so keep a copy if the result must outlive that.  A caller
    that writes the step's tokens into ``static_in`` itself (e.g. as the
    output buffer of the op before) passes ``static_in`` and skips the copy,
    one kernel launch per step.  The graph holds the
    addresses of the layer's parameters; in-place updates of them are seen by
    later replays, replaced parameter tensors are not (capture again).
    """

    def __init__(self, layer: SparseMoESwiGLU, example: Tensor, warmup: int = 2):
        if not example.is_cuda:
            raise RuntimeError("GraphedMoEForward needs a ROCm GPU tensor; there is no CPU path")
        self.layer = layer
        self.static_in = example.detach().clone()
        dev = example.device
        side = torch.cuda.Stream(device=dev)  # default priority
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                layer(self.static_in)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.static_out = layer(self.static_in)

    def __call__(self, x: Tensor) -> Tensor:
        if x.shape != self.static_in.shape or x.dtype != self.static_in.dtype or x.device != self.static_in.device:
            raise ValueError(f"graph captured for {tuple(self.static_in.shape)} {self.static_in.dtype} on "
                             f"{self.static_in.device}, got {tuple(x.shape)} {x.dtype} on {x.device}")
        if x.data_ptr() != self.static_in.data_ptr():
            self.static_in.copy_(x)
        self.graph.replay()
        return self.static_out

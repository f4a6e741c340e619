"""Graph capture of trunk passes: one hipGraph replays a whole pass (or several) of kernels.

The counterpart of the reference's trunk graphs (``src/foldforge/models/execution.py:196-259``
wraps a callable after two warm-up calls on a side stream, captures it once and replays it
with new inputs copied into the captured buffers; the trunk sites are registered at
``execution.py:543-555``). At 128 tokens an eager trunk pass issues ~850 kernels for ~10 ms of
GPU work and is bound by the host (``docs/guides/EXECUTION-SCOPES.md:38-43``); replaying the
captured graph removes the per-launch host work.

Every op of the pair stack and the single track can be captured as it is: the ``hip`` ops
validate shapes on the host only, allocate their workspace from torch's allocator (the
graph's private pool during capture), launch on torch's current stream and use no memset or
host synchronisation. Inputs and outputs of a replay are the captured (static) buffers.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
from typing import Any

import torch

Tensor = torch.Tensor


class CapturedCall:
    """``fn(*tensors, **kwargs)`` captured once as a graph.

    ``__call__(*tensors)`` copies the new inputs into the captured input buffers (same shapes,
    dtypes and device) and replays the graph; it returns the captured output buffers, which
    the next replay overwrites (clone them to keep a result). ``kwargs`` are fixed at capture
    time (e.g. the number of passes). Two warm-up calls run on a side stream first, as the
    reference does, so that one-time work (library loading, allocator growth) stays out of
    the graph.
    """

    def __init__(self, fn: Callable[..., Any], tensors: Sequence[Tensor], *, warmup: int = 2,
                 **kwargs: Any) -> None:
        if not tensors or any(not isinstance(t, Tensor) or not t.is_cuda for t in tensors):
            raise ValueError("graph inputs must be device tensors")
        self.fn, self.kwargs = fn, kwargs
        self.inputs = tuple(t.detach().clone() for t in tensors)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(warmup):
                fn(*self.inputs, **kwargs)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.output = fn(*self.inputs, **kwargs)
        torch.cuda.synchronize()

    def __call__(self, *tensors: Tensor) -> Any:
        if len(tensors) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs, got {len(tensors)}")
        for dst, src in zip(self.inputs, tensors):
            if src.shape != dst.shape or src.dtype != dst.dtype:
                raise ValueError(f"input {tuple(src.shape)} {src.dtype} does not match the "
                                 f"captured {tuple(dst.shape)} {dst.dtype}")
            if src.data_ptr() != dst.data_ptr():
                dst.copy_(src)
        self.graph.replay()
        return self.output


def capture_trunk(model: torch.nn.Module, pair: Tensor, key_mask: Tensor,
                  single: Tensor | None = None, *, passes: int = 1) -> CapturedCall:
    """A trunk (:class:`foldforge_amd.trunk.PairformerTrunk`) run of ``passes`` passes
    captured for inputs of these shapes; call the result with new ``(pair, key_mask[,
    single])``."""
    tensors = (pair, key_mask) if single is None else (pair, key_mask, single)
    return CapturedCall(model, tensors, passes=passes)

"""The Pairformer trunk: 48 blocks run in order for every pass, plus seeded random init.

Call site mirrored: ``Evoformer.trunk_pairformer`` and its loop
(``src/foldforge/models/architectures/af3.py:245-247,813-821`` of the reference); the
recycle embedding between passes is not part of the pair stack, so each pass feeds its
output pair / single straight into the next.
"""

from __future__ import annotations

import torch
from torch import nn

from foldforge_amd.factories import pairformer_block

Tensor = torch.Tensor


def randomise(model: nn.Module, seed: int, *, out_scale: float | None = None) -> nn.Module:
    """Seeded init in the convention of the reference's block tests
    (``tests/models/test_engine_graph.py:40-51``): matrices ``0.08 N(0,1)``, norm weights
    ``1 + 0.1 N(0,1)``, other vectors ``0.05 N(0,1)``. ``out_scale`` additionally
    multiplies every residual-feeding output matrix (``to_out``, ``squeeze``) so that a
    deep stack keeps a bounded residual stream."""
    generator = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            noise = torch.randn(p.shape, generator=generator)
            if p.ndim > 1:
                value = 0.08 * noise
                if out_scale is not None and (name.endswith("to_out.weight") or name.endswith("squeeze.weight")):
                    value = value * out_scale
            elif name.endswith("weight") or "scale" in name:
                value = 1.0 + 0.1 * noise
            else:
                value = 0.05 * noise
            p.copy_(value.to(p.dtype))
    return model


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """The second stream of a device's trunks (one per device and process, default priority)."""
    key = torch.cuda._utils._get_device_index(device)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device)
    return _SIDE_STREAMS[key]


class PairformerTrunk(nn.Module):
    """``n_blocks`` Pairformer blocks with a single track (AF3 trunk widths by default)."""

    overlap_single: bool = True  # run each block's single track beside the next block's pair track

    def __init__(self, n_blocks: int = 48, *, d_pair: int = 128, d_single: int = 384,
                 n_head_single: int = 16, triangle_model: str = "af3",
                 precision: str = "master") -> None:
        super().__init__()
        self.blocks = nn.ModuleList(
            pairformer_block(d_pair=d_pair, triangle_model=triangle_model, d_single=d_single,
                             n_head_single=n_head_single, precision=precision)  # type: ignore[arg-type]
            for _ in range(n_blocks)
        )

    def forward(self, pair: Tensor, key_mask: Tensor, single: Tensor | None = None,
                passes: int = 1, on_block=None):
        """``passes`` times over the blocks; ``on_block(pass, index, pair, single)`` observes each output.

        With a single track on the GPU, block b's single updates (which read only the single
        state and the pair around block b) run on a second stream beside block b + 1's pair
        updates (``overlap_single``, on by default; off while ``on_block`` observes the blocks).
        Every op runs as in the sequential order on the same inputs, so the results are the same
        bit for bit. Under graph capture the second stream joins the capture through the
        per-block events (a fork and a join per block in the graph)."""
        overlap = single is not None and self.overlap_single and on_block is None and pair.is_cuda
        if overlap:
            return self._forward_overlapped(pair, key_mask, single, passes)
        for p in range(passes):
            for i, block in enumerate(self.blocks):
                if single is None:
                    pair = block(pair, key_mask)
                else:
                    pair, single = block(pair, key_mask, single)
                if on_block is not None:
                    on_block(p, i, pair, single)
        return pair if single is None else (pair, single)

    def _forward_overlapped(self, pair: Tensor, key_mask: Tensor, single: Tensor, passes: int):
        main = torch.cuda.current_stream(pair.device)
        side = _side_stream(pair.device)
        # the single track starts from state the main stream produced
        side.wait_stream(main)
        for _ in range(passes):
            for block in self.blocks:
                pair_in = pair
                pair = block.pair_track(pair_in, key_mask)
                ready = torch.cuda.Event()
                ready.record(main)
                with torch.cuda.stream(side):
                    side.wait_event(ready)
                    single = block.single_track(single, pair_in, pair, key_mask)
                # the side stream reads these after the main stream has moved on: their memory
                # must not be handed to a later main-stream allocation before it is done
                pair_in.record_stream(side)
                pair.record_stream(side)
        key_mask.record_stream(side)
        main.wait_stream(side)
        single.record_stream(main)
        return pair, single

"""GPU: a captured trunk pass replays exactly what the eager pass computes, and that is the
oracle's result.

The graph is replayed several times with different inputs copied in, with eager work and
host synchronisations between the replays; every replay must equal the eager run on the same
inputs bitwise (the kernels are deterministic and take no state from earlier calls), and one
replay is compared with the fp64 oracle run through the same blocks and passes.
"""

from __future__ import annotations

import pytest
import torch

import foldforge_amd
from foldforge_amd.execution import capture_trunk
from oracle import pairstack as ps

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from foldforge_amd import _native

    _native.lib()


def _inputs(n: int, length: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(1, n, n, 128, generator=g).bfloat16().cuda()
    s = torch.randn(1, n, 384, generator=g).bfloat16().cuda()
    mask = torch.zeros(1, n, dtype=torch.bool)
    mask[0, :length] = True
    return z, mask.cuda(), s


def test_captured_trunk_pass_replays_the_eager_pass():
    n = 96
    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=2, seed=5, d_single=384,
                               unsupported="error")
    first = _inputs(n, 81, seed=1)
    graph = capture_trunk(model, *first, passes=2)
    for seed, length in ((2, 96), (3, 57), (1, 81)):
        z, mask, s = _inputs(n, length, seed)
        with torch.no_grad():
            want_z, want_s = model(z, mask, s, passes=2)
        torch.cuda.synchronize()
        got_z, got_s = graph(z, mask, s)
        torch.cuda.synchronize()
        assert torch.equal(got_z, want_z), f"pair differs (seed {seed})"
        assert torch.equal(got_s, want_s), f"single differs (seed {seed})"
        # eager work between replays, as a program around the graph would do
        _ = (want_z.float() * 2).sum().item()
        if seed == 3:
            _against_the_oracle(model, (z, mask, s), (got_z, got_s), passes=2)


def _against_the_oracle(model, inputs, outputs, *, passes: int):
    """The replay's change of pair and single over ``passes`` passes against the fp64 oracle's
    (valid pairs / tokens): within the trunk bar for a few block evaluations, 5e-2."""
    z, mask, s = (t.cpu() for t in inputs)
    state = {k: v.cpu() for k, v in model.state_dict().items()}
    blocks = len(model.blocks)
    subs = [{k[len(f"blocks.{i}."):]: v for k, v in state.items() if k.startswith(f"blocks.{i}.")}
            for i in range(blocks)]
    fz, fs = z.double(), s.double()
    for _ in range(passes):
        for sub in subs:
            fz, fs = ps.pairformer_block(fz, mask, sub, n_head_pair=4, s=fs, n_head_single=16, dtype=torch.float64)
    pairs = mask[:, :, None] & mask[:, None, :]
    got_z, got_s = (t.cpu().double() for t in outputs)
    rz = ps.rel_rms(got_z - z.double(), fz - z.double(), pairs)
    rs = ps.rel_rms(got_s - s.double(), fs - s.double(), mask)
    print(f"replay vs fp64 oracle: pair change rel_rms={rz:.3e} single change rel_rms={rs:.3e}", flush=True)
    assert rz <= 5e-2 and rs <= 5e-2


def test_captured_pair_only_trunk():
    n = 64
    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=3, seed=6, d_single=384,
                               unsupported="error")
    z, mask, _ = _inputs(n, 50, seed=4)
    graph = capture_trunk(model, z, mask, passes=1)
    for seed in (5, 6):
        z2, mask2, _ = _inputs(n, 50, seed)
        with torch.no_grad():
            want = model(z2, mask2, passes=1)
        got = graph(z2, mask2)
        torch.cuda.synchronize()
        assert torch.equal(got, want)

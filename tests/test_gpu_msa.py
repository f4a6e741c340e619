"""GPU parity of the MSA-stack ops against the CPU oracle (gfx950 only).

Same conventions as the pair ops: seeded fp32 draws rounded to bf16 feed both sides, the
oracle runs in fp64 on the module's fp32 parameters, the bare update (``residual=False``) is
compared with rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref|, and masking is exact: the
outputs of valid tokens are bitwise independent of the content at masked keys.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import factories
from foldforge_amd.trunk import randomise
from oracle import pairstack as ps
from tests.hip_calls import hip_delta, hip_forward

pytestmark = pytest.mark.gpu

REL_RMS = 1e-2
MAX_ABS = 4e-2


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from foldforge_amd import _native

    _native.lib()


def _check(got: torch.Tensor, want: torch.Tensor, what: str) -> None:
    rr = ps.rel_rms(got, want)
    ma = ps.max_abs(got, want)
    ref = want.abs().max().item()
    print(f"{what}: rel_rms={rr:.2e} max_abs={ma:.2e} max_ref={ref:.2e}", flush=True)
    assert rr <= REL_RMS, f"{what}: rel-RMS {rr:.3e}"
    assert ma <= MAX_ABS * ref, f"{what}: max-abs {ma:.3e} vs {MAX_ABS} * {ref:.3e}"


def _inputs(depth: int, n: int, cm: int, lengths, seed: int):
    g = torch.Generator().manual_seed(seed)
    batch = len(lengths)
    m = torch.randn(batch, depth, n, cm, generator=g).bfloat16()
    z = torch.randn(batch, n, n, 128, generator=g).bfloat16()
    mask = torch.zeros(batch, n, dtype=torch.bool)
    for b, length in enumerate(lengths):
        mask[b, :length] = True
    return m, z, mask


def _pwa(cm: int, heads: int, dh: int | None, seed: int):
    m = randomise(factories.msa_pair_weighted_averaging(cm, 128, heads, dh), seed=seed).cuda()
    m.set_backend("hip")
    return m


# d_head 32 is the released models' width; 24 ends MSA rows inside a 128-row output tile; 12 (not a
# multiple of 8) takes the unstaged 8-byte epilogue
@pytest.mark.parametrize("cm,heads,dh", [(64, 8, None), (64, 4, 16), (128, 8, 8), (64, 8, 32), (64, 8, 24),
                                        (64, 16, 12)])
@pytest.mark.parametrize("depth,n,lengths", [(5, 64, [64]), (7, 100, [77]), (3, 130, [130, 41])])
def test_msa_pair_weighted_averaging_matches_oracle(cm, heads, dh, depth, n, lengths):
    msa, z, mask = _inputs(depth, n, cm, lengths, seed=n + cm + heads)
    mod = _pwa(cm, heads, dh, seed=cm + heads)
    assert mod.unsupported(msa.cuda(), z.cuda(), mask.cuda()) is None
    got = hip_delta(mod, msa.cuda(), z.cuda(), mask.cuda()).cpu()
    want = ps.msa_pair_weighted_averaging(msa, z, mask, mod.state_dict(), n_head=heads,
                                          dtype=torch.float64) - msa.double()
    _check(got, want, f"msa_pwa c_m={cm} heads={heads}x{mod.d_hidden} S={depth} n={n} lengths={lengths}")
    full = hip_forward(mod, msa.cuda(), z.cuda(), mask.cuda()).cpu()
    _check(full, want + msa.double(), "msa_pwa residual")


def test_msa_pair_weighted_averaging_masking_is_exact_and_empty_rows_are_zero():
    depth, n, length = 4, 96, 61
    msa, z, mask = _inputs(depth, n, 64, [length, 0], seed=11)
    mod = _pwa(64, 8, None, seed=12)
    a = hip_delta(mod, msa.cuda(), z.cuda(), mask.cuda()).cpu()
    msa2, z2 = msa.clone(), z.clone()
    msa2[0, :, length:] = 5.0
    z2[0, length:] = -4.0
    z2[0, :, length:] = 9.0
    b = hip_delta(mod, msa2.cuda(), z2.cuda(), mask.cuda()).cpu()
    assert torch.equal(a[0, :, :length], b[0, :, :length])
    assert torch.equal(a[1], torch.zeros_like(a[1]))  # no valid key: zero update


def test_msa_pair_weighted_averaging_full_size_is_finite_and_deterministic():
    depth, n = 512, 384
    msa, z, mask = _inputs(depth, n, 64, [371], seed=21)
    mod = _pwa(64, 8, None, seed=22)
    mc, zc, kc = msa.cuda(), z.cuda(), mask.cuda()
    a = mod(mc, zc, kc)
    b = mod(mc, zc, kc)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("options", [{}, {"parallel": True, "opm_groups": 8, "opm_channel": 8}])
def test_msa_block_overlapped_tracks_are_bitwise_sequential(options):
    """After the outer product mean the MSA block runs its MSA track on a second stream beside
    the pair track: the results equal the sequential order bit for bit (the AF3 order and
    Chai-1's parallel stages with the grouped outer product mean), with every op on ``hip``."""
    from foldforge_amd import dispatch

    n, length, depth, cm, c = 96, 83, 41, 64, 128
    block = randomise(factories.msa_block(cm, c, 4, **options), seed=12).cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")
    g = torch.Generator().manual_seed(13)
    msa = torch.randn(depth, n, cm, generator=g).bfloat16().cuda()
    z = torch.randn(n, n, c, generator=g).bfloat16().cuda()
    tokens = torch.zeros(n, dtype=torch.bool)
    tokens[:length] = True
    msa_mask = ((torch.rand(depth, n, generator=g) > 0.2) & tokens[None]).float()
    msa_mask[0] = tokens.float()
    pair_mask = (tokens[:, None] & tokens[None, :]).float()
    msa_mask, pair_mask = msa_mask.cuda(), pair_mask.cuda()
    with torch.no_grad():
        block.overlap_tracks = False
        want = block(msa, z, msa_mask, pair_mask)
        block.overlap_tracks = True
        got = block(msa, z, msa_mask, pair_mask)
        again = block(msa, z, msa_mask, pair_mask)
    torch.cuda.synchronize()
    assert dispatch.served_count(block, "hip") == 3 * 8
    for a, b, r in zip(got, want, again):
        assert torch.equal(a, b) and torch.equal(r, b)

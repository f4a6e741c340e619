"""GPU parity of the generic-width pair path (template-stack shapes) against the CPU oracle.

The fused kernels serve the AF3 trunk widths (pair 128, hidden 128, 4 x 32 heads); other widths
run the generic path: token-row GEMMs with the LayerNorm prologue, the plane contraction, the
pair-bias kernel and the split-key attention. Same bar as the trunk widths: the bare update on
the valid pairs within rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref| of the fp64 oracle,
masking exact, every call served by ``hip``.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import dispatch, factories
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


def _pair(n: int, c: int, lengths, seed: int):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(len(lengths), n, n, c, generator=g).bfloat16()
    mask = torch.zeros(len(lengths), n, dtype=torch.bool)
    for b, length in enumerate(lengths):
        mask[b, :length] = True
    return z, mask


def _pairs(mask: torch.Tensor) -> torch.Tensor:
    return mask[:, :, None] & mask[:, None, :]


def _check(got, want, where, what):
    rr = ps.rel_rms(got, want, where)
    ma = ps.max_abs(got, want, where)
    ref = want.double()[where].abs().max().item()
    print(f"{what}: rel_rms={rr:.2e} max_abs={ma:.2e} max_ref={ref:.2e}", flush=True)
    assert rr <= REL_RMS, f"{what}: rel-RMS {rr:.3e}"
    assert ma <= MAX_ABS * ref, f"{what}: max-abs {ma:.3e} vs {MAX_ABS} * {ref:.3e}"


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("c,h", [(64, 64), (64, 128), (128, 64), (256, 128), (256, 256)])
@pytest.mark.parametrize("n,lengths", [(37, [37]), (96, [70, 96])])
def test_trimul_generic_widths_match_oracle(outgoing, c, h, n, lengths):
    z, mask = _pair(n, c, lengths, seed=n + c + h)
    m = randomise(factories.triangle_multiplication(c, outgoing=outgoing, d_hidden=h), seed=c + h).cuda()
    m.set_backend("hip")
    assert m.unsupported(z.cuda(), mask.cuda()) is None
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=outgoing, dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"trimul c={c} h={h} outgoing={outgoing} n={n}")
    full = m(z.cuda(), mask.cuda()).cpu()
    torch.testing.assert_close(full.float(), z.float() + got.float(), atol=3e-2, rtol=1e-2)


@pytest.mark.parametrize("outgoing", [True, False])
def test_length_divided_trimul_generic_width_matches_oracle(outgoing):
    """TriangleMultiplicationRF3 at a generic width: the device length (70 of 96) feeds the
    centre norm of the token-row output GEMM."""
    n, c, h = 96, 64, 128
    z, mask = _pair(n, c, [70, 52], seed=31)
    m = randomise(factories.triangle_multiplication(c, outgoing=outgoing, d_hidden=h,
                                                    divide_by_length=True), seed=32).cuda()
    m.set_backend("hip")
    assert m.unsupported(z.cuda(), mask.cuda()) is None
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=outgoing, length_divided=True,
                                      dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"trimul RF3 c={c} h={h} outgoing={outgoing}")


def test_trimul_generic_width_256_tile_contraction():
    """A padded width of 256: the contraction takes its 256 x 256 tiles."""
    n, c, h = 230, 64, 64
    z, mask = _pair(n, c, [230, 177], seed=21)
    m = randomise(factories.triangle_multiplication(c, outgoing=False, d_hidden=h), seed=22).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=False, dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), "trimul c=64 h=64 incoming n=230")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("key", ["rf3", "chai1", "chai1_confidence"])
@pytest.mark.parametrize("d", [16, 64])
def test_triattn_lineage_forms_generic_width_match_oracle(starting, key, d):
    """The RoseTTAFold3 and Chai-1 forms on the generic path (pair 64, 4 x 16 and RoseTTAFold3's
    template width 4 x 64)."""
    from tests.test_gpu_ops import _lineage_module, _lineage_oracle

    n, c = 75, 64
    z, mask = _pair(n, c, [75, 52], seed=41)
    m = _lineage_module(key, c, 4, d, starting, seed=6)
    m.set_backend("hip")
    assert m.unsupported(z.cuda(), mask.cuda()) is None
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    where = _pairs(mask)
    if key.startswith("chai1"):
        where = where & where.transpose(1, 2)
    _check(got, _lineage_oracle(m, z, mask), where, f"triattn {key} c={c} starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("key,c,heads,d", [("chai1", 256, 4, 64), ("chai1_confidence", 256, 4, 64),
                                           ("af3", 128, 4, 48)])
def test_triattn_wide_heads_match_oracle(starting, key, c, heads, d):
    """Heads wider than 32 channels (two 32-channel output tiles per head): Chai-1's trunk and
    confidence shapes (pair 256, 4 x 64) and a 48-channel head (a partial second tile)."""
    from tests.test_gpu_ops import _lineage_module, _lineage_oracle

    n = 44
    z, mask = _pair(n, c, [44, 30], seed=c + d)
    m = _lineage_module(key, c, heads, d, starting, seed=7)
    m.set_backend("hip")
    assert m.unsupported(z.cuda(), mask.cuda()) is None
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    where = _pairs(mask)
    if key.startswith("chai1"):
        where = where & where.transpose(1, 2)
    _check(got, _lineage_oracle(m, z, mask), where, f"triattn {key} {heads}x{d} c={c} starting={starting}")


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("model", ["af3", "protenix"])
@pytest.mark.parametrize("c,heads,d", [(64, 4, 16), (64, 4, 32), (128, 8, 16), (256, 4, 32), (64, 4, 64),
                                          (128, 1, 64)])
@pytest.mark.parametrize("n,lengths", [(40, [40]), (75, [75, 52])])
def test_triattn_generic_widths_match_oracle(starting, model, c, heads, d, n, lengths):
    z, mask = _pair(n, c, lengths, seed=n + c + heads + d)
    m = randomise(factories.triangle_attention(c, heads, starting=starting, model=model,
                                               d_hidden=heads * d), seed=c + d).cuda()
    m.set_backend("hip")
    assert m.unsupported(z.cuda(), mask.cuda()) is None
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_attention(z, mask, m.state_dict(), starting=starting, n_head=heads,
                                 transposed_bias=m.transposed_bias, dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"triattn c={c} {heads}x{d} {model} starting={starting} n={n}")


@pytest.mark.parametrize("op", ["trimul", "triattn"])
def test_generic_path_masking_is_exact(op):
    n, length, c = 58, 41, 64
    z, mask = _pair(n, c, [length], seed=3)
    if op == "trimul":
        m = randomise(factories.triangle_multiplication(c, outgoing=False, d_hidden=128), seed=4).cuda()
    else:
        m = randomise(factories.triangle_attention(c, 4, starting=False, model="af3", d_hidden=64), seed=4).cuda()
    m.set_backend("hip")
    a = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    z2 = z.clone()
    z2[0, length:] = 3.0
    z2[0, :, length:] = -5.0
    b = hip_delta(m, z2.cuda(), mask.cuda()).cpu()
    assert torch.equal(a[0, :length, :length], b[0, :length, :length])


def test_template_stack_block_runs_on_the_kernels():
    """AF3's template-stack block: pair 64, triangle multiplication hidden 64, triangle attention
    4 x 16, transition x 2 (``src/foldforge/modules/dense/template.py:238-247``), a batch of two
    templates, every op on hip."""
    n, c = 72, 64
    z, mask = _pair(n, c, [72, 60], seed=8)
    block = randomise(factories.pairformer_block(d_pair=c, triangle_model="af3", d_hidden_tri_attention=16,
                                                 pair_transition_n=2), seed=9).cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")
    with torch.no_grad():
        got = block(z.cuda(), mask.cuda()).cpu()
    want = ps.pairformer_block(z, mask, block.state_dict(), n_head_pair=4, dtype=torch.float64)
    where = _pairs(mask)
    rr = ps.rel_rms(got - z, want - z.double(), where)
    print(f"template block: update rel_rms={rr:.2e}", flush=True)
    assert rr <= 3e-2


def test_pair_256_block_runs_on_the_kernels():
    """A block at Chai-1's trunk widths in AF3's op forms: pair 256, triangle multiplication
    hidden 256, triangle attention 4 x 64, transition x 2 (256-channel LayerNorm-fed row GEMMs,
    512-channel squeeze), every op on hip."""
    n, c = 52, 256
    z, mask = _pair(n, c, [52, 39], seed=12)
    block = randomise(factories.pairformer_block(d_pair=c, triangle_model="af3", d_hidden_tri_attention=64,
                                                 pair_transition_n=2), seed=13).cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")
    with torch.no_grad():
        got = block(z.cuda(), mask.cuda()).cpu()
    want = ps.pairformer_block(z, mask, block.state_dict(), n_head_pair=4, dtype=torch.float64)
    where = _pairs(mask)
    rr = ps.rel_rms(got - z, want - z.double(), where)
    print(f"pair-256 block: update rel_rms={rr:.2e}", flush=True)
    assert rr <= 3e-2

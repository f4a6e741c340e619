"""GPU: the measured configurations beyond N = 512, in-place calls, and the layout adapter.

* One pair-stack block at N = 384 (the reference's per-op table size): padded width 384 runs
  the 128-tile contraction with three tiles per side. Against the fp64 oracle on valid pairs,
  the block update within rel-RMS 3e-2, one all-real and one ragged batch element.
* Triangle multiplication at N = 320 (padded 384) in both directions, per-op bar.
* The length ladder, one block with the single track at N = 768, 1024, 1536 and 2048: finite,
  bitwise run-to-run, valid region bitwise invariant to padded content, and the update within
  3e-2 of the engine ``pytorch`` backend (fp32 arithmetic inside every op; it is pinned to the
  oracle by the CPU tests) on the same GPU.
* Every entry point whose C-ABI lets ``out`` alias its input, called in place: bitwise the
  out-of-place result.
* ``run_block`` (FoldForge's unbatched layout, fp32 activations under autocast) on ``hip``.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import adapter, dispatch, factories, kernels
from foldforge_amd.modules import TriangleMultiplication
from foldforge_amd.trunk import randomise
from oracle import pairstack as ps
from tests.hip_calls import hip_delta

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from foldforge_amd import _native

    _native.lib()


def _pairs(mask: torch.Tensor) -> torch.Tensor:
    return mask[:, :, None] & mask[:, None, :]


def _hip_block(seed: int, d_single: int = 0):
    block = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3", d_single=d_single),
                      seed=seed, out_scale=0.25 if d_single else None).cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")  # a refused call raises instead of running torch ops
    return block


def test_block_n384_matches_oracle():
    n = 384
    g = torch.Generator().manual_seed(41)
    z = torch.randn(2, n, n, 128, generator=g).bfloat16()
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[1, 300:] = False
    block = _hip_block(42)
    print("block N=384 batch 2 (lengths 384, 300): hip", flush=True)
    with torch.no_grad():
        got = block(z.cuda(), mask.cuda()).cpu()
    assert dispatch.served_count(block, "hip") == 5
    print("block N=384: fp64 oracle", flush=True)
    want = ps.pairformer_block(z, mask, block.state_dict(), n_head_pair=4, dtype=torch.float64)
    for b in range(2):
        where = _pairs(mask[b:b + 1])
        rr = ps.rel_rms(got[b:b + 1].double() - z[b:b + 1].double(), want[b:b + 1] - z[b:b + 1].double(), where)
        print(f"block N=384 element {b}: update rel_rms={rr:.3e}", flush=True)
        assert rr <= 3e-2


@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_n320_three_tiles_per_side(outgoing):
    n = 320
    g = torch.Generator().manual_seed(43)
    z = torch.randn(2, n, n, 128, generator=g).bfloat16()
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 271:] = False
    m = randomise(factories.triangle_multiplication(128, outgoing=outgoing), seed=44).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=outgoing, dtype=torch.float64) - z.double()
    where = _pairs(mask)
    rr, ma = ps.rel_rms(got, want, where), ps.max_abs(got, want, where)
    ref = want[where].abs().max().item()
    print(f"trimul n=320 outgoing={outgoing}: rel_rms={rr:.2e} max_abs={ma:.2e} max_ref={ref:.2e}", flush=True)
    assert rr <= 1e-2 and ma <= 4e-2 * ref


@pytest.mark.parametrize("n,length", [(768, 701), (1024, 977), (1536, 1489), (2048, 1999)])
def test_ladder_block_with_single_track(n, length):
    g = torch.Generator(device="cuda").manual_seed(n)
    z = torch.randn(1, n, n, 128, device="cuda", generator=g).bfloat16()
    s = torch.randn(1, n, 384, device="cuda", generator=g).bfloat16()
    mask = torch.zeros(1, n, dtype=torch.bool, device="cuda")
    mask[0, :length] = True
    block = _hip_block(45, d_single=384)
    print(f"ladder block N={n}: hip runs", flush=True)
    with torch.no_grad():
        za, sa = block(z, mask, s)
        zb, sb = block(z, mask, s)
        assert torch.isfinite(za.float()).all() and torch.isfinite(sa.float()).all()
        assert torch.equal(za, zb) and torch.equal(sa, sb)
        z2, s2 = z.clone(), s.clone()
        z2[0, length:] = 11.0
        z2[0, :, length:] = -6.0
        s2[0, length:] = 4.0
        zc, sc = block(z2, mask, s2)
        assert torch.equal(za[0, :length, :length], zc[0, :length, :length])
        assert torch.equal(sa[0, :length], sc[0, :length])
        assert dispatch.served_count(block, "hip") == 3 * 7
        print(f"ladder block N={n}: pytorch backend", flush=True)
        dispatch.set_refusal(block, None)
        block.set_backend("pytorch")
        zr, sr = block(z, mask, s)
    where = _pairs(mask).cpu()
    rz = ps.rel_rms(za.double() - z.double(), zr.double() - z.double(), where)
    rs = ps.rel_rms(sa.double() - s.double(), sr.double() - s.double(), mask.cpu())
    print(f"ladder block N={n}: update vs pytorch backend pair {rz:.3e} single {rs:.3e}", flush=True)
    assert rz <= 3e-2 and rs <= 3e-2


def _module_args(m):
    if isinstance(m, TriangleMultiplication):
        return dict(ln_pair_weight=m.ln_pair.weight, ln_pair_bias=m.ln_pair.bias, to_left=m.to_left.weight,
                    to_right=m.to_right.weight, to_left_gate=m.to_left_gate.weight,
                    to_right_gate=m.to_right_gate.weight, ln_out_weight=m.ln_out.weight,
                    ln_out_bias=m.ln_out.bias, to_out=m.to_out.weight, to_gate=m.to_gate.weight,
                    outgoing=m.outgoing)
    return dict(ln_pair_weight=m.ln_pair.weight, ln_pair_bias=m.ln_pair.bias, to_bias=m.to_bias.weight,
                to_query=m.to_query.weight, to_key=m.to_key.weight, to_value=m.to_value.weight,
                to_gate=m.to_gate.weight, to_out=m.to_out.weight, n_head=m.n_head, starting=m.starting,
                transposed_bias=m.transposed_bias, gate_bias=m.to_gate.bias, out_bias=m.to_out.bias,
                to_out_t=m.to_out_t.weight if m.dual_output else None,
                out_t_bias=m.to_out_t.bias if m.dual_output else None,
                untransposed_output=m.untransposed_output)


@pytest.mark.parametrize("c,generic", [(128, False), (64, True)])
def test_pair_ops_in_place(c, generic):
    """``out`` aliasing ``z`` (the header's promise) gives the out-of-place result bitwise: both
    triangle multiplications, triangle attention in every lineage's output form (AF3's
    transposed-back ending node, RoseTTAFold3's projection biases, Chai-1's untransposed and
    dual outputs, which stage the ending node's update before adding it to ``out``), the
    transition."""
    n = 100
    g = torch.Generator().manual_seed(46)
    z = torch.randn(2, n, n, c, generator=g).bfloat16().cuda()
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[1, 70:] = False
    mask = mask.cuda()
    hidden = 64 if generic else 128
    heads, dh = (4, 16) if generic else (4, 32)
    mods = [randomise(factories.triangle_multiplication(c, outgoing=o, d_hidden=hidden), seed=47).cuda()
            for o in (True, False)]
    mods += [randomise(factories.triangle_attention(c, heads, starting=st, model=key, d_hidden=heads * dh),
                       seed=48).cuda() for st in (True, False) for key in ("af3", "rf3", "chai1", "chai1_confidence")]
    for m in mods:
        call = kernels.triangle_multiplicative_update if "Multiplication" in type(m).__name__ else kernels.triangle_attention
        want = call(z, mask, **_module_args(m))
        buf = z.clone()
        got = call(buf, mask, **_module_args(m), out=buf)
        assert got.data_ptr() == buf.data_ptr()
        assert torch.equal(got, want), (type(m).__name__, m.starting)
    tr = randomise(factories.transition(c, 4 if not generic else 2), seed=49).cuda()
    targs = dict(ln_weight=tr.ln_in.weight, ln_bias=tr.ln_in.bias, expand_a=tr.expand_a.weight,
                 expand_b=tr.expand_b.weight, squeeze=tr.squeeze.weight)
    want = kernels.transition(z, **targs)
    buf = z.clone()
    assert torch.equal(kernels.transition(buf, **targs, out=buf), want)


def test_single_and_msa_ops_in_place():
    n, depth = 96, 9
    g = torch.Generator().manual_seed(50)
    z = torch.randn(1, n, n, 128, generator=g).bfloat16().cuda()
    s = torch.randn(1, n, 384, generator=g).bfloat16().cuda()
    msa = torch.randn(1, depth, n, 64, generator=g).bfloat16().cuda()
    mask = torch.ones(1, n, dtype=torch.bool, device="cuda")
    mask[0, 80:] = False
    apb = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3", d_single=384).single_attention,
                    seed=51).cuda()
    a = dict(ln_single_weight=apb.ln_single.weight, ln_single_bias=apb.ln_single.bias,
             to_query=apb.to_query.weight, query_bias=apb.to_query.bias, to_key=apb.to_key.weight,
             to_value=apb.to_value.weight, ln_pair_weight=apb.ln_pair.weight, to_bias=apb.to_bias.weight,
             to_gate=apb.to_gate.weight, to_out=apb.to_out.weight, n_head=16)
    want = kernels.attention_pair_bias(s, z, mask, **a)
    buf = s.clone()
    assert torch.equal(kernels.attention_pair_bias(buf, z, mask, **a, out=buf), want)
    pwa = randomise(factories.msa_pair_weighted_averaging(64, 128, 8), seed=52).cuda()
    p = dict(ln_msa_weight=pwa.ln_msa.weight, ln_msa_bias=pwa.ln_msa.bias, ln_pair_weight=pwa.ln_pair.weight,
             to_bias=pwa.to_bias.weight, to_value=pwa.to_value.weight, to_gate=pwa.to_gate.weight,
             to_out=pwa.to_out.weight, n_head=8)
    want = kernels.msa_pair_weighted_averaging(msa, z, mask, **p)
    buf = msa.clone()
    assert torch.equal(kernels.msa_pair_weighted_averaging(buf, z, mask, **p, out=buf), want)
    opm = randomise(factories.outer_product_mean(64, 128, 32, count_offset=1e-3), seed=53).cuda()
    rows = (torch.rand(1, depth, n, generator=g) > 0.2).cuda()
    o = dict(ln_weight=opm.ln_msa.weight, ln_bias=opm.ln_msa.bias, to_left=opm.to_left.weight,
             to_right=opm.to_right.weight, to_out=opm.to_out.weight, to_out_bias=opm.to_out.bias,
             count_offset=1e-3)
    want = kernels.outer_product_mean(msa, rows, **o, residual=z)
    buf = z.clone()
    assert torch.equal(kernels.outer_product_mean(msa, rows, **o, residual=buf, out=buf), want)


def test_run_block_on_hip_matches_the_batched_call_and_the_oracle():
    """FoldForge's layout: ``pair [L, L, c]`` fp32 and ``single [L, c_s]`` under bf16 autocast, the
    outer-product pair mask, the sequence mask. The adapter must give the batched block call's
    result bitwise, and the oracle's within the block bar."""
    n, length = 80, 69
    block = _hip_block(54, d_single=384)
    adapter.place(block, torch.bfloat16, "cuda")
    g = torch.Generator().manual_seed(55)
    pair = torch.randn(n, n, 128, generator=g)
    single = torch.randn(n, 384, generator=g)
    tokens = torch.zeros(n)
    tokens[:length] = 1
    pair_mask = tokens[:, None] * tokens[None, :]
    with torch.no_grad(), adapter.autocast_for(block):
        got_z, got_s = adapter.run_block(block, pair.cuda(), pair_mask.cuda(), single.cuda(), tokens.cuda())
        got_z2 = adapter.run_block(_hip_block(54), pair.cuda(), pair_mask.cuda())  # pair-only block, mask from the pair mask
    assert got_z.shape == (n, n, 128) and got_s.shape == (n, 384) and got_z.dtype == torch.bfloat16
    keys = (tokens > 0)[None].cuda()
    with torch.no_grad():
        want_z, want_s = block(pair.bfloat16()[None].cuda(), keys, single.bfloat16()[None].cuda())
    assert torch.equal(got_z, want_z[0]) and torch.equal(got_s, want_s[0])
    assert got_z2.shape == (n, n, 128)
    zb, sb = pair.bfloat16()[None], single.bfloat16()[None]
    oz, os_ = ps.pairformer_block(zb, keys.cpu(), {k: v.cpu() for k, v in block.state_dict().items()},
                                  n_head_pair=4, s=sb, n_head_single=16, dtype=torch.float64)
    where = _pairs(keys.cpu())
    rz = ps.rel_rms(got_z[None].cpu().double() - zb.double(), oz - zb.double(), where)
    rs = ps.rel_rms(got_s[None].cpu().double() - sb.double(), os_ - sb.double(), keys.cpu())
    print(f"run_block on hip: pair update rel_rms={rz:.3e} single update rel_rms={rs:.3e}", flush=True)
    assert rz <= 3e-2 and rs <= 3e-2
    # the block's extra pair bias ([L, L], OpenDDE's structural bias) on hip, against the oracle
    extra = 1.5 * torch.randn(n, n, generator=g)
    with torch.no_grad(), adapter.autocast_for(block):
        before = dispatch.served_count(block, "hip")
        ez, es = adapter.run_block(block, pair.cuda(), pair_mask.cuda(), single.cuda(), tokens.cuda(),
                                   extra_pair_bias=extra.cuda())
        assert dispatch.served_count(block, "hip") > before
    assert torch.equal(ez, got_z)  # the pair track does not read it
    _, os2 = ps.pairformer_block(zb, keys.cpu(), {k: v.cpu() for k, v in block.state_dict().items()},
                                 n_head_pair=4, s=sb, n_head_single=16,
                                 extra_pair_bias=extra.bfloat16().double(), dtype=torch.float64)
    rs2 = ps.rel_rms(es[None].cpu().double() - sb.double(), os2 - sb.double(), keys.cpu())
    print(f"run_block with extra_pair_bias: single update rel_rms={rs2:.3e}", flush=True)
    assert rs2 <= 3e-2
    assert ps.rel_rms(os2 - sb.double(), os_ - sb.double(), keys.cpu()) > 0.05

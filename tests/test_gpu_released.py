"""GPU: released-layout weights, converted to the engine layout, run through the hip kernels.

A released pairformer block (with its single track) and a released MSA-stack block at the AF3
widths are converted with ``foldforge_amd.released``, loaded strictly, run on the ``hip``
backend in bf16 and compared with the released computation in fp64 on the CPU
(``oracle/released.py``) where the tokens are real: rel-RMS <= 1e-2.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import dispatch, factories, released
from oracle import pairstack as ps
from oracle import released as rel
from tests.test_released import _rand, block_shapes, msa_block_shapes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from foldforge_amd import _native

    _native.lib()


def _rel_rms(got, want, where) -> float:
    return ps.rel_rms(got.double()[where], want.double()[where])


def test_released_pairformer_block_runs_on_the_kernels():
    n, length, c, cs = 64, 53, 128, 384
    state = _rand(block_shapes(c, 4, cs, heads_single=16, d_tri=32), 31, std=0.05)
    block = factories.pairformer_block(d_pair=c, triangle_model="af3", d_single=cs, n_head_single=16)
    released.load(block, released.pairformer_block_from_released(state))
    block = block.cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")  # a refused call would raise instead of running torch ops
    g = torch.Generator().manual_seed(32)
    z = torch.randn(n, n, c, generator=g).bfloat16()
    s = torch.randn(n, cs, generator=g).bfloat16()
    tokens = torch.zeros(n, dtype=torch.bool)
    tokens[:length] = True
    with torch.no_grad():
        for m in block.children_ops():
            assert m.unsupported(*_probe(m, z, s, tokens)) is None, type(m).__name__
        za, sa = block(z[None].cuda(), tokens[None].cuda(), s[None].cuda())
    zw, sw = rel.pairformer_block(z, tokens, state, n_head_pair=4, single=s, n_head_single=16)
    pair = tokens[:, None] & tokens[None, :]
    # the updates, not z + f(z): the N(0, 1) residual would hide an error of several percent in f
    zd, sd = z.double(), s.double()
    r_z = _rel_rms(za[0].cpu().double() - zd, zw.double() - zd, pair)
    r_s = _rel_rms(sa[0].cpu().double() - sd, sw.double() - sd, tokens)
    print(f"released block on hip: pair update rel_rms={r_z:.2e} single update rel_rms={r_s:.2e}", flush=True)
    assert r_z <= 3e-2 and r_s <= 3e-2
    assert dispatch.served_count(block, "hip") == 7  # 5 pair + 2 single-track ops


def _probe(m, z, s, tokens):
    """Device inputs of the right shapes for ``m.unsupported``."""
    zc, sc, kc = z[None].cuda(), s[None].cuda(), tokens[None].cuda()
    name = type(m).__name__
    if name == "AttentionPairBias":
        return sc, zc, kc
    if name == "Transition":
        return (sc,) if m.ln_in.weight.shape[0] == s.shape[-1] else (zc,)
    return zc, kc


def test_released_msa_block_runs_on_the_kernels():
    n, length, depth, cm, c = 48, 41, 37, 64, 128
    shapes = msa_block_shapes(cm, c, 4)
    shapes = {k: v for k, v in shapes.items() if not k.startswith("outer_product_mean.")}
    shapes |= {"outer_product_mean.layer_norm_input.weight": (cm,),
               "outer_product_mean.layer_norm_input.bias": (cm,),
               "outer_product_mean.left_projection.weight": (32, cm),
               "outer_product_mean.right_projection.weight": (32, cm),
               "outer_product_mean.output_w": (32, 32, c), "outer_product_mean.output_b": (c,)}
    # weights of 0.1 N(0, 1): the MSA update is then ~0.4 RMS, well above the bf16 rounding of
    # the MSA stream (~3e-3 RMS per op at |m| ~ 1), which would otherwise set the update's error
    state = _rand(shapes, 33, std=0.1)
    block = factories.msa_block(cm, c, 4)
    released.load(block, released.msa_block_from_released(state))
    block = block.cuda()
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")  # a refused call would raise instead of running torch ops
    g = torch.Generator().manual_seed(34)
    msa = torch.randn(depth, n, cm, generator=g).bfloat16()
    z = torch.randn(n, n, c, generator=g).bfloat16()
    tokens = torch.zeros(n, dtype=torch.bool)
    tokens[:length] = True
    msa_mask = ((torch.rand(depth, n, generator=g) > 0.2) & tokens[None]).float()
    msa_mask[0] = tokens.float()
    pair_mask = (tokens[:, None] & tokens[None, :]).float()
    with torch.no_grad():
        ma, za = block(msa.cuda(), z.cuda(), msa_mask.cuda(), pair_mask.cuda())
    mw, zw = rel.msa_block(msa, z, msa_mask, tokens, state, n_head_pair=4)
    pair = tokens[:, None] & tokens[None, :]
    zd, md = z.double(), msa.double()
    r_z = _rel_rms(za.cpu().double() - zd, zw.double() - zd, pair)
    r_m = _rel_rms(ma.cpu().double() - md, mw.double() - md, (slice(None), tokens))
    print(f"released MSA block on hip: pair update rel_rms={r_z:.2e} msa update rel_rms={r_m:.2e}", flush=True)
    assert r_z <= 3e-2 and r_m <= 3e-2
    hip_calls = dispatch.served_count(block, "hip")
    assert hip_calls == 8, dispatch.ledger_report(block)  # every op of the block ran on the kernels

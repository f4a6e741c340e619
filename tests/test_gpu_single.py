"""GPU parity of the single-track kernels (attention with pair bias, wide transition).

Same conventions as the pair ops: seeded fp32 draws rounded to bf16 feed both sides, the
oracle runs in fp64 on the module's fp32 parameters, and the bare update f(s)
(``residual=False``) is compared: rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref|. Every
query row is compared, padded ones included (they attend over the valid keys like the
others). Masking is exact: the valid rows are bitwise independent of the content of
padded tokens in s and of padded rows / columns in z.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import factories, modules
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


def _inputs(n: int, cs: int, lengths, seed: int):
    g = torch.Generator().manual_seed(seed)
    batch = len(lengths)
    z = torch.randn(batch, n, n, 128, generator=g).bfloat16()
    s = torch.randn(batch, n, cs, generator=g).bfloat16()
    mask = torch.zeros(batch, n, dtype=torch.bool)
    for b, length in enumerate(lengths):
        mask[b, :length] = True
    return s, z, mask


def _apb(cs: int, heads: int, gate_bias: float, seed: int) -> modules.AttentionPairBias:
    m = modules.AttentionPairBias(cs, 128, heads, gate_bias)
    m.set_master_weights()
    m = randomise(m, seed=seed).cuda()
    m.set_backend("hip")
    return m


@pytest.mark.parametrize("cs,heads", [(384, 16), (128, 4), (64, 8)])
@pytest.mark.parametrize("n,lengths", [(64, [64]), (100, [77]), (130, [130, 41])])
def test_attention_pair_bias_matches_oracle(cs, heads, n, lengths):
    s, z, mask = _inputs(n, cs, lengths, seed=n + cs)
    m = _apb(cs, heads, gate_bias=0.5, seed=cs + heads)
    assert m.unsupported(s.cuda(), z.cuda(), mask.cuda()) is None
    got = hip_delta(m, s.cuda(), z.cuda(), mask.cuda()).cpu()
    want = ps.attention_pair_bias(s, z, mask, m.state_dict(), n_head=heads, gate_bias=0.5,
                                  dtype=torch.float64) - s.double()
    _check(got, want, f"attention_pair_bias cs={cs} heads={heads} n={n} lengths={lengths}")
    full = m(s.cuda(), z.cuda(), mask.cuda()).cpu()
    _check(full, want + s.double(), "attention_pair_bias residual")


@pytest.mark.parametrize("form", ["nn_fp32", "bhnn_bf16"])
def test_attention_pair_bias_extra_bias_matches_oracle(form):
    """The block's extra pair bias on hip: an fp32 [N, N] map (broadcast by zero strides, as
    the engine passes it) or a dense bf16 [B, H, N, N]."""
    n, cs, heads = 100, 384, 16
    s, z, mask = _inputs(n, cs, [100, 73], seed=31)
    m = _apb(cs, heads, gate_bias=0.0, seed=32)
    g = torch.Generator().manual_seed(33)
    if form == "nn_fp32":
        extra = 2.0 * torch.randn(n, n, generator=g)
        dev_extra = extra.cuda().expand(2, heads, n, n)
    else:
        extra = (2.0 * torch.randn(2, heads, n, n, generator=g)).bfloat16()
        dev_extra = extra.cuda()
    assert m.unsupported(s.cuda(), z.cuda(), mask.cuda(), dev_extra) is None
    got = hip_delta(m, s.cuda(), z.cuda(), mask.cuda(), dev_extra).cpu()
    want = ps.attention_pair_bias(s, z, mask, m.state_dict(), n_head=heads,
                                  extra_bias=extra.double(), dtype=torch.float64) - s.double()
    _check(got, want, f"attention_pair_bias extra bias {form}")
    plain = ps.attention_pair_bias(s, z, mask, m.state_dict(), n_head=heads, dtype=torch.float64) - s.double()
    assert ps.rel_rms(plain, want) > 0.1  # the bias matters at this size


def test_attention_pair_bias_masking_is_exact_and_empty_rows_are_zero():
    n, length = 96, 61
    s, z, mask = _inputs(n, 384, [length, 0], seed=11)
    m = _apb(384, 16, gate_bias=0.0, seed=12)
    a = hip_delta(m, s.cuda(), z.cuda(), mask.cuda()).cpu()
    s2, z2 = s.clone(), z.clone()
    s2[0, length:] = 5.0
    z2[0, length:] = -4.0
    z2[0, :, length:] = 9.0
    b = hip_delta(m, s2.cuda(), z2.cuda(), mask.cuda()).cpu()
    assert torch.equal(a[0, :length], b[0, :length])
    assert torch.equal(a[1], torch.zeros_like(a[1]))  # no valid key: zero update
    out = m(s.cuda(), z.cuda(), mask.cuda()).cpu()
    assert torch.equal(out[1], s[1])


def test_attention_pair_bias_large_logits_stay_finite():
    n = 64
    s, z, mask = _inputs(n, 384, [50], seed=21)
    m = _apb(384, 16, gate_bias=0.0, seed=22)
    with torch.no_grad():
        m.to_bias.weight.mul_(40.0)  # pair logits of several hundred nats
    got = hip_delta(m, s.cuda(), z.cuda(), mask.cuda()).cpu()
    assert torch.isfinite(got.float()).all()
    want = ps.attention_pair_bias(s, z, mask, m.state_dict(), n_head=16, dtype=torch.float64) - s.double()
    _check(got, want, "attention_pair_bias large logits")


@pytest.mark.parametrize("d,factor,shape", [(384, 4, (2, 77)), (256, 2, (1, 130)), (64, 4, (3, 33))])
def test_wide_transition_matches_oracle(d, factor, shape):
    g = torch.Generator().manual_seed(d + factor)
    x = torch.randn(*shape, d, generator=g).bfloat16()
    m = randomise(factories.transition(d, factor), seed=d).cuda()
    m.set_backend("hip")
    assert m.unsupported(x.cuda()) is None
    got = hip_delta(m, x.cuda()).cpu()
    want = ps.transition(x, m.state_dict(), dtype=torch.float64) - x.double()
    _check(got, want, f"transition d={d} x{factor} rows={shape}")
    full = m(x.cuda()).cpu()
    _check(full, want + x.double(), "transition residual")


def test_trunk_width_single_track_at_full_size_is_finite_and_deterministic():
    n, length = 512, 437
    s, z, mask = _inputs(n, 384, [length], seed=31)
    m = _apb(384, 16, gate_bias=0.0, seed=32)
    tr = randomise(factories.transition(384, 4), seed=33).cuda()
    tr.set_backend("hip")
    sc, zc, mc = s.cuda(), z.cuda(), mask.cuda()
    a = tr(m(sc, zc, mc))
    b = tr(m(sc, zc, mc))
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)

"""GPU parity of the outer product mean against the CPU oracle (gfx950 only).

Seeded fp32 draws rounded to bf16 feed both sides; the oracle runs in fp64 on the module's
fp32 parameters. The update is compared with rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref|
(the kernels round the projections and the per-pair outer products to bf16 before the output
projection, as the reference's bf16 path does). Masking is exact: the update does not depend
on the content of masked MSA entries, bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import factories
from foldforge_amd.trunk import randomise
from oracle import pairstack as ps
from tests.hip_calls import hip_forward

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


def _inputs(batch: int, depth: int, n: int, cm: int, seed: int, keep: float = 0.8):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(batch, depth, n, cm, generator=g).bfloat16()
    rows = torch.rand(batch, depth, n, generator=g) < keep
    rows[:, 0] = True  # every token has at least one MSA entry
    return m, rows


def _opm(cm: int, seed: int, **form):
    mod = randomise(factories.outer_product_mean(cm, 128, 32, **form), seed=seed).cuda()
    mod.set_backend("hip")
    return mod


FORMS = {
    "af3": dict(count_offset=1e-3, normalize_before_proj=False),
    "clamp": dict(count_offset=None, normalize_before_proj=False),
    "before_proj": dict(count_offset=None, normalize_before_proj=True),
    "rf3_bias": dict(count_offset=1e-3, normalize_before_proj=False, projection_bias=True),
}


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("batch,depth,n,cm", [(1, 5, 16, 64), (1, 33, 50, 64), (2, 64, 41, 128),
                                              (1, 1, 9, 64), (1, 100, 130, 64)])
def test_outer_product_mean_matches_oracle(form, batch, depth, n, cm):
    m, rows = _inputs(batch, depth, n, cm, seed=depth + n + cm)
    mod = _opm(cm, seed=n, **FORMS[form])
    mc, rc = m.cuda(), rows.cuda()
    got = hip_forward(mod, mc, rc).cpu()
    oracle_form = {k: v for k, v in FORMS[form].items() if k != "projection_bias"}
    want = ps.outer_product_mean(m, rows, mod.state_dict(), dtype=torch.float64, **oracle_form)
    _check(got, want, f"opm {form} B={batch} S={depth} n={n} c_m={cm}")
    pair = torch.randn(batch, n, n, 128, generator=torch.Generator().manual_seed(3)).bfloat16()
    full = hip_forward(mod, mc, rc, residual=pair.cuda()).cpu()
    _check(full, want + pair.double(), f"opm {form} residual")


def test_outer_product_mean_masked_entries_do_not_leak_and_empty_tokens_use_the_clamp():
    batch, depth, n, cm = 1, 40, 70, 64
    m, rows = _inputs(batch, depth, n, cm, seed=5, keep=0.6)
    rows[0, :, 13] = False  # a token without any MSA entry: count 0, divisor max(0, 1)
    mod = _opm(cm, seed=6, count_offset=None, normalize_before_proj=False)
    a = hip_forward(mod, m.cuda(), rows.cuda()).cpu()
    m2 = m.clone()
    m2[~rows] = 7.0
    b = mod(m2.cuda(), rows.cuda()).cpu()
    assert torch.equal(a, b)
    want = ps.outer_product_mean(m, rows, mod.state_dict(), count_offset=None, dtype=torch.float64)
    _check(a, want, "opm clamp with an empty token")
    # the empty token's row and column are the output bias (zero products, divisor 1)
    bias = mod.to_out.bias.detach().cpu().bfloat16()
    assert torch.equal(a[0, 13, :], bias.expand(n, 128))
    assert torch.equal(a[0, :, 13], bias.expand(n, 128))


def test_outer_product_mean_full_size_matches_the_pytorch_backend():
    """S = 512 MSA rows, L = 384 tokens (the reference's op-table shape), AF3 form."""
    batch, depth, n, cm = 1, 512, 384, 64
    m, rows = _inputs(batch, depth, n, cm, seed=21, keep=0.9)
    mod = _opm(cm, seed=22, count_offset=1e-3, normalize_before_proj=False)
    mc, rc = m.cuda(), rows.cuda()
    with torch.no_grad():
        a = mod(mc, rc)
        b = mod(mc, rc)
        mod.set_backend("pytorch")
        ref = mod(mc, rc).double()
        mod.set_backend("hip")
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)
    _check(a.cpu(), ref.cpu(), "opm full size vs pytorch backend")


@pytest.mark.parametrize("batch,depth,n,cm,cz", [(1, 5, 16, 64, 256), (1, 33, 50, 64, 256), (2, 40, 23, 128, 128),
                                                 (1, 100, 130, 64, 256)])
def test_grouped_outer_product_mean_matches_oracle(batch, depth, n, cm, cz):
    """Chai-1's grouped form (8 groups of 8 channels, products within each group summed over the
    MSA rows, the product norm at eps 0.1, no count division; ``legacy/primitives.py:122-136``)."""
    m, rows = _inputs(batch, depth, n, cm, seed=depth + n + cz)
    mod = randomise(factories.outer_product_mean(cm, cz, 64, groups=8), seed=n + 1).cuda()
    mod.set_backend("hip")
    assert mod.unsupported(m.cuda(), rows.cuda()) is None
    mc, rc = m.cuda(), rows.cuda()
    got = hip_forward(mod, mc, rc).cpu()
    want = ps.outer_product_mean(m, rows, mod.state_dict(), groups=8, dtype=torch.float64)
    _check(got, want, f"opm grouped B={batch} S={depth} n={n} c_m={cm} c_z={cz}")
    pair = torch.randn(batch, n, n, cz, generator=torch.Generator().manual_seed(4)).bfloat16()
    full = hip_forward(mod, mc, rc, residual=pair.cuda()).cpu()
    _check(full, want + pair.double(), "opm grouped residual")
    # masked MSA entries take no part, bit for bit
    m2 = m.clone()
    m2[~rows] = -9.0
    assert torch.equal(hip_forward(mod, m2.cuda(), rc).cpu(), got)

"""GPU parity of the engine's kernel-function entry points that are not whole ops:
``layer_norm_linear`` (LayerNorm prologue + projection + bias + activation) and ``swiglu_ffn``
(the transition's body), through the C-ABI, against the fp64 oracle. Bar: the per-op
tolerance, rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref|; outputs in place where the
header allows it.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import kernels
from oracle import pairstack as ps

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from foldforge_amd import _native

    _native.lib()


def _check(got, want, what):
    rr, ma = ps.rel_rms(got, want), ps.max_abs(got, want)
    ref = want.abs().max().item()
    print(f"{what}: rel_rms={rr:.2e} max_abs={ma:.2e} max_ref={ref:.2e}", flush=True)
    assert rr <= 1e-2 and ma <= 4e-2 * ref, what


@pytest.mark.parametrize("rows,d_in,d_out", [(777, 128, 516 - 4), (4099, 128, 640), (300, 384, 96), (65, 768, 32)])
@pytest.mark.parametrize("activation", ["none", "sigmoid", "silu", "relu"])
def test_layer_norm_linear_matches_oracle(rows, d_in, d_out, activation):
    g = torch.Generator().manual_seed(rows + d_out)
    x = (torch.randn(rows, d_in, generator=g) * 1.5 + 0.2).bfloat16()
    lw = 1 + 0.1 * torch.randn(d_in, generator=g)
    lb = 0.05 * torch.randn(d_in, generator=g)
    w = 0.08 * torch.randn(d_out, d_in, generator=g)
    b = 0.05 * torch.randn(d_out, generator=g)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = kernels.layer_norm_linear(x.cuda(), lw.cuda(), lb.cuda(), w.cuda(), b.cuda(), activation=activation,
                                        out_dtype=out_dtype).cpu()
        assert got.dtype == out_dtype and got.shape == (rows, d_out)
        want = ps.layer_norm_linear(x.double(), lw.double(), lb.double(), w.double(), b.double(),
                                    activation=activation, dtype=torch.float64)
        _check(got, want, f"layer_norm_linear {rows}x{d_in}->{d_out} {activation} {out_dtype}")


def test_layer_norm_linear_without_affine_or_bias():
    g = torch.Generator().manual_seed(71)
    x = torch.randn(2, 33, 17, 128, generator=g).bfloat16()
    w = 0.08 * torch.randn(128, 128, generator=g)
    got = kernels.layer_norm_linear(x.cuda(), None, None, w.cuda()).cpu()
    assert got.shape == (2, 33, 17, 128)
    want = ps.layer_norm_linear(x.double(), None, None, w.double(), dtype=torch.float64)
    _check(got, want, "layer_norm_linear, no affine, no bias")


@pytest.mark.parametrize("rows,d,hidden", [(2 * 96 * 96, 128, 512), (513, 384, 1536), (77, 64, 128),
                                           (300, 768, 1536)])
def test_swiglu_ffn_matches_oracle(rows, d, hidden):
    g = torch.Generator().manual_seed(rows + d)
    x = torch.randn(rows, d, generator=g).bfloat16()
    res = torch.randn(rows, d, generator=g).bfloat16()
    wa = 0.08 * torch.randn(hidden, d, generator=g)
    wb = 0.08 * torch.randn(hidden, d, generator=g)
    wo = 0.08 * torch.randn(d, hidden, generator=g)
    got = kernels.swiglu_ffn(x.cuda(), wa.cuda(), wb.cuda(), wo.cuda()).cpu()
    want = ps.swiglu_ffn(x.double(), wa.double(), wb.double(), wo.double(), dtype=torch.float64)
    _check(got, want, f"swiglu_ffn {rows}x{d} hidden {hidden}")
    xc = x.cuda()
    full = kernels.swiglu_ffn(xc, wa.cuda(), wb.cuda(), wo.cuda(), residual=res.cuda()).cpu()
    _check(full, want + res.double(), "swiglu_ffn with residual")
    inplace = kernels.swiglu_ffn(xc, wa.cuda(), wb.cuda(), wo.cuda(), residual=xc, out=xc)
    assert inplace.data_ptr() == xc.data_ptr()
    assert torch.equal(inplace.cpu(), kernels.swiglu_ffn(x.cuda(), wa.cuda(), wb.cuda(), wo.cuda(),
                                                         residual=x.cuda()).cpu())

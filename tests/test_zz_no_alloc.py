"""GPU: ``ffk_transition_noalloc`` -- the transition with its scratch in the library's static
device array instead of a caller workspace -- called through the C-ABI, against the existing
``ffk_transition`` (with a workspace) on the same inputs: bitwise equal, on two calls in a row
with the second one smaller (the array keeps the first call's contents), for the fused width
(128 x 4, packed weights in the scratch) and the token-row GEMM widths (hidden rows in the
scratch). A call whose scratch would exceed the array is refused with FFK_ERR_WORKSPACE and a
message, before anything is launched.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import _native, factories, kernels
from foldforge_amd.trunk import randomise

pytestmark = pytest.mark.gpu

FFK_ERR_WORKSPACE = 2
SCRATCH_BYTES = 4 << 20


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    _native.lib()


def _module(d: int, factor: int, seed: int):
    return randomise(factories.transition(d, factor), seed=seed).cuda()


def _noalloc(m, x: torch.Tensor, out: torch.Tensor, residual: bool) -> int:
    d = x.shape[-1]
    return _native.lib().ffk_transition_noalloc(
        x.data_ptr(), m.ln_in.weight.data_ptr(), m.ln_in.bias.data_ptr(), m.expand_a.weight.data_ptr(),
        m.expand_b.weight.data_ptr(), m.squeeze.weight.data_ptr(), out.data_ptr(), x.numel() // d, d, m.n,
        int(residual), float(m.ln_in.eps), torch.cuda.current_stream().cuda_stream)


def _with_workspace(m, x: torch.Tensor, residual: bool) -> torch.Tensor:
    return kernels.transition(x, ln_weight=m.ln_in.weight, ln_bias=m.ln_in.bias, expand_a=m.expand_a.weight,
                              expand_b=m.expand_b.weight, squeeze=m.squeeze.weight, residual=residual,
                              eps=m.ln_in.eps)


@pytest.mark.parametrize("d,factor,shapes", [
    (128, 4, [(2, 96, 96), (1, 41, 37)]),   # fused kernel: packed weights in the scratch
    (384, 4, [(1, 682), (2, 77)]),          # token-row GEMMs: 682 rows fill the 4 MiB scratch
    (64, 2, [(5000,), (33,)]),
])
def test_noalloc_matches_the_workspace_entry_point(d, factor, shapes):
    m = _module(d, factor, seed=d + factor)
    g = torch.Generator().manual_seed(d)
    for call, shape in enumerate(shapes):
        residual = call == 0
        x = torch.randn(*shape, d, generator=g).bfloat16().cuda()
        want = _with_workspace(m, x, residual)
        out = torch.full_like(x, float("nan"))
        status = _noalloc(m, x, out, residual)
        assert status == 0, _native.lib().ffk_last_error().decode()
        torch.cuda.synchronize()
        print(f"noalloc transition d={d} x{factor} rows={x.numel() // d} residual={residual}: "
              f"equal={torch.equal(out, want)}", flush=True)
        assert torch.equal(out, want)


def test_noalloc_refuses_a_call_beyond_its_scratch():
    m = _module(384, 4, seed=3)
    rows = SCRATCH_BYTES // (4 * 384 * 4) + 1  # one row more than the array holds
    x = torch.zeros(rows, 384, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros_like(x)
    status = _noalloc(m, x, out, True)
    message = _native.lib().ffk_last_error().decode()
    assert status == FFK_ERR_WORKSPACE, (status, message)
    assert "static scratch" in message and str(rows) in message
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0  # nothing ran

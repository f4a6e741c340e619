"""GPU parity of the HIP kernels against the CPU oracle (gfx950 only).

Inputs are seeded fp32 draws rounded to bf16; the oracle gets the same rounded values and
the module's fp32 parameters and runs in fp64. Op-level parity compares the bare update
``f(x)`` (``residual=False``: the bf16 residual stream would otherwise hide errors in f)
on the valid pairs, to the tolerance stated for bf16 kernels against an fp32 reference:
rel-RMS <= 1e-2 and max-abs <= 4e-2 * max|ref|. Masking is exact: a masked key gets zero
weight, so the valid region is bitwise independent of whatever the padded positions hold.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import factories, kernels
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

    _native.lib()  # a missing library is an error on a GPU box, not a skip
    torch.manual_seed(0)


def _pair(n: int, batch: int = 1, seed: int = 0, lengths=None):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(batch, n, n, 128, generator=g).bfloat16()
    mask = torch.ones(batch, n, dtype=torch.bool)
    for b, length in enumerate(lengths or []):
        mask[b, length:] = False
    return z, mask


def _check(got: torch.Tensor, want: torch.Tensor, where: torch.Tensor | None, what: str) -> None:
    rr = ps.rel_rms(got, want, where)
    ma = ps.max_abs(got, want, where)
    ref = want.double()[where].abs().max().item() if where is not None else want.abs().max().item()
    print(f"{what}: rel_rms={rr:.2e} max_abs={ma:.2e} max_ref={ref:.2e}", flush=True)
    assert rr <= REL_RMS, f"{what}: rel-RMS {rr:.3e}"
    assert ma <= MAX_ABS * ref, f"{what}: max-abs {ma:.3e} vs {MAX_ABS} * {ref:.3e}"


def _pairs(mask: torch.Tensor) -> torch.Tensor:
    return mask[:, :, None] & mask[:, None, :]


def test_layer_norm_matches_oracle():
    g = torch.Generator().manual_seed(1)
    for rows, cols, dtype in ((4097, 128, torch.bfloat16), (300, 384, torch.bfloat16), (77, 100, torch.float32)):
        x = (torch.randn(rows, cols, generator=g) * 2 + 0.5).to(dtype)
        w = 1 + 0.1 * torch.randn(cols, generator=g)
        b = 0.05 * torch.randn(cols, generator=g)
        got = kernels.layer_norm(x.cuda(), w.cuda(), b.cuda(), 1e-5).cpu()
        want = ps.layer_norm(x.double(), w.double(), b.double(), 1e-5)
        assert got.dtype == dtype
        _check(got, want, None, f"layer_norm {rows}x{cols} {dtype}")


def test_layer_norm_multi_pass_and_no_affine():
    # more rows than one pass of the 128-wide kernel's workgroups (32 rows each, at most 32 per
    # CU), with a ragged tail; and the null weight / bias pointers of the C-ABI
    g = torch.Generator().manual_seed(2)
    rows = 32 * 32 * torch.cuda.get_device_properties(0).multi_processor_count * 2 + 37
    x = torch.randn(rows, 128, generator=g).bfloat16()
    w = 1 + 0.1 * torch.randn(128, generator=g)
    b = 0.05 * torch.randn(128, generator=g)
    got = kernels.layer_norm(x.cuda(), w.cuda(), b.cuda(), 1e-5).cpu()
    _check(got, ps.layer_norm(x.double(), w.double(), b.double(), 1e-5), None, f"layer_norm {rows}x128")
    x = x[:4099]
    got = kernels.layer_norm(x.cuda(), None, None, 1e-5).cpu()
    _check(got, ps.layer_norm(x.double(), None, None, 1e-5), None, "layer_norm without affine")


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,lengths", [(64, None), (100, [77]), (130, [130, 41]), (256, [256, 203])])
def test_trimul_matches_oracle(outgoing, n, lengths):
    batch = len(lengths) if lengths else 1
    z, mask = _pair(n, batch, seed=n, lengths=lengths)
    m = randomise(factories.triangle_multiplication(128, outgoing=outgoing), seed=n).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=outgoing, dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"trimul outgoing={outgoing} n={n}")
    full = hip_forward(m, z.cuda(), mask.cuda()).cpu()
    torch.testing.assert_close(full.float(), (z.float() + got.float()), atol=3e-2, rtol=1e-2)


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,lengths", [(64, None), (100, [77, 61])])
def test_length_divided_trimul_matches_oracle(outgoing, n, lengths):
    """RoseTTAFold3's exact triangle multiplication (TriangleMultiplicationRF3) on hip: the real
    length (77 of 100 in the ragged case: the longest element) is counted on the device."""
    batch = len(lengths) if lengths else 1
    z, mask = _pair(n, batch, seed=3 * n, lengths=lengths)
    m = randomise(factories.triangle_multiplication(128, outgoing=outgoing, divide_by_length=True),
                  seed=n + 1).cuda()
    assert m.divide_by_length
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_multiplication(z, mask, m.state_dict(), outgoing=outgoing, length_divided=True,
                                      dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"trimul RF3 outgoing={outgoing} n={n}")


def _lineage_oracle(m, z, mask):
    return ps.triangle_attention(z, mask, m.state_dict(), starting=m.starting, n_head=m.n_head,
                                 transposed_bias=m.transposed_bias,
                                 untransposed_output=m.untransposed_output,
                                 dual_output=m.dual_output, dtype=torch.float64) - z.double()


def _lineage_module(key: str, c: int, heads: int, d: int, starting: bool, seed: int):
    m = randomise(factories.triangle_attention(c, heads, starting=starting, model=key,
                                               d_hidden=heads * d), seed=seed)
    if m.projection_bias:
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            m.to_gate.bias.copy_(torch.randn(m.to_gate.bias.shape, generator=g))
            m.to_out.bias.copy_(0.3 * torch.randn(m.to_out.bias.shape, generator=g))
    return m.cuda()


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("key", ["rf3", "chai1", "chai1_confidence"])
def test_triattn_lineage_forms_match_oracle(starting, key):
    """RoseTTAFold3's projection biases and Chai-1's untransposed / dual outputs on the fused
    kernels, ragged batch of 2, out of place (the same forms in place, bitwise against out of
    place: ``test_gpu_configs.py::test_pair_ops_in_place``)."""
    n, lengths = 100, [100, 61]
    z, mask = _pair(n, 2, seed=11 * n, lengths=lengths)
    m = _lineage_module(key, 128, 4, 32, starting, seed=5)
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    where = _pairs(mask)
    if key.startswith("chai1"):  # the transposed parts reach every pair with a real mirror
        where = where & where.transpose(1, 2)
    _check(got, _lineage_oracle(m, z, mask), where, f"triattn {key} starting={starting}")
    full = hip_forward(m, z.cuda(), mask.cuda()).cpu()
    torch.testing.assert_close(full.float(), z.float() + got.float(), atol=3e-2, rtol=1e-2)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("model", ["af3", "protenix"])
@pytest.mark.parametrize("n,lengths", [(64, None), (100, [61]), (160, [160, 129])])
def test_triattn_matches_oracle(starting, model, n, lengths):
    batch = len(lengths) if lengths else 1
    z, mask = _pair(n, batch, seed=7 * n, lengths=lengths)
    m = randomise(factories.triangle_attention(128, 4, starting=starting, model=model), seed=n).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_attention(z, mask, m.state_dict(), starting=starting, n_head=4,
                                 transposed_bias=m.transposed_bias, dtype=torch.float64) - z.double()
    _check(got, want, _pairs(mask), f"triattn starting={starting} {model} n={n}")


def test_triattn_single_op_workload_shape():
    """The single-op workload the CPU baseline times: starting node on z [1, 128, 128, 128]
    ~N(0, 1) (seed 0), 4 heads x 32, all-ones mask, random init from seed 0."""
    z, mask = _pair(128, 1, seed=0)
    m = randomise(factories.triangle_attention(128, 4, starting=True, model="af3"), seed=0).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda(), mask.cuda()).cpu()
    want = ps.triangle_attention(z, mask, m.state_dict(), starting=True, n_head=4, dtype=torch.float64) - z.double()
    _check(got, want, None, "triattn starting af3 n=128 (single-op workload)")


@pytest.mark.parametrize("n,batch", [(72, 2), (300, 1)])
def test_transition_matches_oracle(n, batch):
    """(300, 1): 90000 positions = 703 full tiles of 128 and a ragged one, more tiles than the
    persistent grid holds, so workgroups carry the weight stream from one tile into the next."""
    z, _ = _pair(n, batch, seed=3)
    m = randomise(factories.transition(128, 4), seed=5).cuda()
    m.set_backend("hip")
    got = hip_delta(m, z.cuda()).cpu()
    want = ps.transition(z, m.state_dict(), dtype=torch.float64) - z.double()
    _check(got, want, None, f"transition n={n} batch={batch}")


def test_padding_is_bitwise_invisible_to_the_valid_region():
    n, length = 96, 70
    z, mask = _pair(n, 1, seed=11, lengths=[length])
    z2 = z.clone()
    g = torch.Generator().manual_seed(12)
    z2[0, length:] = (100 * torch.randn(n - length, n, 128, generator=g)).bfloat16()
    z2[0, :, length:] = (-50 * torch.randn(n, n - length, 128, generator=g)).bfloat16()
    block = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3"), seed=13).cuda()
    block.set_backend("hip")
    a = block(z.cuda(), mask.cuda()).cpu()
    b = block(z2.cuda(), mask.cuda()).cpu()
    assert torch.equal(a[0, :length, :length], b[0, :length, :length])


def test_flash_core_large_logits_and_exact_masking():
    """The core alone, against an fp32 torch softmax, with logits of several hundred nats
    (the failure of a max-free softmax) and masked keys whose values must not matter."""
    B, H, R, n = 1, 4, 4, 256
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, H, R, n, 32, generator=g)
    k = torch.randn(B, H, R, n, 32, generator=g)
    v = torch.randn(B, H, R, n, 32, generator=g)
    bias = 300 * torch.randn(B, H, n, n, generator=g)  # log2 units: up to ~1000 nats
    keep = torch.rand(n, generator=g) > 0.3
    keep[:40] = False  # the first key tiles are fully masked: the offset is set later
    bias_m = torch.where(keep[None, None, None, :], bias, torch.tensor(float("-inf")))
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    vt = kernels.flash_v_layout(vb.transpose(-1, -2))
    blk = kernels.blocked_bias(bias_m)
    out = torch.zeros(B, R, n, H * 32, dtype=torch.bfloat16, device="cuda")
    kernels.flash_attention_bias(qb.cuda(), kb.cuda(), vt.cuda(), blk.cuda(), out, rows_valid=R, n_valid=n)
    logits = qb.float() @ kb.float().transpose(-1, -2) + bias_m[:, :, None]  # [B,H,R,n,n] (log2)
    w = torch.softmax(logits * 0.6931471805599453, dim=-1)
    want = (w @ vb.float()).permute(0, 2, 3, 1, 4).reshape(B, R, n, H * 32)
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    _check(got, want.double(), None, "flash core, large logits")
    v2 = vb.clone()
    v2[..., ~keep, :] = 1e4
    vt2 = kernels.flash_v_layout(v2.transpose(-1, -2))
    out2 = torch.zeros_like(out)
    kernels.flash_attention_bias(qb.cuda(), kb.cuda(), vt2.cuda(), blk.cuda(), out2, rows_valid=R, n_valid=n)
    assert torch.equal(out.cpu(), out2.cpu())


@pytest.mark.parametrize("q_scale", [4.0, 25.0])
def test_flash_core_large_qk_logits(q_scale):
    """Logits dominated by q . k (std 4 x 5.7 and 25 x 5.7 log2 units: about 16 and 100 nats,
    the trained-weight regime), unit-scale bias, a masked key block: the rows' offsets rise
    during the key loop (rescale of l and O), and the result still matches an fp32 softmax."""
    B, H, R, n = 1, 4, 8, 256
    g = torch.Generator().manual_seed(23)
    q = (q_scale * torch.randn(B, H, R, n, 32, generator=g)).bfloat16()
    k = torch.randn(B, H, R, n, 32, generator=g).bfloat16()
    v = torch.randn(B, H, R, n, 32, generator=g).bfloat16()
    bias = torch.randn(B, H, n, n, generator=g)
    bias[..., 96:128] = float("-inf")
    out = torch.zeros(B, R, n, H * 32, dtype=torch.bfloat16, device="cuda")
    kernels.flash_attention_bias(q.cuda(), k.cuda(), kernels.flash_v_layout(v.transpose(-1, -2)).cuda(),
                                 kernels.blocked_bias(bias).cuda(), out, rows_valid=R, n_valid=n)
    logits = q.double() @ k.double().transpose(-1, -2) + bias.double()[:, :, None]
    w = torch.softmax(logits * 0.6931471805599453, dim=-1)
    want = (w @ v.double()).permute(0, 2, 3, 1, 4).reshape(B, R, n, H * 32)
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    _check(got, want, None, f"flash core, q.k logits x{q_scale}")


def test_flash_core_moderate_logits_and_partial_query_block():
    """Unit-scale logits (the lazy offset never moves after the first tile), n = 384 so the
    last 256-query block is half outside, and only some rows / queries are stored."""
    B, H, R, n = 2, 4, 8, 384
    g = torch.Generator().manual_seed(22)
    q = (0.3 * torch.randn(B, H, R, n, 32, generator=g)).bfloat16()
    k = torch.randn(B, H, R, n, 32, generator=g).bfloat16()
    v = torch.randn(B, H, R, n, 32, generator=g).bfloat16()
    bias = 2 * torch.randn(B, H, n, n, generator=g)
    bias[1, :, :, 300:] = float("-inf")
    rows_valid, n_valid = 6, 350
    out = torch.zeros(B, R, n_valid, H * 32, dtype=torch.bfloat16, device="cuda")
    kernels.flash_attention_bias(q.cuda(), k.cuda(), kernels.flash_v_layout(v.transpose(-1, -2)).cuda(),
                                 kernels.blocked_bias(bias).cuda(), out, rows_valid=rows_valid, n_valid=n_valid)
    w = torch.softmax((q.float() @ k.float().transpose(-1, -2) + bias[:, :, None]) * 0.6931471805599453, dim=-1)
    want = (w @ v.float()).permute(0, 2, 3, 1, 4).reshape(B, R, n, H * 32)[:, :, :n_valid]
    got = out.cpu().float()
    _check(got[:, :rows_valid], want[:, :rows_valid].double(), None, "flash core, partial blocks")
    assert (got[:, rows_valid:] == 0).all()


def test_no_valid_key_gives_identity_update():
    z, mask = _pair(64, 1, seed=31, lengths=[0])
    m = randomise(factories.triangle_attention(128, 4, starting=True, model="af3"), seed=1).cuda()
    m.set_backend("hip")
    got = hip_forward(m, z.cuda(), mask.cuda()).cpu()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, z)  # zero attention output -> zero update

"""Pin the CPU oracle (``oracle/pairstack.py``) before trusting it.

Checks, per function: the committed brute-force fixtures (``tests/golden``), fresh
brute-force loops (``oracle/brute.py``), library routines that fix the maths
(``torch.nn.functional.layer_norm``, ``scaled_dot_product_attention``), and invariants a
plausible mistake breaks (outgoing/incoming transpose identity with swapped branches,
softmax shift invariance, key-mask exactness, large-logit stability, the
transposed-bias start/end identity). A planted mistake in the oracle must fail one of
them: see ``test_a_planted_mistake_is_caught``.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import pairstack as ps

GOLDEN = Path(__file__).resolve().parent / "golden" / "pairstack_tiny.npz"
F64 = torch.float64


def _golden() -> dict[str, dict]:
    data = np.load(GOLDEN)
    cases: dict[str, dict] = {}
    for key in data.files:
        case, rest = key.split("/", 1)
        entry = cases.setdefault(case, {"p": {}})
        if rest.startswith("p/"):
            entry["p"][rest[2:]] = torch.from_numpy(data[key])
        else:
            entry[rest] = torch.from_numpy(data[key])
    return cases


def _rand_params(shapes: dict[str, tuple[int, ...]], seed: int) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in shapes.items():
        noise = torch.randn(shape, generator=g, dtype=F64)
        out[name] = 0.3 * noise if len(shape) > 1 else (1 + 0.1 * noise if name.endswith("weight") else 0.1 * noise)
    return out


def _tm_shapes(c: int, h: int) -> dict[str, tuple[int, ...]]:
    return {"ln_pair.weight": (c,), "ln_pair.bias": (c,), "to_left.weight": (h, c),
            "to_right.weight": (h, c), "to_left_gate.weight": (h, c), "to_right_gate.weight": (h, c),
            "ln_out.weight": (h,), "ln_out.bias": (h,), "to_out.weight": (c, h), "to_gate.weight": (c, c)}


def _ta_shapes(c: int, heads: int, d: int) -> dict[str, tuple[int, ...]]:
    return {"ln_pair.weight": (c,), "ln_pair.bias": (c,), "to_bias.weight": (heads, c),
            "to_query.weight": (heads * d, c), "to_key.weight": (heads * d, c),
            "to_value.weight": (heads * d, c), "to_gate.weight": (heads * d, c),
            "to_out.weight": (c, heads * d)}


def _np(p: dict[str, torch.Tensor]) -> dict[str, np.ndarray]:
    return {k: v.numpy() for k, v in p.items()}


# ----------------------------------------------------------------------------- fixtures
def test_golden_fixtures_match_the_oracle():
    cases = _golden()
    assert len(cases) == 8
    for name, c in cases.items():
        p = c["p"]
        if name.startswith("trimul"):
            got = ps.triangle_multiplication(c["z"], c["mask"], p, outgoing=name.endswith("out"), dtype=F64)
        elif name.startswith("triattn"):
            got = ps.triangle_attention(c["z"], c["mask"], p, starting="_start_" in name, n_head=2,
                                        transposed_bias=name.endswith("tb"), dtype=F64)
        elif name == "transition":
            got = ps.transition(c["x"], p, dtype=F64)
        else:
            got = ps.attention_pair_bias(c["s"], c["z"], c["mask"], p, n_head=3, gate_bias=0.5, dtype=F64)
        torch.testing.assert_close(got, c["expected"], rtol=1e-10, atol=1e-10, msg=name)


def test_golden_fixtures_are_reproduced_by_the_brute_force():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN.with_name("make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh = mod.cases()
    data = np.load(GOLDEN)
    assert set(fresh) == set(data.files)
    for k in data.files:
        np.testing.assert_allclose(fresh[k], data[k], rtol=0, atol=1e-12, err_msg=k)


# ----------------------------------------------------------------------------- LayerNorm
def test_layer_norm_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 128, generator=g, dtype=F64) * 3 + 2
    w = torch.randn(128, generator=g, dtype=F64)
    b = torch.randn(128, generator=g, dtype=F64)
    got = ps.layer_norm(x, w, b, 1e-5)
    torch.testing.assert_close(got, F.layer_norm(x, (128,), w, b, 1e-5))
    row = x[3]
    mu = row.sum() / 128
    var = ((row - mu) ** 2).sum() / 128
    torch.testing.assert_close(got[3], (row - mu) / torch.sqrt(var + 1e-5) * w + b)
    # no affine: zero mean, unit (biased) variance up to eps
    y = ps.layer_norm(x, None, None, 0.0)
    torch.testing.assert_close(y.mean(-1), torch.zeros(7, dtype=F64), atol=1e-12, rtol=0)
    torch.testing.assert_close(y.var(-1, unbiased=False), torch.ones(7, dtype=F64))


# ----------------------------------------------------------------------------- triangle multiplication
@pytest.mark.parametrize("outgoing", [True, False])
def test_trimul_matches_brute_force(outgoing):
    n, c, h = 6, 5, 3
    p = _rand_params(_tm_shapes(c, h), 11)
    g = torch.Generator().manual_seed(12)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[1, -2:] = False
    got = ps.triangle_multiplication(z, mask, p, outgoing=outgoing, dtype=F64)
    want = brute.triangle_multiplication(z.numpy(), mask.numpy(), _np(p), outgoing=outgoing)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("outgoing", [True, False])
def test_length_divided_trimul_matches_brute_force(outgoing):
    """RoseTTAFold3's exact form: the length is the count of columns real in ANY batch element
    (here 6 of 7: column 6 is padding in both elements, column 5 only in the second)."""
    n, c, h = 7, 5, 3
    p = _rand_params(_tm_shapes(c, h), 13)
    g = torch.Generator().manual_seed(14)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 5:] = False
    mask[1, 6] = False
    got = ps.triangle_multiplication(z, mask, p, outgoing=outgoing, length_divided=True, dtype=F64)
    want = brute.triangle_multiplication(z.numpy(), mask.numpy(), _np(p), outgoing=outgoing,
                                         length_divided=True)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)
    plain = ps.triangle_multiplication(z, mask, p, outgoing=outgoing, dtype=F64)
    assert (got - plain).abs().max() > 1e-3  # the division changes the centre norm's eps share


def test_length_divided_trimul_is_the_centre_norm_with_eps_times_length_squared():
    """LN(P / L; eps) = LN(P; eps L^2): the identity the kernels use to keep P undivided."""
    n, c, h, eps = 6, 4, 3, 1e-2
    p = _rand_params(_tm_shapes(c, h), 15)
    g = torch.Generator().manual_seed(16)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, -1] = False  # L = 5
    divided = ps.triangle_multiplication(z, mask, p, outgoing=True, length_divided=True, eps=eps,
                                         dtype=F64)
    # the same op with the centre norm's eps scaled by L^2 and no division: split the two
    # norms by running the pair norm at eps and the centre norm at eps * 25 by hand
    x = ps.layer_norm(z, p["ln_pair.weight"], p["ln_pair.bias"], eps)
    pm = (mask[:, :, None] & mask[:, None, :]).to(F64)[..., None]
    a = (x @ p["to_left.weight"].T) * pm * torch.sigmoid(x @ p["to_left_gate.weight"].T)
    b = (x @ p["to_right.weight"].T) * pm * torch.sigmoid(x @ p["to_right_gate.weight"].T)
    pr = torch.einsum("bikc,bjkc->bijc", a, b)
    y = ps.layer_norm(pr, p["ln_out.weight"], p["ln_out.bias"], eps * 25) @ p["to_out.weight"].T
    want = z + y * torch.sigmoid(x @ p["to_gate.weight"].T)
    torch.testing.assert_close(divided, want, rtol=1e-12, atol=1e-12)


def test_trimul_outgoing_is_incoming_on_the_transpose_with_branches_swapped():
    n, c, h = 7, 6, 4
    p = _rand_params(_tm_shapes(c, h), 21)
    g = torch.Generator().manual_seed(22)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, 2] = False
    swapped = dict(p)
    swapped["to_left.weight"], swapped["to_right.weight"] = p["to_right.weight"], p["to_left.weight"]
    swapped["to_left_gate.weight"], swapped["to_right_gate.weight"] = p["to_right_gate.weight"], p["to_left_gate.weight"]
    a = ps.triangle_multiplication(z, mask, p, outgoing=True, dtype=F64)
    b = ps.triangle_multiplication(z.transpose(1, 2), mask, swapped, outgoing=False, dtype=F64).transpose(1, 2)
    torch.testing.assert_close(a, b)


def test_trimul_masked_tokens_contribute_nothing():
    n, c, h = 6, 5, 3
    p = _rand_params(_tm_shapes(c, h), 31)
    g = torch.Generator().manual_seed(32)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, 4:] = False
    z2 = z.clone()
    z2[0, 4:, :, :] = 1e3 * torch.randn(2, n, c, generator=g, dtype=F64)
    z2[0, :, 4:, :] = -1e3
    a = ps.triangle_multiplication(z, mask, p, outgoing=True, dtype=F64)
    b = ps.triangle_multiplication(z2, mask, p, outgoing=True, dtype=F64)
    torch.testing.assert_close(a[0, :4, :4], b[0, :4, :4], rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------------------- triangle attention
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("form", ["rf3", "chai1", "chai1_confidence", "chai1_confidence_biased"])
def test_triattn_forms_match_brute_force(starting, form):
    """The RoseTTAFold3 (gate / output biases) and Chai-1 (untransposed ending output; dual
    output projections) forms against independent loops."""
    n, c, heads, d = 5, 4, 2, 3
    shapes = _ta_shapes(c, heads, d)
    if form in ("rf3", "chai1_confidence_biased"):
        shapes.update({"to_gate.bias": (heads * d,), "to_out.bias": (c,)})
    if form.startswith("chai1_confidence"):
        shapes["to_out_t.weight"] = (c, heads * d)
        if form.endswith("biased"):
            shapes["to_out_t.bias"] = (c,)
    p = _rand_params(shapes, 43)
    g = torch.Generator().manual_seed(44)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 3:] = False
    kw = dict(untransposed_output=form == "chai1", dual_output=form.startswith("chai1_confidence"))
    got = ps.triangle_attention(z, mask, p, starting=starting, n_head=heads, dtype=F64, **kw)
    want = brute.triangle_attention(z.numpy(), mask.numpy(), _np(p), starting=starting,
                                    n_head=heads, **kw)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)


def test_triattn_chai1_forms_reduce_to_the_plain_update():
    """Closed forms: the untransposed ending update is the plain ending update transposed;
    the dual output with a zero second projection is the plain update; with the second
    projection equal to the first it adds the update's own mirror."""
    n, c, heads, d = 6, 4, 2, 2
    p = _rand_params(_ta_shapes(c, heads, d), 45)
    g = torch.Generator().manual_seed(46)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, -2:] = False
    for starting in (True, False):
        plain = ps.triangle_attention(z, mask, p, starting=starting, n_head=heads, dtype=F64) - z
        if not starting:
            untr = ps.triangle_attention(z, mask, p, starting=False, n_head=heads,
                                         untransposed_output=True, dtype=F64) - z
            torch.testing.assert_close(untr, plain.transpose(1, 2), rtol=1e-12, atol=1e-12)
        q = dict(p, **{"to_out_t.weight": torch.zeros(c, heads * d, dtype=F64)})
        dual0 = ps.triangle_attention(z, mask, q, starting=starting, n_head=heads,
                                      dual_output=True, dtype=F64) - z
        torch.testing.assert_close(dual0, plain, rtol=1e-12, atol=1e-12)
        q = dict(p, **{"to_out_t.weight": p["to_out.weight"]})
        dual = ps.triangle_attention(z, mask, q, starting=starting, n_head=heads,
                                     dual_output=True, dtype=F64) - z
        torch.testing.assert_close(dual, plain + plain.transpose(1, 2), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("transposed", [False, True])
def test_triattn_matches_brute_force(starting, transposed):
    n, c, heads, d = 6, 5, 2, 3
    p = _rand_params(_ta_shapes(c, heads, d), 41)
    g = torch.Generator().manual_seed(42)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 1] = False
    mask[1, :] = False  # no valid key at all: the stated zero-output convention
    got = ps.triangle_attention(z, mask, p, starting=starting, n_head=heads,
                                transposed_bias=transposed, dtype=F64, row_chunk=2)
    want = brute.triangle_attention(z.numpy(), mask.numpy(), _np(p), starting=starting,
                                    n_head=heads, transposed_bias=transposed)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)


def test_triattn_core_equals_sdpa_math():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(3, 4, 9, 8, generator=g, dtype=F64) for _ in range(3))
    bias = torch.randn(1, 4, 9, 9, generator=g, dtype=F64)
    keep = torch.ones(1, 1, 1, 9, dtype=torch.bool)
    got = ps._masked_softmax_attention(q, k, v, bias, keep, 8**-0.5)
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=bias.expand(3, 4, 9, 9), scale=8**-0.5)
    torch.testing.assert_close(got, want)


def test_triattn_softmax_shift_invariance_and_mask_exactness():
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(2, 4, 7, 8, generator=g, dtype=F64) for _ in range(3))
    bias = torch.randn(1, 4, 7, 7, generator=g, dtype=F64)
    keep = torch.tensor([True, True, False, True, False, True, True])[None, None, None, :]
    base = ps._masked_softmax_attention(q, k, v, bias, keep, 0.3)
    shifted = ps._masked_softmax_attention(q, k, v, bias + torch.randn(1, 4, 7, 1, generator=g, dtype=F64) * 50,
                                           keep, 0.3)
    torch.testing.assert_close(base, shifted)
    # a masked key's value has no influence at all
    v2 = v.clone()
    v2[..., 2, :] = 1e6
    v2[..., 4, :] = float("nan")
    torch.testing.assert_close(ps._masked_softmax_attention(q, k, torch.nan_to_num(v2, nan=0.0), bias, keep, 0.3), base)


def test_triattn_large_logits_stay_finite_and_match_brute_force():
    n, c, heads, d = 5, 4, 2, 2
    p = _rand_params(_ta_shapes(c, heads, d), 51)
    p["to_bias.weight"] = p["to_bias.weight"] * 150.0  # logits of several hundred nats
    g = torch.Generator().manual_seed(52)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    got = ps.triangle_attention(z, mask, p, starting=True, n_head=heads, dtype=F64)
    assert torch.isfinite(got).all()
    want = brute.triangle_attention(z.numpy(), mask.numpy(), _np(p), starting=True, n_head=heads)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-10, atol=1e-10)


def test_transposed_bias_ending_node_is_starting_node_on_the_transpose():
    n, c, heads, d = 6, 5, 2, 3
    p = _rand_params(_ta_shapes(c, heads, d), 61)
    g = torch.Generator().manual_seed(62)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, 0] = False
    end = ps.triangle_attention(z, mask, p, starting=False, n_head=heads, transposed_bias=True, dtype=F64)
    start_t = ps.triangle_attention(z.transpose(1, 2), mask, p, starting=True, n_head=heads, dtype=F64)
    torch.testing.assert_close(end, start_t.transpose(1, 2))
    # the AF3 (un-transposed bias) ending node is a different function
    af3 = ps.triangle_attention(z, mask, p, starting=False, n_head=heads, transposed_bias=False, dtype=F64)
    assert (af3 - end).abs().max() > 1e-3


# ----------------------------------------------------------------------------- transition / APB
def test_transition_matches_brute_force_and_closed_form():
    c = 6
    p = _rand_params({"ln_in.weight": (c,), "ln_in.bias": (c,), "expand_a.weight": (4 * c, c),
                      "expand_b.weight": (4 * c, c), "squeeze.weight": (c, 4 * c)}, 71)
    g = torch.Generator().manual_seed(72)
    x = torch.randn(2, 3, 4, c, generator=g, dtype=F64)
    got = ps.transition(x, p, dtype=F64)
    np.testing.assert_allclose(got.numpy(), brute.transition(x.numpy(), _np(p)), rtol=1e-11, atol=1e-11)
    h = F.layer_norm(x, (c,), p["ln_in.weight"], p["ln_in.bias"], 1e-5)
    a, b = h @ p["expand_a.weight"].T, h @ p["expand_b.weight"].T
    torch.testing.assert_close(got, x + (a * torch.sigmoid(a) * b) @ p["squeeze.weight"].T)


def test_attention_pair_bias_matches_brute_force():
    n, cs, c, hs = 6, 8, 5, 2
    p = _rand_params({"ln_single.weight": (cs,), "ln_single.bias": (cs,), "to_query.weight": (cs, cs),
                      "to_query.bias": (cs,), "to_key.weight": (cs, cs), "to_value.weight": (cs, cs),
                      "ln_pair.weight": (c,), "to_bias.weight": (hs, c), "to_gate.weight": (cs, cs),
                      "to_out.weight": (cs, cs)}, 81)
    g = torch.Generator().manual_seed(82)
    s = torch.randn(2, n, cs, generator=g, dtype=F64)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, -3:] = False
    got = ps.attention_pair_bias(s, z, mask, p, n_head=hs, gate_bias=-1.0, dtype=F64)
    want = brute.attention_pair_bias(s.numpy(), z.numpy(), mask.numpy(), _np(p), n_head=hs, gate_bias=-1.0)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)
    # the block's extra pair bias: an [N, N] map broadcast over samples and heads
    extra = 2.0 * torch.randn(n, n, generator=g, dtype=F64)
    got = ps.attention_pair_bias(s, z, mask, p, n_head=hs, extra_bias=extra, dtype=F64)
    want = brute.attention_pair_bias(s.numpy(), z.numpy(), mask.numpy(), _np(p), n_head=hs,
                                     extra_bias=extra.expand(2, hs, n, n).numpy())
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)
    assert (got - ps.attention_pair_bias(s, z, mask, p, n_head=hs, dtype=F64)).abs().max() > 1e-2


def _pwa_params(cm: int, c: int, heads: int, d: int, seed: int) -> dict[str, torch.Tensor]:
    return _rand_params({"ln_msa.weight": (cm,), "ln_msa.bias": (cm,), "ln_pair.weight": (c,),
                         "to_bias.weight": (heads, c), "to_value.weight": (heads * d, cm),
                         "to_gate.weight": (heads * d, cm), "to_out.weight": (cm, heads * d)}, seed)


def test_msa_pair_weighted_averaging_matches_brute_force():
    depth, n, cm, c, heads, d = 3, 5, 6, 4, 2, 3
    p = _pwa_params(cm, c, heads, d, 91)
    g = torch.Generator().manual_seed(92)
    m = torch.randn(2, depth, n, cm, generator=g, dtype=F64)
    z = torch.randn(2, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(2, n, dtype=torch.bool)
    mask[0, 1] = mask[0, 4] = False
    mask[1, :] = False  # no valid key: zero update
    got = ps.msa_pair_weighted_averaging(m, z, mask, p, n_head=heads, dtype=F64)
    want = brute.msa_pair_weighted_averaging(m.numpy(), z.numpy(), mask.numpy(), _np(p), n_head=heads)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)
    assert torch.equal(got[1], m[1])


def test_msa_pair_weighted_averaging_closed_forms():
    """Zero pair logits give the plain mean of the values over the valid keys; the weights do
    not depend on the MSA row, so permuting MSA rows permutes the update."""
    depth, n, cm, c, heads, d = 4, 6, 8, 4, 2, 4
    p = _pwa_params(cm, c, heads, d, 93)
    p["to_bias.weight"] = torch.zeros(heads, c, dtype=F64)
    g = torch.Generator().manual_seed(94)
    m = torch.randn(1, depth, n, cm, generator=g, dtype=F64)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.tensor([[True, False, True, True, False, True]])
    got = ps.msa_pair_weighted_averaging(m, z, mask, p, n_head=heads, dtype=F64)
    x = F.layer_norm(m, (cm,), p["ln_msa.weight"], p["ln_msa.bias"], 1e-5)
    v = x @ p["to_value.weight"].T
    mean = v[:, :, mask[0]].mean(dim=2, keepdim=True)
    want = m + (torch.sigmoid(x @ p["to_gate.weight"].T) * mean) @ p["to_out.weight"].T
    torch.testing.assert_close(got, want)
    perm = torch.tensor([2, 0, 3, 1])
    p2 = _pwa_params(cm, c, heads, d, 95)
    a = ps.msa_pair_weighted_averaging(m, z, mask, p2, n_head=heads, dtype=F64)
    b = ps.msa_pair_weighted_averaging(m[:, perm], z, mask, p2, n_head=heads, dtype=F64)
    torch.testing.assert_close(b, a[:, perm])


def _opm_params(cm: int, hidden: int, cz: int, seed: int, *, groups: int = 1,
                bias: bool = False) -> dict[str, torch.Tensor]:
    k = hidden // groups
    shapes = {"ln_msa.weight": (cm,), "ln_msa.bias": (cm,), "to_left.weight": (hidden, cm),
              "to_right.weight": (hidden, cm), "to_out.weight": (cz, groups * k * k),
              "to_out.bias": (cz,)}
    if bias:
        shapes |= {"to_left.bias": (hidden,), "to_right.bias": (hidden,)}
    if groups > 1:
        shapes |= {"product_norm.weight": (groups * k * k,), "product_norm.bias": (groups * k * k,)}
    return _rand_params(shapes, seed)


def _opm_inputs(batch: int, depth: int, n: int, cm: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(batch, depth, n, cm, generator=g, dtype=F64)
    rows = torch.rand(batch, depth, n, generator=g) > 0.25
    rows[:, 0] = True
    return m, rows


@pytest.mark.parametrize("form", [
    dict(count_offset=1e-3, normalize_before_proj=False),
    dict(count_offset=None, normalize_before_proj=False),
    dict(count_offset=None, normalize_before_proj=True),
    dict(count_offset=1e-3, normalize_before_proj=True),
    dict(count_offset=None, normalize_before_proj=False, groups=2),
])
@pytest.mark.parametrize("bias", [False, True])
def test_outer_product_mean_matches_brute_force(form, bias):
    depth, n, cm, hidden, cz = 3, 4, 6, 4, 5
    groups = form.get("groups", 1)
    p = _opm_params(cm, hidden, cz, 101, groups=groups, bias=bias)
    m, rows = _opm_inputs(2, depth, n, cm, 102)
    rows[1, :, 2] = False  # a token with no MSA entry: count 0
    got = ps.outer_product_mean(m, rows, p, dtype=F64, **form)
    want = brute.outer_product_mean(m.numpy(), rows.numpy(), _np(p), **form)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)


def test_outer_product_mean_closed_forms():
    """A mean over MSA rows: with the divisor n (offset 0) repeating every MSA row leaves the
    output unchanged and a masked row adds nothing; one MSA row gives the outer product of its
    two projections, flattened left channel first (a single nonzero output weight picks
    left channel c times right channel e); the AF3 form puts the bias before the divide."""
    depth, n, cm, hidden, cz = 3, 5, 8, 4, 3
    p = _opm_params(cm, hidden, cz, 103)
    m, rows = _opm_inputs(1, depth, n, cm, 104)
    mean = dict(count_offset=0.0, normalize_before_proj=True)
    base = ps.outer_product_mean(m, rows, p, dtype=F64, **mean)
    twice = ps.outer_product_mean(torch.cat([m, m], 1), torch.cat([rows, rows], 1), p,
                                  dtype=F64, **mean)
    torch.testing.assert_close(twice, base)
    # the AF3 form divides the bias too: repeating the rows scales the bias term by 1 / 2
    af3_1 = ps.outer_product_mean(m, rows, p, count_offset=0.0, dtype=F64)
    af3_2 = ps.outer_product_mean(torch.cat([m, m], 1), torch.cat([rows, rows], 1), p,
                                  count_offset=0.0, dtype=F64)
    count = torch.einsum("bsi,bsj->bij", rows.double(), rows.double())[..., None]
    torch.testing.assert_close(af3_1 - af3_2, p["to_out.bias"] / (2 * count))
    extra = torch.zeros(1, 1, n, dtype=torch.bool)
    padded = ps.outer_product_mean(torch.cat([m, torch.randn(1, 1, n, cm, dtype=F64)], 1),
                                   torch.cat([rows, extra], 1), p, dtype=F64, **mean)
    torch.testing.assert_close(padded, base)

    one = torch.ones(1, 1, n, dtype=torch.bool)
    x = F.layer_norm(m[:, :1], (cm,), p["ln_msa.weight"], p["ln_msa.bias"], 1e-5)[0, 0]
    left, right = x @ p["to_left.weight"].T, x @ p["to_right.weight"].T
    c, e = 1, 3
    q = dict(p)
    q["to_out.weight"] = torch.zeros(cz, hidden * hidden, dtype=F64)
    q["to_out.weight"][0, c * hidden + e] = 1.0
    q["to_out.bias"] = torch.zeros(cz, dtype=F64)
    got = ps.outer_product_mean(m[:, :1], one, q, count_offset=0.0, dtype=F64)[0, :, :, 0]
    torch.testing.assert_close(got, torch.outer(left[:, c], right[:, e]))
    af3 = ps.outer_product_mean(m[:, :1], one, p, count_offset=1e-3, dtype=F64)
    plain = ps.outer_product_mean(m[:, :1], one, p, count_offset=0.0, dtype=F64)
    torch.testing.assert_close(af3, plain / (1 + 1e-3))


def test_block_is_the_composition_of_the_pinned_ops():
    n, c, h, heads, d, cs, hs = 5, 6, 4, 2, 3, 6, 2
    params = {}
    for prefix, shapes, seed in (
        ("tri_multi_outgoing", _tm_shapes(c, h), 1), ("tri_multi_incoming", _tm_shapes(c, h), 2),
        ("tri_atten_starting", _ta_shapes(c, heads, d), 3), ("tri_atten_ending", _ta_shapes(c, heads, d), 4),
    ):
        params.update({f"{prefix}.{k}": v for k, v in _rand_params(shapes, seed).items()})
    tr = {"ln_in.weight": (c,), "ln_in.bias": (c,), "expand_a.weight": (4 * c, c),
          "expand_b.weight": (4 * c, c), "squeeze.weight": (c, 4 * c)}
    params.update({f"transition_pair.{k}": v for k, v in _rand_params(tr, 5).items()})
    g = torch.Generator().manual_seed(9)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, -1] = False
    got = ps.pairformer_block(z, mask, params, n_head_pair=heads, dtype=F64)
    x = z.numpy()
    sub = lambda pre: {k[len(pre) + 1:]: v.numpy() for k, v in params.items() if k.startswith(pre + ".")}  # noqa: E731
    x = brute.triangle_multiplication(x, mask.numpy(), sub("tri_multi_outgoing"), outgoing=True)
    x = brute.triangle_multiplication(x, mask.numpy(), sub("tri_multi_incoming"), outgoing=False)
    x = brute.triangle_attention(x, mask.numpy(), sub("tri_atten_starting"), starting=True, n_head=heads)
    x = brute.triangle_attention(x, mask.numpy(), sub("tri_atten_ending"), starting=False, n_head=heads)
    x = brute.transition(x, sub("transition_pair"))
    np.testing.assert_allclose(got.numpy(), x, rtol=1e-10, atol=1e-10)


def test_parallel_block_is_the_sum_of_updates_on_the_block_input():
    """The parallel schedule (``legacy/pairformer.py:176-190``, single ``:208-226``): every
    update is computed by the brute-force loops from the block's input and added once. The
    schedule that feeds the triangle attentions the already-updated pair must differ."""
    n, c, h, heads, d, cs, hs = 5, 6, 4, 2, 3, 8, 2
    params = {}
    for prefix, shapes, seed in (
        ("tri_multi_outgoing", _tm_shapes(c, h), 21), ("tri_multi_incoming", _tm_shapes(c, h), 22),
        ("tri_atten_starting", _ta_shapes(c, heads, d), 23), ("tri_atten_ending", _ta_shapes(c, heads, d), 24),
    ):
        params.update({f"{prefix}.{k}": v for k, v in _rand_params(shapes, seed).items()})
    tr = lambda w: {"ln_in.weight": (w,), "ln_in.bias": (w,), "expand_a.weight": (4 * w, w),  # noqa: E731
                    "expand_b.weight": (4 * w, w), "squeeze.weight": (w, 4 * w)}
    params.update({f"transition_pair.{k}": v for k, v in _rand_params(tr(c), 25).items()})
    params.update({f"single_transition.{k}": v for k, v in _rand_params(tr(cs), 26).items()})
    apb = {"ln_single.weight": (cs,), "ln_single.bias": (cs,), "to_query.weight": (cs, cs),
           "to_query.bias": (cs,), "to_key.weight": (cs, cs), "to_value.weight": (cs, cs),
           "ln_pair.weight": (c,), "to_bias.weight": (hs, c), "to_gate.weight": (cs, cs),
           "to_out.weight": (cs, cs)}
    params.update({f"single_attention.{k}": v for k, v in _rand_params(apb, 27).items()})
    g = torch.Generator().manual_seed(28)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    s = torch.randn(1, n, cs, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    mask[0, -1] = False
    got_z, got_s = ps.pairformer_block(z, mask, params, n_head_pair=heads, s=s, n_head_single=hs,
                                       dtype=F64, parallel=True)
    x, m = z.numpy(), mask.numpy()
    sub = lambda pre: {k[len(pre) + 1:]: v.numpy() for k, v in params.items() if k.startswith(pre + ".")}  # noqa: E731
    tm = (brute.triangle_multiplication(x, m, sub("tri_multi_outgoing"), outgoing=True) - x
          + brute.triangle_multiplication(x, m, sub("tri_multi_incoming"), outgoing=False) - x)
    ta = lambda y: (brute.triangle_attention(y, m, sub("tri_atten_starting"), starting=True, n_head=heads) - y  # noqa: E731
                    + brute.triangle_attention(y, m, sub("tri_atten_ending"), starting=False, n_head=heads) - y)
    tr_pair = brute.transition(x, sub("transition_pair")) - x
    want_z = x + tm + ta(x) + tr_pair
    np.testing.assert_allclose(got_z.numpy(), want_z, rtol=1e-10, atol=1e-10)
    sv = s.numpy()
    want_s = (sv + (brute.attention_pair_bias(sv, x, m, sub("single_attention"), n_head=hs) - sv)
              + (brute.transition(sv, sub("single_transition")) - sv))
    np.testing.assert_allclose(got_s.numpy(), want_s, rtol=1e-10, atol=1e-10)
    # the mistake of feeding the attentions the pair after the other updates is visible
    z1 = x + tm + tr_pair
    wrong = z1 + ta(z1)
    assert np.abs(wrong - want_z)[0][np.outer(m[0], m[0])].max() > 1e-3


def test_a_planted_mistake_is_caught(monkeypatch):
    """A transposed operand planted in the oracle's contraction breaks the brute-force check."""
    n, c, h = 5, 4, 3
    p = _rand_params(_tm_shapes(c, h), 91)
    g = torch.Generator().manual_seed(92)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    want = brute.triangle_multiplication(z.numpy(), mask.numpy(), _np(p), outgoing=True)
    real = ps.triangle_multiplication(z, mask, p, outgoing=True, dtype=F64)
    np.testing.assert_allclose(real.numpy(), want, rtol=1e-11, atol=1e-11)
    broken = dict(p)
    broken["to_left.weight"], broken["to_right.weight"] = p["to_right.weight"], p["to_left.weight"]
    wrong = ps.triangle_multiplication(z, mask, broken, outgoing=True, dtype=F64)
    assert np.abs(wrong.numpy() - want).max() > 1e-3


def test_block_io_dtype_rounds_the_stream_between_ops():
    n, c, h, heads, d = 5, 6, 4, 2, 3
    params = {}
    for prefix, shapes, seed in (
        ("tri_multi_outgoing", _tm_shapes(c, h), 11), ("tri_multi_incoming", _tm_shapes(c, h), 12),
        ("tri_atten_starting", _ta_shapes(c, heads, d), 13), ("tri_atten_ending", _ta_shapes(c, heads, d), 14),
    ):
        params.update({f"{prefix}.{k}": v for k, v in _rand_params(shapes, seed).items()})
    tr = {"ln_in.weight": (c,), "ln_in.bias": (c,), "expand_a.weight": (4 * c, c),
          "expand_b.weight": (4 * c, c), "squeeze.weight": (c, 4 * c)}
    params.update({f"transition_pair.{k}": v for k, v in _rand_params(tr, 15).items()})
    g = torch.Generator().manual_seed(16)
    z = torch.randn(1, n, n, c, generator=g, dtype=F64)
    mask = torch.ones(1, n, dtype=torch.bool)
    plain = ps.pairformer_block(z, mask, params, n_head_pair=heads, dtype=F64)
    assert torch.equal(plain, ps.pairformer_block(z, mask, params, n_head_pair=heads, dtype=F64, io_dtype=None))
    rounded = ps.pairformer_block(z, mask, params, n_head_pair=heads, dtype=F64, io_dtype=torch.bfloat16)
    assert torch.equal(rounded, rounded.bfloat16().double())  # the stream leaves each op in bf16
    assert 0 < ps.rel_rms(rounded, plain) < 2e-2


@pytest.mark.parametrize("activation", ["none", "sigmoid", "silu", "relu"])
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm_linear_matches_brute_force(activation, affine):
    """Row by row: the brute-force LayerNorm, a mat-vec, the activation's closed form."""
    import math

    g = torch.Generator().manual_seed(61)
    x = torch.randn(7, 12, generator=g, dtype=F64) * 2 + 0.3
    w = torch.randn(5, 12, generator=g, dtype=F64) * 0.4
    b = torch.randn(5, generator=g, dtype=F64) * 0.1
    lw = 1 + 0.1 * torch.randn(12, generator=g, dtype=F64) if affine else None
    lb = 0.1 * torch.randn(12, generator=g, dtype=F64) if affine else None
    got = ps.layer_norm_linear(x, lw, lb, w, b, activation=activation, dtype=F64)
    act = {"none": lambda t: t, "sigmoid": lambda t: 1 / (1 + math.exp(-t)),
           "silu": lambda t: t / (1 + math.exp(-t)), "relu": lambda t: max(t, 0.0)}[activation]
    for r in range(7):
        h = brute.layer_norm_vec(x[r].numpy(), None if lw is None else lw.numpy(),
                                 None if lb is None else lb.numpy(), 1e-5)
        y = brute._matvec(w.numpy(), h)
        want = [act(y[o] + float(b[o])) for o in range(5)]
        np.testing.assert_allclose(got[r].numpy(), want, rtol=1e-12, atol=1e-12)
    if activation == "none" and affine:
        torch.testing.assert_close(got, F.linear(F.layer_norm(x, (12,), lw, lb, 1e-5), w, b))


def test_swiglu_ffn_is_the_transition_without_its_norm():
    """``x + swiglu_ffn(LN(x))`` equals the brute-force transition, which pins the SwiGLU body."""
    c = 8
    p = _rand_params({"ln_in.weight": (c,), "ln_in.bias": (c,), "expand_a.weight": (4 * c, c),
                      "expand_b.weight": (4 * c, c), "squeeze.weight": (c, 4 * c)}, 62)
    g = torch.Generator().manual_seed(63)
    x = torch.randn(2, 5, c, generator=g, dtype=F64)
    h = ps.layer_norm(x, p["ln_in.weight"], p["ln_in.bias"], 1e-5)
    got = ps.swiglu_ffn(h, p["expand_a.weight"], p["expand_b.weight"], p["squeeze.weight"], residual=x, dtype=F64)
    want = brute.transition(x.numpy(), _np(p))
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-11, atol=1e-11)
    bare = ps.swiglu_ffn(h, p["expand_a.weight"], p["expand_b.weight"], p["squeeze.weight"], dtype=F64)
    torch.testing.assert_close(bare + x, got)
    # the gate branches are not interchangeable: swapping expand_a and expand_b changes the result
    swapped = ps.swiglu_ffn(h, p["expand_b.weight"], p["expand_a.weight"], p["squeeze.weight"], dtype=F64)
    assert (swapped - bare).abs().max() > 1e-3

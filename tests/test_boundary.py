"""The drop-in boundary on the CPU: backend names and plans, the refusal policies (engine
error, fallback, error), the parity helpers of the GPU tests, factories and precision, dead
modules, the residual contract, and the ``pytorch`` backend against the oracle.

Mirrors the reference's ``tests/kernels/test_backends.py``, ``test_engine_factories.py``,
``tests/models/test_dead_modules.py:97-136`` and ``test_released_conversions.py`` (the
parity is checked only where the pair is real, ``:61-64``). The ``hip`` backend's
refusals are forced from the host with CPU tensors and a faked device capability.
"""

from __future__ import annotations

import logging

import pytest
import torch
from torch import nn

from foldforge_amd import adapter, dispatch, factories
from foldforge_amd.modules import (
    AttentionPairBias,
    BackendUnsupported,
    MSAPairWeightedAveraging,
    MasterWeights,
    PairformerBlock,
    Transition,
    TriangleAttention,
    TriangleAttentionAF3,
    TriangleAttentionChai1,
    TriangleAttentionChai1Confidence,
    TriangleAttentionOpenFold,
    TriangleAttentionRF3,
    TriangleMultiplication,
    TriangleMultiplicationRF3,
)
from foldforge_amd.trunk import PairformerTrunk, randomise
from oracle import pairstack as ps
from tests.hip_calls import hip_delta, hip_forward


def fake_gfx950(monkeypatch):
    monkeypatch.setattr(dispatch, "device_arch", lambda _d=None: "gfx950")


def test_names_and_aliases():
    assert set(dispatch.BACKEND_NAMES) >= {"pytorch", "hip", "cuda", "triton", "anthropic", "cueq"}
    assert "miniworld" in dispatch.REQUESTABLE and "cuequivariance" in dispatch.REQUESTABLE
    with pytest.raises(ValueError, match="Unknown backend"):
        dispatch.Plan.of("magma")
    with pytest.raises(ValueError, match="unknown op"):
        dispatch.check_ops({"nope": "pytorch"})
    with pytest.raises(ValueError, match="unknown backend"):
        dispatch.check_ops({"trimul": "nope"})
    with pytest.raises(ValueError, match="engine.unsupported"):
        dispatch.Plan.of("pytorch", unsupported="ignore")
    with pytest.raises(ValueError, match="Unknown backend"):
        dispatch.pick("magma", Transition, "gfx950")


def test_serves_is_derived_from_the_classes():
    table = dispatch.SERVES
    assert set(table) == set(dispatch.OP_NAMES)
    for op in ("trimul", "triangle_attention", "transition", "layernorm", "single_attention",
               "msa_pwa", "opm"):
        assert table[op] == ("miniworld", "pytorch", "hip"), op
    assert table["dit_blocks"] == ()  # named, no class in this build


def test_pick():
    assert dispatch.pick("miniworld", Transition, None) == ("pytorch", None)
    name, why = dispatch.pick("hip", Transition, None)
    assert name == "pytorch" and "gfx950" in why
    assert dispatch.pick("miniworld", Transition, "gfx950") == ("hip", None)
    assert dispatch.pick("hip", TriangleMultiplication, "gfx950") == ("hip", None)
    assert dispatch.pick("miniworld", AttentionPairBias, "gfx950") == ("hip", None)
    assert dispatch.pick("pytorch", AttentionPairBias, "gfx950") == ("pytorch", None)
    for cls in (AttentionPairBias, Transition):
        name, why = dispatch.pick("cuda", cls, "gfx950")
        assert name == "pytorch" and "no 'cuda' backend" in why
    name, why = dispatch.pick("cuequivariance", Transition, "gfx950")
    assert name == "pytorch" and "'cueq'" in why
    # another ROCm card: the hip kernels are gfx950 code objects
    assert dispatch.pick("miniworld", Transition, "gfx942") == ("pytorch", None)
    assert dispatch.pick("hip", Transition, "gfx942")[0] == "pytorch"


def test_plan_resolve_reports_refused_ops(caplog):
    plan = dispatch.Plan.of("pytorch", {"transition": "hip", "single_attention": "cuda"})
    assert plan.requested("transition") == "hip" and plan.requested("trimul") == "pytorch"
    with caplog.at_level(logging.WARNING, logger="foldforge.backend"):
        picks = plan.resolve("gfx950")
    assert picks["transition"] == ("hip", None)
    assert picks["single_attention"].reason is not None
    summary = plan.summary(picks)
    assert summary["fallbacks"].keys() == {"single_attention"}
    assert summary["ops"]["trimul"] == "pytorch"
    assert sum("single_attention" in r.message for r in caplog.records) == 1
    strict = dispatch.Plan.of("pytorch", {"single_attention": "cuda"}, "error")
    with pytest.raises(dispatch.BackendUnsupportedError):
        strict.resolve("gfx950")


class _Model(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.transition = factories.transition(16, 2, precision="fp32")
        self.trimul = factories.triangle_multiplication(16, outgoing=True, precision="fp32")
        self.norm = factories.layer_norm(16)


def _x(batch: int = 1) -> torch.Tensor:
    torch.manual_seed(0)
    return torch.randn(batch, 4, 16)


def test_install_sets_the_backend_per_module(monkeypatch):
    fake_gfx950(monkeypatch)
    model = _Model()
    placed = dispatch.install(model, dispatch.Plan.of("miniworld", {"trimul": "pytorch"}))
    assert model.transition.backend == "hip"
    assert model.norm.backend == "hip"
    assert model.trimul.backend == "pytorch"
    assert model.trimul.ln_pair.backend == "pytorch"  # an op's own sub-modules are its business
    assert placed["transition"]["backend"] == "hip"
    assert placed["trimul"]["op"] == "trimul"
    assert set(placed) == {"transition", "trimul", "norm"}


def test_without_a_policy_a_refused_call_raises_in_forward_and_delta(monkeypatch):
    """The engine's own contract: a module outside its backend's range never falls back."""
    fake_gfx950(monkeypatch)
    m = factories.transition(16, 2, precision="fp32")
    m.set_backend("hip")
    assert m.unsupported(_x()) is not None  # a CPU tensor is outside the hip backend
    with pytest.raises(BackendUnsupported):
        m(_x())
    with pytest.raises(BackendUnsupported):
        m.delta(_x())
    assert dispatch.ledger_of(m).served == {}


def test_parity_helpers_fail_when_hip_refuses(monkeypatch):
    """The GPU parity tests call through these helpers; a refusal must fail them."""
    m = factories.transition(16, 2, precision="fp32")
    m.set_backend("hip")
    monkeypatch.setattr(type(m), "_unsupported_hip", lambda self, x: "planted refusal")
    with pytest.raises(AssertionError, match="planted refusal"):
        hip_delta(m, _x())
    with pytest.raises(AssertionError, match="planted refusal"):
        hip_forward(m, _x())
    m.refusal_policy = "fallback"  # even a module that would fall back fails the helper
    with pytest.raises(AssertionError, match="refused"):
        hip_delta(m, _x())
    m.set_backend("pytorch")
    with pytest.raises(AssertionError, match="not hip"):
        hip_delta(m, _x())


def test_parity_helpers_count_a_served_call(monkeypatch):
    m = factories.transition(16, 2, precision="fp32")
    m.set_backend("hip")
    monkeypatch.setattr(type(m), "_unsupported_hip", lambda self, x: None)
    monkeypatch.setattr(type(m), "_forward_hip", lambda self, x, residual=True: x * 0 + 7)
    assert torch.equal(hip_delta(m, _x()), torch.full((1, 4, 16), 7.0))
    assert dispatch.ledger_of(m).served["hip"] == 1
    monkeypatch.setattr(type(m), "_route", lambda self, a, k: "hip")  # a route that forgets to count
    with pytest.raises(AssertionError, match="did not serve"):
        hip_delta(m, _x())


def test_fallback_policy_runs_pytorch_once_logged(monkeypatch, caplog):
    fake_gfx950(monkeypatch)
    model = _Model()
    expected = Transition.forward(model.transition, _x())  # pytorch backend
    dispatch.install(model, dispatch.Plan.of("hip"))
    dispatch.clear_ledgers(model)
    assert model.transition.backend == "hip"
    with caplog.at_level(logging.WARNING, logger="foldforge.backend"):
        first = model.transition(_x())
        second = model.transition(_x())
        third = model.transition.delta(_x())
    torch.testing.assert_close(first, expected)
    torch.testing.assert_close(second, expected)
    torch.testing.assert_close(_x() + third, expected)
    assert model.transition.backend == "hip"  # the module keeps its backend
    assert sum("refused a call" in r.message for r in caplog.records) == 1
    entry = dispatch.ledger_report(model)["transition"]
    assert entry["served"] == {"pytorch": 3}
    assert sum(entry["refused"].values()) == 3 and len(entry["refused"]) == 1
    assert dispatch.served_count(model, "hip") == 0
    dispatch.clear_ledgers(model)
    assert dispatch.ledger_report(model)["transition"]["served"] == {}


def test_error_policy_raises(monkeypatch):
    fake_gfx950(monkeypatch)
    model = _Model()
    dispatch.install(model, dispatch.Plan.of("hip", unsupported="error"))
    with pytest.raises(dispatch.BackendUnsupportedError, match=r"engine.unsupported: error"):
        model.transition(_x())
    with pytest.raises(dispatch.BackendUnsupportedError):
        model.transition.delta(_x())
    with pytest.raises(dispatch.BackendUnsupportedError, match="no 'cuda' backend"):
        dispatch.install(_Model(), dispatch.Plan.of("cuda", unsupported="error"))


def test_composite_children_are_set_one_by_one(monkeypatch):
    fake_gfx950(monkeypatch)
    block = factories.pairformer_block(d_pair=32, triangle_model="af3", d_single=64,
                                       n_head_single=4, precision="fp32")
    holder = nn.ModuleList([block])
    dispatch.install(holder, dispatch.Plan.of("miniworld"))
    assert block.backend == "pytorch"
    assert block.tri_multi_outgoing.backend == "hip"
    assert block.tri_atten_ending.backend == "hip"
    assert block.transition_pair.backend == "hip"
    assert block.single_attention.backend == "hip"
    assert block.single_transition.backend == "hip"
    # widths outside the kernels (32 != 128) are refused per call even on a gfx950
    from foldforge_amd import modules

    monkeypatch.setattr(modules, "hip_reason", lambda *_t: None)
    reason = block.tri_multi_outgoing.unsupported(
        torch.zeros(1, 4, 4, 32, dtype=torch.bfloat16), torch.ones(1, 4, dtype=torch.bool))
    assert reason is not None and "128" in reason
    reason = block.tri_atten_starting.unsupported(
        torch.zeros(1, 4, 4, 32, dtype=torch.float32), torch.ones(1, 4, dtype=torch.bool))
    assert reason is not None and "bf16" in reason


def test_factories_precision_and_model_keys():
    for precision in ("master", "fp32"):
        m = factories.transition(32, 4, precision=precision)
        assert {p.dtype for p in m.parameters()} == {torch.float32}
        assert m.master_weights is (precision == "master")
        m.to(torch.bfloat16)
        assert m.expand_a.weight.dtype == (torch.float32 if precision == "master" else torch.bfloat16)
        assert m.ln_in.weight.dtype == torch.float32
    with pytest.raises(ValueError, match="precision"):
        factories.finish(Transition(8, 2), "bf16")
    assert type(factories.triangle_attention(32, 4, starting=True, model="af3")) is TriangleAttentionAF3
    assert type(factories.triangle_attention(32, 4, starting=False, model="protenix")) is TriangleAttentionOpenFold
    assert type(factories.triangle_multiplication(32, outgoing=True)) is TriangleMultiplication
    assert type(factories.triangle_multiplication(32, outgoing=True, divide_by_length=True)) is TriangleMultiplicationRF3
    assert factories.triangle_multiplication(64, outgoing=False, d_hidden=128).to_left.weight.shape == (128, 64)
    with pytest.raises(ValueError, match="no triangle attention class"):
        TriangleAttention(32, 4, model="chai2")
    assert factories.model_keys("alphafold3").triangle == "af3"
    with pytest.raises(ValueError, match="no engine selector keys"):
        factories.model_keys("nope")


def test_triangle_attention_classes_follow_the_model_keys():
    """The reference's class per key (tests/kernels/test_engine_factories.py:75-90) and each
    lineage's parameters: RF3's projection biases, Chai-1 confidence's to_out_t."""
    cases = {"af3": TriangleAttentionAF3, "rf3": TriangleAttentionRF3,
             "chai1": TriangleAttentionChai1, "chai1_confidence": TriangleAttentionChai1Confidence}
    for key, cls in cases.items():
        m = factories.triangle_attention(32, 4, starting=key != "rf3", model=key)
        assert type(m) is cls
        assert (m.to_gate.bias is not None) == (key == "rf3")
        assert (m.to_out.bias is not None) == (key == "rf3")
        assert hasattr(m, "to_out_t") == (key == "chai1_confidence")
    fast = factories.pairformer_block(d_pair=32, triangle_model="rf3", parallel=True)
    assert type(fast.tri_atten_starting) is TriangleAttentionRF3
    assert type(fast.tri_multi_outgoing) is TriangleMultiplication
    exact = factories.pairformer_block(d_pair=32, triangle_model="rf3", parallel=True,
                                       divide_by_length=True)
    assert type(exact.tri_multi_outgoing) is TriangleMultiplicationRF3
    conf = factories.pairformer_block(d_pair=32, triangle_model="chai1_confidence", d_single=64,
                                      n_head_single=4, single_gate_bias=1.0, parallel=True)
    assert type(conf.tri_atten_starting) is TriangleAttentionChai1Confidence
    assert conf.single_attention.gate_bias == 1.0


@pytest.mark.parametrize("key", ["rf3", "chai1", "chai1_confidence"])
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_lineage_forms_match_the_oracle(key, starting):
    """The pytorch backend's RF3 / Chai-1 forms against the fp64 oracle (pinned by loops)."""
    m = randomise(factories.triangle_attention(16, 2, starting=starting, model=key), seed=3)
    if key == "rf3":
        with torch.no_grad():
            m.to_gate.bias.normal_(0, 0.5)
            m.to_out.bias.normal_(0, 0.5)
    g = torch.Generator().manual_seed(4)
    z = torch.randn(2, 9, 9, 16, generator=g)
    mask = torch.ones(2, 9, dtype=torch.bool)
    mask[1, 6:] = False
    got = m.delta(z, mask)
    want = ps.triangle_attention(z, mask, m.state_dict(), starting=starting, n_head=2,
                                 untransposed_output=m.untransposed_output,
                                 dual_output=m.dual_output, dtype=torch.float64) - z.double()
    torch.testing.assert_close(got.double(), want, rtol=1e-4, atol=1e-4)


def test_master_flag_reaches_every_mixin_below():
    block = factories.pairformer_block(d_pair=32, triangle_model="af3", d_single=64, n_head_single=4)
    mixins = [m for m in block.modules() if isinstance(m, MasterWeights)]
    assert mixins and all(m.master_weights for m in mixins)
    assert {p.dtype for p in block.parameters()} == {torch.float32}


def test_engine_state_dict_keys():
    block = factories.pairformer_block(d_pair=128, triangle_model="af3", d_single=384)
    keys = set(block.state_dict())
    for key in (
        "tri_multi_outgoing.to_left.weight", "tri_multi_incoming.ln_out.bias",
        "tri_multi_outgoing.to_gate.weight", "tri_atten_starting.to_bias.weight",
        "tri_atten_ending.to_query.weight", "transition_pair.expand_a.weight",
        "transition_pair.squeeze.weight", "single_attention.to_query.bias",
        "single_attention.ln_pair.weight", "single_transition.ln_in.weight",
    ):
        assert key in keys, key
    assert "single_attention.ln_pair.bias" not in keys
    assert block.tri_multi_outgoing.to_out.weight.shape == (128, 128)
    assert block.tri_atten_starting.to_bias.weight.shape == (4, 128)


def test_dead_flag_and_identity():
    for cls in (Transition, TriangleAttention, TriangleMultiplication, AttentionPairBias,
                MSAPairWeightedAveraging):
        assert cls.dead is False
    module = factories.transition(16, 2, precision="fp32").eval()
    module.dead = True
    x = torch.randn(3, 16, dtype=torch.bfloat16)
    assert torch.equal(module(x), x)
    module.dead = False
    assert not torch.equal(module(x), x)


def test_residual_contract_and_delta():
    torch.manual_seed(0)
    m = randomise(factories.triangle_multiplication(16, outgoing=False, precision="fp32"), 3)
    x = torch.randn(1, 5, 5, 16)
    mask = torch.ones(1, 5, dtype=torch.bool)
    torch.testing.assert_close(m(x, mask), x + m.delta(x, mask))


def _valid(x, mask):
    pm = mask[:, :, None] & mask[:, None, :]
    return x[pm]


@pytest.mark.parametrize("outgoing", [True, False])
def test_pytorch_backend_trimul_matches_oracle(outgoing):
    m = randomise(factories.triangle_multiplication(32, outgoing=outgoing, precision="fp32"), 1)
    torch.manual_seed(2)
    x = torch.randn(2, 9, 9, 32)
    mask = torch.ones(2, 9, dtype=torch.bool)
    mask[1, -3:] = False
    got = m(x, mask)
    want = ps.triangle_multiplication(x, mask, m.state_dict(), outgoing=outgoing, dtype=torch.float64)
    torch.testing.assert_close(_valid(got.double(), mask), _valid(want, mask), atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("model", ["af3", "boltz2"])
def test_pytorch_backend_triattn_matches_oracle(starting, model):
    m = randomise(factories.triangle_attention(32, 4, starting=starting, model=model, precision="fp32"), 1)
    torch.manual_seed(3)
    x = torch.randn(1, 10, 10, 32)
    mask = torch.ones(1, 10, dtype=torch.bool)
    mask[0, -2:] = False
    got = m(x, mask)
    want = ps.triangle_attention(x, mask, m.state_dict(), starting=starting, n_head=4,
                                 transposed_bias=m.transposed_bias, dtype=torch.float64)
    torch.testing.assert_close(_valid(got.double(), mask), _valid(want, mask), atol=2e-5, rtol=2e-5)


def test_msa_pair_weighted_averaging_class_contract_and_pytorch_backend():
    m = randomise(factories.msa_pair_weighted_averaging(64, 32, 8, precision="fp32"), 6)
    keys = set(m.state_dict())
    assert {"ln_msa.weight", "ln_msa.bias", "ln_pair.weight", "to_bias.weight", "to_value.weight",
            "to_gate.weight", "to_out.weight"} == keys  # no pair-norm offset
    assert m.to_value.weight.shape == (64, 64) and m.d_hidden == 8
    assert dispatch.op_name(m) == "msa_pwa"
    torch.manual_seed(7)
    msa = torch.randn(1, 3, 7, 64)
    z = torch.randn(1, 7, 7, 32)
    mask = torch.ones(1, 7, dtype=torch.bool)
    mask[0, -2:] = False
    got = m(msa, z, mask)
    want = ps.msa_pair_weighted_averaging(msa, z, mask, m.state_dict(), n_head=8, dtype=torch.float64)
    torch.testing.assert_close(got.double(), want, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(m(msa, z, mask), msa + m.delta(msa, z, mask))


@pytest.mark.parametrize("form", [
    dict(count_offset=1e-3, normalize_before_proj=False),
    dict(count_offset=None, normalize_before_proj=True, projection_bias=True),
    dict(count_offset=None, normalize_before_proj=False, groups=2),
])
def test_outer_product_mean_class_contract_and_pytorch_backend(form):
    groups = form.get("groups", 1)
    hidden = 8 if groups > 1 else 4
    m = randomise(factories.outer_product_mean(16, 24, hidden, precision="fp32", **form), 8)
    keys = set(m.state_dict())
    want_keys = {"ln_msa.weight", "ln_msa.bias", "to_left.weight", "to_right.weight",
                 "to_out.weight", "to_out.bias"}
    if form.get("projection_bias"):
        want_keys |= {"to_left.bias", "to_right.bias"}
    if groups > 1:
        want_keys |= {"product_norm.weight", "product_norm.bias"}
    assert keys == want_keys
    k = hidden // groups
    assert m.to_out.weight.shape == (24, groups * k * k)
    assert dispatch.op_name(m) == "opm"
    torch.manual_seed(9)
    msa = torch.randn(2, 5, 7, 16)
    rows = torch.rand(2, 5, 7) > 0.3
    rows[1, :, -1] = False
    got = m(msa, rows)
    oracle_form = {k_: v for k_, v in form.items() if k_ != "projection_bias"}
    want = ps.outer_product_mean(msa, rows, m.state_dict(), dtype=torch.float64, **oracle_form)
    torch.testing.assert_close(got.double(), want, atol=2e-5, rtol=2e-5)
    pair = torch.randn(2, 7, 7, 24)
    torch.testing.assert_close(m(msa, rows, residual=pair), pair + m.delta(msa, rows))
    assert m.unsupported(msa, rows) is None  # pytorch serves every form


def test_outer_product_mean_hip_refusals():
    m = factories.outer_product_mean(64, 128, 32, groups=1)
    m.set_backend("hip")
    msa = torch.randn(1, 3, 5, 64).bfloat16()
    rows = torch.ones(1, 3, 5, dtype=torch.bool)
    assert "device" in (m.unsupported(msa, rows) or "")  # a CPU tensor is not served
    g = factories.outer_product_mean(64, 128, 32, groups=4)
    g.set_backend("hip")
    assert g.unsupported(msa, rows) is not None


def test_pytorch_backend_block_and_run_block_match_oracle():
    block = randomise(factories.pairformer_block(d_pair=32, triangle_model="af3", d_single=48,
                                                 n_head_single=4, precision="fp32"), 4)
    torch.manual_seed(5)
    n = 8
    pair = torch.randn(n, n, 32)
    single = torch.randn(n, 48)
    tokens = torch.ones(n)
    tokens[-2:] = 0
    pair_mask = tokens[:, None] * tokens[None, :]
    got_pair, got_single = adapter.run_block(block, pair, pair_mask, single.clone(), tokens)
    mask = (tokens > 0)[None]
    want_pair, want_single = ps.pairformer_block(pair[None], mask, block.state_dict(), n_head_pair=4,
                                                 s=single[None], n_head_single=4, dtype=torch.float64)
    torch.testing.assert_close(_valid(got_pair[None].double(), mask), _valid(want_pair, mask), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(got_single[tokens > 0].double(), want_single[0][tokens > 0], atol=1e-4, rtol=1e-4)


def test_token_mask_is_the_pair_mask_diagonal():
    tokens = torch.tensor([1.0, 1.0, 0.0, 1.0])
    pm = tokens[:, None] * tokens[None, :]
    assert factories.token_mask(pm).tolist() == [True, True, False, True]
    assert factories.residue_mask(pm).shape == (1, 4)


def test_trunk_runs_passes_on_cpu():
    trunk = randomise(PairformerTrunk(2, d_pair=32, d_single=48, n_head_single=4, precision="fp32"), 7)
    assert isinstance(trunk.blocks[0], PairformerBlock)
    z = torch.randn(1, 6, 6, 32)
    s = torch.randn(1, 6, 48)
    mask = torch.ones(1, 6, dtype=torch.bool)
    seen = []
    pair, single = trunk(z, mask, s, passes=2, on_block=lambda p, i, *_: seen.append((p, i)))
    assert seen == [(0, 0), (0, 1), (1, 0), (1, 1)]
    assert torch.isfinite(pair).all() and torch.isfinite(single).all()


def test_parallel_block_matches_the_oracle_schedule():
    """``parallel=True`` (Chai-1 / RF3): every pair update and both single updates read the
    block's input (``legacy/pairformer.py:176-190,208-226``)."""
    block = randomise(factories.pairformer_block(d_pair=32, triangle_model="af3", d_single=48,
                                                 n_head_single=4, parallel=True, precision="fp32"), 11)
    torch.manual_seed(12)
    z = torch.randn(2, 7, 7, 32)
    s = torch.randn(2, 7, 48)
    mask = torch.ones(2, 7, dtype=torch.bool)
    mask[1, -2:] = False
    got_z, got_s = block(z, mask, s)
    want_z, want_s = ps.pairformer_block(z, mask, block.state_dict(), n_head_pair=4, s=s, n_head_single=4,
                                         dtype=torch.float64, parallel=True)
    torch.testing.assert_close(_valid(got_z.double(), mask), _valid(want_z, mask), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(got_s.double()[mask], want_s[mask], atol=1e-4, rtol=1e-4)
    seq_z = ps.pairformer_block(z, mask, block.state_dict(), n_head_pair=4, dtype=torch.float64)
    assert (_valid(seq_z, mask) - _valid(want_z, mask)).abs().max() > 1e-2  # the schedules differ

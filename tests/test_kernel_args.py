"""Host-side argument checks of :mod:`foldforge_amd.kernels` (CPU).

The C-ABI receives raw pointers without sizes for parameters and outputs, so a parameter
of the wrong shape or an ``out=`` of the wrong shape, dtype or layout has to be stopped in
Python with a ``ValueError``; otherwise it becomes an out-of-bounds device access. These
tests point the checks at CPU tensors (``kernels.DEVICE_TYPE``) and expect every bad
argument to raise before anything reaches the library.
"""

from __future__ import annotations

import pytest
import torch

from foldforge_amd import factories, kernels
from foldforge_amd.trunk import randomise


@pytest.fixture(autouse=True)
def _cpu_checks(monkeypatch):
    monkeypatch.setattr(kernels, "DEVICE_TYPE", "cpu")

    def refuse_native():
        raise AssertionError("an argument check let a bad call reach the library")

    monkeypatch.setattr(kernels._native, "lib", refuse_native)


def _pair(n=8, c=128, batch=1):
    return torch.zeros(batch, n, n, c, dtype=torch.bfloat16), torch.ones(batch, n, dtype=torch.bool)


def _trimul_args(m):
    return dict(ln_pair_weight=m.ln_pair.weight, ln_pair_bias=m.ln_pair.bias, to_left=m.to_left.weight,
                to_right=m.to_right.weight, to_left_gate=m.to_left_gate.weight,
                to_right_gate=m.to_right_gate.weight, ln_out_weight=m.ln_out.weight,
                ln_out_bias=m.ln_out.bias, to_out=m.to_out.weight, to_gate=m.to_gate.weight, outgoing=True)


def _triattn_args(m):
    return dict(ln_pair_weight=m.ln_pair.weight, ln_pair_bias=m.ln_pair.bias, to_bias=m.to_bias.weight,
                to_query=m.to_query.weight, to_key=m.to_key.weight, to_value=m.to_value.weight,
                to_gate=m.to_gate.weight, to_out=m.to_out.weight, n_head=4, starting=True)


@pytest.mark.parametrize("name,shape", [
    ("to_out", (128, 64)), ("to_gate", (128, 127)), ("ln_out_weight", (64,)), ("ln_pair_bias", (129,)),
    ("to_right_gate", (128, 64)),
])
def test_trimul_rejects_a_parameter_of_the_wrong_shape(name, shape):
    m = randomise(factories.triangle_multiplication(128, outgoing=True), 1)
    args = _trimul_args(m)
    args[name] = torch.zeros(shape)
    z, mask = _pair()
    with pytest.raises(ValueError, match=name):
        kernels.triangle_multiplicative_update(z, mask, **args)


@pytest.mark.parametrize("name,shape", [
    ("to_bias", (8, 128)), ("to_gate", (128, 64)), ("to_out", (64, 128)), ("ln_pair_weight", (64,)),
])
def test_triattn_rejects_a_parameter_of_the_wrong_shape(name, shape):
    m = randomise(factories.triangle_attention(128, 4, starting=True, model="af3"), 1)
    args = _triattn_args(m)
    args[name] = torch.zeros(shape)
    z, mask = _pair()
    with pytest.raises(ValueError, match=name):
        kernels.triangle_attention(z, mask, **args)


@pytest.mark.parametrize("bad", [
    torch.zeros(1, 8, 8, 64, dtype=torch.bfloat16),          # shape
    torch.zeros(1, 8, 8, 128, dtype=torch.float32),          # dtype
    torch.zeros(1, 8, 128, 8, dtype=torch.bfloat16).transpose(2, 3),  # layout
])
def test_out_must_match_the_input(bad):
    z, mask = _pair()
    m = randomise(factories.triangle_multiplication(128, outgoing=True), 1)
    with pytest.raises(ValueError, match="out"):
        kernels.triangle_multiplicative_update(z, mask, **_trimul_args(m), out=bad)
    t = randomise(factories.triangle_attention(128, 4, starting=True, model="af3"), 1)
    with pytest.raises(ValueError, match="out"):
        kernels.triangle_attention(z, mask, **_triattn_args(t), out=bad)
    tr = randomise(factories.transition(128, 4), 1)
    with pytest.raises(ValueError, match="out"):
        kernels.transition(z, ln_weight=tr.ln_in.weight, ln_bias=tr.ln_in.bias, expand_a=tr.expand_a.weight,
                           expand_b=tr.expand_b.weight, squeeze=tr.squeeze.weight, out=bad)


def test_transition_rejects_mismatched_weights():
    tr = randomise(factories.transition(128, 4), 1)
    z, _ = _pair()
    with pytest.raises(ValueError, match="squeeze"):
        kernels.transition(z, ln_weight=tr.ln_in.weight, ln_bias=tr.ln_in.bias, expand_a=tr.expand_a.weight,
                           expand_b=tr.expand_b.weight, squeeze=torch.zeros(128, 256))
    with pytest.raises(ValueError, match="ln_bias"):
        kernels.transition(z, ln_weight=tr.ln_in.weight, ln_bias=torch.zeros(64), expand_a=tr.expand_a.weight,
                           expand_b=tr.expand_b.weight, squeeze=tr.squeeze.weight)


def test_single_and_msa_ops_reject_bad_parameters():
    apb = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3", d_single=384).single_attention, 2)
    z, mask = _pair()
    s = torch.zeros(1, 8, 384, dtype=torch.bfloat16)
    args = dict(ln_single_weight=apb.ln_single.weight, ln_single_bias=apb.ln_single.bias,
                to_query=apb.to_query.weight, query_bias=apb.to_query.bias, to_key=apb.to_key.weight,
                to_value=apb.to_value.weight, ln_pair_weight=apb.ln_pair.weight, to_bias=apb.to_bias.weight,
                to_gate=apb.to_gate.weight, to_out=apb.to_out.weight, n_head=16)
    for name, shape in (("query_bias", (383,)), ("to_bias", (16, 64)), ("ln_pair_weight", (384,))):
        bad = dict(args, **{name: torch.zeros(shape)})
        with pytest.raises(ValueError, match=name):
            kernels.attention_pair_bias(s, z, mask, **bad)
    with pytest.raises(ValueError, match="out"):
        kernels.attention_pair_bias(s, z, mask, **args, out=torch.zeros(1, 8, 383, dtype=torch.bfloat16))
    pwa = randomise(factories.msa_pair_weighted_averaging(64, 128, 8), 3)
    msa = torch.zeros(1, 3, 8, 64, dtype=torch.bfloat16)
    pargs = dict(ln_msa_weight=pwa.ln_msa.weight, ln_msa_bias=pwa.ln_msa.bias, ln_pair_weight=pwa.ln_pair.weight,
                 to_bias=pwa.to_bias.weight, to_value=pwa.to_value.weight, to_gate=pwa.to_gate.weight,
                 to_out=pwa.to_out.weight, n_head=8)
    with pytest.raises(ValueError, match="to_out"):
        kernels.msa_pair_weighted_averaging(msa, z, mask, **dict(pargs, to_out=torch.zeros(64, 32)))
    opm = randomise(factories.outer_product_mean(64, 128, 32), 4)
    rows = torch.ones(1, 3, 8, dtype=torch.bool)
    oargs = dict(ln_weight=opm.ln_msa.weight, ln_bias=opm.ln_msa.bias, to_left=opm.to_left.weight,
                 to_right=opm.to_right.weight, to_out=opm.to_out.weight, to_out_bias=opm.to_out.bias)
    with pytest.raises(ValueError, match="left_bias"):
        kernels.outer_product_mean(msa, rows, **oargs, left_bias=torch.zeros(31))
    with pytest.raises(ValueError, match="out"):
        kernels.outer_product_mean(msa, rows, **oargs, out=torch.zeros(1, 8, 8, 64, dtype=torch.bfloat16))


def test_flash_core_rejects_an_output_too_small():
    q = torch.zeros(1, 4, 4, 128, 32, dtype=torch.bfloat16)
    vt = torch.zeros(1, 4, 4, 128 // 32, 32, 32, dtype=torch.bfloat16)  # the key-blocked v^T layout
    blk = torch.zeros(1 * 4 * 128 * 128)
    with pytest.raises(ValueError, match="cover"):
        kernels.flash_attention_bias(q, q, vt, blk, torch.zeros(1, 4, 100, 128, dtype=torch.bfloat16),
                                     rows_valid=4, n_valid=128)
    with pytest.raises(ValueError, match="valid extents"):
        kernels.flash_attention_bias(q, q, vt, blk, torch.zeros(1, 4, 128, 128, dtype=torch.bfloat16),
                                     rows_valid=5, n_valid=128)


def test_pair_weighted_averaging_head_split_bounds():
    # the gated average feeds the output projection as bf16 rows of heads x d_head <= 768 channels
    assert kernels.msa_pair_weighted_averaging_supported(64, 8, 32)
    assert kernels.msa_pair_weighted_averaging_supported(64, 24, 32)
    assert not kernels.msa_pair_weighted_averaging_supported(64, 32, 32)
    assert not kernels.msa_pair_weighted_averaging_supported(64, 8, 6)


def _attn_transition_args(t, tr):
    return dict(ln_pair_weight=t.ln_pair.weight, ln_pair_bias=t.ln_pair.bias, to_bias=t.to_bias.weight,
                to_query=t.to_query.weight, to_key=t.to_key.weight, to_value=t.to_value.weight,
                to_gate=t.to_gate.weight, to_out=t.to_out.weight, ln_weight=tr.ln_in.weight,
                ln_bias=tr.ln_in.bias, expand_a=tr.expand_a.weight, expand_b=tr.expand_b.weight,
                squeeze=tr.squeeze.weight)


@pytest.mark.parametrize("name,shape", [
    ("to_bias", (8, 128)), ("to_gate", (128, 64)), ("to_out", (64, 128)), ("ln_weight", (64,)),
    ("expand_b", (256, 128)), ("squeeze", (128, 256)),
])
def test_attention_transition_rejects_a_parameter_of_the_wrong_shape(name, shape):
    t = randomise(factories.triangle_attention(128, 4, starting=False, model="af3"), 1)
    tr = randomise(factories.transition(128, 4), 1)
    args = _attn_transition_args(t, tr)
    args[name] = torch.zeros(shape)
    z, mask = _pair()
    with pytest.raises(ValueError, match=name):
        kernels.triangle_attention_transition(z, mask, **args)


def test_attention_transition_checks_out_and_width():
    t = randomise(factories.triangle_attention(128, 4, starting=False, model="af3"), 1)
    tr = randomise(factories.transition(128, 4), 1)
    z, mask = _pair()
    with pytest.raises(ValueError, match="out"):
        kernels.triangle_attention_transition(z, mask, **_attn_transition_args(t, tr),
                                              out=torch.zeros(1, 8, 8, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="pair width"):
        kernels.triangle_attention_transition(*_pair(c=64), **_attn_transition_args(t, tr))

"""The released (dense) parameter layout converts to the engine modules' own.

As the reference checks its conversions (``tests/kernels/test_released_conversions.py``):
random released-layout tensors, converted with ``foldforge_amd.released``, loaded strictly
into the engine module on the ``pytorch`` backend (fp32, CPU), compared with the released
computation (``oracle/released.py``, fp64) where the pair / tokens are real. The
miniworld-format file round trip and the conversion's exactness errors are checked too.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from foldforge_amd import checkpoint, factories, released
from foldforge_amd.modules import MSABlock, PairformerBlock
from foldforge_amd.trunk import PairformerTrunk
from oracle import released as rel

L = 12
TOL = 2e-5


def _rand(shapes: dict[str, tuple[int, ...]], seed: int, std: float = 0.15) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in shapes.items():
        t = torch.randn(shape, generator=g)
        if len(shape) > 1:
            out[name] = std * t
        elif name.endswith("weight"):
            out[name] = 1.0 + 0.1 * t
        else:
            out[name] = 0.1 * t
    return out


def _norm(key: str, c: int) -> dict[str, tuple[int, ...]]:
    return {f"{key}.weight": (c,), f"{key}.bias": (c,)}


def trimul_shapes(c: int, h: int) -> dict[str, tuple[int, ...]]:
    return {**_norm("left_norm_input", c), "projection.weight": (2 * h, c), "gate.weight": (2 * h, c),
            **_norm("center_norm", h), "output_projection.weight": (c, h), "gating_linear.weight": (c, c)}


def triattn_shapes(c: int, heads: int, d: int) -> dict[str, tuple[int, ...]]:
    hd = heads * d
    return {**_norm("act_norm", c), "pair_bias_projection.weight": (heads, c),
            "q_projection.weight": (hd, c), "k_projection.weight": (hd, c),
            "v_projection.weight": (hd, c), "gating_query.weight": (hd, c),
            "output_projection.weight": (c, hd)}


def transition_shapes(c: int, n: int = 4) -> dict[str, tuple[int, ...]]:
    return {**_norm("input_layer_norm", c), "transition1.weight": (2 * n * c, c),
            "transition2.weight": (c, n * c)}


def msa_attention_shapes(cm: int, cz: int, heads: int, vd: int) -> dict[str, tuple[int, ...]]:
    return {**_norm("act_norm", cm), **_norm("pair_norm", cz), "pair_logits.weight": (heads, cz),
            "v_projection.weight": (heads * vd, cm), "gating_query.weight": (heads * vd, cm),
            "output_projection.weight": (cm, heads * vd)}


def opm_shapes(cm: int, k: int, cz: int) -> dict[str, tuple[int, ...]]:
    return {**_norm("layer_norm_input", cm), "left_projection.weight": (k, cm),
            "right_projection.weight": (k, cm), "output_w": (k, k, cz), "output_b": (cz,)}


def single_shapes(cs: int, cz: int, heads: int) -> dict[str, tuple[int, ...]]:
    a = "single_attention_."
    return {f"{a}adaptive_layernorm.layer_norm.weight": (cs,), f"{a}adaptive_layernorm.layer_norm.bias": (cs,),
            f"{a}q_projection.weight": (cs, cs), f"{a}q_projection.bias": (cs,),
            f"{a}k_projection.weight": (cs, cs), f"{a}v_projection.weight": (cs, cs),
            f"{a}gating_query.weight": (cs, cs), f"{a}adaptive_zero_init.transition2.weight": (cs, cs),
            **_norm("single_pair_logits_norm", cz), "single_pair_logits_projection.weight": (heads, cz)}


def _prefixed(prefix: str, shapes: dict[str, tuple[int, ...]]) -> dict[str, tuple[int, ...]]:
    return {f"{prefix}.{k}": v for k, v in shapes.items()}


def block_shapes(c: int, heads: int, cs: int = 0, heads_single: int = 4,
                 d_tri: int | None = None) -> dict[str, tuple[int, ...]]:
    d = d_tri or c // heads
    out = {**_prefixed("triangle_multiplication_outgoing", trimul_shapes(c, c)),
           **_prefixed("triangle_multiplication_incoming", trimul_shapes(c, c)),
           **_prefixed("pair_attention1", triattn_shapes(c, heads, d)),
           **_prefixed("pair_attention2", triattn_shapes(c, heads, d)),
           **_prefixed("pair_transition", transition_shapes(c))}
    if cs:
        out |= single_shapes(cs, c, heads_single) | _prefixed("single_transition", transition_shapes(cs))
    return out


def msa_block_shapes(cm: int, c: int, heads: int) -> dict[str, tuple[int, ...]]:
    return {**_prefixed("outer_product_mean", opm_shapes(cm, 4, c)),
            **_prefixed("msa_attention1", msa_attention_shapes(cm, c, 8, cm // 8)),
            **_prefixed("msa_transition", transition_shapes(cm)),
            **_prefixed("triangle_multiplication_outgoing", trimul_shapes(c, c)),
            **_prefixed("triangle_multiplication_incoming", trimul_shapes(c, c)),
            **_prefixed("pair_attention1", triattn_shapes(c, heads, c // heads)),
            **_prefixed("pair_attention2", triattn_shapes(c, heads, c // heads)),
            **_prefixed("pair_transition", transition_shapes(c))}


def _masks():
    tokens = torch.ones(L, dtype=torch.bool)
    tokens[-3:] = False
    return tokens, tokens[:, None] & tokens[None, :]


def _close(actual, expected, where=None, tol=TOL):
    actual, expected = actual.double(), expected.double()
    if where is not None:
        actual, expected = actual[where], expected[where]
    torch.testing.assert_close(actual, expected, atol=tol, rtol=tol)


@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication(outgoing):
    state = _rand(trimul_shapes(32, 16), 1)
    engine = factories.triangle_multiplication(32, outgoing=outgoing, d_hidden=16, precision="fp32")
    released.load(engine, released.triangle_multiplication_from_released(state, outgoing=outgoing))
    x = torch.randn(L, L, 32)
    tokens, pair = _masks()
    with torch.no_grad():
        actual = engine(x[None], tokens[None])[0]
    _close(actual, rel.triangle_multiplication(x, pair, state, outgoing=outgoing), pair)


def test_triangle_multiplication_branches_are_interleaved_rows():
    """Row 2k of the released projection / gate is branch a of channel k, row 2k + 1 branch b;
    the outgoing module takes a as ``left``, the incoming one takes b."""
    state = _rand(trimul_shapes(8, 4), 2)
    out = released.triangle_multiplication_from_released(state, outgoing=True)
    torch.testing.assert_close(out["to_left.weight"], state["projection.weight"][0::2])
    torch.testing.assert_close(out["to_right.weight"], state["projection.weight"][1::2])
    inc = released.triangle_multiplication_from_released(state, outgoing=False)
    torch.testing.assert_close(inc["to_left.weight"], state["projection.weight"][1::2])
    torch.testing.assert_close(inc["to_right_gate.weight"], state["gate.weight"][0::2])


@pytest.mark.parametrize("ending", [False, True])
def test_triangle_attention(ending):
    state = _rand(triattn_shapes(32, 4, 8), 3)
    engine = factories.triangle_attention(32, 4, starting=not ending, model="af3", precision="fp32")
    released.load(engine, released.triangle_attention_from_released(state))
    x = torch.randn(L, L, 32)
    tokens, pair = _masks()
    with torch.no_grad():
        actual = engine(x[None], tokens[None])[0]
    _close(actual, rel.triangle_attention(x, pair, state, n_head=4, ending=ending), pair)


def test_transition():
    state = _rand(transition_shapes(24), 4)
    engine = factories.transition(24, 4, precision="fp32")
    released.load(engine, released.transition_from_released(state))
    x = torch.randn(2, L, 24)
    with torch.no_grad():
        _close(engine(x), rel.transition(x, state))


def test_msa_pair_weighted_averaging_discards_the_pair_norm_offset():
    state = _rand(msa_attention_shapes(16, 32, 4, 4), 5)
    converted = released.msa_pair_weighted_averaging_from_released(state)
    assert released.is_discarded("pair_norm.bias") and "ln_pair.bias" not in converted
    engine = factories.msa_pair_weighted_averaging(16, 32, 4, precision="fp32")
    released.load(engine, converted)
    msa, pair = torch.randn(5, L, 16), torch.randn(L, L, 32)
    tokens, _ = _masks()
    msa_mask = (torch.rand(5, L, generator=torch.Generator().manual_seed(1)) > 0.1) & tokens[None]
    msa_mask[0] = tokens
    with torch.no_grad():
        actual = engine(msa[None], pair[None], msa_mask.any(0)[None])[0]
    _close(actual, rel.msa_attention(msa, msa_mask, pair, state, n_head=4), (slice(None), tokens))


def test_outer_product_mean():
    state = _rand(opm_shapes(16, 6, 32), 6, std=0.2)
    converted = released.outer_product_mean_from_released(state)
    assert converted["to_out.weight"].shape == (32, 36)
    engine = factories.outer_product_mean(16, 32, 6, normalize_before_proj=False, count_offset=1e-3,
                                          precision="fp32")
    released.load(engine, converted)
    msa = torch.randn(5, L, 16)
    tokens, pair = _masks()
    mask = (torch.rand(5, L, generator=torch.Generator().manual_seed(2)) > 0.1) & tokens[None]
    mask[0] = tokens
    with torch.no_grad():
        actual = engine(msa[None], mask[None])[0]
    _close(actual, rel.outer_product_mean(msa, mask, state), pair, tol=1e-4)


def test_pairformer_block_with_single_track():
    c, heads, cs = 32, 4, 48
    state = _rand(block_shapes(c, heads, cs, heads_single=4), 7, std=0.1)
    block = factories.pairformer_block(d_pair=c, triangle_model="af3", d_single=cs, n_head_single=4,
                                       d_hidden_tri_attention=c // heads, precision="fp32")
    released.load(block, released.pairformer_block_from_released(state))
    z, s = torch.randn(L, L, c), torch.randn(L, cs)
    tokens, pair = _masks()
    with torch.no_grad():
        za, sa = block(z[None], tokens[None], s[None])
    zw, sw = rel.pairformer_block(z, tokens, state, n_head_pair=heads, single=s, n_head_single=4)
    _close(za[0], zw, pair, tol=1e-4)
    _close(sa[0], sw, tokens, tol=1e-4)


def test_msa_block():
    cm, c, heads = 16, 32, 4
    state = _rand(msa_block_shapes(cm, c, heads), 8, std=0.1)
    block = factories.msa_block(cm, c, heads, opm_channel=4, precision="fp32")
    released.load(block, released.msa_block_from_released(state))
    msa, z = torch.randn(5, L, cm), torch.randn(L, L, c)
    tokens, pair = _masks()
    msa_mask = ((torch.rand(5, L, generator=torch.Generator().manual_seed(3)) > 0.1) & tokens[None]).float()
    msa_mask[0] = tokens.float()
    with torch.no_grad():
        ma, za = block(msa, z, msa_mask, pair.float())
    mw, zw = rel.msa_block(msa, z, msa_mask, tokens, state, n_head_pair=heads)
    _close(za, zw, pair, tol=1e-4)
    _close(ma, mw, (slice(None), tokens), tol=1e-4)


class _Model(nn.Module):
    """A whole-model stand-in: two trunk blocks, one MSA block and a plain parameter."""

    def __init__(self, c: int, cs: int, cm: int) -> None:
        super().__init__()
        self.evoformer = nn.Module()
        self.evoformer.trunk_pairformer = nn.ModuleList(
            factories.pairformer_block(d_pair=c, triangle_model="af3", d_single=cs, n_head_single=4)
            for _ in range(2))
        self.evoformer.msa_stack = nn.ModuleList([factories.msa_block(cm, c, 4, opm_channel=4)])
        self.evoformer.prev_single_embedding = nn.Linear(cs, cs, bias=False)


def _model_state(c: int, cs: int, cm: int) -> dict[str, torch.Tensor]:
    shapes = {}
    for i in range(2):
        shapes |= _prefixed(f"evoformer.trunk_pairformer.{i}", block_shapes(c, 4, cs, d_tri=32))
    shapes |= _prefixed("evoformer.msa_stack.0", msa_block_shapes(cm, c, 4))
    shapes["evoformer.prev_single_embedding.weight"] = (cs, cs)
    return _rand(shapes, 9)


def test_convert_state_is_exact_and_the_file_round_trips(tmp_path):
    c, cs, cm = 32, 48, 16
    model = _Model(c, cs, cm)
    state = _model_state(c, cs, cm)
    converted = checkpoint.convert_state(state, model)
    assert set(converted) == set(model.state_dict())
    path = checkpoint.write(tmp_path / "af3.miniworld.pt", converted, family="alphafold3", source="test")
    assert checkpoint.is_native(path)
    report = checkpoint.load_into(model, path, family="alphafold3")
    assert report["mapped_records"] == len(converted)
    for k, v in model.state_dict().items():
        assert torch.equal(v, converted[k]), k
    # the trunk blocks of the whole-model file load into a PairformerTrunk
    trunk = PairformerTrunk(2, d_pair=c, d_single=cs, n_head_single=4)
    checkpoint.load_into(trunk, path, family="alphafold3", prefix=checkpoint.TRUNK_PREFIX,
                         renumber_as="blocks")
    assert torch.equal(trunk.blocks[1].tri_multi_incoming.to_left.weight,
                       state["evoformer.trunk_pairformer.1.triangle_multiplication_incoming.projection.weight"][1::2])
    with pytest.raises(ValueError, match="family"):
        checkpoint.load_into(model, path, family="boltz2")


def test_conversion_errors(tmp_path):
    c, cs, cm = 32, 48, 16
    model = _Model(c, cs, cm)
    state = _model_state(c, cs, cm)
    unknown = dict(state)
    unknown["evoformer.trunk_pairformer.0.pair_attention1.mystery.weight"] = torch.zeros(3)
    with pytest.raises(checkpoint.ConversionError, match="mystery"):
        checkpoint.convert_state(unknown, model)
    discarded = dict(state)
    discarded["evoformer.msa_stack.0.msa_attention1.pair_norm.bias"] = torch.zeros(c)
    checkpoint.convert_state(discarded, model)  # a known discard is fine
    stray = dict(state)
    stray["evoformer.not_a_parameter"] = torch.zeros(1)
    with pytest.raises(checkpoint.ConversionError, match="not_a_parameter"):
        checkpoint.convert_state(stray, model)
    missing = {k: v for k, v in state.items() if not k.endswith("pair_transition.transition2.weight")}
    with pytest.raises(KeyError):
        checkpoint.convert_state(missing, model)
    torch.save({"format": "other", "state_dict": {}}, tmp_path / "x.pt")
    with pytest.raises(ValueError, match="not a miniworld"):
        checkpoint.read(tmp_path / "x.pt")
    torch.save({"format": "miniworld", "version": 2, "state_dict": {}}, tmp_path / "y.pt")
    with pytest.raises(ValueError, match="version"):
        checkpoint.read(tmp_path / "y.pt")


def test_trunk_loader_reads_a_miniworld_file(tmp_path):
    import foldforge_amd

    c, cs, cm = 128, 384, 64
    trunk = PairformerTrunk(2)
    state = {f"evoformer.trunk_pairformer.{i}.{k}": v for i in range(2)
             for k, v in _rand(block_shapes(c, 4, cs, heads_single=16), 10 + i, std=0.05).items()}
    model = nn.Module()
    model.evoformer = nn.Module()
    model.evoformer.trunk_pairformer = trunk.blocks
    converted = checkpoint.convert_state(state, model)
    path = checkpoint.write(tmp_path / "t.miniworld.pt", converted, family="alphafold3", source="t")
    loaded = foldforge_amd.load(checkpoint=path, device="cpu", blocks=2, backend="pytorch")
    got = loaded.blocks[0].single_attention.to_bias.weight
    torch.testing.assert_close(got.float(), state["evoformer.trunk_pairformer.0.single_pair_logits_projection.weight"])
    assert isinstance(loaded.blocks[0], PairformerBlock) and not isinstance(loaded.blocks[0], MSABlock)

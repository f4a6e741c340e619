"""Released parameter layout (the AlphaFold 3 family's dense names) -> engine state dicts.

The counterpart of the reference's ``src/foldforge/models/checkpoints/legacy/released.py``
for the modules this build serves: the pair stack (triangle multiplication, triangle
attention, transition), the pairformer block with its single track, and the MSA-stack
ops (outer product mean, MSA pair-weighted averaging) with their block. Each function maps
a released state dict (optionally below ``prefix``) to the engine module's own keys by
views only (``chunk``, strided selection, ``reshape``/``T``) and copies no value; all run on
the CPU and keep the dtype. The rules:

* split -- ``transition1 [2 n c, c]`` -> ``expand_a`` / ``expand_b`` (first / second half);
  the triangle multiplication's ``projection`` / ``gate [2 h, c]`` -> ``to_left`` /
  ``to_right`` (and gates) by the per-channel interleave (row ``2 k`` is branch a of channel
  ``k``, row ``2 k + 1`` branch b; the incoming module takes branch b as ``left``, since the
  engine contracts ``left[k, i] right[k, j]`` where the release writes ``"ckj,cki->cij"``);
  the outer product mean's ``output_w [K, K, c_z]`` -> ``to_out.weight [c_z, K K]``;
* discard -- the pair-LayerNorm offsets that only add one constant per head to softmax
  logits (``DISCARDED``);
* rename -- everything else.
"""

from __future__ import annotations

import re
from collections.abc import Mapping

import torch
from torch import nn

Tensor = torch.Tensor
State = Mapping[str, Tensor]

#: Released keys (regular expressions) with no engine parameter: offsets of pair norms whose
#: output only feeds softmax logits, so the offset adds a per-head constant that cancels.
DISCARDED = (
    r"(^|\.)pair_norm\.bias$",                  # MSA pair-weighted averaging
    r"(^|\.)single_pair_logits_norm\.bias$",    # the pairformer's single attention
)


class ConversionError(RuntimeError):
    """A released state that does not convert exactly (a key left unread that is not a known
    discard; a missing, extra or mis-shaped key)."""


def is_discarded(key: str) -> bool:
    return any(re.search(p, key) for p in DISCARDED)


class Tracked(dict):
    """A released state dict that records which full keys a conversion read."""

    def __init__(self, items: Mapping[str, Tensor], used: set[str] | None = None,
                 prefix: str = "") -> None:
        super().__init__(items)
        self.used = set() if used is None else used
        self.prefix = prefix

    def __getitem__(self, key: str) -> Tensor:
        self.used.add(self.prefix + key)
        return super().__getitem__(key)

    def below(self, prefix: str) -> Tracked:
        head = prefix + "." if prefix else ""
        return Tracked({k[len(head):]: v for k, v in self.items() if k.startswith(head)},
                       self.used, self.prefix + head)


def _below(state: State, prefix: str) -> dict[str, Tensor] | Tracked:
    if isinstance(state, Tracked):
        return state.below(prefix)
    head = prefix + "." if prefix else ""
    return {k[len(head):]: v for k, v in state.items() if k.startswith(head)}


def _require(state: State, *keys: str) -> None:
    missing = [k for k in keys if k not in state]
    if missing:
        raise KeyError(f"released state lacks {missing} (has {sorted(state)[:10]} ...)")


def _copy_norm(out: dict[str, Tensor], name: str, s: State, key: str, bias: bool = True) -> None:
    _require(s, f"{key}.weight", *([f"{key}.bias"] if bias else []))
    out[f"{name}.weight"] = s[f"{key}.weight"]
    if bias:
        out[f"{name}.bias"] = s[f"{key}.bias"]


def _copy_linear(out: dict[str, Tensor], name: str, s: State, key: str) -> None:
    """Weight, and the bias when the release has one."""
    out[f"{name}.weight"] = s[f"{key}.weight"]
    if f"{key}.bias" in s:
        out[f"{name}.bias"] = s[f"{key}.bias"]


# ------------------------------------------------------------------------------- pair track
def triangle_multiplication_from_released(state: State, *, outgoing: bool,
                                          prefix: str = "") -> dict[str, Tensor]:
    """Released ``left_norm_input projection gate center_norm output_projection gating_linear``
    (``legacy/triangle_multiplication.py:38-47``) -> engine ``TriangleMultiplication``."""
    s = _below(state, prefix)
    _require(s, "projection.weight", "gate.weight", "output_projection.weight", "gating_linear.weight")
    proj, gate = s["projection.weight"], s["gate.weight"]
    if proj.dim() != 2 or proj.shape[0] % 2 or gate.shape != proj.shape:
        raise ValueError(f"projection {tuple(proj.shape)} / gate {tuple(gate.shape)} must both "
                         "be [2 * hidden, c]")
    a_rows, b_rows = slice(0, None, 2), slice(1, None, 2)  # branch a = even rows, b = odd
    left, right = (a_rows, b_rows) if outgoing else (b_rows, a_rows)
    out: dict[str, Tensor] = {}
    _copy_norm(out, "ln_pair", s, "left_norm_input")
    _copy_norm(out, "ln_out", s, "center_norm")
    out["to_left.weight"], out["to_right.weight"] = proj[left], proj[right]
    out["to_left_gate.weight"], out["to_right_gate.weight"] = gate[left], gate[right]
    out["to_out.weight"] = s["output_projection.weight"]
    out["to_gate.weight"] = s["gating_linear.weight"]
    return {k: v.contiguous() for k, v in out.items()}


_TRIATTN_NAMES = (("to_bias", "pair_bias_projection"), ("to_query", "q_projection"),
                  ("to_key", "k_projection"), ("to_value", "v_projection"),
                  ("to_gate", "gating_query"), ("to_out", "output_projection"))


def triangle_attention_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """Released grid self-attention ``act_norm pair_bias_projection q/k/v_projection
    gating_query output_projection [output_projection_transposed]``
    (``legacy/attention.py:89-106``) -> engine ``TriangleAttention`` (a rename; gate / output
    biases carried when present, RoseTTAFold3's; Chai-1's confidence head's second output
    projection becomes ``to_out_t``)."""
    s = _below(state, prefix)
    _require(s, *(f"{key}.weight" for _, key in _TRIATTN_NAMES))
    out: dict[str, Tensor] = {}
    _copy_norm(out, "ln_pair", s, "act_norm")
    for name, key in _TRIATTN_NAMES:
        _copy_linear(out, name, s, key)
    if "output_projection_transposed.weight" in s:
        _copy_linear(out, "to_out_t", s, "output_projection_transposed")
    return out


def transition_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """Released ``input_layer_norm transition1 [2 n c, c] transition2``
    (``legacy/primitives.py:20-37``) -> engine ``Transition``."""
    s = _below(state, prefix)
    _require(s, "transition1.weight", "transition2.weight")
    t1 = s["transition1.weight"]
    half = t1.shape[0] // 2
    out: dict[str, Tensor] = {}
    _copy_norm(out, "ln_in", s, "input_layer_norm")
    out["expand_a.weight"] = t1[:half].contiguous()
    out["expand_b.weight"] = t1[half:].contiguous()
    out["squeeze.weight"] = s["transition2.weight"]
    return out


# -------------------------------------------------------------------------------- MSA stack
def outer_product_mean_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """Released ``layer_norm_input left/right_projection output_w output_b
    [product_norm]`` (``legacy/primitives.py:62-78``) -> engine ``OuterProductMean``;
    ``output_w [(G,) K, K, c_z]`` flattens to ``to_out.weight [c_z, G K K]``."""
    s = _below(state, prefix)
    _require(s, "left_projection.weight", "right_projection.weight", "output_w", "output_b")
    out: dict[str, Tensor] = {}
    _copy_norm(out, "ln_msa", s, "layer_norm_input")
    _copy_linear(out, "to_left", s, "left_projection")
    _copy_linear(out, "to_right", s, "right_projection")
    w = s["output_w"]
    out["to_out.weight"] = w.reshape(-1, w.shape[-1]).T.contiguous()
    out["to_out.bias"] = s["output_b"]
    if "product_norm.weight" in s:
        _copy_norm(out, "product_norm", s, "product_norm")
    return out


def msa_pair_weighted_averaging_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """Released MSA attention ``act_norm pair_norm pair_logits v_projection gating_query
    output_projection`` (``legacy/attention.py:193-200``) -> engine
    ``MSAPairWeightedAveraging``; the pair norm's offset is discarded."""
    s = _below(state, prefix)
    _require(s, "pair_norm.weight", "pair_logits.weight", "v_projection.weight",
             "gating_query.weight", "output_projection.weight")
    out: dict[str, Tensor] = {}
    _copy_norm(out, "ln_msa", s, "act_norm")
    out["ln_pair.weight"] = s["pair_norm.weight"]
    for name, key in (("to_bias", "pair_logits"), ("to_value", "v_projection"),
                      ("to_gate", "gating_query"), ("to_out", "output_projection")):
        out[f"{name}.weight"] = s[f"{key}.weight"]
    return out


# ------------------------------------------------------------------------------------ blocks
def attention_pair_bias_from_released(attention: State, norm: State,
                                      projection: State) -> dict[str, Tensor]:
    """The pairformer's single attention (``single_attention_``, ``legacy/transformer.py:
    28-90``) with its pair-logit norm and projection -> engine ``AttentionPairBias``; the
    norm's offset is discarded."""
    a = attention
    _require(a, "adaptive_layernorm.layer_norm.weight", "adaptive_layernorm.layer_norm.bias",
             "q_projection.weight", "q_projection.bias", "k_projection.weight",
             "v_projection.weight", "gating_query.weight", "adaptive_zero_init.transition2.weight")
    _require(norm, "weight")
    _require(projection, "weight")
    return {
        "ln_single.weight": a["adaptive_layernorm.layer_norm.weight"],
        "ln_single.bias": a["adaptive_layernorm.layer_norm.bias"],
        "to_query.weight": a["q_projection.weight"],
        "to_query.bias": a["q_projection.bias"],
        "to_key.weight": a["k_projection.weight"],
        "to_value.weight": a["v_projection.weight"],
        "ln_pair.weight": norm["weight"],
        "to_bias.weight": projection["weight"],
        "to_gate.weight": a["gating_query.weight"],
        "to_out.weight": a["adaptive_zero_init.transition2.weight"],
    }


def _nest(out: dict[str, Tensor], name: str, tensors: Mapping[str, Tensor]) -> None:
    out.update({f"{name}.{k}": v for k, v in tensors.items()})


def pairformer_block_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """A released pairformer block (``legacy/pairformer.py:153-230`` names) -> this build's
    ``PairformerBlock``: ``triangle_multiplication_outgoing / incoming`` ->
    ``tri_multi_outgoing / incoming``, ``pair_attention1 / 2`` -> ``tri_atten_starting /
    ending``, ``pair_transition`` -> ``transition_pair``, and when present ``single_attention_``
    + ``single_pair_logits_*`` -> ``single_attention``, ``single_transition``."""
    s = _below(state, prefix)
    out: dict[str, Tensor] = {}
    _nest(out, "tri_multi_outgoing", triangle_multiplication_from_released(
        s, outgoing=True, prefix="triangle_multiplication_outgoing"))
    _nest(out, "tri_multi_incoming", triangle_multiplication_from_released(
        s, outgoing=False, prefix="triangle_multiplication_incoming"))
    if any(k.startswith("pair_attention1.") for k in s):
        _nest(out, "tri_atten_starting", triangle_attention_from_released(s, prefix="pair_attention1"))
        _nest(out, "tri_atten_ending", triangle_attention_from_released(s, prefix="pair_attention2"))
    _nest(out, "transition_pair", transition_from_released(s, prefix="pair_transition"))
    if any(k.startswith("single_attention_.") for k in s):
        _nest(out, "single_attention", attention_pair_bias_from_released(
            _below(s, "single_attention_"), _below(s, "single_pair_logits_norm"),
            _below(s, "single_pair_logits_projection")))
        _nest(out, "single_transition", transition_from_released(s, prefix="single_transition"))
    return out


def msa_block_from_released(state: State, *, prefix: str = "") -> dict[str, Tensor]:
    """A released MSA-stack block (the dense ``EvoformerBlock``) -> this build's ``MSABlock``
    (same attribute names: ``outer_product_mean``, ``msa_attention1``, ``msa_transition``, the
    two triangle multiplications, ``pair_attention1 / 2`` when present, ``pair_transition``)."""
    s = _below(state, prefix)
    out: dict[str, Tensor] = {}
    _nest(out, "outer_product_mean", outer_product_mean_from_released(s, prefix="outer_product_mean"))
    _nest(out, "msa_attention1", msa_pair_weighted_averaging_from_released(s, prefix="msa_attention1"))
    _nest(out, "msa_transition", transition_from_released(s, prefix="msa_transition"))
    for name, outgoing in (("triangle_multiplication_outgoing", True),
                           ("triangle_multiplication_incoming", False)):
        _nest(out, name, triangle_multiplication_from_released(s, outgoing=outgoing, prefix=name))
    for name in ("pair_attention1", "pair_attention2"):
        if any(k.startswith(name + ".") for k in s):
            _nest(out, name, triangle_attention_from_released(s, prefix=name))
    _nest(out, "pair_transition", transition_from_released(s, prefix="pair_transition"))
    return out


@torch.no_grad()
def load(module: nn.Module, converted: Mapping[str, Tensor]) -> nn.Module:
    """Strict load keeping the module's parameter dtypes (fp32 masters stay fp32: the released
    values are copied in, never rounded)."""
    own = module.state_dict()
    extra = sorted(set(converted) - set(own))
    if extra:
        raise ConversionError(f"{type(module).__name__} has no parameter for {extra[:8]}")
    wrong = sorted(k for k in converted if tuple(converted[k].shape) != tuple(own[k].shape))
    if wrong:
        raise ConversionError(f"mis-shaped: {[(k, tuple(converted[k].shape), tuple(own[k].shape)) for k in wrong[:4]]}")
    module.load_state_dict(dict(converted), strict=True)
    return module

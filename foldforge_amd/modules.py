"""Engine-compatible op classes of the pair stack with a native ``hip`` backend.

These mirror the classes FoldForge's graph holds from ``miniworld_engine.modules``
(imported at ``src/foldforge/modules/engine/modules.py:23-31`` of the reference) and
keep their contract (``src/foldforge/modules/engine/policy.py:85-101``,
``tests/kernels/test_backends.py``, ``tests/models/test_dead_modules.py:97-136``):

* ``backends`` (class attribute), ``backend``, ``set_backend(name)``;
* ``unsupported(*args) -> str | None``: whether the CURRENT backend takes the call,
  asked before the call; ``forward`` and ``delta`` raise :class:`BackendUnsupported` for a
  call outside the backend's range (the engine never falls back; FoldForge's guard does,
  and so does a module given the refusal policy ``"fallback"`` by
  :func:`foldforge_amd.dispatch.install`);
* ``_forward_<backend>(*args)`` for every listed backend;
* residual-owning forwards (``x + f(x)``) and ``delta(*args)`` for the bare update;
* ``dead = False`` class attribute; a dead module returns its input unchanged;
* fp32 master parameters (:class:`MasterWeights`) that stay fp32 under a bulk
  ``.to(torch.bfloat16)``; LayerNorm affines are fp32 under any cast;
* the engine's ``state_dict`` keys (``legacy/released.py:135-368``).

The ``hip`` backend calls :mod:`foldforge_amd.kernels` (one C-ABI call per op) and has
no fallback of its own: if the native library is missing the call raises.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from typing import Any

import torch
from torch import nn

from foldforge_amd import dispatch, torch_ops

Tensor = torch.Tensor

HIP_ARCH = "gfx950"


class BackendUnsupported(RuntimeError):
    """A call outside the selected backend's range (the engine's own refusal error)."""


def device_arch(device: torch.device) -> str | None:
    """gfx architecture of a ROCm device (``"gfx950"`` on an MI355X), None elsewhere."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return None
    name = torch.cuda.get_device_properties(device).gcnArchName
    return name.split(":")[0]


def hip_reason(*tensors: Tensor) -> str | None:
    """Why the hip backend cannot take tensors on these devices (None: it can)."""
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            return f"a {t.device.type} tensor (the hip backend needs a gfx950 device)"
        arch = device_arch(t.device)
        if arch != HIP_ARCH:
            return f"device arch {arch} (the hip kernels are built for {HIP_ARCH})"
    return None


# ------------------------------------------------------------------------------------ mixins
class MasterWeights:
    """fp32 master parameters: under ``master_weights`` a bulk cast moves them but keeps fp32.

    Activations are bf16 (autocast) while the parameters stay fp32 masters
    (``src/foldforge/modules/engine/configure.py:1-6`` of the reference).
    """

    master_weights: bool = False

    def set_master_weights(self) -> None:
        for m in self.modules():  # type: ignore[attr-defined]
            if isinstance(m, MasterWeights):
                m.master_weights = True
        self.float()  # type: ignore[attr-defined]

    def _apply(self, fn, recurse=True):  # type: ignore[override]
        if not self.master_weights:
            return super()._apply(fn, recurse)  # type: ignore[misc]

        def keep_fp32(t: Tensor) -> Tensor:
            out = fn(t)
            if t.dtype == torch.float32 and out.dtype != torch.float32:
                return t.to(device=out.device)
            return out

        return super()._apply(keep_fp32, recurse)  # type: ignore[misc]


class EngineOp:
    """Backend dispatch of one op class (mixed into an ``nn.Module``).

    A call goes to ``_forward_<backend>``. When the backend refuses it (``unsupported``
    returns a reason) the module's ``refusal_policy`` decides: ``None`` (the engine's own
    behaviour) raises :class:`BackendUnsupported`; ``"error"`` raises
    :class:`foldforge_amd.dispatch.BackendUnsupportedError`; ``"fallback"`` runs ``pytorch``
    and logs the reason once. ``forward`` and ``delta`` take the same route, so a refused
    call never changes backend silently. Every call is counted in the module's ledger.
    """

    backends: tuple[str, ...] = ("pytorch", "hip")
    dead: bool = False
    refusal_policy: str | None = None

    def _init_backend(self, backend: str) -> None:
        self.backend = "pytorch"
        self.set_backend(backend)

    def set_backend(self, name: str) -> None:
        if name not in self.backends:
            raise ValueError(
                f"{type(self).__name__} has no {name!r} backend (available: {', '.join(self.backends)})"
            )
        self.backend = name

    def unsupported(self, *args: Any, **kwargs: Any) -> str | None:
        """Why the current backend cannot take this call (None: it can)."""
        if self.backend == "pytorch":
            return None
        return getattr(self, f"_unsupported_{self.backend}")(*args, **kwargs)

    def _route(self, args: tuple, kwargs: dict) -> str:
        """The backend this call runs on (refusals handled by the policy, the call counted)."""
        backend = self.backend
        if backend != "pytorch":
            reason = self.unsupported(*args, **kwargs)
            if reason is not None:
                backend = dispatch.on_refusal(self, reason, BackendUnsupported)  # type: ignore[arg-type]
        dispatch.note_call(self, backend)  # type: ignore[arg-type]
        return backend

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return getattr(self, f"_forward_{self._route(args, kwargs)}")(*args, **kwargs)

    def delta(self, *args: Any, **kwargs: Any) -> Tensor:
        """The bare update ``f(x)`` (the forward returns ``x + f(x)``)."""
        return getattr(self, f"_forward_{self._route(args, kwargs)}")(*args, residual=False, **kwargs)


def _linear(d_in: int, d_out: int, bias: bool = False) -> nn.Linear:
    return nn.Linear(d_in, d_out, bias=bias)


# ------------------------------------------------------------------------------------ LayerNorm
class LayerNorm(EngineOp, nn.LayerNorm):
    """The engine LayerNorm: fp32 affine under any cast, output in the input dtype
    (``src/foldforge/modules/engine/modules.py:230-238``)."""

    def __init__(self, normalized_shape, eps: float = 1e-5, bias: bool = True,
                 elementwise_affine: bool = True, backend: str = "pytorch") -> None:
        nn.LayerNorm.__init__(self, normalized_shape, eps=eps,
                              elementwise_affine=elementwise_affine, bias=bias)
        self._init_backend(backend)

    def _apply(self, fn, recurse=True):  # type: ignore[override]
        def keep_fp32(t: Tensor) -> Tensor:
            out = fn(t)
            if t.dtype == torch.float32 and out.dtype != torch.float32:
                return t.to(device=out.device)
            return out

        return super()._apply(keep_fp32, recurse)

    def _unsupported_hip(self, x: Tensor) -> str | None:
        reason = hip_reason(x)
        if reason is not None:
            return reason
        if x.dtype not in (torch.bfloat16, torch.float32):
            return f"dtype {x.dtype} (the kernel takes bf16 or fp32)"
        if len(self.normalized_shape) != 1:
            return "normalisation over more than one axis"
        return None

    def _forward_pytorch(self, x: Tensor) -> Tensor:
        return torch_ops.layer_norm(self, x)

    def _forward_hip(self, x: Tensor) -> Tensor:
        from foldforge_amd import kernels

        return kernels.layer_norm(x.contiguous(), self.weight, self.bias, self.eps)


# ------------------------------------------------------------------------------------ pair ops
def _pair_reason(z: Tensor, mask: Tensor) -> str | None:
    reason = hip_reason(z, mask)
    if reason is not None:
        return reason
    if z.dtype != torch.bfloat16:
        return f"{z.dtype} activations (the kernels take bf16)"
    if z.dim() != 4 or z.shape[1] != z.shape[2]:
        return f"pair shape {tuple(z.shape)} (the kernels take [B, N, N, c])"
    if mask is None or mask.shape != z.shape[:2]:
        return "the kernels need a [B, N] key mask"
    if z.shape[0] * 128 > 65535 or z.shape[1] > 65535 - 127:
        return f"pair shape {tuple(z.shape)} exceeds the launch grid"
    return None


class TriangleMultiplication(EngineOp, MasterWeights, nn.Module):
    """Triangle multiplicative update (outgoing / incoming), residual included
    (equations ``legacy/reference/triangle.py:19-49``; parameters ``legacy/released.py:166-173``)."""

    divide_by_length = False

    def __init__(self, d_pair: int, d_hidden: int | None = None, outgoing: bool = True,
                 p_drop: float = 0.0, model: str | None = None, backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        hidden = d_pair if d_hidden is None else d_hidden
        self.d_pair, self.d_hidden, self.outgoing, self.p_drop = d_pair, hidden, outgoing, p_drop
        self.ln_pair = LayerNorm(d_pair)
        self.to_left = _linear(d_pair, hidden)
        self.to_right = _linear(d_pair, hidden)
        self.to_left_gate = _linear(d_pair, hidden)
        self.to_right_gate = _linear(d_pair, hidden)
        self.ln_out = LayerNorm(hidden)
        self.to_out = _linear(hidden, d_pair)
        self.to_gate = _linear(d_pair, d_pair)
        self._init_backend(backend)

    def __new__(cls, *args: Any, **kwargs: Any):
        if cls is TriangleMultiplication and kwargs.get("model") == "rf3":
            cls = TriangleMultiplicationRF3
        return super().__new__(cls)

    def _unsupported_hip(self, x: Tensor, mask: Tensor) -> str | None:
        reason = _pair_reason(x, mask)
        if reason is not None:
            return reason
        from foldforge_amd.kernels import trimul_supported

        if x.shape[-1] != self.d_pair or not trimul_supported(self.d_pair, self.d_hidden):
            return (f"d_pair={x.shape[-1]} d_hidden={self.d_hidden} (the kernels take 128 / 128, or a "
                    "pair width a multiple of 64 up to 256 with a hidden width a multiple of 64 up to 768)")
        return None

    def _forward_pytorch(self, x: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        return torch_ops.triangle_multiplication(self, x, mask, residual=residual)

    def _forward_hip(self, x: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        from foldforge_amd import kernels

        return kernels.triangle_multiplicative_update(
            x.contiguous(), mask.contiguous(),
            ln_pair_weight=self.ln_pair.weight, ln_pair_bias=self.ln_pair.bias,
            to_left=self.to_left.weight, to_right=self.to_right.weight,
            to_left_gate=self.to_left_gate.weight, to_right_gate=self.to_right_gate.weight,
            ln_out_weight=self.ln_out.weight, ln_out_bias=self.ln_out.bias,
            to_out=self.to_out.weight, to_gate=self.to_gate.weight,
            outgoing=self.outgoing, residual=residual, length_divided=self.divide_by_length,
            eps=self.ln_pair.eps,
        )


class TriangleMultiplicationRF3(TriangleMultiplication):
    """RoseTTAFold3's exact form: the contraction divided by the real length
    (``legacy/routing.py:33-55``, ``legacy/reference/triangle.py:46-48``)."""

    divide_by_length = True


#: ``TriangleAttention(model=...)`` key -> the key's class. The lineages differ in four places
#: (``src/foldforge/modules/dense/spec.py``): the ending node's bias from the transposed pair
#: (the OpenFold lineage, ``:116-125``), gate and output projection biases (RoseTTAFold3,
#: ``:437,645``), the ending node's update added without turning it back (Chai-1's trunk,
#: ``:463-470,716``) and a second, transposed output projection (Chai-1's confidence head,
#: ``:476-478,694``).
TRIANGLE_ATTENTION_MODELS: dict[str, str] = {
    "af3": "TriangleAttentionAF3",
    "openfold3": "TriangleAttentionAF3",
    "intellifold2": "TriangleAttentionAF3",
    "openfold3_preview2": "TriangleAttentionOpenFold",
    "protenix": "TriangleAttentionOpenFold",
    "boltz2": "TriangleAttentionOpenFold",
    "opendde": "TriangleAttentionOpenFold",
    "rf3": "TriangleAttentionRF3",
    "chai1": "TriangleAttentionChai1",
    "chai1_confidence": "TriangleAttentionChai1Confidence",
}


class TriangleAttention(EngineOp, MasterWeights, nn.Module):
    """Triangle attention around the starting / ending node, residual included
    (``legacy/attention.py:60-171``; parameters ``legacy/released.py:176-208``).

    ``TriangleAttention(..., model=key)`` builds the key's class (``TRIANGLE_ATTENTION_MODELS``).
    ``d_hidden`` is the total hidden width (default ``d_pair``). The class attributes name the
    lineage's form: ``transposed_bias``, ``projection_bias`` (``to_gate`` / ``to_out`` carry
    biases), ``untransposed_output`` and ``dual_output`` (``to_out_t``).
    """

    transposed_bias = False
    projection_bias = False
    untransposed_output = False
    dual_output = False

    def __new__(cls, *args: Any, **kwargs: Any):
        if cls is TriangleAttention:
            model = kwargs.get("model", "af3")
            if model not in TRIANGLE_ATTENTION_MODELS:
                raise ValueError(
                    f"no triangle attention class for model {model!r} in this build "
                    f"(known: {', '.join(TRIANGLE_ATTENTION_MODELS)})"
                )
            cls = globals()[TRIANGLE_ATTENTION_MODELS[model]]
        return super().__new__(cls)

    def __init__(self, d_pair: int, n_head: int, d_hidden: int | None = None,
                 starting: bool = True, p_drop: float = 0.0, model: str = "af3",
                 backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        hidden = d_pair if d_hidden is None else d_hidden
        self.d_pair, self.n_head, self.d_hidden = d_pair, n_head, hidden
        self.starting, self.p_drop, self.model = starting, p_drop, model
        self.ln_pair = LayerNorm(d_pair)
        self.to_bias = _linear(d_pair, n_head)
        self.to_query = _linear(d_pair, hidden)
        self.to_key = _linear(d_pair, hidden)
        self.to_value = _linear(d_pair, hidden)
        self.to_gate = _linear(d_pair, hidden, bias=self.projection_bias)
        self.to_out = _linear(hidden, d_pair, bias=self.projection_bias)
        if self.dual_output:
            self.to_out_t = _linear(hidden, d_pair, bias=self.projection_bias)
        self._init_backend(backend)

    def _unsupported_hip(self, x: Tensor, mask: Tensor) -> str | None:
        reason = _pair_reason(x, mask)
        if reason is not None:
            return reason
        from foldforge_amd.kernels import triangle_attention_supported

        d = self.d_hidden // self.n_head
        if (x.shape[-1] != self.d_pair or self.d_hidden % self.n_head
                or not triangle_attention_supported(self.d_pair, self.n_head, d, self.transposed_bias)):
            return (f"d_pair={x.shape[-1]} heads={self.n_head} hidden={self.d_hidden} (the kernels "
                    "take 128 with 4 x 32, or pair 64 / 128 / 256 with at most 32 heads of 8 to 64 "
                    "channels, heads x d_head a multiple of 64)")
        if (self.d_pair, self.n_head, d) != (128, 4, 32) and x.shape[0] * x.shape[1] > 65535:
            return f"batch x n = {x.shape[0] * x.shape[1]} exceeds the launch grid"
        return None

    def _forward_pytorch(self, x: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        return torch_ops.triangle_attention(self, x, mask, residual=residual)

    def _forward_hip(self, x: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        from foldforge_amd import kernels

        return kernels.triangle_attention(
            x.contiguous(), mask.contiguous(),
            ln_pair_weight=self.ln_pair.weight, ln_pair_bias=self.ln_pair.bias,
            to_bias=self.to_bias.weight, to_query=self.to_query.weight,
            to_key=self.to_key.weight, to_value=self.to_value.weight,
            to_gate=self.to_gate.weight, to_out=self.to_out.weight, n_head=self.n_head,
            gate_bias=self.to_gate.bias, out_bias=self.to_out.bias,
            to_out_t=self.to_out_t.weight if self.dual_output else None,
            out_t_bias=self.to_out_t.bias if self.dual_output else None,
            starting=self.starting, transposed_bias=self.transposed_bias,
            untransposed_output=self.untransposed_output, residual=residual, eps=self.ln_pair.eps,
        )


class TriangleAttentionAF3(TriangleAttention):
    """AF3: the ending node's bias comes from the un-transposed pair (``legacy/attention.py:144-147``)."""

    transposed_bias = False


class TriangleAttentionOpenFold(TriangleAttention):
    """OpenFold lineage: the ending node's bias comes from the transposed pair."""

    transposed_bias = True


class TriangleAttentionRF3(TriangleAttentionAF3):
    """RoseTTAFold3: AF3's form with biases on the gate and output projections
    (``legacy/attention.py:97-102`` with ``spec.triangle_attention_bias``)."""

    projection_bias = True


class TriangleAttentionChai1(TriangleAttentionAF3):
    """Chai-1's trunk: the ending node's update is added in the attention's own orientation,
    not turned back (``legacy/attention.py:84-88,160-163``)."""

    untransposed_output = True


class TriangleAttentionChai1Confidence(TriangleAttentionAF3):
    """Chai-1's confidence head: a second output projection ``to_out_t`` of the same gated
    values, added transposed over the pair axes (``legacy/attention.py:103-106,129-131,152-158``;
    released ``output_projection_transposed``)."""

    dual_output = True


class Transition(EngineOp, MasterWeights, nn.Module):
    """SwiGLU transition, residual included (``legacy/reference/transition.py:28-59``;
    parameters ``legacy/released.py:211-224``)."""

    def __init__(self, d_hidden: int, n: int = 4, backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        self.d, self.n = d_hidden, n
        self.ln_in = LayerNorm(d_hidden)
        self.expand_a = _linear(d_hidden, n * d_hidden)
        self.expand_b = _linear(d_hidden, n * d_hidden)
        self.squeeze = _linear(n * d_hidden, d_hidden)
        self._init_backend(backend)

    def _unsupported_hip(self, x: Tensor) -> str | None:
        reason = hip_reason(x)
        if reason is not None:
            return reason
        if x.dtype != torch.bfloat16:
            return f"{x.dtype} activations (the kernel takes bf16)"
        from foldforge_amd.kernels import transition_supported

        if not transition_supported(self.d, self.n):
            return (f"width {self.d} x {self.n} (the kernels take 128 x 4, or d and "
                    "n * d multiples of 64)")
        return None

    def _forward_pytorch(self, x: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        return torch_ops.transition(self, x, residual=residual)

    def _forward_hip(self, x: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return x if residual else torch.zeros_like(x)
        from foldforge_amd import kernels

        return kernels.transition(
            x.contiguous(), ln_weight=self.ln_in.weight, ln_bias=self.ln_in.bias,
            expand_a=self.expand_a.weight, expand_b=self.expand_b.weight,
            squeeze=self.squeeze.weight, residual=residual, eps=self.ln_in.eps,
        )


class AttentionPairBias(EngineOp, MasterWeights, nn.Module):
    """Single-track attention with pair bias, residual included
    (``legacy/transformer.py:28-137``; parameters ``legacy/released.py:281-315``).
    The pair norm has no offset (a per-head constant is softmax-invariant)."""

    def __init__(self, d_single: int, d_pair: int, n_head: int = 16, gate_bias: float = 0.0,
                 backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        self.d_single, self.d_pair, self.n_head, self.gate_bias = d_single, d_pair, n_head, gate_bias
        self.ln_single = LayerNorm(d_single)
        self.to_query = _linear(d_single, d_single, bias=True)
        self.to_key = _linear(d_single, d_single)
        self.to_value = _linear(d_single, d_single)
        self.ln_pair = LayerNorm(d_pair, bias=False)
        self.to_bias = _linear(d_pair, n_head)
        self.to_gate = _linear(d_single, d_single)
        self.to_out = _linear(d_single, d_single)
        self._init_backend(backend)

    def _unsupported_hip(self, s: Tensor, z: Tensor, mask: Tensor,
                         extra_bias: Tensor | None = None) -> str | None:
        reason = _pair_reason(z, mask) or hip_reason(s)
        if reason is not None:
            return reason
        if s.dtype != torch.bfloat16:
            return f"{s.dtype} single activations (the kernels take bf16)"
        if s.dim() != 3 or s.shape[:2] != z.shape[:2] or s.shape[-1] != self.d_single:
            return f"single shape {tuple(s.shape)} for pair {tuple(z.shape)}"
        if z.shape[-1] != 128 or self.d_pair != 128:
            return f"d_pair={z.shape[-1]} (the kernels take 128)"
        from foldforge_amd.kernels import single_attention_heads_supported

        if not single_attention_heads_supported(self.d_single, self.n_head):
            return (f"d_single={self.d_single} heads={self.n_head} (the kernels take a multiple "
                    "of 64 split into at most 32 heads of 8, 16, 24 or 32)")
        if extra_bias is not None:
            if extra_bias.dtype not in (torch.float32, torch.bfloat16) or extra_bias.device != s.device:
                return f"extra bias {extra_bias.dtype} on {extra_bias.device} (the kernels take fp32 / bf16 on the device)"
            want = (s.shape[0], self.n_head, s.shape[1], s.shape[1])
            try:
                fits = torch.broadcast_shapes(tuple(extra_bias.shape), want) == torch.Size(want)
            except RuntimeError:
                fits = False
            if not fits:
                return f"extra bias {tuple(extra_bias.shape)} does not broadcast to {want}"
        return None

    def _forward_pytorch(self, s: Tensor, z: Tensor, mask: Tensor, extra_bias: Tensor | None = None,
                         *, residual: bool = True) -> Tensor:
        if self.dead:
            return s if residual else torch.zeros_like(s)
        return torch_ops.attention_pair_bias(self, s, z, mask, extra_bias, residual=residual)

    def _forward_hip(self, s: Tensor, z: Tensor, mask: Tensor, extra_bias: Tensor | None = None,
                     *, residual: bool = True) -> Tensor:
        if self.dead:
            return s if residual else torch.zeros_like(s)
        from foldforge_amd import kernels

        return kernels.attention_pair_bias(
            s.contiguous(), z.contiguous(), mask.contiguous(),
            ln_single_weight=self.ln_single.weight, ln_single_bias=self.ln_single.bias,
            to_query=self.to_query.weight, query_bias=self.to_query.bias,
            to_key=self.to_key.weight, to_value=self.to_value.weight,
            ln_pair_weight=self.ln_pair.weight, to_bias=self.to_bias.weight,
            to_gate=self.to_gate.weight, to_out=self.to_out.weight, n_head=self.n_head,
            gate_bias=self.gate_bias, extra_bias=extra_bias, residual=residual,
            eps_single=self.ln_single.eps, eps_pair=self.ln_pair.eps,
        )


# ------------------------------------------------------------------------------------ MSA stack
class MSAPairWeightedAveraging(EngineOp, MasterWeights, nn.Module):
    """MSA pair-weighted averaging, residual included (``legacy/attention.py:174-229``;
    parameters ``legacy/released.py:253-278``): every MSA row is averaged over the keys with
    one set of softmax weights per head taken from the pair. The pair norm has no offset
    (a per-head constant is softmax-invariant). ``d_hidden`` is the per-head value width
    (default ``d_msa // n_head``, the legacy ``value_dim``)."""

    def __init__(self, d_msa: int, d_pair: int, n_head: int = 8, d_hidden: int | None = None,
                 p_drop: float = 0.0, backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        dh = d_msa // n_head if d_hidden is None else d_hidden
        self.d_msa, self.d_pair, self.n_head, self.d_hidden, self.p_drop = d_msa, d_pair, n_head, dh, p_drop
        self.ln_msa = LayerNorm(d_msa)
        self.ln_pair = LayerNorm(d_pair, bias=False)
        self.to_bias = _linear(d_pair, n_head)
        self.to_value = _linear(d_msa, n_head * dh)
        self.to_gate = _linear(d_msa, n_head * dh)
        self.to_out = _linear(n_head * dh, d_msa)
        self._init_backend(backend)

    def _unsupported_hip(self, m: Tensor, z: Tensor, mask: Tensor) -> str | None:
        reason = _pair_reason(z, mask) or hip_reason(m)
        if reason is not None:
            return reason
        if m.dtype != torch.bfloat16:
            return f"{m.dtype} MSA activations (the kernels take bf16)"
        if m.dim() != 4 or m.shape[0] != z.shape[0] or m.shape[2] != z.shape[1] or m.shape[3] != self.d_msa:
            return f"MSA shape {tuple(m.shape)} for pair {tuple(z.shape)}"
        if z.shape[-1] != 128 or self.d_pair != 128:
            return f"d_pair={z.shape[-1]} (the kernels take 128)"
        from foldforge_amd.kernels import msa_pair_weighted_averaging_supported

        if not msa_pair_weighted_averaging_supported(self.d_msa, self.n_head, self.d_hidden):
            return (f"d_msa={self.d_msa} heads={self.n_head} x {self.d_hidden} (the kernels take "
                    "d_msa a multiple of 64 up to 768, at most 32 heads of a multiple of 4, "
                    "heads x d_head a multiple of 64 up to 768)")
        return None

    def _forward_pytorch(self, m: Tensor, z: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return m if residual else torch.zeros_like(m)
        return torch_ops.msa_pair_weighted_averaging(self, m, z, mask, residual=residual)

    def _forward_hip(self, m: Tensor, z: Tensor, mask: Tensor, *, residual: bool = True) -> Tensor:
        if self.dead:
            return m if residual else torch.zeros_like(m)
        from foldforge_amd import kernels

        return kernels.msa_pair_weighted_averaging(
            m.contiguous(), z.contiguous(), mask.contiguous(),
            ln_msa_weight=self.ln_msa.weight, ln_msa_bias=self.ln_msa.bias,
            ln_pair_weight=self.ln_pair.weight, to_bias=self.to_bias.weight,
            to_value=self.to_value.weight, to_gate=self.to_gate.weight, to_out=self.to_out.weight,
            n_head=self.n_head, residual=residual, eps_msa=self.ln_msa.eps,
            eps_pair=self.ln_pair.eps,
        )


class OuterProductMean(EngineOp, MasterWeights, nn.Module):
    """Outer product mean, the raw MSA-to-pair update (``legacy/primitives.py:40-136``,
    ``legacy/reference/attention.py:57-74``; engine factory ``modules/engine/modules.py:184-210``;
    parameters ``legacy/released.py:227-251``). The forward returns the update alone, or
    ``residual + update`` when ``residual=`` is given (the model owns the residual,
    ``graph.py:303``).

    ``l, r = mask * (LN(m) W^T + b)``; ``o[i, j] = sum_s l[s, i] (x) r[s, j]`` (left channel
    major); ``n[i, j] = sum_s mask[s, i] mask[s, j]``; divisor ``n + count_offset`` or, with
    ``count_offset=None``, ``max(n, 1)``. ``normalize_before_proj=False`` is AF3's
    ``(o W^T + b) / d``, ``True`` is ``(o / d) W^T + b``. ``groups > 1`` (Chai-1) takes the
    products within each of ``groups`` channel groups, normalises them with ``product_norm``
    and divides by nothing; ``d_hidden`` is the total width of all groups.
    """

    def __init__(self, d_msa: int, d_pair: int, d_hidden: int = 32, *,
                 normalize_before_proj: bool = True, projection_bias: bool = False,
                 groups: int = 1, product_norm_eps: float = 0.1, count_offset: float | None = None,
                 backend: str = "pytorch") -> None:
        nn.Module.__init__(self)
        if d_hidden % groups != 0:
            raise ValueError(f"d_hidden={d_hidden} is not a multiple of groups={groups}")
        if count_offset is not None and count_offset < 0:
            raise ValueError(f"count_offset={count_offset} must be >= 0 (or None for the clamp)")
        self.d_msa, self.d_pair, self.d_hidden, self.groups = d_msa, d_pair, d_hidden, groups
        self.normalize_before_proj, self.count_offset = normalize_before_proj, count_offset
        k = d_hidden // groups
        self.ln_msa = LayerNorm(d_msa)
        self.to_left = _linear(d_msa, d_hidden, bias=projection_bias)
        self.to_right = _linear(d_msa, d_hidden, bias=projection_bias)
        self.to_out = _linear(groups * k * k, d_pair, bias=True)
        if groups > 1:
            self.product_norm = LayerNorm(groups * k * k, eps=product_norm_eps)
        self._init_backend(backend)

    def _unsupported_hip(self, m: Tensor, mask: Tensor, residual: Tensor | None = None) -> str | None:
        reason = hip_reason(m, mask)
        if reason is not None:
            return reason
        if m.dtype != torch.bfloat16:
            return f"{m.dtype} MSA activations (the kernels take bf16)"
        if m.dim() != 4 or m.shape[3] != self.d_msa:
            return f"MSA shape {tuple(m.shape)} (expected [B, S, N, {self.d_msa}])"
        if mask.dtype != torch.bool or tuple(mask.shape) != tuple(m.shape[:3]):
            return f"row mask {tuple(mask.shape)} {mask.dtype} (expected bool {tuple(m.shape[:3])})"
        if min(m.shape[:3]) == 0:
            return "empty MSA"
        if residual is not None and (residual.dtype != torch.bfloat16
                                     or tuple(residual.shape) != (m.shape[0], m.shape[2], m.shape[2], self.d_pair)):
            return f"residual {tuple(residual.shape)} {residual.dtype}"
        from foldforge_amd.kernels import outer_product_mean_grouped_supported, outer_product_mean_supported

        if self.groups != 1:
            dg = self.d_hidden // self.groups
            if not outer_product_mean_grouped_supported(self.d_msa, self.groups, dg, self.d_pair):
                return (f"d_msa={self.d_msa} {self.groups} groups of {dg} d_pair={self.d_pair} (the "
                        "grouped kernels take d_msa a multiple of 64 up to 768, 8 groups of 8, "
                        "d_pair 128 or 256)")
            return None
        if not outer_product_mean_supported(self.d_msa, self.d_hidden, self.d_pair):
            return (f"d_msa={self.d_msa} d_hidden={self.d_hidden} d_pair={self.d_pair} (the kernels "
                    "take d_msa a multiple of 64 up to 768, d_hidden 32, d_pair 128)")
        return None

    def _forward_pytorch(self, m: Tensor, mask: Tensor, residual: Tensor | None = None) -> Tensor:
        if self.dead:
            return residual if residual is not None else torch.zeros(
                *m.shape[:1], m.shape[2], m.shape[2], self.d_pair, dtype=m.dtype, device=m.device)
        return torch_ops.outer_product_mean(self, m, mask, residual=residual)

    def _forward_hip(self, m: Tensor, mask: Tensor, residual: Tensor | None = None) -> Tensor:
        if self.dead:
            return self._forward_pytorch(m, mask, residual)
        from foldforge_amd import kernels

        if self.groups != 1:
            return kernels.outer_product_mean_grouped(
                m.contiguous(), mask.contiguous(), groups=self.groups, ln_weight=self.ln_msa.weight,
                ln_bias=self.ln_msa.bias, to_left=self.to_left.weight, to_right=self.to_right.weight,
                norm_weight=self.product_norm.weight, norm_bias=self.product_norm.bias,
                to_out=self.to_out.weight, to_out_bias=self.to_out.bias, left_bias=self.to_left.bias,
                right_bias=self.to_right.bias,
                residual=None if residual is None else residual.contiguous(),
                eps=self.ln_msa.eps, norm_eps=self.product_norm.eps,
            )
        return kernels.outer_product_mean(
            m.contiguous(), mask.contiguous(), ln_weight=self.ln_msa.weight,
            ln_bias=self.ln_msa.bias, to_left=self.to_left.weight, to_right=self.to_right.weight,
            to_out=self.to_out.weight, to_out_bias=self.to_out.bias, left_bias=self.to_left.bias,
            right_bias=self.to_right.bias,
            residual=None if residual is None else residual.contiguous(),
            count_offset=self.count_offset, normalize_before_proj=self.normalize_before_proj,
            eps=self.ln_msa.eps,
        )

    def delta(self, m: Tensor, mask: Tensor, residual: Tensor | None = None) -> Tensor:
        """The update alone (what the forward returns without ``residual``)."""
        return getattr(self, f"_forward_{self._route((m, mask), {})}")(m, mask)


# ------------------------------------------------------------------------------------ block

def _fused_attention_transition(att: "TriangleAttention", tr: "Transition") -> bool:
    """Whether ``att`` then ``tr`` fit the fused kernel (AF3 trunk widths, the z-frame update,
    no projection biases, neither op dead)."""
    return (not att.dead and not tr.dead and not att.untransposed_output and not att.dual_output
            and att.to_gate.bias is None and att.to_out.bias is None
            and (att.d_pair, att.n_head, att.d_hidden) == (128, 4, 128) and (tr.d, tr.n) == (128, 4))


def attention_then_transition(att: "TriangleAttention", tr: "Transition", z: Tensor, mask: Tensor,
                              fuse: bool = True) -> Tensor:
    """``tr(att(z, mask))``: a sequential block's last two pair updates
    (``legacy/pairformer.py:200-202``). Where both ops route to ``hip`` and their widths fit,
    one call runs them with the attention's output projection inside the transition kernel
    (``kernels.triangle_attention_transition``: the same results, the attention output never
    written). Each op is routed (refusal policy, ledger) exactly as its own call would be."""
    b_att = att._route((z, mask), {})
    if b_att == "hip" and fuse and _fused_attention_transition(att, tr):
        # the transition's refusal reasons (device, dtype, width) read the same on z as on the
        # attention's output, which has z's shape, dtype and device
        b_tr = tr._route((z,), {})
        if b_tr == "hip":
            from foldforge_amd import kernels

            return kernels.triangle_attention_transition(
                z.contiguous(), mask.contiguous(),
                ln_pair_weight=att.ln_pair.weight, ln_pair_bias=att.ln_pair.bias,
                to_bias=att.to_bias.weight, to_query=att.to_query.weight,
                to_key=att.to_key.weight, to_value=att.to_value.weight,
                to_gate=att.to_gate.weight, to_out=att.to_out.weight,
                ln_weight=tr.ln_in.weight, ln_bias=tr.ln_in.bias, expand_a=tr.expand_a.weight,
                expand_b=tr.expand_b.weight, squeeze=tr.squeeze.weight, starting=att.starting,
                transposed_bias=att.transposed_bias, eps_pair=att.ln_pair.eps, eps=tr.ln_in.eps,
            )
        return getattr(tr, f"_forward_{b_tr}")(att._forward_hip(z, mask))
    z = getattr(att, f"_forward_{b_att}")(z, mask)
    return tr(z)


@dataclass(frozen=True)
class PairformerConfig:
    """The engine's block configuration (``src/foldforge/modules/engine/pairformer.py:38-52``).
    ``d_hidden_tri_attention`` is the per-head width."""

    d_pair: int = 128
    d_hidden_tri_multi: int = 128
    d_hidden_tri_attention: int = 32
    n_head_tri_attention: int = 4
    p_drop: float = 0.0
    use_triangle_attention: bool = True
    model: str = "af3"
    d_single: int = 0
    n_head_single: int = 16
    single_gate_bias: float = 0.0
    pair_transition_n: int = 4
    single_transition_n: int = 4
    parallel: bool = False

    def as_dict(self) -> dict[str, Any]:
        return {f.name: getattr(self, f.name) for f in fields(self)}


class PairformerBlock(MasterWeights, nn.Module):
    """One Pairformer block: a composite that stays on ``pytorch`` itself while every child
    op carries its own backend (``src/foldforge/modules/engine/policy.py:118-121``).

    ``block(pair, key_mask)`` -> pair; ``block(pair, key_mask, single[, bias])`` ->
    ``(pair, single)`` (``src/foldforge/modules/engine/graph.py:226-233``). Order: the
    sequential AF3 schedule of ``legacy/pairformer.py:191-230`` (``parallel``: every update
    reads the block's input, ``legacy/pairformer.py:176-190``).
    """

    backends = ("pytorch",)
    #: the ending node's attention and the pair transition as one fused call where both run
    #: on ``hip`` (``attention_then_transition``; False: two calls, the same results)
    fuse_attention_transition: bool = True

    def __init__(self, config: PairformerConfig) -> None:
        super().__init__()
        self.config = config
        c = config
        self.tri_multi_outgoing = TriangleMultiplication(c.d_pair, c.d_hidden_tri_multi, outgoing=True)
        self.tri_multi_incoming = TriangleMultiplication(c.d_pair, c.d_hidden_tri_multi, outgoing=False)
        if c.use_triangle_attention:
            hidden = c.n_head_tri_attention * c.d_hidden_tri_attention
            self.tri_atten_starting = TriangleAttention(
                c.d_pair, c.n_head_tri_attention, d_hidden=hidden, starting=True, model=c.model)
            self.tri_atten_ending = TriangleAttention(
                c.d_pair, c.n_head_tri_attention, d_hidden=hidden, starting=False, model=c.model)
        self.transition_pair = Transition(c.d_pair, c.pair_transition_n)
        if c.d_single > 0:
            self.single_attention = AttentionPairBias(
                c.d_single, c.d_pair, c.n_head_single, c.single_gate_bias)
            self.single_transition = Transition(c.d_single, c.single_transition_n)
        self.backend = "pytorch"

    def children_ops(self) -> list[nn.Module]:
        return [m for m in self.children() if isinstance(m, EngineOp)]

    def set_backend(self, name: str) -> None:
        """The block itself stays ``pytorch``; each child takes ``name`` where it has it."""
        self.backend = "pytorch"
        for m in self.children_ops():
            m.set_backend(name if name in m.backends else "pytorch")

    def forward(self, pair: Tensor, key_mask: Tensor, single: Tensor | None = None,
                bias: Tensor | None = None):
        pair_out = self.pair_track(pair, key_mask)
        if single is None or self.config.d_single == 0:
            return pair_out
        return pair_out, self.single_track(single, pair, pair_out, key_mask, bias)

    def pair_track(self, pair: Tensor, key_mask: Tensor) -> Tensor:
        """The block's pair updates (``forward`` without the single track)."""
        c = self.config
        if c.parallel:
            # every pair update reads the block's input (legacy/pairformer.py:176-190)
            z0 = pair
            upd = self.tri_multi_outgoing.delta(z0, key_mask) + self.tri_multi_incoming.delta(z0, key_mask)
            if c.use_triangle_attention:
                upd = upd + self.tri_atten_starting.delta(z0, key_mask) + self.tri_atten_ending.delta(z0, key_mask)
            return z0 + upd + self.transition_pair.delta(z0)
        z = self.tri_multi_outgoing(pair, key_mask)
        z = self.tri_multi_incoming(z, key_mask)
        if c.use_triangle_attention:
            z = self.tri_atten_starting(z, key_mask)
            return attention_then_transition(self.tri_atten_ending, self.transition_pair, z,
                                             key_mask, self.fuse_attention_transition)
        return self.transition_pair(z)

    def single_track(self, single: Tensor, pair: Tensor, pair_out: Tensor, key_mask: Tensor,
                     bias: Tensor | None = None) -> Tensor:
        """The block's single updates from its pair input (parallel schedule) or output
        (sequential schedule): they read no other state, so they may run beside the next
        block's pair track."""
        c = self.config
        if c.parallel:
            return single + self.single_attention.delta(single, pair, key_mask, bias) \
                + self.single_transition.delta(single)
        s = self.single_attention(single, pair_out, key_mask, bias)
        return self.single_transition(s)


class MSABlock(MasterWeights, nn.Module):
    """One MSA-stack block composed of the op classes (the reference's engine graph builds it
    the same way, ``src/foldforge/modules/engine/graph.py:240-340``; the engine has no MSA
    block class): outer product mean -> MSA pair-weighted averaging -> MSA transition (or the
    Boltz order, ``msa_first``), then the pair track (two triangle multiplications, two
    triangle attentions when ``with_pair_attention``, the transition). Every part owns its
    residual except the outer product mean, whose raw update is added here. ``parallel`` is
    Chai-1's block (every update of a stage reads the stage's input, ``graph.py:316-340``).

    ``block(msa [M, L, c_m], pair [L, L, c_z], msa_mask [M, L], pair_mask [L, L])`` ->
    ``(msa, pair)``: unbatched, like the reference's block; MSA rows are real where
    ``msa_mask > 0``, a token column is a key when any row has it, and the token mask is the
    pair mask's diagonal.
    """

    backends = ("pytorch",)

    def __init__(self, c_msa: int, c_pair: int, n_heads_pair: int = 4, *,
                 msa_value_dim: int | None = None, with_pair_attention: bool = True,
                 triangle_model: str = "af3", msa_first: bool = False, parallel: bool = False,
                 opm_channel: int = 32, opm_groups: int = 1, opm_projection_bias: bool = False,
                 opm_normalize_before_proj: bool = False,
                 opm_count_offset: float | None = 1e-3) -> None:
        super().__init__()
        if parallel and msa_first:
            raise ValueError("a parallel MSA block runs the outer product mean first")
        self.msa_first, self.parallel, self.with_pair_attention = msa_first, parallel, with_pair_attention
        self.outer_product_mean = OuterProductMean(
            c_msa, c_pair, opm_channel * opm_groups, groups=opm_groups,
            projection_bias=opm_projection_bias, normalize_before_proj=opm_normalize_before_proj,
            count_offset=None if opm_groups > 1 else opm_count_offset)
        self.msa_attention1 = MSAPairWeightedAveraging(c_msa, c_pair, 8, msa_value_dim)
        self.msa_transition = Transition(c_msa, 4)
        self.triangle_multiplication_outgoing = TriangleMultiplication(c_pair, outgoing=True)
        self.triangle_multiplication_incoming = TriangleMultiplication(c_pair, outgoing=False)
        if with_pair_attention:
            self.pair_attention1 = TriangleAttention(c_pair, n_heads_pair, starting=True, model=triangle_model)
            self.pair_attention2 = TriangleAttention(c_pair, n_heads_pair, starting=False, model=triangle_model)
        self.pair_transition = Transition(c_pair, 4)
        self.backend = "pytorch"

    def children_ops(self) -> list[nn.Module]:
        return [m for m in self.children() if isinstance(m, EngineOp)]

    def set_backend(self, name: str) -> None:
        self.backend = "pytorch"
        for m in self.children_ops():
            m.set_backend(name if name in m.backends else "pytorch")

    # after the outer product mean the MSA track and the pair track read only the stage's MSA
    # and pair: on the GPU the MSA track runs on a second stream beside the pair track (the
    # same ops on the same inputs, so the same results bit for bit)
    overlap_tracks: bool = True
    #: the ending node's attention and the pair transition as one fused call where both run
    #: on ``hip`` (``attention_then_transition``; False: two calls, the same results)
    fuse_attention_transition: bool = True

    def forward(self, msa: Tensor, pair: Tensor, msa_mask: Tensor, pair_mask: Tensor):
        m, z = msa[None], pair[None]
        rows = (msa_mask > 0)[None].contiguous()
        columns = (msa_mask.max(dim=0).values > 0)[None].contiguous()
        tokens = (pair_mask.diagonal(dim1=-2, dim2=-1) > 0)[None].contiguous()
        if self.msa_first:
            m = self.msa_transition(self.msa_attention1(m, z, columns))
        z = self.outer_product_mean(m, rows, residual=z)

        def msa_track() -> Tensor:
            if self.parallel:
                return m + self.msa_attention1.delta(m, z, columns) + self.msa_transition.delta(m)
            if self.msa_first:
                return m
            return self.msa_transition(self.msa_attention1(m, z, columns))

        side = None
        if self.overlap_tracks and z.is_cuda and not self.msa_first:
            from foldforge_amd.trunk import _side_stream

            main, side = torch.cuda.current_stream(z.device), _side_stream(z.device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                m_out = msa_track()
            for t in (m, z, columns):  # read on the side stream after the main one moves on
                t.record_stream(side)
        else:
            m_out = msa_track()
        z = self.pair_track(z, tokens)
        if side is not None:
            main.wait_stream(side)
            m_out.record_stream(main)
        return m_out[0], z[0]

    def pair_track(self, z: Tensor, tokens: Tensor) -> Tensor:
        """The block's pair updates after the outer product mean."""
        if self.parallel:
            z = z + (self.triangle_multiplication_outgoing.delta(z, tokens)
                     + self.triangle_multiplication_incoming.delta(z, tokens)
                     + self.pair_transition.delta(z))
            if self.with_pair_attention:
                z = z + self.pair_attention1.delta(z, tokens) + self.pair_attention2.delta(z, tokens)
            return z
        z = self.triangle_multiplication_outgoing(z, tokens)
        z = self.triangle_multiplication_incoming(z, tokens)
        if self.with_pair_attention:
            z = self.pair_attention1(z, tokens)
            return attention_then_transition(self.pair_attention2, self.pair_transition, z, tokens,
                                             self.fuse_attention_transition)
        return self.pair_transition(z)

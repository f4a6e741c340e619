"""Which backend runs each op module, and what happens to a call the backend refuses.

An op module (:mod:`foldforge_amd.modules`) carries a backend name and answers
``unsupported(*args)`` before every call. This module holds the table the rest of the
library reads -- the engine's op names, the classes behind each, the backend names a
configuration may request -- and three steps built on it:

* :func:`pick` turns a requested name into the backend one class runs on a device, with the
  reason whenever the answer differs from the request;
* :class:`Plan` is one model's request (a default, per-op overrides, a refusal policy);
  :meth:`Plan.resolve` says what each op of the table gets on a device;
* :func:`install` hands every op module of a model its backend and its refusal policy.

The refusal itself runs inside the op module (``EngineOp.forward``, via :func:`on_refusal`):
without an installed policy the module raises the engine's ``BackendUnsupported``; under
``"error"`` it raises :class:`BackendUnsupportedError`; under ``"fallback"`` the call runs the
``pytorch`` backend and the reason is logged once per (class, backend, reason). Each module
counts its calls in a :class:`CallLedger` (:func:`ledger_report`): host calls, not a kernel
trace, and graph replays are not seen.

Kept from the reference because configurations and callers name them
(``src/foldforge/modules/engine/backends.py:35-70``, ``policy.py:43-60``): the op names of
``engine.ops`` with their class names, the backend and alias names, the policy names
``fallback`` / ``error`` and the error class name ``BackendUnsupportedError``. FoldForge's own
policy can drive these modules unchanged through the engine contract (``backends``,
``set_backend``, ``unsupported``, ``_forward_<backend>``).
"""

from __future__ import annotations

import logging
from collections import Counter
from collections.abc import Iterator, Mapping
from dataclasses import dataclass, field
from typing import Any, NamedTuple

import torch
from torch import nn

log = logging.getLogger("foldforge.backend")

#: The device architecture the ``hip`` code objects are built for.
KERNEL_ARCH = "gfx950"
#: Backend names of the engine: the reference's five and this library's ``hip``.
BACKEND_NAMES = ("pytorch", "hip", "cuda", "triton", "anthropic", "cueq")
#: Family names a configuration may request; ``None`` means "the engine's own kernels",
#: decided per class and device by :func:`pick`.
ALIASES: dict[str, str | None] = {"miniworld": None, "cuequivariance": "cueq"}
REQUESTABLE = (*ALIASES, *BACKEND_NAMES)
REFUSAL_POLICIES = ("fallback", "error")

#: ``engine.ops`` name -> the op classes that carry it. Names without a class in
#: :mod:`foldforge_amd.modules` (the diffusion and sampler ops) still validate in a
#: configuration; nothing of theirs is served here.
OP_TABLE: dict[str, tuple[str, ...]] = {
    "trimul": ("TriangleMultiplication", "TriangleMultiplicationRF3", "BidirectionalTriangleMultiplication"),
    "triangle_attention": (
        "TriangleAttention", "TriangleAttentionAF3", "TriangleAttentionOpenFold",
        "TriangleAttentionRF3", "TriangleAttentionChai1", "TriangleAttentionChai1Confidence",
    ),
    "opm": ("OuterProductMean",),
    "msa_pwa": ("MSAPairWeightedAveraging",),
    "single_attention": ("AttentionPairBias",),
    "transition": ("Transition",),
    "layernorm": ("LayerNorm",),
    "conditioning": ("ConditionedTransition", "AdaptiveLayerNorm", "IdentityAdaptiveLayerNorm", "AdaptiveRMSNorm"),
    "dit_blocks": ("TokenDiTProtenix", "TokenDiTMiniWorldBiasOnly"),
    "atom_blocks": (
        "AtomDiTProtenix", "AtomDiTOpenFold3", "AtomDiTBoltz2", "AtomDiTRoseTTAFold3",
        "AtomDiTChai1", "AtomDiTMiniWorld", "AtomDiTESMFold2Pair",
    ),
    "sampler_ops": ("AugmentNoise", "AlignEuler", "PoolAtoms"),
}
OP_NAMES = tuple(OP_TABLE)


class BackendUnsupportedError(RuntimeError):
    """A refused call, or an op no class serves, under the refusal policy ``"error"``."""


# ------------------------------------------------------------------------------- the table
def classes_of(op: str) -> tuple[type, ...]:
    """The classes of ``op`` that exist in :mod:`foldforge_amd.modules`."""
    from foldforge_amd import modules

    return tuple(c for c in (getattr(modules, name, None) for name in OP_TABLE[op]) if c is not None)


def op_name(obj: object) -> str | None:
    """The op a module instance or class carries (None for composites and plain modules)."""
    cls = obj if isinstance(obj, type) else type(obj)
    for op in OP_NAMES:
        if any(issubclass(cls, c) for c in classes_of(op)):
            return op
    return None


def offered(op: str) -> tuple[str, ...]:
    """The requestable names that reach a backend some class of ``op`` has."""
    have: set[str] = set()
    for cls in classes_of(op):
        have.update(cls.backends)
    names = [n for n in REQUESTABLE if ALIASES.get(n, n) in have]
    if "hip" in have:
        names.insert(0, "miniworld")
    return tuple(dict.fromkeys(names))


def __getattr__(name: str) -> object:
    if name == "SERVES":  # computed on access: the classes register lazily
        return {op: offered(op) for op in OP_NAMES}
    raise AttributeError(name)


def device_arch(device: object | None) -> str | None:
    """The gfx architecture of a ROCm device (``"gfx950"``); None without one."""
    if not torch.cuda.is_available():
        return None
    dev = torch.device("cuda") if device is None else torch.device(device)  # type: ignore[arg-type]
    if dev.type != "cuda":
        return None
    return torch.cuda.get_device_properties(dev.index or 0).gcnArchName.split(":")[0]


class Pick(NamedTuple):
    """The backend a class runs on, and why it is not the requested one (None: it is)."""

    backend: str
    reason: str | None = None


def pick(requested: str, cls: type, arch: str | None) -> Pick:
    """The backend ``cls`` runs on a device of architecture ``arch`` when ``requested`` is asked."""
    if requested not in REQUESTABLE:
        raise ValueError(f"Unknown backend: {requested}")
    target = ALIASES.get(requested, requested)
    has = tuple(cls.backends)
    native = arch == KERNEL_ARCH
    if target is None:  # the engine's own kernels, where this class and device have them
        return Pick("hip" if native and "hip" in has else "pytorch")
    if target == "pytorch":
        return Pick("pytorch")
    if target not in has:
        return Pick("pytorch", f"{cls.__name__} has no {target!r} backend (it has {', '.join(has)})")
    if target == "hip" and not native:
        return Pick("pytorch", f"the hip backend runs on {KERNEL_ARCH} (MI355X) devices only, this is {arch}")
    return Pick(target)


def check_ops(ops: Mapping[str, str]) -> dict[str, str]:
    """Validate an ``engine.ops`` mapping: known op names, requestable backends."""
    stray = sorted(k for k in ops if k not in OP_TABLE)
    if stray:
        raise ValueError(f"engine.ops names unknown op(s) {stray}; known: {list(OP_NAMES)}")
    wrong = {k: v for k, v in ops.items() if v not in REQUESTABLE}
    if wrong:
        raise ValueError(f"engine.ops names unknown backend(s) {wrong}; known: {list(REQUESTABLE)}")
    return dict(ops)


# -------------------------------------------------------------------------------- the plan
@dataclass(frozen=True)
class Plan:
    """One model's backend request: ``default`` for every op, ``overrides`` per op name, and
    the policy for calls a backend refuses."""

    default: str = "miniworld"
    overrides: tuple[tuple[str, str], ...] = ()
    refusal: str = "fallback"

    @classmethod
    def of(cls, backend: str = "miniworld", ops: Mapping[str, str] | None = None,
           unsupported: str = "fallback") -> Plan:
        if backend not in REQUESTABLE:
            raise ValueError(f"Unknown backend: {backend}")
        if unsupported not in REFUSAL_POLICIES:
            raise ValueError(f"engine.unsupported must be one of {REFUSAL_POLICIES}, got {unsupported!r}")
        return cls(backend, tuple(sorted(check_ops(ops or {}).items())), unsupported)

    def requested(self, op: str) -> str:
        for name, backend in self.overrides:
            if name == op:
                return backend
        return self.default

    def pick_for(self, cls: type, arch: str | None) -> Pick:
        op = op_name(cls)
        if op is None:
            raise TypeError(f"{cls.__name__} carries no op of the table")
        return pick(self.requested(op), cls, arch)

    def resolve(self, arch: str | None) -> dict[str, Pick]:
        """What each op with a class here resolves to on ``arch``: the first class that takes
        the request, else the first class's reason. Ops nobody serves are logged once, or
        raise under the policy ``"error"``."""
        out: dict[str, Pick] = {}
        for op in OP_NAMES:
            picks = [pick(self.requested(op), c, arch) for c in classes_of(op)]
            if picks:
                out[op] = next((p for p in picks if p.reason is None), picks[0])
        lost = {op: p.reason for op, p in out.items() if p.reason is not None}
        if lost:
            text = "; ".join(f"{op} ({self.requested(op)}): {why}" for op, why in lost.items())
            if self.refusal == "error":
                raise BackendUnsupportedError(f"no class serves the requested backend (engine.unsupported: error): {text}")
            log.warning("plan %s: ops run on the pytorch backend instead: %s", self.default, text)
        return out

    def summary(self, picks: Mapping[str, Pick]) -> dict[str, object]:
        return {
            "backend": self.default,
            "requested": {op: self.requested(op) for op in picks},
            "ops": {op: p.backend for op, p in picks.items()},
            "fallbacks": {op: p.reason for op, p in picks.items() if p.reason is not None},
            "unsupported": self.refusal,
        }


def op_modules(model: nn.Module, prefix: str = "") -> Iterator[tuple[str, nn.Module]]:
    """Every op module of ``model`` (a composite's op children included, ops not descended)."""
    if op_name(model) is not None:
        yield prefix, model
        return
    for name, child in model.named_children():
        yield from op_modules(child, f"{prefix}.{name}" if prefix else name)


def install(model: nn.Module, plan: Plan, device: object | None = None) -> dict[str, dict[str, Any]]:
    """Give every op module of ``model`` its backend under ``plan`` on ``device`` and the plan's
    refusal policy. Composites keep ``pytorch`` (they only call their children). Returns,
    per module name, its op, the requested and chosen backend, and the reason they differ."""
    arch = device_arch(device)
    placed: dict[str, dict[str, Any]] = {}
    for name, module in op_modules(model):
        op = op_name(module)
        chosen = plan.pick_for(type(module), arch)
        if chosen.reason is not None and plan.refusal == "error":
            raise BackendUnsupportedError(f"{name or type(module).__name__}: {chosen.reason}")
        module.set_backend(chosen.backend)  # type: ignore[operator]
        module.refusal_policy = plan.refusal
        placed[name] = {"op": op, "requested": plan.requested(str(op)), "backend": chosen.backend,
                        "reason": chosen.reason}
    moved = sorted((n, p) for n, p in placed.items() if p["reason"] is not None)
    if moved:
        head = "; ".join(f"{n}: {p['reason']}" for n, p in moved[:6])
        log.warning("%d op module(s) run on pytorch instead of %s: %s%s", len(moved), plan.default,
                    head, " ..." if len(moved) > 6 else "")
    return placed


# ----------------------------------------------------------------------- refusals and ledger
@dataclass
class CallLedger:
    """Host calls of one op module: by the backend that ran them, and refusals by reason."""

    served: Counter[str] = field(default_factory=Counter)
    refused: Counter[str] = field(default_factory=Counter)


_LEDGER = "_call_ledger"
_ANNOUNCED: set[tuple[str, str, str]] = set()


def ledger_of(module: nn.Module) -> CallLedger:
    book = module.__dict__.get(_LEDGER)
    if book is None:
        book = CallLedger()
        module.__dict__[_LEDGER] = book
    return book


def note_call(module: nn.Module, backend: str) -> None:
    if not torch.compiler.is_compiling():
        ledger_of(module).served[backend] += 1


def on_refusal(module: nn.Module, reason: str, engine_error: type[Exception]) -> str:
    """The backend a refused call runs on, under the module's refusal policy (or raise)."""
    policy = getattr(module, "refusal_policy", None)
    cls, backend = type(module).__name__, str(getattr(module, "backend", "?"))
    if policy is None:
        raise engine_error(f"{cls} backend {backend!r}: {reason}")
    if policy == "error":
        raise BackendUnsupportedError(f"{cls} backend {backend!r} refused a call (engine.unsupported: error): {reason}")
    if not torch.compiler.is_compiling():
        ledger_of(module).refused[reason] += 1
    key = (cls, backend, reason)
    if key not in _ANNOUNCED:
        _ANNOUNCED.add(key)
        log.warning("%s: the %s backend refused a call (%s); it ran on pytorch", cls, backend, reason)
    return "pytorch"


def set_refusal(model: nn.Module, policy: str | None) -> nn.Module:
    """Give every op module of ``model`` the refusal ``policy`` (``None``: the engine's raise)."""
    if policy is not None and policy not in REFUSAL_POLICIES:
        raise ValueError(f"refusal policy must be one of {REFUSAL_POLICIES} or None, got {policy!r}")
    for _, module in op_modules(model):
        module.refusal_policy = policy
    return model


def forget_announcements() -> None:
    """Let every refusal be logged again."""
    _ANNOUNCED.clear()


def ledger_report(model: nn.Module) -> dict[str, dict[str, Any]]:
    """Per op module of ``model``: class, current backend, host calls served per backend and
    refusals per reason."""
    report: dict[str, dict[str, Any]] = {}
    for name, module in op_modules(model):
        book = module.__dict__.get(_LEDGER) or CallLedger()
        report[name or "<root>"] = {"class": type(module).__name__, "backend": module.backend,
                                    "served": dict(book.served), "refused": dict(book.refused)}
    return report


def clear_ledgers(model: nn.Module) -> None:
    for module in model.modules():
        module.__dict__.pop(_LEDGER, None)


def served_count(model: nn.Module, backend: str) -> int:
    """Host calls ``backend`` ran, summed over every op module of ``model``."""
    return sum(entry["served"].get(backend, 0) for entry in ledger_report(model).values())

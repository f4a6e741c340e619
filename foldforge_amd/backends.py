"""Which backend serves which op: the table behind ``backend``, ``engine.ops`` and ``engine.unsupported``.

Mirrors ``src/foldforge/modules/engine/backends.py`` of the reference with this build's
engine: the op classes of :mod:`foldforge_amd.modules` list ``pytorch`` (the reference)
and ``hip`` (the gfx950 kernels). The reference's backend names stay valid so that an
existing configuration validates; a class that lacks a named backend is refused with a
reason (the guard then runs ``pytorch``). The ``miniworld`` alias means "the engine's own
kernels": ``hip`` on a gfx950 device where the class has it, else ``pytorch``
(``backends.py:137-165`` of the reference, with ``hip`` where it chose ``cuda``).
"""

from __future__ import annotations

import logging
from collections.abc import Mapping
from dataclasses import dataclass, field

logger = logging.getLogger("foldforge.backend")

#: The engine's backend names (the reference's five plus ``hip``).
ENGINE_BACKENDS = ("pytorch", "hip", "cuda", "triton", "anthropic", "cueq")
#: Policy aliases -> what they mean; ``None``: decided per class by :func:`choose_backend`.
ALIASES: dict[str, str | None] = {"miniworld": None, "cuequivariance": "cueq"}
BACKENDS = ("miniworld", "cuequivariance", *ENGINE_BACKENDS)
#: The device architecture the ``hip`` kernels are built for.
HIP_ARCH = "gfx950"

#: op -> the class names (in :mod:`foldforge_amd.modules`) that carry it; the keys are the
#: names ``engine.ops`` takes (``backends.py:35-70`` of the reference). Ops outside the
#: pair stack keep their names (a configuration naming them validates) but have no
#: class in this build.
OP_CLASSES: dict[str, tuple[str, ...]] = {
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
OPS = tuple(OP_CLASSES)
UNSUPPORTED = ("fallback", "error")


class BackendUnsupportedError(RuntimeError):
    """A (backend, module) combination the engine does not serve, with ``engine.unsupported: error``."""


def op_classes(op: str) -> tuple[type, ...]:
    """The classes of ``op`` that exist in this build."""
    from foldforge_amd import modules

    return tuple(getattr(modules, name) for name in OP_CLASSES[op] if hasattr(modules, name))


def op_of(module: object) -> str | None:
    """The op an op-module instance carries, or None."""
    for op in OPS:
        classes = op_classes(op)
        if classes and isinstance(module, classes):
            return op
    return None


def serves(op: str) -> tuple[str, ...]:
    """The backends some class of ``op`` has, in the policy's names."""
    have = {b for cls in op_classes(op) for b in cls.backends}
    named = [b for b in ENGINE_BACKENDS if b in have]
    return (*(["miniworld"] if "hip" in have else []), *named,
            *(["cuequivariance"] if "cueq" in have else []))


def __getattr__(name: str) -> object:
    if name == "SERVES":
        return {op: serves(op) for op in OPS}
    raise AttributeError(name)


def validate_ops(ops: Mapping[str, str]) -> dict[str, str]:
    """``engine.ops``: known op names, known backends."""
    unknown = sorted(set(ops) - set(OPS))
    if unknown:
        raise ValueError(f"engine.ops names unknown op(s) {unknown}; known: {list(OPS)}")
    bad = {op: b for op, b in ops.items() if b not in BACKENDS}
    if bad:
        raise ValueError(f"engine.ops names unknown backend(s) {bad}; known: {list(BACKENDS)}")
    return dict(ops)


def capability(device: object | None) -> str | None:
    """The gfx architecture of a ROCm ``device`` (``"gfx950"``), None without one."""
    import torch

    if not torch.cuda.is_available() or getattr(device, "type", "cuda") != "cuda":
        return None
    index = getattr(device, "index", None)
    return torch.cuda.get_device_properties(index if index is not None else 0).gcnArchName.split(":")[0]


def choose_backend(requested: str, cls: type, device: object | None = None) -> tuple[str, str | None]:
    """``(backend, reason)`` of one class under ``requested``; ``reason`` says why it differs."""
    name = ALIASES.get(requested, requested)
    have = tuple(cls.backends)
    arch = capability(device)
    if name is None:
        if "hip" in have and arch == HIP_ARCH:
            return "hip", None
        return "pytorch", None
    if name == "pytorch":
        return "pytorch", None
    if name not in have:
        return "pytorch", f"{cls.__name__} has no {name!r} backend (available: {', '.join(have)})"
    if name == "hip" and arch != HIP_ARCH:
        return "pytorch", f"the hip backend needs a {HIP_ARCH} (MI355X) device (found {arch})"
    return name, None


@dataclass(frozen=True)
class Resolved:
    op: str
    requested: str
    backend: str
    reason: str | None = None


@dataclass(frozen=True)
class BackendPlan:
    """The backend of every op for one loaded model."""

    backend: str = "miniworld"
    ops: tuple[tuple[str, str], ...] = ()
    unsupported: str = "fallback"
    resolved: dict[str, Resolved] = field(default_factory=dict, compare=False, hash=False)

    @classmethod
    def make(cls, backend: str = "miniworld", ops: Mapping[str, str] | None = None,
             unsupported: str = "fallback") -> BackendPlan:
        if backend not in BACKENDS:
            raise ValueError(f"Unknown backend: {backend}")
        if unsupported not in UNSUPPORTED:
            raise ValueError(f"engine.unsupported must be one of {UNSUPPORTED}, got {unsupported!r}")
        return cls(backend, tuple(sorted(validate_ops(ops or {}).items())), unsupported)

    def requested(self, op: str) -> str:
        return dict(self.ops).get(op, self.backend)

    def of(self, op: str) -> str:
        resolved = self.resolved.get(op)
        return resolved.backend if resolved is not None else self.requested(op)

    def for_class(self, cls: type, device: object | None = None) -> tuple[str, str | None]:
        op = next(op for op in OPS if op_classes(op) and issubclass(cls, op_classes(op)))
        return choose_backend(self.requested(op), cls, device)

    def resolve(self, device: object | None = None) -> BackendPlan:
        """Check every op that has classes here against the machine; one log line for refusals."""
        self.resolved.clear()
        for op in OPS:
            classes = op_classes(op)
            if not classes:
                continue
            asked = self.requested(op)
            choices = [choose_backend(asked, cls, device) for cls in classes]
            ok = [name for name, reason in choices if reason is None]
            if ok:
                self.resolved[op] = Resolved(op, asked, ok[0])
            else:
                self.resolved[op] = Resolved(op, asked, "pytorch", choices[0][1])
        missing = [r for r in self.resolved.values() if r.reason is not None]
        if missing and self.unsupported == "error":
            lines = "; ".join(f"{r.op} on {r.requested}: {r.reason}" for r in missing)
            raise BackendUnsupportedError(
                f"backend ops no engine class serves (engine.unsupported: error): {lines}")
        if missing:
            lines = "; ".join(f"{r.op} ({r.requested}: {r.reason})" for r in missing)
            logger.warning("backend %s: running the engine pytorch backend for %s", self.backend, lines)
        return self

    def report(self) -> dict[str, object]:
        return {
            "backend": self.backend,
            "ops": {op: r.backend for op, r in self.resolved.items()},
            "fallbacks": {op: f"{r.requested}: {r.reason}" for op, r in self.resolved.items()
                          if r.reason is not None},
            "unsupported": self.unsupported,
        }

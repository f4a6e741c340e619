"""Host-side observations of the op modules: which backend each call ran on and which
calls were refused (``src/foldforge/modules/engine/serving.py`` of the reference).

The guard counts calls per module; graph replays and compiled regions are not counted.
These are host-call counters, not a kernel trace.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field
from typing import Any

import torch

_STATS_ATTR = "_foldforge_observations"


@dataclass
class Observations:
    served: Counter[str] = field(default_factory=Counter)
    refused: Counter[str] = field(default_factory=Counter)


def observations_of(module: torch.nn.Module) -> Observations:
    stats = module.__dict__.get(_STATS_ATTR)
    if stats is None:
        stats = Observations()
        object.__setattr__(module, _STATS_ATTR, stats)
    return stats


def observe_call(module: torch.nn.Module, backend: str, refusal: str | None,
                 served_by: str = "pytorch") -> None:
    if torch.compiler.is_compiling():
        return
    stats = observations_of(module)
    if refusal is None:
        stats.served[backend] += 1
    else:
        stats.refused[refusal] += 1
        stats.served[served_by] += 1


def reset_observations(model: torch.nn.Module) -> None:
    for module in model.modules():
        module.__dict__.pop(_STATS_ATTR, None)


def report_observations(model: torch.nn.Module) -> dict[str, Any]:
    modules = {}
    for name, module in model.named_modules():
        stats = module.__dict__.get(_STATS_ATTR)
        if stats is None and not getattr(module, "_foldforge_guarded", False):
            continue
        modules[name or "<root>"] = {
            "class": type(module).__name__,
            "backend": getattr(module, "backend", None),
            "host_observed": stats is not None,
            "served_host_calls": {} if stats is None else dict(stats.served),
            "refused_host_calls": {} if stats is None else dict(stats.refused),
        }
    return {
        "coverage": "engine_modules_with_a_backend_guard",
        "counting": "host_calls_including_capture; excludes_compiled_regions_and_graph_replays",
        "selections_are_kernel_traces": False,
        "modules": modules,
    }

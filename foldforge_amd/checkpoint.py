"""The miniworld checkpoint format for this build's modules: an fp32 ``state_dict`` in engine
keys plus a format tag, written with ``torch.save`` and read with ``weights_only=True``.

The format of the reference (``src/foldforge/models/checkpoints/miniworld.py:1-25``)::

    {"format": "miniworld", "version": 1, "family": "alphafold3",
     "source": "<released blob name>", "state_dict": {engine key: fp32 tensor}}

* :func:`read` checks the tag and version; :func:`load_into` is a strict
  ``load_state_dict`` (no translation at load time). A whole-model file keeps the trunk
  blocks under ``evoformer.trunk_pairformer.<i>`` and the MSA-stack blocks under
  ``evoformer.msa_stack.<i>`` (``src/foldforge/models/architectures/af3.py:245``);
  :func:`submodule_state` cuts such a prefix out, so those blocks load into a
  :class:`foldforge_amd.trunk.PairformerTrunk` or a list of :class:`MSABlock`.
* :func:`convert_state` is the offline conversion of a released-layout state dict into the
  engine keys of a model built from this build's classes, with the reference's exactness
  rules (``miniworld.py:288-357``): every released key under a converted block is read by
  its conversion or is a known discard, every other key is a key of the model, and the
  result has exactly the model's keys and shapes.
"""

from __future__ import annotations

from collections.abc import Mapping
from pathlib import Path
from typing import Any

import torch
from torch import nn

from foldforge_amd import released
from foldforge_amd.modules import MSABlock, PairformerBlock

Tensor = torch.Tensor

FORMAT = "miniworld"
VERSION = 1
SUFFIX = ".miniworld.pt"
TRUNK_PREFIX = "evoformer.trunk_pairformer"
MSA_STACK_PREFIX = "evoformer.msa_stack"

ConversionError = released.ConversionError


def is_native(path: Path) -> bool:
    return Path(path).name.endswith(SUFFIX)


def read(path: Path | str) -> dict[str, Any]:
    """The checked contents of a miniworld-format file (``weights_only`` load)."""
    blob = torch.load(path, map_location="cpu", weights_only=True)
    tag = blob.get("format") if isinstance(blob, dict) else None
    if tag != FORMAT:
        raise ValueError(f"{path} is not a miniworld-format checkpoint (format tag {tag!r})")
    if blob.get("version") != VERSION:
        raise ValueError(f"{path} is miniworld format version {blob.get('version')}; this code "
                         f"reads version {VERSION}")
    if not isinstance(blob.get("state_dict"), dict):
        raise ValueError(f"{path} has no state_dict")
    return blob


def write(path: Path | str, state: Mapping[str, Tensor], *, family: str, source: str) -> Path:
    """Write ``state`` (made fp32 and contiguous) as a miniworld-format file, atomically."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(path.name + ".part")
    torch.save({"format": FORMAT, "version": VERSION, "family": family, "source": source,
                "state_dict": {k: v.detach().to(torch.float32).contiguous().clone()
                               for k, v in state.items()}}, tmp)
    tmp.replace(path)
    return path


def submodule_state(state: Mapping[str, Tensor], prefix: str, *,
                    renumber_as: str | None = None) -> dict[str, Tensor]:
    """The entries of ``state`` below ``prefix.``, prefix removed; ``renumber_as="blocks"``
    turns ``<i>.<key>`` into ``blocks.<i>.<key>`` (a :class:`PairformerTrunk`'s keys)."""
    head = prefix + "."
    out = {k[len(head):]: v for k, v in state.items() if k.startswith(head)}
    if renumber_as:
        out = {f"{renumber_as}.{k}": v for k, v in out.items()}
    return out


def load_into(model: nn.Module, source: Path | str | Mapping[str, Any], *, family: str,
              prefix: str | None = None, renumber_as: str | None = None) -> dict[str, Any]:
    """Strict load of a miniworld file (or its already-read contents) into ``model``;
    ``prefix`` selects a sub-tree of a whole-model file. Parameters keep their dtypes."""
    blob = read(source) if not isinstance(source, Mapping) else dict(source)
    if blob.get("family") != family:
        raise ValueError(f"the checkpoint holds family {blob.get('family')!r}, the model is {family!r}")
    state = dict(blob["state_dict"])
    if prefix is not None:
        state = submodule_state(state, prefix, renumber_as=renumber_as)
    released.load(model, state)
    return {"format": FORMAT, "format_version": VERSION, "source": blob.get("source"),
            "mapped_records": len(state)}


def _converters(model: nn.Module) -> list[tuple[str, Any]]:
    """``(prefix, convert)`` of the outermost convertible blocks of ``model``."""
    found: list[tuple[str, Any]] = []
    for name, module in model.named_modules():
        if not name or any(name.startswith(p + ".") for p, _ in found):
            continue
        if isinstance(module, PairformerBlock):
            found.append((name, released.pairformer_block_from_released))
        elif isinstance(module, MSABlock):
            found.append((name, released.msa_block_from_released))
    return found


def convert_state(released_state: Mapping[str, Tensor], model: nn.Module) -> dict[str, Tensor]:
    """Convert a released-layout state dict to ``model``'s engine keys (fp32 copies)."""
    tracked = released.Tracked(released_state)
    out: dict[str, Tensor] = {}
    prefixes = []
    for prefix, convert in _converters(model):
        for key, value in convert(tracked, prefix=prefix).items():
            out[f"{prefix}.{key}"] = value
        prefixes.append(prefix)

    def converted(key: str) -> bool:
        return any(key.startswith(p + ".") for p in prefixes)

    unread = sorted(k for k in released_state
                    if converted(k) and k not in tracked.used and not released.is_discarded(k))
    if unread:
        raise ConversionError(f"released keys neither read by a conversion nor a known discard: "
                              f"{unread[:8]}{' ...' if len(unread) > 8 else ''}")
    target = model.state_dict()
    for key, value in released_state.items():
        if converted(key):
            continue
        if key not in target:
            raise ConversionError(f"released key {key!r} is not a parameter of the model and no "
                                  "conversion covers it")
        out[key] = value
    missing = sorted(set(target) - set(out))
    extra = sorted(set(out) - set(target))
    wrong = sorted(k for k in set(out) & set(target) if tuple(out[k].shape) != tuple(target[k].shape))
    if missing or extra or wrong:
        raise ConversionError(f"conversion does not match the model: missing={missing[:6]}, "
                              f"extra={extra[:6]}, mis-shaped={wrong[:6]}")
    return {k: v.detach().to(torch.float32).contiguous().clone() for k, v in out.items()}

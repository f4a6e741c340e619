"""foldforge_amd: MI355X-native (gfx950) kernels for the Pairformer pair stack behind the
FoldForge engine-op contract.

``foldforge_amd.load(...)`` builds a trunk of engine-compatible blocks and applies a backend
plan (``miniworld`` = the native ``hip`` kernels on a gfx950, ``pytorch`` = the reference
equations in torch ops), the counterpart of ``foldforge.load(..., backend=...)``
(``src/foldforge/models/__init__.py:134-148`` of the reference).
"""

from __future__ import annotations

__version__ = "0.1.0"


def load(name: str = "pairformer-trunk", checkpoint=None, *, backend: str = "miniworld",
         dtype=None, device="cuda", blocks: int = 48, seed: int = 0, d_single: int = 384,
         engine_ops=None, unsupported: str = "fallback", out_scale: float | None = 0.25,
         family: str = "alphafold3"):
    """A configured trunk on ``device`` with ``backend`` applied to every op module.

    ``checkpoint``: a miniworld-format file (``*.miniworld.pt`` of ``family``; a whole-model
    file contributes its ``evoformer.trunk_pairformer.<i>`` blocks), a ``.safetensors`` file or
    a weights-only torch state dict in the trunk's keys
    (``blocks.<i>.tri_multi_outgoing.to_left.weight`` ...); without one the parameters are
    seeded random init (:func:`foldforge_amd.trunk.randomise`).
    """
    import torch

    from foldforge_amd import dispatch
    from foldforge_amd.adapter import place
    from foldforge_amd.trunk import PairformerTrunk, randomise

    if name != "pairformer-trunk":
        raise ValueError(f"unknown model {name!r}; this build serves 'pairformer-trunk'")
    dtype = torch.bfloat16 if dtype is None else dtype
    plan = dispatch.Plan.of(backend, engine_ops, unsupported)
    model = PairformerTrunk(blocks, d_single=d_single)
    if checkpoint is None:
        randomise(model, seed, out_scale=out_scale)
    else:
        path = str(checkpoint)
        if path.endswith(".miniworld.pt"):
            from foldforge_amd import checkpoint as ckpt

            blob = ckpt.read(path)
            whole = any(k.startswith(ckpt.TRUNK_PREFIX + ".") for k in blob["state_dict"])
            ckpt.load_into(model, blob, family=family,
                           prefix=ckpt.TRUNK_PREFIX if whole else None,
                           renumber_as="blocks" if whole else None)
            state = None
        elif path.endswith(".safetensors"):
            from safetensors.torch import load_file

            state = load_file(path)
        else:
            state = torch.load(path, map_location="cpu", weights_only=True)
        if state is not None:
            model.load_state_dict(state, strict=True)
    device = torch.device(device)
    place(model, dtype, device)
    picks = plan.resolve(dispatch.device_arch(device))
    model.foldforge_load_report = {"engine_backends": {"plan": plan.summary(picks),
                                                       "modules": dispatch.install(model, plan, device)}}
    return model

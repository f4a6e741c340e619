"""Helpers that make a GPU parity test prove the ``hip`` kernels served the call.

Each helper asks the module whether its backend takes the call, runs it, and checks that the
module's call ledger counted exactly one more ``hip`` call. A refused call therefore fails the
test instead of comparing another backend with the oracle.
"""

from __future__ import annotations

from foldforge_amd import dispatch


def _served(module) -> int:
    return dispatch.ledger_of(module).served["hip"]


def _run(module, call, args, kwargs):
    assert module.backend == "hip", f"{type(module).__name__} is on {module.backend!r}, not hip"
    reason = module.unsupported(*args, **kwargs)
    assert reason is None, f"{type(module).__name__}: the hip backend refused the call: {reason}"
    before = _served(module)
    out = call(*args, **kwargs)
    assert _served(module) == before + 1, f"{type(module).__name__}: the hip backend did not serve the call"
    return out


def hip_delta(module, *args, **kwargs):
    """``module.delta(*args)``, served by ``hip``."""
    return _run(module, module.delta, args, kwargs)


def hip_forward(module, *args, **kwargs):
    """``module(*args)``, served by ``hip``."""
    return _run(module, module, args, kwargs)

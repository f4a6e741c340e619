"""Write ``pairstack_tiny.npz``: tiny seeded pair-stack cases with fp64 brute-force outputs.

The reference holds no golden vectors for these ops (its tests compare two
implementations on seeded random weights), so the fixtures are produced by the
element-by-element loops of ``oracle/brute.py`` from the equations. Run from the
repository root: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import brute  # noqa: E402

OUT = Path(__file__).resolve().with_name("pairstack_tiny.npz")


def _params(rng: np.random.Generator, shapes: dict[str, tuple[int, ...]]) -> dict[str, np.ndarray]:
    out = {}
    for name, shape in shapes.items():
        if len(shape) > 1:
            out[name] = 0.3 * rng.standard_normal(shape)
        elif name.endswith("weight"):
            out[name] = 1.0 + 0.1 * rng.standard_normal(shape)
        else:
            out[name] = 0.1 * rng.standard_normal(shape)
    return out


def cases() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    n, c, hid, heads, d = 5, 6, 4, 2, 3
    mask = np.ones((1, n), dtype=bool)
    mask[0, -1] = False
    store: dict[str, np.ndarray] = {}

    def put(case: str, inputs: dict[str, np.ndarray], params: dict[str, np.ndarray], expected):
        for k, v in inputs.items():
            store[f"{case}/{k}"] = v
        for k, v in params.items():
            store[f"{case}/p/{k}"] = v
        store[f"{case}/expected"] = expected

    tm_shapes = {
        "ln_pair.weight": (c,), "ln_pair.bias": (c,), "to_left.weight": (hid, c),
        "to_right.weight": (hid, c), "to_left_gate.weight": (hid, c),
        "to_right_gate.weight": (hid, c), "ln_out.weight": (hid,), "ln_out.bias": (hid,),
        "to_out.weight": (c, hid), "to_gate.weight": (c, c),
    }
    for outgoing in (True, False):
        z = rng.standard_normal((1, n, n, c))
        p = _params(rng, tm_shapes)
        put(f"trimul_{'out' if outgoing else 'in'}", {"z": z, "mask": mask}, p,
            brute.triangle_multiplication(z, mask, p, outgoing=outgoing))
    ta_shapes = {
        "ln_pair.weight": (c,), "ln_pair.bias": (c,), "to_bias.weight": (heads, c),
        "to_query.weight": (heads * d, c), "to_key.weight": (heads * d, c),
        "to_value.weight": (heads * d, c), "to_gate.weight": (heads * d, c),
        "to_out.weight": (c, heads * d),
    }
    for starting in (True, False):
        for transposed in (False, True):
            z = rng.standard_normal((1, n, n, c))
            p = _params(rng, ta_shapes)
            name = f"triattn_{'start' if starting else 'end'}_{'tb' if transposed else 'af3'}"
            put(name, {"z": z, "mask": mask}, p,
                brute.triangle_attention(z, mask, p, starting=starting, n_head=heads,
                                         transposed_bias=transposed))
    tr_shapes = {"ln_in.weight": (c,), "ln_in.bias": (c,), "expand_a.weight": (2 * c, c),
                 "expand_b.weight": (2 * c, c), "squeeze.weight": (c, 2 * c)}
    x = rng.standard_normal((1, n, n, c))
    p = _params(rng, tr_shapes)
    put("transition", {"x": x}, p, brute.transition(x, p))
    cs, hs = 9, 3
    apb_shapes = {
        "ln_single.weight": (cs,), "ln_single.bias": (cs,), "to_query.weight": (cs, cs),
        "to_query.bias": (cs,), "to_key.weight": (cs, cs), "to_value.weight": (cs, cs),
        "ln_pair.weight": (c,), "to_bias.weight": (hs, c), "to_gate.weight": (cs, cs),
        "to_out.weight": (cs, cs),
    }
    s = rng.standard_normal((1, n, cs))
    z = rng.standard_normal((1, n, n, c))
    p = _params(rng, apb_shapes)
    put("apb", {"s": s, "z": z, "mask": mask}, p,
        brute.attention_pair_bias(s, z, mask, p, n_head=hs, gate_bias=0.5))
    return store


if __name__ == "__main__":
    np.savez_compressed(OUT, **cases())
    print(OUT)

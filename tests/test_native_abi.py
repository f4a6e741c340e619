"""The C-ABI library on the CPU: it builds for gfx950, loads next to torch's HIP runtime and
exports exactly what ``include/foldforge_amd.h`` declares. No kernel is launched here (no
device); the workspace-size queries are pure host arithmetic and are checked against the
layouts they describe.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from foldforge_amd import _native, build

HEADER = Path(__file__).resolve().parents[1] / "include" / "foldforge_amd.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ffk_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not build.LIBRARY.exists():
        build.build()
    return _native.lib()


def test_header_and_binding_agree():
    names = declared()
    assert names, "no ffk_ entry point parsed from the header"
    assert set(names) == set(_native.SIGNATURES), set(names) ^ set(_native.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    for name in declared():
        assert hasattr(lib, name), name


def test_version_and_error_text(lib):
    assert lib.ffk_version() >= 100
    assert isinstance(lib.ffk_last_error(), bytes)


def test_workspace_sizes_follow_the_layouts(lib):
    def up(x):
        return (x + 255) // 256 * 256

    b, n = 2, 300
    np_ = 384
    tm = lib.ffk_triangle_multiplication_workspace(b, n, 128, 128)
    weights = up(4 * 128 * 128 * 2) + up(128 * 128 * 2) + up(128 * 128 * 2)
    # one float: the centre norm's epsilon of a length-divided call
    assert tm == up(4) + weights + 3 * up(b * 128 * np_ * np_ * 2) + up(b * np_ * 4) + up(b * 4)
    ta = lib.ffk_triangle_attention_workspace(b, n, 128, 4, 32, 0)
    weights = up(3 * 128 * 128 * 2) + up(32 * 128 * 2) + 2 * up(128 * 128 * 2)
    qkv = 3 * up(b * 4 * np_ * np_ * 32 * 2)
    assert ta == weights + qkv + up(b * 4 * np_ * np_ * 4) + up(b * n * n * 128 * 2) + up(b * np_ * 4) + up(b * 4)
    # the untransposed form stages one update; the dual form also packs its second projection
    update = up(b * n * n * 128 * 2)
    assert lib.ffk_triangle_attention_workspace(b, n, 128, 4, 32, 1) == ta + update
    assert lib.ffk_triangle_attention_workspace(b, n, 128, 4, 32, 2) == ta + update + up(128 * 128 * 2)
    assert lib.ffk_triangle_attention_workspace(b, n, 128, 4, 32, 3) == 0
    # generic widths: 16- and 32-wide heads take the flash core's layouts (rows padded to 4,
    # keys to 32, blocked bias) and stage the attention output in bf16; others the token layouts
    # with an fp32 gated output; the gate is staged (bf16) except where the output kernel
    # computes it
    np32, r4 = 320, 300
    tok = b * n * n * 64
    # (pair 64 with 64 or 128 gated channels: the output kernel computes the gate, none staged)
    flash16 = 3 * up(b * 4 * r4 * np32 * 16 * 2) + up(b * 4 * np32 * np32 * 4) + up(tok * 2)
    assert lib.ffk_triangle_attention_workspace(b, n, 64, 4, 16, 0) == flash16
    assert lib.ffk_triangle_attention_workspace(b, n, 64, 2, 32, 0) == (
        3 * up(b * 2 * r4 * np32 * 32 * 2) + up(b * 2 * np32 * np32 * 4) + up(tok * 2))
    tok128 = b * n * n * 128
    assert lib.ffk_triangle_attention_workspace(b, n, 128, 8, 16, 0) == (
        3 * up(b * 8 * r4 * np32 * 16 * 2) + up(tok128 * 2) + up(b * 8 * np32 * np32 * 4) + up(tok128 * 2))
    assert lib.ffk_triangle_attention_workspace(b, n, 64, 8, 8, 0) == (
        3 * up(tok * 2) + up(b * n * 64 * np32 * 2) + up(b * 8 * n * np32 * 4) + up(tok * 4))
    assert lib.ffk_transition_workspace(1000, 128, 4) == 3 * up(4 * 128 * 128 * 2)
    assert lib.ffk_transition_workspace(700, 384, 4) == up(700 * 1536 * 4)
    # hidden rows within the LayerNorm-fed GEMM's k limit (768) are staged in bf16
    assert lib.ffk_transition_workspace(700, 64, 2) == up(700 * 128 * 2)
    assert lib.ffk_transition_workspace(700, 256, 3) == up(700 * 768 * 2)
    apb = lib.ffk_attention_pair_bias_workspace(b, n, 384, 128, 16)
    tokens = up(b * n * 384 * 2)
    assert apb == 3 * tokens + up(b * n * 384 * 4) + up(b * 384 * np32 * 2) + up(b * 16 * n * np32 * 4)
    assert lib.ffk_attention_pair_bias_workspace(b, 0, 384, 128, 16) == 0
    depth, sp = 45, 64
    opm = lib.ffk_outer_product_mean_workspace(b, depth, n, 64, 32, 128)
    assert opm == 2 * up(b * n * 32 * sp * 2) + up(b * n * sp * 2) + up(b * n * n * 4) + up(128 * 1024 * 2)
    assert lib.ffk_outer_product_mean_workspace(b, 0, n, 64, 32, 128) == 0
    # the grouped (Chai-1) form: 64 channels a side, no count, the 512-wide output weight
    og = lib.ffk_outer_product_mean_grouped_workspace(b, depth, n, 64, 8, 8, 256)
    assert og == 2 * up(b * n * 64 * sp * 2) + up(b * n * sp * 2) + up(256 * 512 * 2)
    assert lib.ffk_outer_product_mean_grouped_workspace(b, depth, 0, 64, 8, 8, 256) == 0
    assert lib.ffk_triangle_multiplication_workspace(0, n, 128, 128) == 0


def test_build_recipe_targets_gfx950_without_packed_fp32():
    srcs = build.sources()
    assert srcs and all(str(s).endswith(".hip") for s in srcs)
    for src in srcs:
        cmd = build.compile_command(src, src.with_suffix(".o"))
        assert "--offload-arch=gfx950" in cmd
        assert "-packed-fp32-ops" in cmd
    assert "--offload-arch=gfx950" in build.link_command([s.with_suffix(".o") for s in srcs])

"""Host logic of bench.py that runs without a GPU: the traffic figure it reports must come from a
counter summary taken on the current flash-core sources."""
from __future__ import annotations

import importlib.util
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench(tmp_path=None):
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if tmp_path is not None:
        mod.ROOT = tmp_path
    return mod


def _fake_tree(tmp_path, digest_of_sources: bool, text: str = "int x;\n"):
    for p in ("foldforge_amd/csrc/triattn.hip", "foldforge_amd/csrc/ffk_device.h", "foldforge_amd/csrc/ffk_kernels.h"):
        (tmp_path / p).parent.mkdir(parents=True, exist_ok=True)
        (tmp_path / p).write_text(text)
    b = _bench(tmp_path)
    digest = b.source_digest() if digest_of_sources else "0" * 64
    (tmp_path / "profiles").mkdir(exist_ok=True)
    (tmp_path / "profiles" / "flash_attn_bias_n512_traffic.md").write_text(
        f"# summary\n\nsource_sha256: {digest}\n\ntraffic_bytes_per_launch: 123456\n")
    return b


def test_traffic_is_read_when_the_summary_names_the_current_sources(tmp_path):
    b = _fake_tree(tmp_path, True)
    assert b.recorded_traffic("flash_attn_bias_n512") == 123456.0


def test_stale_or_missing_traffic_summary_gives_none(tmp_path):
    b = _fake_tree(tmp_path, False)
    assert b.recorded_traffic("flash_attn_bias_n512") is None
    b = _fake_tree(tmp_path, True)
    (tmp_path / "foldforge_amd/csrc/triattn.hip").write_text("int y;\n")  # source changed after profiling
    assert b.recorded_traffic("flash_attn_bias_n512") is None
    assert b.recorded_traffic("no_such_kernel") is None


def test_committed_traffic_summary_parses():
    text = (ROOT / "profiles" / "flash_attn_bias_n512_traffic.md").read_text()
    keys = {ln.split(":", 1)[0].strip() for ln in text.splitlines() if ":" in ln}
    assert {"source_sha256", "traffic_bytes_per_launch"} <= keys

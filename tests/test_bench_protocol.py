"""bench.py's measurement bookkeeping on the CPU: a committed counter summary is only
reported while the kernel sources it was measured on are unchanged."""
import os

import bench


def _setup(tmp_path, source_text):
    (tmp_path / "profiles").mkdir()
    (tmp_path / "k.hip").write_text(source_text)
    return tmp_path


def test_traffic_reported_only_for_the_measured_sources(tmp_path, monkeypatch):
    root = _setup(tmp_path, "kernel v1\n")
    monkeypatch.setattr(bench, "ROOT", str(root))
    digest = bench.source_digest(["k.hip"])
    (root / "profiles" / "traffic_w.txt").write_text(
        "# header\nhbm_bytes_per_launch: 12345\nsource_sha256: %s\n" % digest)
    assert bench.read_traffic("w", ["k.hip"]) == 12345
    (root / "k.hip").write_text("kernel v2\n")  # the kernel changed since the counters ran
    assert bench.read_traffic("w", ["k.hip"]) is None


def test_traffic_without_a_source_line_or_file_is_not_reported(tmp_path, monkeypatch):
    root = _setup(tmp_path, "kernel\n")
    monkeypatch.setattr(bench, "ROOT", str(root))
    (root / "profiles" / "traffic_old.txt").write_text("hbm_bytes_per_launch: 99\n")
    assert bench.read_traffic("old", ["k.hip"]) is None
    assert bench.read_traffic("missing", ["k.hip"]) is None


def test_committed_decode_summary_matches_the_sources():
    """The decode traffic in profiles/ was measured on the kernel in this tree."""
    path = os.path.join(bench.ROOT, "profiles", "traffic_decode_qwen3_8b.txt")
    assert os.path.exists(path)
    assert bench.read_traffic("decode_qwen3_8b") is not None


def test_median_runs_and_cpu_model():
    calls = []
    ms = bench._median_ms(lambda: calls.append(1), runs=5, budget_s=0.0)
    assert len(calls) == 6 and ms >= 0.0  # one warm-up, then five timed runs
    assert isinstance(bench._cpu_model(), str)

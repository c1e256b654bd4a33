"""bench.py's command line and the build's tuning-knob switch, on the CPU (nothing here
touches a GPU: every case ends before the first HIP call)."""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_reason():
    out = _bench("--gpus", "2")
    assert out.returncode == 2
    assert "single MI355X" in out.stderr and out.stdout == ""


def test_unknown_sections_are_refused():
    out = _bench("--only", "headline,no_such_section")
    assert out.returncode == 2
    assert "no_such_section" in out.stderr


def test_build_refuses_definitions_that_are_not_tuning_knobs(monkeypatch):
    from marathon_amd import build

    monkeypatch.setenv(build.DEFINES_ENV, "MKV_XCDS=1 NDEBUG=1")
    with pytest.raises(ValueError, match="NDEBUG"):
        build.build_library()


def test_bench_reports_the_library_build_definitions(tmp_path, monkeypatch):
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    from marathon_amd import build

    f = tmp_path / "build_defines.txt"
    monkeypatch.setattr(build, "DEFINES_FILE", str(f))
    assert bench.build_defines() == "unknown"
    f.write_text("MKV_XCDS=1\n")
    assert bench.build_defines() == "MKV_XCDS=1"
    f.write_text("\n")
    assert bench.build_defines() == ""

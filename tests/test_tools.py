"""The command-line tools (drop-ins for the reference's build_global and
search_pipeline executables) on the CPU: they are built, and their argument
and file errors end the process with status 1 before any GPU work, as the
reference's do (build_global.cu:22-25, search_pipeline.cu:590-592,
utils.h:27-34)."""
import os
import subprocess

import numpy as np
import pytest

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fusiongpu_amd", "_lib", "bin")


def _run(*args, cwd=None):
    return subprocess.run([os.path.join(BIN, args[0]), *args[1:]], capture_output=True, text=True, timeout=60,
                          cwd=cwd)


@pytest.mark.parametrize("tool", ["build_global", "search_pipeline"])
def test_usage_without_arguments(tool):
    r = _run(tool)
    assert r.returncode == 1 and "Usage" in r.stderr


def test_missing_and_malformed_inputs(tmp_path):
    r = _run("build_global", str(tmp_path / "none.fvecs"))
    assert r.returncode == 1 and "cannot open" in r.stderr
    bad = tmp_path / "bad.fvecs"
    bad.write_bytes(np.array([0], np.int32).tobytes())
    r = _run("build_global", str(bad))
    assert r.returncode == 1 and "bad fvecs header" in r.stderr
    r = _run("build_global", "--bogus")
    assert r.returncode == 1 and "unknown argument" in r.stderr
    r = _run("search_pipeline", str(tmp_path / "none.fvecs"), str(tmp_path / "q.fvecs"))
    assert r.returncode == 1 and "cannot open" in r.stderr
    r = _run("search_pipeline", str(tmp_path / "none.fvecs"), str(tmp_path / "q.fvecs"), "--coarse", "cagra")
    assert r.returncode == 1 and "--coarse must be exact or graph" in r.stderr


def test_dimension_not_divisible_by_pq_m(tmp_path):
    f = tmp_path / "d30.fvecs"
    rows = np.concatenate([np.full((5, 1), 30, np.int32).view(np.float32), np.zeros((5, 30), np.float32)], 1)
    f.write_bytes(rows.astype(np.float32).tobytes())
    r = _run("build_global", str(f))
    assert r.returncode == 1 and "not a multiple" in r.stderr

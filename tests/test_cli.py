"""The shlo_hip CLI: the shlo_mlx surface of the reference (Main.lean:16-48)."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "contract-stablehlo-mlx_amd", "shlo_hip", "shlo_hip")


def test_usage_without_arguments():
    r = subprocess.run([CLI], capture_output=True, text=True)
    assert r.returncode == 2 and "usage: shlo_hip" in r.stderr


def test_wrong_argument_count(tmp_path):
    mod = tmp_path / "m.mlir"
    mod.write_text('module { func.func public @main(%a: tensor<4xf32>) -> tensor<4xf32> {\n'
                   '  func.return %a : tensor<4xf32>\n} }\n')
    r = subprocess.run([CLI, str(mod), str(tmp_path / "out")], capture_output=True, text=True)
    assert r.returncode == 2 and "@main takes 1 arguments, 0 files given" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [["--repeat", "3"], ["--no-compile"]])
def test_cli_runs_module(oracle, tmp_path, flags):
    import sys
    sys.path.insert(0, os.path.join(ROOT, "contract-stablehlo-mlx_amd"))
    from shlo_hip import configs
    N, K, M = 33, 70, 45
    a, st = oracle.fill_unif(1, 1.0, N * K)
    b, _ = oracle.fill_unif(1, 1.0, K * M, state=st)
    (tmp_path / "m.mlir").write_text(configs.dot_module(N, K, M))
    a.tofile(tmp_path / "a.bin")
    b.tofile(tmp_path / "b.bin")
    r = subprocess.run([CLI, str(tmp_path / "m.mlir"), str(tmp_path / "out"), str(tmp_path / "a.bin"),
                        str(tmp_path / "b.bin")] + flags, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "first call (trace + compile + run):" in r.stdout
    if "--repeat" in flags:
        assert "per call over 2:" in r.stdout
    got = np.fromfile(tmp_path / "out0.bin", dtype=np.float32).reshape(N, M)
    want = oracle.dot_general_bnk(a.reshape(1, N, K), np.ascontiguousarray(b.reshape(K, M).T)[None])[0]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

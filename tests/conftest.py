"""Shared test setup: import paths, the `gpu` marker, built libraries."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "mlx-llm_amd"
ORACLE = ROOT / "oracle"
for p in (PKG, ORACLE, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmlxq.so on cuda:0)")


def _ensure_built():
    """Build what is missing; a libmlxq.so built from other sources than this
    tree's is rebuilt where there is no GPU (the build host) and refused where
    there is one (GPU runs use the library built beforehand, never a stale one)."""
    if not (ORACLE / "liboracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ORACLE)], check=True)
    if not (PKG / "libmlxq.so").exists():
        subprocess.run([sys.executable, str(PKG / "build.py")], check=True)
    from provenance import library_hash, source_hash

    out = subprocess.run([sys.executable, "-c", "import mlxq; print(mlxq.version())"], cwd=str(PKG),
                         capture_output=True, text=True)
    if library_hash(out.stdout.strip()) == source_hash():
        return
    import torch

    if torch.cuda.device_count() > 0:
        pytest.exit(f"libmlxq.so is stale ({out.stdout.strip()}, tree src={source_hash()}): "
                    "rebuild with mlx-llm_amd/build.py before running the GPU tests", returncode=3)
    subprocess.run([sys.executable, str(PKG / "build.py")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch


@pytest.fixture(autouse=True)
def _kernel_overrides(monkeypatch):
    """The library reads its MLXQ_* kernel overrides once; a test that sets or
    removes one through monkeypatch has them read again, and again after the
    environment is restored."""
    import mlxq

    set_env, del_env = monkeypatch.setenv, monkeypatch.delenv
    touched = []

    def setenv(name, value, prepend=None):
        set_env(name, value, prepend)
        if name.startswith("MLXQ_"):
            touched.append(name)
            mlxq.reload_overrides()

    def delenv(name, raising=True):
        del_env(name, raising)
        if name.startswith("MLXQ_"):
            touched.append(name)
            mlxq.reload_overrides()

    monkeypatch.setenv, monkeypatch.delenv = setenv, delenv
    yield
    monkeypatch.undo()
    if touched:
        mlxq.reload_overrides()

"""The C-ABI libraries load and export every function their headers declare
(no device work: this runs without a GPU), and the registry knows "hip"."""

import ctypes
import pathlib
import re

import pytest

import mlvc_hip

REPO = pathlib.Path(__file__).resolve().parents[1]


def declared(header: str) -> list[str]:
    text = (REPO / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlvc_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("mlvc_hip_device.h", mlvc_hip.DEVICE_LIB),
                                        ("mlvc_hip_backend.h", mlvc_hip.BACKEND_LIB)])
def test_library_exports_every_declared_symbol(header, lib):
    names = declared(header)
    assert len(names) > 10
    so = ctypes.CDLL(str(lib))
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_registry_has_hip_backend():
    assert "hip" in mlvc_hip.available_backends()


def test_unknown_backend_and_missing_model_fail_loudly(tmp_path):
    with pytest.raises(mlvc_hip.MlvcError, match="unknown inference backend"):
        mlvc_hip.Backend(tmp_path, "cuda")
    with pytest.raises(mlvc_hip.MlvcError):
        mlvc_hip.aot_inspect(tmp_path, "missing")

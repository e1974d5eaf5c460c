"""The C-ABI library loads and exports every function include/tessery_hip.h declares; loader
errors keep tessery's stable codes. No compute call is made (no GPU needed)."""

import ctypes as ct
import re
from types import SimpleNamespace

import pytest

from tessery_amd import runtime
from tessery_amd.errors import HipUnavailableError, MetalUnavailableError, NativeBuildError
from tests.conftest import ROOT

HEADER = (ROOT / "include" / "tessery_hip.h").read_text()
DECLARED = sorted(set(re.findall(r"\b(mi_\w+)\s*\(", HEADER)))


def test_header_and_loader_agree():
    assert DECLARED == sorted(runtime.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ct.CDLL(str(runtime.library_path()))
    for name in DECLARED:
        assert hasattr(lib, name), name
    bound = runtime._library()
    assert bound.mi_abi_version() == runtime.ABI_VERSION


def test_missing_library_is_native_build_error(tmp_path):
    with pytest.raises(NativeBuildError) as error:
        runtime._library(tmp_path / "absent.so")
    assert str(error.value) == "native_engine_not_built"


@pytest.mark.parametrize("changed_during_load", [False, True])
def test_stale_or_changing_library_has_stable_error(tmp_path, monkeypatch, changed_during_load):
    library = tmp_path / "libtessery_hip.so"
    library.write_bytes(b"placeholder")

    def fake_load(path):
        if changed_during_load:
            library.write_bytes(b"changed")
        return SimpleNamespace()  # no ABI symbols

    monkeypatch.setattr(runtime.ct, "CDLL", fake_load)
    with pytest.raises(NativeBuildError):
        runtime._library(library)


def test_wrong_abi_version_is_native_build_error(tmp_path, monkeypatch):
    library = tmp_path / "libtessery_hip.so"
    library.write_bytes(b"x")
    functions = {name: SimpleNamespace() for name in runtime.SIGNATURES}
    functions["mi_abi_version"] = lambda: runtime.ABI_VERSION + 1
    monkeypatch.setattr(runtime.ct, "CDLL", lambda path: SimpleNamespace(**functions))
    with pytest.raises(NativeBuildError):
        runtime._library(library)


def test_no_device_is_hip_unavailable(monkeypatch):
    """mi_create returns NULL without a gfx950 device; the error is tessery's Metal one."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(MetalUnavailableError) as error:
        runtime.HipRuntime()
    assert isinstance(error.value, HipUnavailableError)

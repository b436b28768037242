"""The C-ABI library loads and exports every entry point include/wanmi.h declares (no GPU calls)."""

import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "wanmi.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wanmi_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "wanmi_adaln_quant" in names and "wanmi_abi_version" in names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"libwanmi.so does not export {name}"
    assert set(_declared()) == set(pkg._lib.exported_symbols())


def test_abi_version_and_error_reporting(pkg):
    lib = pkg._lib.load()
    header = (ROOT / "include" / "wanmi.h").read_text()
    assert lib.wanmi_abi_version() == int(re.search(r"WANMI_ABI_VERSION (\d+)", header).group(1)) == 3
    # an argument error is reported without touching the GPU
    st = lib.wanmi_adaln_quant(None, None, None, None, None, 4, 100, 1e-6, 1, 1, None, None, None, None)
    assert st == pkg._lib.WANMI_ERR_ARG
    assert b"multiple of 32" in lib.wanmi_last_error()


def test_missing_library_raises(pkg, monkeypatch, tmp_path):
    """Without the built library every op fails loudly; nothing falls back to the CPU."""
    import pytest
    import torch

    lib_mod = pkg._lib
    monkeypatch.setattr(lib_mod, "_LIB", None)
    monkeypatch.setattr(lib_mod, "LIB_PATH", tmp_path / "libwanmi.so")
    with pytest.raises(RuntimeError, match="is missing"):
        lib_mod.load()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.adaln_modulate(torch.zeros(4, 64, dtype=torch.bfloat16), eps=1e-6)


def test_cpu_tensor_is_rejected(pkg):
    import pytest
    import torch

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pkg.adaln_modulate(x, eps=1e-6)

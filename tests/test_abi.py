"""The C ABI library loads and exports every symbol include/mxmoe.h declares (no GPU needed)."""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mxmoe.h"
LIB = ROOT / "vesper_amd" / "libmxmoe.so"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_documented_entry_points():
    names = declared_symbols()
    for required in ("mx_create", "mx_destroy", "mx_last_error", "mx_malloc", "mx_dequant_mxfp4",
                     "mx_act_quant32", "mx_expert_forward", "mx_router", "mx_moe_decode", "mx_acc_add_rows"):
        assert required in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "build the library first: python -m vesper_amd.build"
    lib = C.CDLL(str(LIB))
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    from vesper_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES), set(declared_symbols()) - set(_lib.SIGNATURES)


def test_loader_reports_devices_without_failing_and_errors_map_to_python():
    from vesper_amd import _lib
    lib = _lib.load()
    n = lib.device_count()
    assert n >= 0
    if n == 0:
        with pytest.raises(ValueError):
            _lib.Context(0)
        assert "not present" in lib.last_error()


def test_tiled_expert_size_is_the_reference_byte_count():
    """mx_tiled_expert_bytes is host arithmetic (no device): same bytes as the six reference tensors."""
    from vesper_amd import _lib
    from vesper_amd.config import BASELINE, REFERENCE
    lib = _lib.load()
    for cfg in (BASELINE, REFERENCE):
        assert lib.cdll.mx_tiled_expert_bytes(cfg.hidden, cfg.intermediate) == cfg.expert_bytes
    assert lib.cdll.mx_tiled_expert_bytes(7168, 2048) == 23_396_352
    for bad in ((100, 128), (128, 0), (-128, 128)):
        assert lib.cdll.mx_tiled_expert_bytes(*bad) == 0


def test_expert_keys_round_trip_and_refuse_bad_forms():
    from vesper_amd.tiered import expert_key, parse_key
    assert expert_key(*parse_key("7:255")) == (7 << 32) | 255
    assert parse_key("0:0") == (0, 0)
    for bad in ("7", "a:b", "1:2:3", None):
        with pytest.raises(ValueError):
            parse_key(bad)
    with pytest.raises(ValueError):
        expert_key(-1, 0)


def test_product_package_never_imports_the_oracle():
    """oracle/ is test infrastructure: the vesper_amd package must not import it (no CPU fallback path)."""
    import re as _re
    pkg = ROOT / "vesper_amd"
    offenders = [p.name for p in pkg.glob("*.py")
                 if _re.search(r"^\s*(from|import)\s+oracle\b", p.read_text(), flags=_re.M)]
    assert not offenders, offenders

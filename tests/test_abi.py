"""CPU checks of the C-ABI library: it loads and exports every declared symbol.

No compute call is made (no GPU here)."""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "pdscope_moe.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pdscope_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_api():
    syms = declared_symbols()
    for name in ("pdscope_route_topk", "pdscope_route_hist", "pdscope_pack", "pdscope_swiglu_grouped",
                 "pdscope_swiglu_decode", "pdscope_merge", "pdscope_stage_expert", "pdscope_stage_merge",
                 "pdscope_last_error"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    from pdscope_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail("libpdscope_moe.so is not built (run python -m pdscope_amd.build)")
    lib = _lib.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == set(declared_symbols())
    assert lib.pdscope_version().decode().startswith("pdscope_moe gfx950")
    assert lib.pdscope_route_workspace_bytes() >= 4
    assert [lib.pdscope_grouped_block_m(r) for r in (8, 32, 80, 128, 256, 600)] == [32, 64, 128, 256, 384, 256]


def test_invalid_arguments_raise_before_any_launch():
    """Argument validation happens on the host and maps to ValueError."""
    from pdscope_amd import _lib
    with pytest.raises(ValueError):
        _lib.call("pdscope_pack", None, 1, 1, 1, None, None, None, None, None, None, None)
    with pytest.raises(ValueError):
        _lib.call("pdscope_route_topk", None, None, None, 1, 2048, 128, 8, 1, None, None, None, None, None, None)
    with pytest.raises(ValueError):
        _lib.call("pdscope_schedule", None, 128, None, 0, 48, None, None)
    msg = _lib.load().pdscope_last_error().decode()
    assert "schedule" in msg
    # the bound decode layer checks its out-pointer, read-back words and
    # binding before touching the device
    import ctypes
    handle = ctypes.c_void_p()
    with pytest.raises(ValueError, match="null binding out-pointer"):
        _lib.call("pdscope_decode_bind", None, None, 2048, 128, 8, 1, 1, None, 768, None, None, None, None, None,
                  None, None, None, None)
    with pytest.raises(ValueError, match="null read-back pointer"):
        _lib.call("pdscope_decode_bind", None, None, 2048, 128, 8, 1, 1, None, 768, None, None, None, None, None,
                  None, None, None, ctypes.byref(handle))
    assert handle.value is None
    with pytest.raises(ValueError, match="null binding"):
        _lib.call("pdscope_decode_run", None, None, None, None, None, None, 1, None)
    _lib.load().pdscope_decode_unbind(None)   # freeing no binding is a no-op

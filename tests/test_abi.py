"""CPU checks of the C ABI: the library loads, exports every function that
include/sulimo_hip.h declares, and the Python binding declares the same set.
No device call is made here beyond the probe, which reports absence cleanly."""
import ctypes

import pytest

from sulimo_amd import hip


def test_header_symbols_exported():
    L = hip.lib()
    names = hip.header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_header():
    L = ctypes.CDLL(hip.LIB_PATH)
    hip._declare(L)  # raises AttributeError if a declared binding has no symbol
    declared = set(hip.header_functions())
    bound = {n for n in dir(hip) if n.startswith("sulimo_hip_")}
    assert not bound - declared


def test_probe_never_raises():
    r = hip.probe()
    assert r.available in (0, 1)
    if not r.available:
        assert r.reason


def test_errors_without_device_are_reported():
    r = hip.probe()
    if r.available:
        pytest.skip("a device is present")
    with pytest.raises(hip.HipError) as e:
        hip.HipContext.get_or_init(0)
    assert e.value.code == hip.ERR_DEVICE_NOT_FOUND


def _header_struct_fields(name):
    """Member names of `typedef struct { ... } name;` in include/sulimo_hip.h."""
    import re
    from pathlib import Path
    text = (Path(hip.LIB_PATH).parent.parent / "include" / "sulimo_hip.h").read_text()
    body = re.search(r"typedef struct \{([^}]*)\}\s*" + name + r";", text).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        if decl.strip():
            fields += [re.findall(r"\w+", part)[-1] for part in decl.split(",")]
    return fields


@pytest.mark.parametrize("cname,cls", [("sulimo_hip_layer_tensors", "LayerTensorsC"),
                                       ("sulimo_hip_prefill_scratch", "PrefillScratchC")])
def test_ctypes_structs_match_header(cname, cls):
    names = [f[0] for f in getattr(hip, cls)._fields_]
    assert names == _header_struct_fields(cname)

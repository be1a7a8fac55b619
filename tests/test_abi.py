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


# Every struct of include/sulimo_hip.h and its ctypes mirror in sulimo_amd/hip.py.
STRUCTS = [
    ("sulimo_hip_device_info", "DeviceInfo"),
    ("sulimo_hip_probe_result", "ProbeResult"),
    ("sulimo_hip_gemm_profile", "GemmProfile"),
    ("sulimo_hip_model_config", "ModelConfigC"),
    ("sulimo_hip_layer_tensors", "LayerTensorsC"),
    ("sulimo_hip_model_tensors", "ModelTensorsC"),
    ("sulimo_hip_kv_cache", "KvCacheC"),
    ("sulimo_hip_prefill_scratch", "PrefillScratchC"),
    ("sulimo_hip_prefill_outputs", "PrefillOutputsC"),
    ("sulimo_hip_kernel_stat", "KernelStat"),
    ("sulimo_hip_prefill_stats", "PrefillStats"),
]


def _header_text():
    from pathlib import Path
    return Path(hip.HEADER_PATH).read_text()


def _header_struct_fields(name):
    """Member names of `typedef struct { ... } name;` in include/sulimo_hip.h."""
    import re
    body = re.search(r"typedef struct \{([^}]*)\}\s*" + name + r";", _header_text()).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    body = re.sub(r"\[[^\]]*\]", "", body)  # array extents
    fields = []
    for decl in body.split(";"):
        if decl.strip():
            fields += [re.findall(r"\w+", part)[-1] for part in decl.split(",")]
    return fields


def test_every_header_struct_has_a_mirror():
    import re
    declared = set(re.findall(r"\}\s*(sulimo_hip_\w+)\s*;", _header_text()))
    assert declared == {c for c, _ in STRUCTS}


@pytest.mark.parametrize("cname,cls", STRUCTS)
def test_ctypes_structs_match_header(cname, cls):
    names = [f[0] for f in getattr(hip, cls)._fields_]
    assert names == _header_struct_fields(cname)


def test_compiled_c_consumer_layout_and_calls(tmp_path):
    """A C program compiled by gcc against include/sulimo_hip.h and linked to the
    library: sizeof and offsetof of every member of every struct equal the ctypes
    mirror (a size_t/int32_t or ordering mismatch changes them), and sulimo_hip_probe /
    sulimo_hip_get_or_init / sulimo_hip_last_error behave through the real C ABI."""
    import os
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not installed")
    lines = ["#include <stddef.h>", "#include <stdio.h>", "#include <string.h>",
             '#include "sulimo_hip.h"', "int main(void) {"]
    want = []
    for cname, cls in STRUCTS:
        ct = getattr(hip, cls)
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        want.append(f"{cname} {ctypes.sizeof(ct)}")
        for fname, _ in ct._fields_:
            lines.append(f'  printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
            want.append(f"{cname}.{fname} {getattr(ct, fname).offset}")
    lines += [
        "  sulimo_hip_probe_result r;",
        "  memset(&r, 0x5a, sizeof r);",
        "  int rc = sulimo_hip_probe(&r);",
        '  printf("probe rc %d available %d\\n", rc, r.available);',
        "  if (!r.available) {",
        '    if (r.reason[0] == 0) { printf("no reason\\n"); return 2; }',
        "    sulimo_hip_ctx *ctx = NULL;",
        "    int e = sulimo_hip_get_or_init(0, &ctx);",
        '    printf("init %d %s\\n", e, sulimo_hip_last_error()[0] ? "message" : "empty");',
        "  } else {",
        '    printf("device %s wave %d\\n", r.info.arch_name, r.info.wavefront_size);',
        "  }",
        "  return 0;", "}"]
    src = tmp_path / "consumer.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "consumer"
    libdir = os.path.dirname(hip.LIB_PATH)
    cc = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(hip.HEADER_PATH),
                         str(src), "-o", str(exe), "-L", libdir, "-lsulimo_hip",
                         f"-Wl,-rpath,{libdir}"], capture_output=True, text=True)
    assert cc.returncode == 0, cc.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    out = run.stdout.splitlines()
    assert out[:len(want)] == want
    tail = out[len(want):]
    assert tail[0].startswith("probe rc 0 available ")
    if tail[0].endswith("available 0"):
        assert tail[1] == f"init {hip.ERR_DEVICE_NOT_FOUND} message"
    else:
        assert tail[1].startswith("device gfx950") and tail[1].endswith("wave 64")

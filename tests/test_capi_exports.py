"""The C-ABI library loads and exports every entry point include/ffnerf_hip.h
declares (no compute calls: this runs on the CPU-only container too)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "ffnerf_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ffn_\w+)\s*\(", text, re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ("ffn_create", "ffn_destroy", "ffn_bind_params", "ffn_train_step", "ffn_occ_decay", "ffn_sample",
              "ffn_hash_encode_fwd", "ffn_hash_encode_bwd", "ffn_adam", "ffn_last_error", "ffn_version",
              "ffn_occ_bitfield", "ffn_march", "ffn_render"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import ffn_lib
    if not ffn_lib.LIB_PATH.exists():
        pytest.fail("libffnerf_hip.so is not built (run __graft_entry__.build())")
    lib = ffn_lib.load()
    for n in declared_functions():
        assert hasattr(lib, n), n
    assert sorted(ffn_lib.EXPORTS) == declared_functions()
    assert ffn_lib.load().ffn_version() == ffn_lib.ABI_VERSION == 3


def test_binding_refuses_another_abi_version(monkeypatch):
    """The binding checks ffn_version() on load: a library built from another header (other struct layouts)
    is refused with an error instead of being called with structures of the wrong size."""
    import ffn_lib
    if not ffn_lib.LIB_PATH.exists():
        pytest.fail("libffnerf_hip.so is not built (run __graft_entry__.build())")
    monkeypatch.setattr(ffn_lib, "ABI_VERSION", 1)
    with pytest.raises(ffn_lib.FfnError, match="ABI version 3"):
        ffn_lib.load(ffn_lib.LIB_PATH)


def test_invalid_config_is_an_error_not_a_silent_return():
    import ffn_lib as fl
    from common import spec_cfg0
    lib = fl.load()
    cfg = fl.make_config(spec_cfg0(nd=5))
    h = ctypes.c_void_p()
    rc = lib.ffn_create(ctypes.byref(cfg), ctypes.byref(h))
    assert rc < 0 and b"nd=5" in lib.ffn_last_error()
    cfg = fl.make_config(spec_cfg0(f_per_level=3))
    assert lib.ffn_create(ctypes.byref(cfg), ctypes.byref(h)) < 0
    assert b"f_per_level" in lib.ffn_last_error()


def test_one_hip_runtime_per_process():
    """Loading the library must leave one HIP runtime in the process: torch's (ffn_lib.load imports torch
    before the library, whose own dependency would otherwise map the system runtime beside torch's)."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); import ffn_lib; ffn_lib.load(); "
            "print(sorted({l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}))")
    out = subprocess.run([sys.executable, "-c", code % str(ROOT / "ffnerf-experimental_amd")],
                         capture_output=True, text=True, check=True).stdout
    maps = eval(out.strip().splitlines()[-1])
    assert len(maps) == 1, maps

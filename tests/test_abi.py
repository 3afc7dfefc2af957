"""The C ABI library loads and exports every entry point include/mx_sampler.h
declares (no GPU needed: nothing is called that touches a device)."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "mx_sampler.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|void)\s+(mxs_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from metallix_amd import sampler

    lib = sampler.load_library()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
        assert name in sampler.PROTOTYPES, f"{name} missing from the Python prototypes"


def test_abi_version_and_status_strings():
    from metallix_amd import sampler

    lib = sampler.load_library()
    assert lib.mxs_abi_version() == sampler.ABI_VERSION == 2
    assert lib.mxs_status_string(0) == b"ok"
    assert b"temperature" in lib.mxs_status_string(-4)


def test_create_rejects_bad_arguments_without_a_device():
    import ctypes
    from metallix_amd import sampler

    lib = sampler.load_library()
    ctx = ctypes.c_void_p()
    assert lib.mxs_create(0, None, 0, 10, ctypes.byref(ctx)) == -1
    assert lib.mxs_create(0, None, 1, 0, ctypes.byref(ctx)) == -1
    assert lib.mxs_create(0, None, 1, 10, None) == -1


def test_noalloc_topn_rejects_bad_arguments_without_a_device():
    from metallix_amd import sampler

    lib = sampler.load_library()
    # null logits: rejected by the argument checks, before any HIP call
    assert lib.mxs_logsoftmax_topn_noalloc(None, None, 0, 4, 100, 100, 5, None, None, None, None, None) == -1
    assert b"required" in lib.mxs_last_error(None)

"""The C-ABI library loads and exports every entry point include/freeml_hip.h declares.

No compute call is made here: this suite runs without a GPU.
"""
import ctypes
import os
import re

import pytest

import freeml_amd

HEADER = freeml_amd.HEADER


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmlh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_op_set():
    names = declared_functions()
    for op in ("fmlh_mul", "fmlh_matmul_strided", "fmlh_softmax", "fmlh_layernorm", "fmlh_gelu",
               "fmlh_add", "fmlh_copy", "fmlh_gather_rows", "fmlh_split_qkv", "fmlh_scale_add",
               "fmlh_nanollm_create", "fmlh_nanollm_prefill", "fmlh_nanollm_decode"):
        assert op in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(freeml_amd.LIB_PATH), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(freeml_amd.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_probe_library_is_separate():
    """The exchange-latency probe lives in its own library (include/freeml_probe.h), not in the
    product one."""
    probe = declared_functions(freeml_amd.PROBE_HEADER)
    assert probe == ["fmlh_probe_exchange"]
    assert not set(probe) & set(declared_functions())
    assert os.path.exists(freeml_amd.PROBE_LIB_PATH), "run __graft_entry__.build() first"
    main = ctypes.CDLL(freeml_amd.LIB_PATH)
    assert not hasattr(main, "fmlh_probe_exchange")
    lib = ctypes.CDLL(freeml_amd.PROBE_LIB_PATH)
    assert all(hasattr(lib, n) for n in probe)
    assert set(probe) <= set(freeml_amd._PROBE_SIGS)


def test_python_binding_covers_the_header():
    bound = set(freeml_amd._SIGS) | {"fmlh_last_error", "fmlh_get_stream"}
    assert set(declared_functions()) <= bound


def test_header_compiles_as_c():
    import subprocess
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.c")
        with open(src, "w") as f:
            f.write('#include "freeml_hip.h"\n#include "freeml_probe.h"\nint main(void){ return FMLH_OK; }\n')
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER),
                        src, "-o", os.path.join(d, "t")], check=True)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device error path")
def test_no_device_reports_error_instead_of_crashing():
    with pytest.raises(freeml_amd.FreeMLHipError) as e:
        freeml_amd.init(0)
    assert e.value.code in (-3, -2)
    assert freeml_amd.lib().fmlh_last_error()

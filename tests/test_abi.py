"""CPU checks of the C-ABI boundary: the library loads, exports every entry point include/cdclq.h
declares, its structs match the reference-mirroring layout, and it fails cleanly without a GPU.
No compute calls are made here."""
import ctypes as C
import os
import re
import subprocess

import pytest

import cdclq
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cdclq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cdclq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_boundary():
    names = declared_functions()
    for required in ("cdclq_quantize_layer", "cdclq_gram_accumulate", "cdclq_upper_chol_of_inverse",
                     "cdclq_proxy_loss", "cdclq_ctx_create", "cdclq_ctx_destroy", "cdclq_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = cdclq.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", cdclq.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (cdclq_\w+)", out))
    assert set(declared_functions()) <= exported
    assert set(cdclq.exported_symbols()) == set(declared_functions())


def test_struct_layouts_match_oracle_and_binding():
    lib = cdclq.lib()
    assert lib.cdclq_sizeof_config() == O.lib().orc_sizeof_config() == C.sizeof(cdclq._Config)
    assert lib.cdclq_sizeof_stats() == O.lib().orc_sizeof_stats() == C.sizeof(cdclq._Stats)
    assert lib.cdclq_abi_version() == 1


def test_default_config_is_reference_default():
    """src/engine.rs:146-167, through the library, the oracle and the Python mirror."""
    c = cdclq._Config()
    cdclq.lib().cdclq_default_config(C.byref(c))
    o = O.config()
    py = cdclq.Config()._c()
    for name, _ in cdclq._Config._fields_:
        assert getattr(c, name) == getattr(o, name) == getattr(py, name), name
    assert (c.bits, c.group, c.block, c.damp, c.act_order, c.passes, c.tol) == (3, 128, 128, 0.01, 1, 10, 1e-3)


@pytest.mark.parametrize("group,n,ng", [(128, 4096, 32), (128, 300, 3), (0, 300, 1), (512, 300, 1), (64, 64, 1)])
def test_num_groups(group, n, ng):
    c = cdclq.Config(group=group)._c()
    assert cdclq.lib().cdclq_num_groups(C.byref(c), n) == ng == O.lib().orc_num_groups(C.byref(O.config(group=group)),
                                                                                         n)


def test_no_gpu_fails_cleanly():
    """Without a usable GPU the context constructor reports an error instead of falling back."""
    p = C.c_void_p()
    rc = cdclq.lib().cdclq_ctx_create(10_000, C.byref(p))
    assert rc == cdclq.DEVICE and not p.value
    assert cdclq.lib().cdclq_quantize_layer(None, None, 0, 0, None, None, None, None, 0, None, None, None, None, None,
                                            None) == cdclq.INVALID_ARG


def test_product_never_imports_the_oracle():
    """The product package must not load or reference the test oracle."""
    pkg = os.path.join(ROOT, "cdcl-gptq_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower().replace("no oracle", ""), os.path.join(dirpath, f)

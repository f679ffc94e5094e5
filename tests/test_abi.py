"""The C ABI boundary without a GPU: the library loads, exports exactly what
include/mxdecode.h declares, the ctypes table matches the header, and bad
arguments come back as error codes (checked on the host before any launch).
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from gemmagemini4hackathon2026_10_2425_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mxdecode.h"


def header_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(mxd_\w+)\s*\(", text))


def test_header_and_ctypes_table_agree():
    assert header_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert _lib.LIB_PATH.exists(), "libmxdecode.so is not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mxd_\w+)", out))
    missing = header_functions() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_library_loads_and_reports_version():
    lib = _lib.load()
    assert lib.mxd_abi_version() == 2
    for name in _lib.SIGNATURES:
        assert hasattr(lib, name)


P = ctypes.c_void_p(16)  # a non-null dummy: argument checks fail before any dereference


@pytest.mark.parametrize(
    "name,args,code",
    [
        ("mxd_matvec_f16", (P, P, _lib.MXD_F32, P, 64, 12, 0, None, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_matvec_f16", (None, P, _lib.MXD_F32, P, 64, 16, 0, None, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_matvec_f16", (P, P, 7, P, 64, 16, 0, None, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_matvec_f16", (P, P, _lib.MXD_F32, P, 64, 16, _lib.MXD_EPI_GELU_MUL, None, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_matvec_f16", (P, P, _lib.MXD_F32, P, 0, 16, 0, None, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_matvec_q8b32", (P, P, P, _lib.MXD_F16, P, 64, 48, 0, None, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_matvec_q8b32", (P, None, P, _lib.MXD_F16, P, 64, 64, 0, None, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_gemv_f32", (P, P, P, 8, 6, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_matvec_gate_up", (5, P, None, P, None, P, _lib.MXD_F32, P, 64, 64, 0, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_matvec_gate_up", (_lib.MXD_W_Q8B32, P, None, P, None, P, _lib.MXD_F32, P, 64, 64, 0, None),
         _lib.MXD_ERR_INVALID_ARG),
        ("mxd_rmsnorm", (P, P, P, 3, 1, 64, 1e-6, 1, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_rope_kv", (P, P, P, P, 8, 1, 255, 64, 0, 1, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_rope_kv", (P, P, P, P, 8, 1, 256, 64, 64, 1, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_attention", (P, P, P, P, 32, 8, 96, 512, 10, None, 0.1, None, 0, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_attention", (P, P, P, P, 32, 8, 128, 500, 10, None, 0.1, None, 0, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_attention", (P, P, P, P, 48, 3, 128, 512, 10, None, 0.1, None, 0, None), _lib.MXD_ERR_UNSUPPORTED),
        ("mxd_attention", (P, P, P, P, 32, 8, 128, 512, 0, None, 0.1, None, 0, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_attention", (P, P, P, P, 32, 8, 128, 512, 513, None, 0.1, None, 0, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_attention", (P, P, P, P, 32, 8, 128, 32768, 32768, None, 0.1, None, 0, None), _lib.MXD_ERR_WORKSPACE),
        ("mxd_argmax", (P, P, 100, 0, None, 0, None), _lib.MXD_ERR_WORKSPACE),
        ("mxd_argmax", (P, P, 0, 0, P, 64, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_fill_normal", (P, 9, 10, 0, 0, 0.02, None), _lib.MXD_ERR_INVALID_ARG),
        ("mxd_embed", (P, P, -1, 1, P, 64, 1.0, 10, None), _lib.MXD_ERR_INVALID_ARG),
    ],
)
def test_host_side_argument_errors(name, args, code):
    with pytest.raises(_lib.MxdValueError) as ei:
        _lib.call(name, *args)
    assert ei.value.code == code
    assert _lib.last_error()  # the failure is described


def test_tunable_names():
    _lib.set_tunable("MV_NR", 2)
    _lib.set_tunable("MV_NR", 0)
    with pytest.raises(_lib.MxdValueError):
        _lib.call("mxd_set_tunable", b"", 1)


def test_workspace_queries():
    n = _lib.query("mxd_attention_workspace_size", 32, 8, 128, 32768)
    assert n >= 64 * 32 * (128 + 2) * 4
    assert _lib.query("mxd_argmax_workspace_size", 256000) >= 12


@pytest.mark.parametrize("bad", [dict(head_dim=96), dict(rope_factor=32.0, rope_low_freq_factor=4.0,
                                                          rope_high_freq_factor=1.0, rope_original_max_positions=8192),
                                  dict(rope_factor=0.5, rope_low_freq_factor=1.0, rope_high_freq_factor=4.0,
                                       rope_original_max_positions=8192)])
def test_engine_config_rejected_before_allocation(bad):
    """mxd_engine_create checks the config on the host before any device call."""
    from gemmagemini4hackathon2026_10_2425_amd.engine import LLAMA32_1B

    cfg = LLAMA32_1B.to_c()
    for k, v in bad.items():
        setattr(cfg, k, v)
    out = ctypes.c_void_p()
    with pytest.raises(_lib.MxdValueError):
        _lib.call("mxd_engine_create", ctypes.byref(cfg), 256, ctypes.byref(out))
    assert not out.value

# SPDX-License-Identifier: Apache-2.0
"""The C-ABI library loads and exports exactly what include/k3kda.h declares, and the
struct mirrors match the reference's byte layout. No GPU compute is called here."""
from __future__ import annotations

import ctypes as C
import re
import subprocess

import pytest

from conftest import REPO
import k3kda

HEADER = REPO / "include" / "k3kda.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(k3(?:hip)?_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_path():
    names = declared_functions()
    for must in ("k3_kda_layer", "k3_kda_scratch", "k3hip_kda_decode", "k3hip_kda_prep",
                 "k3hip_kda_chunk", "k3hip_kda_epilogue", "k3hip_kda_layer_dev"):
        assert must in names
    assert set(names) == set(k3kda.EXPORTS), set(names) ^ set(k3kda.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = k3kda.lib()
    for n in declared_functions():
        assert hasattr(L, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", str(k3kda.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert set(declared_functions()) <= exported


def test_version_and_error_string_without_gpu():
    L = k3kda.lib()
    assert b"gfx950" in L.k3hip_version()
    assert isinstance(L.k3hip_last_error(), bytes)
    assert L.k3hip_device_count() >= 0


def test_scratch_size_matches_reference_formula():
    """k3_kda_scratch returns the reference's float count 6TP + TH + 2P + D
    (src/core/k3_ops.c:853-862)."""
    L = k3kda.lib()
    for hidden, H, D, T in ((128, 4, 16, 8), (7168, 96, 128, 4), (4096, 32, 128, 8192)):
        c = k3kda.make_cfg(hidden, H, D)
        P = H * D
        assert L.k3_kda_scratch(C.byref(c), T) == 6 * T * P + T * H + 2 * P + D


def test_struct_mirrors_match_reference_layout():
    assert C.sizeof(k3kda.K3Cfg) == 128
    assert C.sizeof(k3kda.K3KdaW) == 120
    lay = REPO / "oracle" / "_ref" / "layout.txt"
    if not lay.exists():
        pytest.skip("reference layout probe not built (reference sources absent)")
    fields = dict(l.rsplit(" ", 1) for l in lay.read_text().splitlines())
    assert int(fields["K3Cfg"]) == C.sizeof(k3kda.K3Cfg)
    assert int(fields["K3KdaW"]) == C.sizeof(k3kda.K3KdaW)
    for key, off in fields.items():
        if "." in key:
            st, f = key.split(".")
            cls = getattr(k3kda, st)
            assert getattr(cls, f).offset == int(off), key


def test_invalid_arguments_are_refused_before_any_launch():
    """Argument checks run on the host and need no device."""
    L = k3kda.lib()
    rc = L.k3hip_kda_decode(-1, 1, 128, None, None, None, None, None, None, None, 1.0, None)
    assert rc == k3kda.EINVAL and b"B=-1" in L.k3hip_last_error()
    rc = L.k3hip_kda_decode(1, 1, 48, None, None, None, None, None, None, None, 1.0, None)
    assert rc == k3kda.EUNSUPPORTED
    rc = L.k3hip_kda_prep(4, 1, 128, 9, -5.0, 0, *([None] * 17), None)
    assert rc in (k3kda.EINVAL, k3kda.EUNSUPPORTED)
    rc = L.k3hip_kda_epilogue(1, 1, 128, 1e-5, None, None, 0, None, None, 0, None)
    assert rc == k3kda.EINVAL


def test_projection_gemm_selector_without_gpu():
    """The layer prefill's GEMM selector is a host-side setting: unknown values are refused
    and the default (hipBLASLt) is restored."""
    L = k3kda.lib()
    assert L.k3hip_set_projection_gemm(2) == k3kda.EINVAL and b"impl=2" in L.k3hip_last_error()
    assert L.k3hip_set_projection_gemm(k3kda.GEMM_HANDWRITTEN) == k3kda.OK
    assert L.k3hip_set_projection_gemm(k3kda.GEMM_HIPBLASLT) == k3kda.OK

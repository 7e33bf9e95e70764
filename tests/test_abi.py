"""The C ABI: libinet_nr.so loads (no GPU needed), exports every function include/inet_nr.h and include/inet_wifi.h
declare, and the ctypes mirrors of the structs have the C layout (checked against sizeof / offsetof from the headers
compiled by gcc). No compute entry point is called here."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from conftest import ROOT
from isaac_net_amd import _lib

HEADER = os.path.join(ROOT, "include", "inet_nr.h")
WIFI_HEADER = os.path.join(ROOT, "include", "inet_wifi.h")


def _lib_path():
    if not os.path.exists(_lib.LIB_PATH):
        from isaac_net_amd import build
        build.build()
    return _lib.LIB_PATH


def declared_functions(header=HEADER, prefix="inet_nr_"):
    src = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|const char \*)\s*(" + prefix + r"\w+)\s*\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib_path())
    names = declared_functions()
    assert names == sorted(["inet_nr_abi_version", "inet_nr_build_info", "inet_nr_step", "inet_nr_submit",
                            "inet_nr_reset", "inet_nr_dl_step", "inet_nr_dl_submit", "inet_nr_dl_reset",
                            "inet_nr_submit_step", "inet_nr_step_cells", "inet_nr_cells_reset"])
    for n in names:
        assert hasattr(lib, n), n
    lib.inet_nr_abi_version.restype = ctypes.c_int32
    assert lib.inet_nr_abi_version() == _lib.ABI_VERSION == 15
    lib.inet_nr_build_info.restype = ctypes.c_char_p
    assert b"gfx950" in lib.inet_nr_build_info()
    wifi = declared_functions(WIFI_HEADER, "inet_wifi_")
    assert wifi == sorted(["inet_wifi_abi_version", "inet_wifi_step", "inet_wifi_submit", "inet_wifi_reset",
                           "inet_wifi_dcf_step", "inet_wifi_dcf_reset"])
    for n in wifi:
        assert hasattr(lib, n), n
    lib.inet_wifi_abi_version.restype = ctypes.c_int32
    assert lib.inet_wifi_abi_version() == _lib.WIFI_ABI_VERSION == 7


STRUCTS = ("InetNrState", "InetNrTables", "InetNrParams", "InetNrOutputs", "InetNrRow", "InetNrDlState",
           "InetNrArrivals", "InetNrCells", "InetWifiState", "InetWifiParams", "InetWifiOutputs", "InetDcfState", "InetDcfParams")


def test_ctypes_layout_matches_header():
    py = {n: getattr(_lib, n) for n in STRUCTS if hasattr(_lib, n)}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', f'#include "{WIFI_HEADER}"',
             "int main(void) {"]
    for n, cls in py.items():
        lines.append(f'printf("{n} %zu\\n", sizeof({n}));')
        for f, _ in cls._fields_:
            lines.append(f'printf("{n}.{f} %zu\\n", offsetof({n}, {f}));')
    lines += ['printf("InetNrRow %zu\\n", sizeof(InetNrRow));', "return 0; }"]
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        open(c, "w").write("\n".join(lines))
        exe = os.path.join(d, "layout")
        subprocess.run(["gcc", "-std=c11", "-o", exe, c], check=True)
        out = dict(l.rsplit(" ", 1) for l in subprocess.run([exe], check=True, capture_output=True,
                                                              text=True).stdout.split("\n") if l)
    for n, cls in py.items():
        assert int(out[n]) == ctypes.sizeof(cls), n
        for f, _ in cls._fields_:
            assert int(out[f"{n}.{f}"]) == getattr(cls, f).offset, f"{n}.{f}"
    assert int(out["InetNrRow"]) == 4 * len(_lib.ROW_DTYPE_FIELDS)


def test_load_refuses_missing_library(tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        _lib._LIB, saved = None, _lib._LIB
        try:
            _lib.load(str(tmp_path / "nope.so"))
        finally:
            _lib._LIB = saved

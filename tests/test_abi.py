"""CPU checks of the C ABI: the library loads, exports every symbol that
include/apus_hip.h declares, and honours the forced-fallback switch
(APUS_HIP_DISABLE, the analogue of the reference's APUS_METAL_NO_* nulling
of its hook table, c/backend_metal.mm:490-495). No compute runs here."""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np

import apus_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "apus_hip.h")


def declared():
    txt = open(HDR).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(apus_hip_\w+)\s*\(", txt)))


def test_header_matches_binding_list():
    assert declared() == sorted(apus_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", apus_hip.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    have = set(re.findall(r"\bT (apus_hip_\w+)", out))
    missing = [s for s in declared() if s not in have]
    assert not missing, missing
    lib = apus_hip.load()
    for s in declared():
        assert getattr(lib, s) is not None


def test_forced_fallback_returns_disabled():
    """With APUS_HIP_DISABLE=1 every op returns APUS_HIP_ERR_DISABLED (2)
    without touching a device; a host engine then runs its CPU op."""
    code = r"""
import ctypes as C, numpy as np, sys
sys.path.insert(0, %r)
import apus_hip
lib = apus_hip.load()
b = np.zeros(4, np.uint16); beta = np.zeros(4, np.uint16)
rc = lib.apus_hip_gdn_beta(b.ctypes.data_as(C.POINTER(C.c_uint16)),
                           beta.ctypes.data_as(C.POINTER(C.c_uint16)), C.c_size_t(4))
print(rc, apus_hip.last_error())
""" % os.path.dirname(apus_hip.__file__)
    env = dict(os.environ, APUS_HIP_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stderr
    rc, msg = r.stdout.split(" ", 1)
    assert int(rc) == 2 and "APUS_HIP_DISABLE" in msg


def test_binding_raises_on_error():
    err = apus_hip.ApusHipError(3, "x")
    assert err.code == 3 and "x" in str(err)

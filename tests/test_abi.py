"""The C ABI library loads, exports every declared symbol, and rejects
malformed arguments before touching the device (CPU-only checks)."""
import ctypes as C
import os

from conftest import ROOT


def test_library_exports_every_declared_symbol(mx):
    header = os.path.join(ROOT, "include", "mx355.h")
    names = mx.declared_symbols(header)
    assert "mx_qmv" in names and len(names) >= 20
    missing = [n for n in names if not hasattr(mx.lib, n)]
    assert not missing, missing


def test_abi_version(mx):
    assert mx.lib.mx_abi_version() == 1


def test_qmv_rejects_bad_geometry_without_device(mx):
    fake = 256  # never dereferenced: validation fails first
    q = mx.QWeightC(fake, fake, fake, 64, 512, 3, 64)  # 3-bit is unsupported
    rc = mx.lib.mx_qmv(C.byref(q), fake, 1, fake, None)
    assert rc == mx.MX_EINVAL
    assert b"bits" in mx.lib.mx_last_error()
    q = mx.QWeightC(fake, fake, fake, 64, 500, 4, 64)  # k not a multiple of 32
    assert mx.lib.mx_qmv(C.byref(q), fake, 1, fake, None) == mx.MX_EINVAL
    q = mx.QWeightC(fake, fake, fake, 64, 512, 4, 64)
    assert mx.lib.mx_qmv(C.byref(q), fake, 9, fake, None) == mx.MX_EUNSUPPORTED
    assert mx.lib.mx_qmv(C.byref(q), None, 1, fake, None) == mx.MX_EINVAL

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


def test_layer_entry_points_reject_bad_geometry_without_device(mx):
    fake = 256
    ok_bank = mx.QBankC(fake, fake, fake, 8, 64, 256, 4, 64)
    down = mx.QBankC(fake, fake, fake, 8, 256, 64, 5, 64)
    sg = mx.QWeightC(fake, fake, fake, 64, 256, 4, 64)
    sd = mx.QWeightC(fake, fake, fake, 256, 64, 5, 64)
    args = [fake, fake, fake, 9, 4, C.byref(ok_bank), C.byref(ok_bank), C.byref(down),
            C.byref(sg), C.byref(sg), C.byref(sd), fake, fake, None]
    assert mx.lib.mx_moe_experts(*args) == mx.MX_EUNSUPPORTED  # rows > 8
    args[3] = 2
    bad_down = mx.QBankC(fake, fake, fake, 8, 128, 64, 5, 64)  # down.n != hidden
    args[7] = C.byref(bad_down)
    assert mx.lib.mx_moe_experts(*args) == mx.MX_EINVAL
    assert mx.lib.mx_moe_route(fake, 100, fake, 1, 2, 100, 10, fake, fake, fake, None) == \
        mx.MX_EUNSUPPORTED
    assert mx.lib.mx_moe_route(fake, 512, fake, 1, 2, 512, 17, fake, fake, fake, None) == \
        mx.MX_EUNSUPPORTED
    dims = mx.GdnDimsC(16, 32, 64, 128, 4)
    assert mx.lib.mx_gdn_recurrence(fake, 8192, fake, fake, fake, 4160, fake, fake, fake, 1e-6,
                                    C.byref(dims), 1, 1, fake, fake, None, fake, None) == \
        mx.MX_EUNSUPPORTED
    dims = mx.GdnDimsC(16, 24, 128, 128, 4)  # 24 % 16 != 0
    assert mx.lib.mx_gdn_scan(fake, fake, fake, fake, fake, C.byref(dims), 1, 1, fake, fake,
                              None, fake, None) == mx.MX_EINVAL
    assert mx.lib.mx_gdn_conv(fake, 8192, 1, 1, fake, fake, fake, 8192, 9, fake, 8192, None,
                              None) == mx.MX_EUNSUPPORTED
    head = mx.QWeightC(fake, fake, fake, 1000, 512, 8, 64)
    assert mx.lib.mx_head_argmax(C.byref(head), fake, 0, fake, fake, None) == mx.MX_EUNSUPPORTED
    assert mx.lib.mx_head_workspace_bytes(151936, 2048, 8) > 0
    assert mx.lib.mx_moe_workspace_bytes(8, 10, 512) >= 8 * 11 * 512 * 2
    # engine measurement hooks: null engine or outputs are refused
    prof = mx.StepProfileC()
    tok = (C.c_uint32 * 4)(1, 2, 3, 4)
    out = (C.c_uint32 * 4)()
    assert mx.lib.mx_engine_profile_verify(None, 0, tok, 4, out, C.byref(prof)) == mx.MX_EINVAL
    assert mx.lib.mx_engine_draft_bytes(None, 0, None) == mx.MX_EINVAL


def test_noalloc_head_refuses_oversized_heads_without_device(mx):
    """The static-scratch head rejects a head whose partials exceed its
    1 MiB array before any launch (pointers are never dereferenced)."""
    fake = 256
    assert mx.lib.mx_head_noalloc_max_bytes() == 1 << 20
    big = mx.QWeightC(fake, fake, fake, 300000, 2048, 8, 64)
    assert mx.lib.mx_head_workspace_bytes(300000, 2048, 8) > mx.lib.mx_head_noalloc_max_bytes()
    assert mx.lib.mx_head_argmax_noalloc(C.byref(big), fake, 8, fake, None) == mx.MX_EUNSUPPORTED
    assert b"static scratch" in mx.lib.mx_last_error()
    ok = mx.QWeightC(fake, fake, fake, 1000, 512, 8, 64)
    assert mx.lib.mx_head_argmax_noalloc(C.byref(ok), fake, 9, fake, None) == mx.MX_EUNSUPPORTED
    assert mx.lib.mx_head_argmax_noalloc(C.byref(ok), None, 1, fake, None) == mx.MX_EINVAL

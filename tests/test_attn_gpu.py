"""Gated decode attention (mx_attn_decode): the fixed-order kernel is bit-exact
with the CPU oracle's restatement, and the matrix-core kernel is within
tolerance of the float64 closed form, for rows at ragged positions (chunk
boundaries of both kernels, a single cached position, and the last position
of the cache), rows that share a slot, and 1, 4 and 8 q heads per kv head."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _sigmoid_bf16(x):
    return 1.0 / (1.0 + np.exp(-x))


@pytest.mark.parametrize("heads,kv_heads,hd", [(16, 2, 256), (4, 1, 128), (8, 8, 128), (8, 1, 256)])
def test_attn_decode_exact_and_fast(mx, orc, heads, kv_heads, hd):
    S, max_ctx = 5, 1100
    rng = np.random.default_rng(heads * 1000 + hd)
    pos = np.array([0, 62, 63, 64, 255, 256, 700, max_ctx - 1], np.int32)
    rows = len(pos)
    slots = rng.integers(0, S, rows).astype(np.int32)
    slots[1] = slots[0]  # two rows of one slot (a verify block)
    kc = orc.f32_to_bf16(rng.standard_normal((S, kv_heads, max_ctx, hd)).astype(np.float32))
    vc = orc.f32_to_bf16(rng.standard_normal((S, kv_heads, max_ctx, hd)).astype(np.float32))
    q = orc.f32_to_bf16((rng.standard_normal((rows, heads, hd)) * 0.3).astype(np.float32))
    qkv_stride = 2 * heads * hd + 64
    qkv = orc.f32_to_bf16(rng.standard_normal((rows, qkv_stride)).astype(np.float32))
    slot_stride = kv_heads * max_ctx * hd
    want = np.empty((rows, heads, hd), np.uint16)
    orc.lib.mxo_attention(q.ctypes.data, qkv.ctypes.data, qkv_stride, rows, slots.ctypes.data,
                          pos.ctypes.data, kc.ctypes.data, vc.ctypes.data, heads, kv_heads, hd,
                          max_ctx, slot_stride, want.ctypes.data)
    # float64 closed form
    G = heads // kv_heads
    ref = np.empty((rows, heads, hd))
    for r in range(rows):
        for h in range(heads):
            k = bf(kc[slots[r], h // G, : pos[r] + 1]).astype(np.float64)
            v = bf(vc[slots[r], h // G, : pos[r] + 1]).astype(np.float64)
            s = k @ bf(q[r, h]).astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            gate = bf(qkv[r, h * 2 * hd + hd: h * 2 * hd + 2 * hd]).astype(np.float64)
            ref[r, h] = (p @ v) / p.sum() * _sigmoid_bf16(gate)
    dims = mx.AttnDimsC(heads, kv_heads, hd, max_ctx, slot_stride)
    ws = mx.DeviceArray((mx.lib.mx_attn_workspace_bytes(rows, heads, hd, max_ctx),), np.uint8)
    dq, dqkv, dsl, dpos, dk, dv = (mx.DeviceArray.from_numpy(np.ascontiguousarray(a))
                                   for a in (q, qkv, slots, pos, kc, vc))
    for flags in (0, 1):
        out = mx.DeviceArray((rows, heads, hd), np.uint16)
        mx.check(mx.lib.mx_attn_decode(dq.ptr, dqkv.ptr, qkv_stride, rows, dsl.ptr, dpos.ptr,
                                       dk.ptr, dv.ptr, C.byref(dims), flags, ws.ptr, out.ptr, None))
        got = out.numpy()
        if flags == 0:
            assert (got == want).all(), np.argwhere(got != want)[:5]
        g = bf(got).astype(np.float64)
        scale = np.abs(ref).max(axis=2, keepdims=True)
        # two bf16 roundings (attention, gated output) plus fp32 sums
        assert np.all(np.abs(g - ref) <= 2.0 ** -6 * np.abs(ref) + 2.0 ** -9 * scale), flags


@pytest.mark.parametrize("heads,kv_heads,hd,p0,rows", [(16, 2, 256, 0, 40), (16, 2, 256, 700, 129),
                                                        (8, 2, 128, 250, 37), (8, 4, 256, 31, 17)])
def test_attn_prefill_form_within_tolerance(mx, orc, heads, kv_heads, hd, p0, rows):
    """The prefill form (flags bit 1: the rows of one slot's chunk at positions
    p0 .. p0 + rows - 1, query blocks sharing each 64-key tile, partials per
    256-key split) against the float64 closed form with the matrix-core
    kernel's bound, and within that bound of the per-row matrix-core kernel;
    the chunks start at 0, inside a split and across split boundaries, with
    rows that do not fill the last query block."""
    S, max_ctx = 3, 1100
    rng = np.random.default_rng(heads * 100 + hd + p0 + rows)
    slot = 1
    pos = np.arange(p0, p0 + rows, dtype=np.int32)
    slots = np.full(rows, slot, np.int32)
    kc = orc.f32_to_bf16(rng.standard_normal((S, kv_heads, max_ctx, hd)).astype(np.float32))
    vc = orc.f32_to_bf16(rng.standard_normal((S, kv_heads, max_ctx, hd)).astype(np.float32))
    q = orc.f32_to_bf16((rng.standard_normal((rows, heads, hd)) * 0.3).astype(np.float32))
    qkv_stride = 2 * heads * hd
    qkv = orc.f32_to_bf16(rng.standard_normal((rows, qkv_stride)).astype(np.float32))
    slot_stride = kv_heads * max_ctx * hd
    G = heads // kv_heads
    ref = np.empty((rows, heads, hd))
    for r in range(rows):
        for h in range(heads):
            k = bf(kc[slot, h // G, : pos[r] + 1]).astype(np.float64)
            v = bf(vc[slot, h // G, : pos[r] + 1]).astype(np.float64)
            s = k @ bf(q[r, h]).astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            gate = bf(qkv[r, h * 2 * hd + hd: h * 2 * hd + 2 * hd]).astype(np.float64)
            ref[r, h] = (p @ v) / p.sum() * _sigmoid_bf16(gate)
    dims = mx.AttnDimsC(heads, kv_heads, hd, max_ctx, slot_stride)
    ws = mx.DeviceArray((mx.lib.mx_attn_workspace_bytes(rows, heads, hd, max_ctx),), np.uint8)
    dq, dqkv, dsl, dpos, dk, dv = (mx.DeviceArray.from_numpy(np.ascontiguousarray(a))
                                   for a in (q, qkv, slots, pos, kc, vc))
    got = {}
    for flags in (1, 3, 3):
        out = mx.DeviceArray((rows, heads, hd), np.uint16)
        mx.check(mx.lib.mx_attn_decode(dq.ptr, dqkv.ptr, qkv_stride, rows, dsl.ptr, dpos.ptr,
                                       dk.ptr, dv.ptr, C.byref(dims), flags, ws.ptr, out.ptr, None))
        g = out.numpy()
        if flags in got:
            assert (g == got[flags]).all()  # deterministic
        got[flags] = g
    scale = np.abs(ref).max(axis=2, keepdims=True)
    for flags, g in got.items():
        g = bf(g).astype(np.float64)
        assert np.all(np.abs(g - ref) <= 2.0 ** -6 * np.abs(ref) + 2.0 ** -9 * scale), flags
    a, b = bf(got[1]).astype(np.float64), bf(got[3]).astype(np.float64)
    assert np.all(np.abs(a - b) <= 2.0 ** -6 * np.abs(ref) + 2.0 ** -9 * scale)

"""ctypes wrapper of liboracle.so — the CPU restatement used as the checker.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py; never by the product library.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} not built; run make -C oracle")
    lib = C.CDLL(LIB_PATH)
    vp, i32, i64, u64, sz, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_size_t, C.c_float
    sig = {
        "mxo_bf16_to_f32": ([C.c_uint16], f32),
        "mxo_f32_to_bf16": ([f32], C.c_uint16),
        "mxo_expf": ([f32], f32),
        "mxo_log1pf": ([f32], f32),
        "mxo_sigmoidf": ([f32], f32),
        "mxo_softplusf": ([f32], f32),
        "mxo_eval_math": ([i32, vp, vp, i64], None),
        "mxo_rng_u64": ([u64, u64], u64),
        "mxo_fill_bf16": ([vp, sz, u64, i32, f32, f32], None),
        "mxo_fill_codes": ([vp, i64, i32, i32, u64], None),
        "mxo_code": ([vp, i32, i32], C.c_uint32),
        "mxo_dequant_rows": ([vp, vp, vp, i32, i32, i32, i32, vp, i32, vp], None),
        "mxo_qmv": ([vp, vp, vp, i32, i32, i32, i32, vp, i32, vp], None),
        "mxo_qmv_f64": ([vp, vp, vp, i32, i32, i32, i32, vp, i32, vp], None),
        "mxo_num_threads": ([], i32),
        "mxo_qmv_row": ([vp, vp, vp, i32, i32, i32, vp], f32),
        "mxo_xq_slices": ([i32], i32),
        "mxo_xq_int": ([C.c_uint16, i32], i64),
        "mxo_xq_group_exp": ([vp], i32),
        "mxo_xq_row": ([vp, vp, vp, i32, i32, vp], f32),
        "mxo_xq": ([vp, vp, vp, i32, i32, i32, vp, i32, vp], None),
        "mxo_sigmoid_bf16": ([f32], f32),
        "mxo_softplus_bf16": ([f32], f32),
        "mxo_moe_route": ([vp, i64, vp, i64, i32, i32, i32, vp, vp, vp], None),
        "mxo_moe_experts": ([vp, vp, vp, i32, i32, vp, vp, vp, vp, vp, vp, vp], None),
        "mxo_moe_reduce": ([vp, i32, i32, i32, vp], None),
        "mxo_moe_hc_epilogue": ([vp, vp, vp, vp, vp, i32, i32, i32, vp], None),
        "mxo_gdn_conv": ([vp, i64, i32, i32, vp, vp, vp, i32, i32, vp, i64, vp], None),
        "mxo_gdn_recurrence": ([vp, i64, vp, vp, vp, i64, vp, vp, vp, f32, i32, i32, i32, i32,
                                vp, vp, vp, vp], None),
        "mxo_gdn_scan": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp], None),
        "mxo_argmax_bf16": ([vp, i32, i32, vp], None),
        "mxo_gemv_bf16": ([vp, i32, i32, vp, i32, vp], None),
        "mxo_head_argmax": ([vp, vp, i32, vp, vp], None),
        "mxo_hc_norm": ([vp, vp, i32, i32, i32, f32, vp], None),
        "mxo_hc_down": ([vp, vp, i32, i32, i32, vp, vp], None),
        "mxo_hc_up_mix": ([vp, vp, vp, i32, i32, vp], None),
        "mxo_hc_write": ([vp, vp, i32, i32, vp, vp], None),
        "mxo_embed": ([vp, vp, i32, i32, vp], None),
        "mxo_attn_prep": ([vp, i64, i32, vp, vp, vp, vp, f32, vp, vp, i32, i32, i32, i32, i32,
                           i64, vp, vp, vp], None),
        "mxo_rope_table": ([i32, i32, f32, vp, vp], None),
        "mxo_attention": ([vp, vp, i64, i32, vp, vp, vp, vp, i32, i32, i32, i32, i64, vp], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


lib = _load()


# projection arithmetic of a weight struct: the fixed fp32 order of
# mxo_qmv_row, or the exact-integer projection of mxo_xq_row
FIXED, XQ = 0, 1


class QW(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("n", C.c_int), ("k", C.c_int), ("bits", C.c_int), ("gs", C.c_int),
                ("mode", C.c_int)]


class QBank(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("experts", C.c_int), ("n", C.c_int), ("k", C.c_int), ("bits", C.c_int),
                ("gs", C.c_int), ("mode", C.c_int)]


def qw(codes, scales, biases, n, k, bits, gs, mode=FIXED) -> QW:
    """Struct view of host arrays (the caller keeps the arrays alive)."""
    for a in (codes, scales, biases):
        assert a.flags["C_CONTIGUOUS"]
    assert mode == FIXED or gs == 64
    return QW(codes.ctypes.data, scales.ctypes.data, biases.ctypes.data, n, k, bits, gs, mode)


def qbank(codes, scales, biases, experts, n, k, bits, gs, mode=FIXED) -> QBank:
    for a in (codes, scales, biases):
        assert a.flags["C_CONTIGUOUS"]
    assert mode == FIXED or gs == 64
    return QBank(codes.ctypes.data, scales.ctypes.data, biases.ctypes.data, experts, n, k, bits, gs,
                 mode)


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- numpy helpers ----
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    flat, of = f.reshape(-1), out.reshape(-1)
    u = flat.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = (0x7FC0 | ((u[nan] >> 16) & 0x8000)).astype(np.uint16)
    of[:] = r
    return out


def eval_math(op: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib.mxo_eval_math(op, _p(x), _p(out), x.size)
    return out


def fill_bf16(count: int, seed: int, dist: int, a: float, b: float) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib.mxo_fill_bf16(_p(out), count, seed, dist, a, b)
    return out


def fill_codes(rows: int, k: int, bits: int, seed: int) -> np.ndarray:
    out = np.empty((rows, k * bits // 32), np.uint32)
    lib.mxo_fill_codes(_p(out), rows, k, bits, seed)
    return out


def random_qweight(n: int, k: int, bits: int, gs: int, seed: int,
                   s_range=(0.005, 0.03), b_range=(-0.2, 0.2)):
    """Host copy of the same tensors rust-mlx_amd.QWeight.random makes on device."""
    codes = fill_codes(n, k, bits, seed)
    scales = fill_bf16(n * (k // gs), seed + 1, 0, *s_range).reshape(n, k // gs)
    biases = fill_bf16(n * (k // gs), seed + 2, 0, *b_range).reshape(n, k // gs)
    return codes, scales, biases


def unpack_codes(codes: np.ndarray, k: int, bits: int) -> np.ndarray:
    """All codes of a [n, k*bits/32] word matrix as uint8 [n, k]."""
    n = codes.shape[0]
    out = np.empty((n, k), np.uint8)
    for r in range(n):
        row = np.ascontiguousarray(codes[r])
        for c in range(k):
            out[r, c] = lib.mxo_code(_p(row), c, bits)
    return out


def dequant_rows(codes, scales, biases, k, bits, gs, ids) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.uint32)
    n = codes.shape[0]
    out = np.empty((ids.size, k), np.uint16)
    lib.mxo_dequant_rows(_p(codes), _p(scales), _p(biases), n, k, bits, gs, _p(ids), ids.size,
                         _p(out))
    return out


def qmv(codes, scales, biases, k, bits, gs, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    n = codes.shape[0]
    y = np.empty((m, n), np.uint16)
    lib.mxo_qmv(_p(codes), _p(scales), _p(biases), n, k, bits, gs, _p(x), m, _p(y))
    return y


def xq(codes, scales, biases, k, bits, x) -> np.ndarray:
    """Exact-integer projection (mxo_xq): fp32 y [m, n] before bf16 rounding."""
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    n = codes.shape[0]
    y = np.empty((m, n), np.float32)
    lib.mxo_xq(_p(codes), _p(scales), _p(biases), n, k, bits, _p(x), m, _p(y))
    return y


def qmv_f64(codes, scales, biases, k, bits, gs, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    n = codes.shape[0]
    y = np.empty((m, n), np.float64)
    lib.mxo_qmv_f64(_p(codes), _p(scales), _p(biases), n, k, bits, gs, _p(x), m, _p(y))
    return y


def num_threads() -> int:
    return lib.mxo_num_threads()


# ---- MoE ----
def sigmoid_bf16(x: float) -> float:
    return lib.mxo_sigmoid_bf16(x)


def moe_route(logits: np.ndarray, shared_logit: np.ndarray, top_k: int):
    logits = np.ascontiguousarray(logits, np.uint16)
    shared_logit = np.ascontiguousarray(shared_logit, np.uint16).reshape(-1)
    rows, experts = logits.shape
    ids = np.empty((rows, top_k), np.uint32)
    scores = np.empty((rows, top_k), np.uint16)
    factor = np.empty(rows, np.uint16)
    lib.mxo_moe_route(_p(logits), experts, _p(shared_logit), 1, rows, experts, top_k, _p(ids),
                      _p(scores), _p(factor))
    return ids, scores, factor


def moe_experts(x, ids, scores, top_k, gate: QBank, up: QBank, down: QBank, sgate: QW, sup: QW,
                sdown: QW, hidden: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    ids = np.ascontiguousarray(ids, np.uint32)
    scores = np.ascontiguousarray(scores, np.uint16)
    rows = x.shape[0]
    p = np.empty((rows, top_k + 1, hidden), np.uint16)
    lib.mxo_moe_experts(_p(x), _p(ids), _p(scores), rows, top_k, C.byref(gate), C.byref(up),
                        C.byref(down), C.byref(sgate), C.byref(sup), C.byref(sdown), _p(p))
    return p


def moe_reduce(p: np.ndarray, top_k: int) -> np.ndarray:
    p = np.ascontiguousarray(p, np.uint16)
    rows, _, hidden = p.shape
    out = np.empty((rows, hidden), np.uint16)
    lib.mxo_moe_reduce(_p(p), rows, top_k, hidden, _p(out))
    return out


def moe_hc_epilogue(routed, shared, factor, residual, gate, hc: int) -> np.ndarray:
    routed, shared, factor, residual, gate = (np.ascontiguousarray(a, np.uint16)
                                              for a in (routed, shared, factor, residual, gate))
    rows, hidden = routed.shape
    out = np.empty((rows, hc * hidden), np.uint16)
    lib.mxo_moe_hc_epilogue(_p(routed), _p(shared), _p(factor), _p(residual), _p(gate), rows, hc,
                            hidden, _p(out))
    return out


# ---- GDN ----
def gdn_conv(qkv, groups, t, slots, conv_state, conv_w, window_history=False):
    """Returns (out, new conv_state, window or None); inputs are not modified."""
    qkv = np.ascontiguousarray(qkv, np.uint16)
    channels = conv_w.shape[1]
    taps = conv_w.shape[0]
    conv_state = np.array(conv_state, np.uint16, copy=True, order="C")
    slots = np.ascontiguousarray(slots, np.int32)
    conv_w = np.ascontiguousarray(conv_w, np.float32)
    out = np.empty((groups * t, channels), np.uint16)
    hist = np.empty((groups, taps - 1 + t, channels), np.uint16) if window_history else None
    lib.mxo_gdn_conv(_p(qkv), qkv.shape[1], groups, t, _p(slots), _p(conv_state), _p(conv_w),
                     channels, taps, _p(out), channels, _p(hist) if hist is not None else None)
    return out, conv_state, hist


def gdn_recurrence(conv_out, z, a, b, a_log, dt_bias, norm_w, eps, hk, hv, groups, t, slots,
                   state, history=False):
    """z, a, b are separate [rows, *] arrays here. Returns (y, new state, history)."""
    conv_out = np.ascontiguousarray(conv_out, np.uint16)
    rows = groups * t
    zab = np.ascontiguousarray(np.concatenate([z, a, b], axis=1), np.uint16)
    zs = zab.shape[1]
    zp = zab.ctypes.data
    ap = zp + 2 * z.shape[1]
    bp = ap + 2 * a.shape[1]
    state = np.array(state, np.float32, copy=True, order="C")
    slots = np.ascontiguousarray(slots, np.int32)
    a_log = np.ascontiguousarray(a_log, np.float32)
    dt_bias = np.ascontiguousarray(dt_bias, np.uint16)
    norm_w = np.ascontiguousarray(norm_w, np.uint16)
    y = np.empty((rows, hv * 128), np.uint16)
    hist = np.empty((rows, hv, 128, 128), np.float32) if history else None
    lib.mxo_gdn_recurrence(_p(conv_out), conv_out.shape[1], zp, ap, bp, zs, _p(a_log),
                           _p(dt_bias), _p(norm_w), eps, hk, hv, groups, t, _p(slots),
                           _p(state), _p(hist) if hist is not None else None, _p(y))
    return y, state, hist


def gdn_scan(q, k, v, g, beta, hk, hv, groups, t, slots, state, history=False):
    q, k, v, beta = (np.ascontiguousarray(a, np.uint16) for a in (q, k, v, beta))
    g = np.ascontiguousarray(g, np.float32)
    rows = groups * t
    state = np.array(state, np.float32, copy=True, order="C")
    slots = np.ascontiguousarray(slots, np.int32)
    y = np.empty((rows, hv, 128), np.uint16)
    hist = np.empty((rows, hv, 128, 128), np.float32) if history else None
    lib.mxo_gdn_scan(_p(q), _p(k), _p(v), _p(g), _p(beta), hk, hv, groups, t, _p(slots),
                     _p(state), _p(hist) if hist is not None else None, _p(y))
    return y, state, hist


# ---- unquantised GEMV ----
def gemv_bf16(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.uint16)
    n, k = w.shape
    rows = x.shape[0]
    y = np.empty((rows, n), np.uint16)
    lib.mxo_gemv_bf16(_p(w), n, k, _p(x), rows, _p(y))
    return y


# ---- head ----
def argmax_bf16(logits: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(logits, np.uint16)
    rows, n = logits.shape
    out = np.empty(rows, np.uint32)
    lib.mxo_argmax_bf16(_p(logits), rows, n, _p(out))
    return out


def head_argmax(w: QW, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    out = np.empty(m, np.uint32)
    scratch = np.empty(w.n, np.float32)
    lib.mxo_head_argmax(C.byref(w), _p(x), m, _p(out), _p(scratch))
    return out

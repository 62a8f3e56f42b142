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
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


lib = _load()


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


def qmv_f64(codes, scales, biases, k, bits, gs, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    m = x.shape[0]
    n = codes.shape[0]
    y = np.empty((m, n), np.float64)
    lib.mxo_qmv_f64(_p(codes), _p(scales), _p(biases), n, k, bits, gs, _p(x), m, _p(y))
    return y


def num_threads() -> int:
    return lib.mxo_num_threads()

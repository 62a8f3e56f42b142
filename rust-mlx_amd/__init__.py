"""ctypes binding of libmx355.so — the MI355X batched-decode-step library.

This module is a thin host-side harness over the C ABI declared in
include/mx355.h; it is used by the tests and by bench.py.  It never falls back
to another implementation: if the native library is missing or fails to load,
importing this module raises.

The package directory name contains a hyphen, so load it with
``load_package()`` below (or importlib) rather than a plain import.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmx355.so")

MX_OK = 0
MX_EINVAL = 1
MX_EUNSUPPORTED = 2
MX_EHIP = 3
MX_ENOMEM = 4
MX_ESTATE = 5


class MxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"mx error {code}: {msg}")
        self.code = code


class QWeightC(C.Structure):
    _fields_ = [
        ("codes", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("n", C.c_int32),
        ("k", C.c_int32),
        ("bits", C.c_int32),
        ("group_size", C.c_int32),
    ]


class QBankC(C.Structure):
    _fields_ = [
        ("codes", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("experts", C.c_int32),
        ("n", C.c_int32),
        ("k", C.c_int32),
        ("bits", C.c_int32),
        ("group_size", C.c_int32),
    ]


class GdnDimsC(C.Structure):
    _fields_ = [("hk", C.c_int32), ("hv", C.c_int32), ("dk", C.c_int32), ("dv", C.c_int32),
                ("conv_k", C.c_int32)]


class AttnDimsC(C.Structure):
    _fields_ = [("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("max_ctx", C.c_int32), ("slot_stride", C.c_int64)]


MAX_LAYERS = 128  # MX_MAX_LAYERS


class ModelConfigC(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "layers", "attn_every", "vocab", "hc", "hc_rank", "gdn_hk", "gdn_hv", "gdn_dk",
        "gdn_dv", "conv_k", "heads", "kv_heads", "head_dim", "rotary_dim")] + [
        ("rope_theta", C.c_float), ("rms_eps", C.c_float)] + [(n, C.c_int32) for n in (
            "experts", "top_k", "moe_inter", "shared_inter", "bits", "down_bits", "embed_bits",
            "head_bits", "group_size", "mixed_bits", "max_slots", "max_context", "max_verify")] + [
        ("seed", C.c_uint64), ("mtp", C.c_int32),
        ("layer_widths", C.c_uint8 * (2 * (MAX_LAYERS + 1)))]


def config_c(cfg: dict) -> ModelConfigC:
    """The mx_model_config of an engine configuration dict (its optional
    "layer_widths" list fills the per-layer width table, zeros elsewhere)."""
    d = dict(cfg)
    widths = d.pop("layer_widths", None) or []
    cc = ModelConfigC(**d)
    if len(widths) > 2 * (MAX_LAYERS + 1):
        raise ValueError("layer_widths longer than the engine's table")
    for i, w in enumerate(widths):
        cc.layer_widths[i] = int(w)
    return cc


class GenerateStatsC(C.Structure):
    _fields_ = [("rounds", C.c_int32), ("drafted", C.c_int32), ("accepted", C.c_int32)]


class StepProfileC(C.Structure):
    _fields_ = [("rows", C.c_int32), ("layers", C.c_int32)] + [(n, C.c_double) for n in (
        "distinct_experts", "gate_up_ms", "down_ms", "gate_up_bytes", "down_bytes", "step_ms",
        "step_bytes")]


SCHED_PREFILL = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_int32, C.POINTER(C.c_uint32), C.c_int32,
                            C.POINTER(C.c_uint32))
SCHED_DECODE = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_uint32),
                           C.c_int32, C.POINTER(C.c_uint32))
SCHED_CLONE = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_int32, C.c_int32)


class SchedBackendC(C.Structure):
    _fields_ = [("ctx", C.c_void_p), ("prefill", SCHED_PREFILL), ("decode", SCHED_DECODE),
                ("clone", SCHED_CLONE)]


class ExpertTimingC(C.Structure):
    _fields_ = [("launches", C.c_int32)] + [(n, C.c_double) for n in (
        "distinct_experts", "gate_up_ms", "gate_up_bytes", "down_ms", "down_bytes")]


class SchedConfigC(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("batch_size", "slots", "prefix_entries", "prefix_tokens",
                                         "max_context", "n_stop")] + [("stop", C.c_uint32 * 8)]


class SchedEventC(C.Structure):
    _fields_ = [("job", C.c_uint64), ("token", C.c_uint32), ("kind", C.c_int32),
                ("detail", C.c_int32)]


SCHED_TOKEN, SCHED_STOP, SCHED_LENGTH, SCHED_ERROR = 0, 1, 2, 3


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C rust-mlx_amd/csrc)"
        )
    lib = C.CDLL(LIB_PATH)
    vp, sz, i32, i64, u64, f32 = C.c_void_p, C.c_size_t, C.c_int32, C.c_int64, C.c_uint64, C.c_float
    sig = {
        "mx_last_error": ([], C.c_char_p),
        "mx_abi_version": ([], i32),
        "mx_prefill_chunk_tokens": ([], i32),
        "mx_malloc": ([C.POINTER(vp), sz], i32),
        "mx_free": ([vp], i32),
        "mx_memcpy_htod": ([vp, vp, sz], i32),
        "mx_memcpy_dtoh": ([vp, vp, sz], i32),
        "mx_memcpy_dtod": ([vp, vp, sz, vp], i32),
        "mx_memset": ([vp, C.c_int, sz, vp], i32),
        "mx_stream_create": ([C.POINTER(vp)], i32),
        "mx_stream_destroy": ([vp], i32),
        "mx_stream_sync": ([vp], i32),
        "mx_device_sync": ([], i32),
        "mx_event_create": ([C.POINTER(vp)], i32),
        "mx_event_destroy": ([vp], i32),
        "mx_event_record": ([vp, vp], i32),
        "mx_event_elapsed_ms": ([vp, vp, C.POINTER(f32)], i32),
        "mx_fill_bf16": ([vp, sz, u64, i32, f32, f32, vp], i32),
        "mx_fill_codes": ([vp, i64, i32, i32, u64, vp], i32),
        "mx_eval_math": ([i32, vp, vp, i64, vp], i32),
        "mx_qmv": ([C.POINTER(QWeightC), vp, i32, vp, vp], i32),
        "mx_dequant_rows": ([C.POINTER(QWeightC), vp, i32, vp, vp], i32),
        "mx_moe_route": ([vp, i64, vp, i64, i32, i32, i32, vp, vp, vp, vp], i32),
        "mx_moe_workspace_bytes": ([i32, i32, i32], sz),
        "mx_moe_experts": ([vp, vp, vp, i32, i32, C.POINTER(QBankC), C.POINTER(QBankC),
                            C.POINTER(QBankC), C.POINTER(QWeightC), C.POINTER(QWeightC),
                            C.POINTER(QWeightC), vp, vp, vp], i32),
        "mx_moe_reduce": ([vp, i32, i32, i32, vp, vp], i32),
        "mx_moe_hc_epilogue": ([vp, vp, vp, vp, vp, i32, i32, i32, vp, vp], i32),
        "mx_moe_reduce_hc_epilogue": ([vp, vp, vp, vp, i32, i32, i32, i32, vp, vp], i32),
        "mx_head_workspace_bytes": ([i32, i32, i32], sz),
        "mx_head_argmax": ([C.POINTER(QWeightC), vp, i32, vp, vp, vp], i32),
        "mx_argmax_bf16": ([vp, i32, i32, vp, vp], i32),
        "mx_gdn_conv": ([vp, i64, i32, i32, vp, vp, vp, i32, i32, vp, i64, vp, vp], i32),
        "mx_gdn_recurrence": ([vp, i64, vp, vp, vp, i64, vp, vp, vp, f32, C.POINTER(GdnDimsC),
                               i32, i32, vp, vp, vp, vp, vp], i32),
        "mx_gdn_scan": ([vp, vp, vp, vp, vp, C.POINTER(GdnDimsC), i32, i32, vp, vp, vp, vp,
                         vp], i32),
        "mx_gdn_recurrence_fast": ([vp, i64, vp, vp, vp, i64, vp, vp, vp, f32,
                                    C.POINTER(GdnDimsC), i32, i32, vp, vp, vp, vp, vp], i32),
        "mx_gdn_prefill_workspace_bytes": ([i32, i32, i32], sz),
        "mx_gdn_prefill_chunked": ([vp, vp, vp, vp, vp, C.POINTER(GdnDimsC), i32, i32, vp, vp, vp,
                                    vp, vp], i32),
        "mx_gemv_bf16": ([vp, i32, i32, vp, i32, vp, vp], i32),
        "mx_attn_workspace_bytes": ([i32, i32, i32, i32], sz),
        "mx_attn_decode": ([vp, vp, i64, i32, vp, vp, vp, vp, C.POINTER(AttnDimsC), i32, vp, vp,
                            vp], i32),
        "mx_engine_create": ([C.POINTER(ModelConfigC), C.POINTER(vp)], i32),
        "mx_engine_destroy": ([vp], i32),
        "mx_engine_reset_slot": ([vp, i32], i32),
        "mx_engine_clone_slot": ([vp, i32, i32], i32),
        "mx_engine_offset": ([vp, i32], i32),
        "mx_engine_decode_batch": ([vp, vp, vp, i32, vp], i32),
        "mx_engine_decode_rows": ([vp, vp, vp, i32, vp], i32),
        "mx_engine_decode_batch_outputs": ([vp, vp, vp, i32, vp, vp, vp], i32),
        "mx_engine_decode_forced": ([vp, vp, vp, i32, vp, vp, vp, vp], i32),
        "mx_engine_prefill": ([vp, i32, vp, i32, vp], i32),
        "mx_engine_prefill_chunked": ([vp, i32, vp, i32, vp], i32),
        "mx_engine_verify": ([vp, i32, vp, i32, vp], i32),
        "mx_engine_commit": ([vp, i32, i32], i32),
        "mx_engine_generate": ([vp, i32, vp, i32, i32, i32, vp, vp, C.POINTER(GenerateStatsC), vp],
                               i32),
        "mx_engine_set_flags": ([vp, i32], i32),
        "mx_engine_fill_slot": ([vp, i32, i32, u64], i32),
        "mx_qmm": ([C.POINTER(QWeightC), vp, i32, vp, vp], i32),
        "mx_xq": ([C.POINTER(QWeightC), vp, i32, vp, vp], i32),
        "mx_hc_workspace_bytes": ([i32], sz),
        "mx_hc_forward_mfma": ([C.POINTER(QWeightC), C.POINTER(QWeightC), vp, vp, i32, i32, i32,
                                i32, f32, vp, vp, vp, vp], i32),
        "mx_qmm_conv": ([C.POINTER(QWeightC), vp, i32, i32, i32, vp, vp, vp, vp, i64, vp, i64, vp],
                        i32),
        "mx_head_argmax_mfma": ([C.POINTER(QWeightC), vp, i32, vp, vp, vp], i32),
        "mx_head_noalloc_max_bytes": ([], C.c_size_t),
        "mx_head_argmax_noalloc": ([C.POINTER(QWeightC), vp, i32, vp, vp], i32),
        "mx_moe_experts_mfma": ([vp, vp, vp, i32, i32, C.POINTER(QBankC), C.POINTER(QBankC),
                                 C.POINTER(QBankC), C.POINTER(QWeightC), C.POINTER(QWeightC),
                                 C.POINTER(QWeightC), vp, vp, vp], i32),
        "mx_moe_routed_experts_mfma": ([vp, i64, vp, i64, i32, vp, i32, i32, C.POINTER(QBankC),
                                        C.POINTER(QBankC), C.POINTER(QBankC),
                                        C.POINTER(QWeightC), C.POINTER(QWeightC),
                                        C.POINTER(QWeightC), vp, vp, vp, vp, vp, vp], i32),
        "mx_moe_routed_experts_hc_mfma": ([vp, i64, vp, i64, i32, vp, i32, i32, i32,
                                           C.POINTER(QBankC), C.POINTER(QBankC),
                                           C.POINTER(QBankC), C.POINTER(QWeightC),
                                           C.POINTER(QWeightC), C.POINTER(QWeightC), vp, vp, vp,
                                           vp, vp, vp, vp], i32),
        "mx_engine_profile_step": ([vp, vp, vp, i32, vp, C.POINTER(StepProfileC)], i32),
        "mx_engine_profile_verify": ([vp, i32, vp, i32, vp, C.POINTER(StepProfileC)], i32),
        "mx_engine_draft_bytes": ([vp, i32, C.POINTER(C.c_double)], i32),
        "mx_engine_read": ([vp, C.c_char_p, vp, sz], i32),
        "mx_engine_time_experts": ([vp, i32, C.POINTER(ExpertTimingC)], i32),
        "mx_sched_create": ([C.POINTER(SchedConfigC), C.POINTER(SchedBackendC), C.POINTER(vp)], i32),
        "mx_sched_create_for_engine": ([vp, C.POINTER(SchedConfigC), C.POINTER(vp)], i32),
        "mx_sched_destroy": ([vp], i32),
        "mx_sched_submit": ([vp, u64, vp, i32, i32, i32], i32),
        "mx_sched_cancel": ([vp, u64], i32),
        "mx_sched_step": ([vp, C.POINTER(SchedEventC), i32, C.POINTER(i32), C.POINTER(i32)], i32),
        "mx_sched_pending": ([vp], i32),
        "mx_sched_cached": ([vp], i32),
        "mx_engine_tensor": ([vp, C.c_char_p, C.POINTER(vp), C.POINTER(sz)], i32),
        "mx_engine_load_tensor": ([vp, C.c_char_p, i32, C.POINTER(C.c_int64), i32, vp, sz], i32),
        "mx_engine_load_safetensors": ([vp, C.c_char_p, C.POINTER(i32)], i32),
        "mx_checkpoint_target": ([C.POINTER(ModelConfigC), C.c_char_p, C.c_char_p, sz,
                                  C.POINTER(i32)], i32),
        "mx_checkpoint_check": ([C.POINTER(ModelConfigC), C.c_char_p, C.POINTER(i32)], i32),
        "mx_engine_slot_failed": ([vp, i32], i32),
        "mx_engine_inject_failure": ([vp, i32], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


lib = _load()
# tokens per chunk of mx_engine_prefill_chunked
PREFILL_CHUNK = int(lib.mx_prefill_chunk_tokens())


def check(rc: int) -> None:
    if rc != MX_OK:
        raise MxError(rc, (lib.mx_last_error() or b"").decode())


def declared_symbols(header: str) -> list[str]:
    """Names of every function the C header declares (for export checks)."""
    import re

    text = open(header).read()
    # a name followed by "(" declares a function; "mx_status (*field)" is a
    # function-pointer member of a struct
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\((?!\*)", text)))


class DeviceArray:
    """A device allocation with a numpy dtype/shape view for tests and bench."""

    def __init__(self, shape, dtype, zero: bool = False):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib.mx_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value
        if zero:
            check(lib.mx_memset(self.ptr, 0, self.nbytes, None))

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        check(lib.mx_memcpy_htod(d.ptr, a.ctypes.data, d.nbytes))
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(lib.mx_memcpy_htod(self.ptr, a.ctypes.data, self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib.mx_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib.mx_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class QWeight:
    """An affine-quantised matrix resident on the device (MLX layout)."""

    codes: DeviceArray
    scales: DeviceArray
    biases: DeviceArray
    n: int
    k: int
    bits: int
    group_size: int

    def c(self) -> QWeightC:
        return QWeightC(self.codes.ptr, self.scales.ptr, self.biases.ptr, self.n, self.k,
                        self.bits, self.group_size)

    @classmethod
    def random(cls, n: int, k: int, bits: int, gs: int, seed: int,
               s_range=(0.005, 0.03), b_range=(-0.2, 0.2)) -> "QWeight":
        """Random codes, scales ~ U(s_range), biases ~ U(b_range), on device."""
        codes = DeviceArray((n, k * bits // 32), np.uint32)
        scales = DeviceArray((n, k // gs), np.uint16)
        biases = DeviceArray((n, k // gs), np.uint16)
        check(lib.mx_fill_codes(codes.ptr, n, k, bits, seed, None))
        check(lib.mx_fill_bf16(scales.ptr, scales.nbytes // 2, seed + 1, 0, s_range[0], s_range[1], None))
        check(lib.mx_fill_bf16(biases.ptr, biases.nbytes // 2, seed + 2, 0, b_range[0], b_range[1], None))
        return cls(codes, scales, biases, n, k, bits, gs)

    def host(self):
        return self.codes.numpy(), self.scales.numpy(), self.biases.numpy()


@dataclass
class QBank:
    """A bank of equally shaped quantised expert matrices on the device."""

    codes: DeviceArray
    scales: DeviceArray
    biases: DeviceArray
    experts: int
    n: int
    k: int
    bits: int
    group_size: int

    def c(self) -> QBankC:
        return QBankC(self.codes.ptr, self.scales.ptr, self.biases.ptr, self.experts, self.n,
                      self.k, self.bits, self.group_size)

    @classmethod
    def random(cls, experts: int, n: int, k: int, bits: int, gs: int, seed: int,
               s_range=(0.005, 0.03), b_range=(-0.2, 0.2)) -> "QBank":
        """Same streams as QWeight.random of an [experts*n, k] matrix."""
        q = QWeight.random(experts * n, k, bits, gs, seed, s_range, b_range)
        return cls(q.codes, q.scales, q.biases, experts, n, k, bits, gs)

    def host(self):
        return self.codes.numpy(), self.scales.numpy(), self.biases.numpy()


def qmv(w: QWeight, x: DeviceArray, m: int, y: DeviceArray, stream=None) -> None:
    qc = w.c()
    check(lib.mx_qmv(C.byref(qc), x.ptr, m, y.ptr, stream))


def dequant_rows(w: QWeight, ids: DeviceArray, count: int, out: DeviceArray, stream=None) -> None:
    qc = w.c()
    check(lib.mx_dequant_rows(C.byref(qc), ids.ptr, count, out.ptr, stream))


def fill_bf16(d: DeviceArray, seed: int, dist: int, a: float, b: float) -> None:
    check(lib.mx_fill_bf16(d.ptr, d.nbytes // 2, seed, dist, a, b, None))


def sync() -> None:
    check(lib.mx_device_sync())


# ---- model configurations (benchmark configs 3 and 4, and a tiny test model) ----
MX_DT_U32, MX_DT_BF16, MX_DT_F16, MX_DT_F32 = 0, 1, 2, 3

CONFIG3 = dict(hidden=2048, layers=48, attn_every=4, vocab=151936, hc=4, hc_rank=256, gdn_hk=16,
               gdn_hv=32, gdn_dk=128, gdn_dv=128, conv_k=4, heads=16, kv_heads=2, head_dim=256,
               rotary_dim=64, rope_theta=1e7, rms_eps=1e-6, experts=512, top_k=10, moe_inter=512,
               shared_inter=512, bits=4, down_bits=5, embed_bits=8, head_bits=8, group_size=64,
               mixed_bits=0, max_slots=8, max_context=4096, max_verify=8, seed=20250)

def checkpoint_target(cfg: dict, name: str):
    """mx_checkpoint_target: (status, engine tensor name, info dict) for an
    MLX tensor name under configuration cfg, no device needed."""
    cc = config_c(cfg)
    buf = C.create_string_buffer(256)
    info = (C.c_int32 * 8)()
    rc = lib.mx_checkpoint_target(C.byref(cc), name.encode(), buf, 256, info)
    keys = ("kind", "part", "row0", "rows", "n", "k", "bits", "count")
    return rc, buf.value.decode(), dict(zip(keys, list(info)))


# The quantised modules of one layer by width role (0: projections,
# hyper-connections, router, expert and shared-expert gate/up; 1: expert and
# shared-expert down), as the reference names them (src/hybrid.rs:56-66,
# 130-142, 335-352, 529-567; src/mtp.rs:39-70).  The engine fuses each
# role's modules of a layer at one width.
_HC_MODULES = ("input_mix_weight_down", "input_mix_weight_up")
_ROLE0 = {
    "linear_attention": ("linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.in_proj_a",
                         "linear_attn.in_proj_b", "linear_attn.out_proj"),
    "full_attention": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                       "self_attn.o_proj"),
}
_MOE0 = ("mlp.gate", "mlp.shared_expert_gate", "mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj",
         "mlp.shared_expert.gate_proj", "mlp.shared_expert.up_proj")
_MOE1 = ("mlp.switch_mlp.down_proj", "mlp.shared_expert.down_proj")


def _layer_modules(prefix: str, kind: str):
    """(role, module prefix) of every quantised module of one layer."""
    out = []
    for hc in ("attn_hyper_connection", "mlp_hyper_connection"):
        out += [(0, f"{prefix}.{hc}.{m}") for m in _HC_MODULES + ("block_inject_weight",)]
    out += [(0, f"{prefix}.{m}") for m in _ROLE0[kind] + _MOE0]
    out += [(1, f"{prefix}.{m}") for m in _MOE1]
    return out


def config_from_mlx(config: dict, max_slots=8, max_context=4096, max_verify=8, seed=1,
                    mtp=0) -> dict:
    """Engine configuration of an MLX checkpoint's config.json (the fields
    HybridConfig reads, src/hybrid.rs; rope defaults as src/qsa.rs:35-40):
    the layer pattern must repeat k-1 linear-attention layers then one full
    attention layer.  Widths come from "quantization": its default, and the
    per-module entries that override it (src/weights.rs:70-90) for the
    embedding, the head, and each layer's width table entries
    (`layer_widths`; the MTP draft layer at index `layers`).  Raises
    ValueError naming the module when the engine cannot hold a width as
    given: two modules the engine fuses at one width differ (one width per
    layer for its projections, hyper-connections, router and expert gate/up;
    one for its expert and shared-expert down), the mixer differs from the
    default width, a module's group size differs from the default's, or the
    mode is not affine.  (The engine itself takes group size 64 only:
    mx_engine_create refuses others.)"""
    t = config.get("text_config", config)
    q = config.get("quantization") or config.get("quantization_config")
    if not q:
        raise ValueError("config.json has no quantization (the engine runs quantised weights)")
    types = t["layer_types"]
    n = t["num_hidden_layers"]
    k = types.index("full_attention") + 1
    if n % k or types != (["linear_attention"] * (k - 1) + ["full_attention"]) * (n // k):
        raise ValueError("layer pattern is not (k-1 linear attention, 1 full attention) repeated")
    if n > MAX_LAYERS:
        raise ValueError(f"{n} layers: the engine holds at most {MAX_LAYERS}")
    gs0 = q["group_size"]
    if q.get("mode", "affine") != "affine":
        raise ValueError(f"quantization mode {q.get('mode')}: the engine runs affine weights")

    def quant_of(module):
        """(bits, group size) of a module: its own entry (with or without the
        language_model. prefix) or the default."""
        for key in (module, "language_model." + module):
            e = q.get(key)
            if isinstance(e, dict):
                if e.get("mode", "affine") != "affine":
                    raise ValueError(f"{module}: quantization mode {e.get('mode')} is not affine")
                if e["group_size"] != gs0:
                    raise ValueError(f"{module}: group size {e['group_size']}, the engine uses one "
                                     f"group size for every module ({gs0})")
                return e["bits"]
        return q["bits"]

    def one_width(modules, what):
        widths = {}
        for m in modules:
            widths.setdefault(quant_of(m), m)
        if len(widths) > 1:
            (a, ma), (b, mb) = list(widths.items())[:2]
            raise ValueError(f"{what}: {ma} is {a}-bit and {mb} is {b}-bit; the engine fuses them "
                             "at one width")
        return next(iter(widths))

    table = [0] * (2 * (MAX_LAYERS + 1))
    for i in range(n):
        mods = _layer_modules(f"model.layers.{i}", types[i])
        for role in (0, 1):
            table[2 * i + role] = one_width([m for r, m in mods if r == role], f"layer {i}")
    if mtp:
        mods = _layer_modules("mtp.layers.0", "full_attention")
        extra = ["mtp.fc_embedding", "mtp.fc_hidden"] + \
            [f"mtp.hyper_connection_mixer.{m}" for m in _HC_MODULES]
        table[2 * n] = one_width([m for r, m in mods if r == 0] + extra, "MTP layer")
        table[2 * n + 1] = one_width([m for r, m in mods if r == 1], "MTP layer")
    mixer = one_width([f"model.hyper_connection_mixer.{m}" for m in _HC_MODULES], "mixer")
    if mixer != q["bits"]:
        raise ValueError(f"model.hyper_connection_mixer: {mixer}-bit, the engine runs the mixer at "
                         f"the default width ({q['bits']}-bit)")
    rope = t.get("rope_parameters") or {}
    head_dim = t["head_dim"]
    return dict(
        hidden=t["hidden_size"], layers=n, attn_every=k, vocab=t["vocab_size"], hc=t["hc_count"],
        hc_rank=t["hc_lowrank"], gdn_hk=t["linear_num_key_heads"], gdn_hv=t["linear_num_value_heads"],
        gdn_dk=t["linear_key_head_dim"], gdn_dv=t["linear_value_head_dim"],
        conv_k=t["linear_conv_kernel_dim"], heads=t["num_attention_heads"],
        kv_heads=t["num_key_value_heads"], head_dim=head_dim,
        rotary_dim=int(head_dim * rope.get("partial_rotary_factor", 0.25)),
        rope_theta=float(rope.get("rope_theta", 1e7)), rms_eps=t["rms_norm_eps"],
        experts=t["num_experts"], top_k=t["num_experts_per_tok"],
        moe_inter=t["moe_intermediate_size"], shared_inter=t["shared_expert_intermediate_size"],
        bits=q["bits"], down_bits=table[1],
        embed_bits=quant_of("model.embed_tokens"), head_bits=quant_of("lm_head"),
        group_size=gs0, mixed_bits=0, max_slots=max_slots, max_context=max_context,
        max_verify=max_verify, seed=seed, mtp=mtp, layer_widths=table)


def checkpoint_check(cfg: dict, path) -> int:
    """mx_checkpoint_check: every check of loading `path` into an engine of
    configuration cfg, without a device; returns the tensors checked
    (raises MxError naming the first failing tensor)."""
    n = C.c_int32()
    check(lib.mx_checkpoint_check(C.byref(config_c(cfg)), os.fspath(path).encode(), C.byref(n)))
    return n.value


TINY = dict(hidden=256, layers=4, attn_every=4, vocab=1024, hc=4, hc_rank=64, gdn_hk=1, gdn_hv=2,
            gdn_dk=128, gdn_dv=128, conv_k=4, heads=2, kv_heads=1, head_dim=128, rotary_dim=32,
            rope_theta=1e7, rms_eps=1e-6, experts=64, top_k=4, moe_inter=64, shared_inter=128,
            bits=4, down_bits=5, embed_bits=8, head_bits=8, group_size=64, mixed_bits=0,
            max_slots=6, max_context=600, max_verify=8, seed=77)


class Engine:
    """Host handle of an mx_engine (synchronous calls, one owning thread)."""

    def __init__(self, cfg: dict):
        self.cfg = dict(cfg)
        cc = config_c(self.cfg)
        h = C.c_void_p()
        check(lib.mx_engine_create(C.byref(cc), C.byref(h)))
        self.h = h.value

    def close(self):
        if self.h:
            lib.mx_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _u32(a):
        return np.ascontiguousarray(a, np.uint32)

    def decode_batch(self, slots, tokens, equal=True) -> np.ndarray:
        s = np.ascontiguousarray(slots, np.int32)
        t = self._u32(tokens)
        out = np.empty(len(s), np.uint32)
        fn = lib.mx_engine_decode_batch if equal else lib.mx_engine_decode_rows
        check(fn(self.h, s.ctypes.data, t.ctypes.data, len(s), out.ctypes.data))
        return out

    def decode_batch_outputs(self, slots, tokens, logits=True, hidden=True):
        """mx_engine_decode_batch_outputs: (next tokens, bf16 logits [rows, vocab]
        or None, bf16 hidden streams [rows, hc*hidden] or None)."""
        s = np.ascontiguousarray(slots, np.int32)
        t = self._u32(tokens)
        rows = len(s)
        out = np.empty(rows, np.uint32)
        c = self.cfg
        lg = DeviceArray((rows, c["vocab"]), np.uint16) if logits else None
        hd = DeviceArray((rows, c["hc"] * c["hidden"]), np.uint16) if hidden else None
        check(lib.mx_engine_decode_batch_outputs(self.h, s.ctypes.data, t.ctypes.data, rows,
                                                 out.ctypes.data, lg.ptr if lg else None,
                                                 hd.ptr if hd else None))
        return out, (lg.numpy() if lg else None), (hd.numpy() if hd else None)

    def decode_forced(self, slots, tokens, h_in):
        """mx_engine_decode_forced: h_in bf16 [layers + 1, rows, hc*hidden];
        returns (next tokens, per-layer outputs [layers, rows, hc*hidden],
        per-layer expert ids [layers, rows, top_k])."""
        s = np.ascontiguousarray(slots, np.int32)
        t = self._u32(tokens)
        rows = len(s)
        c = self.cfg
        h_in = np.ascontiguousarray(h_in, np.uint16)
        assert h_in.shape == (c["layers"] + 1, rows, c["hc"] * c["hidden"]), h_in.shape
        h_out = np.empty((c["layers"], rows, c["hc"] * c["hidden"]), np.uint16)
        ids = np.empty((c["layers"], rows, c["top_k"]), np.uint32)
        out = np.empty(rows, np.uint32)
        check(lib.mx_engine_decode_forced(self.h, s.ctypes.data, t.ctypes.data, rows,
                                          h_in.ctypes.data, h_out.ctypes.data, ids.ctypes.data,
                                          out.ctypes.data))
        return out, h_out, ids

    def prefill(self, slot, tokens, chunked=False) -> int:
        """Feeds tokens to a slot; returns the greedy token after the last one.
        chunked: mx_engine_prefill_chunked (512-token chunks on the matrix
        cores, within tolerance of the exact 8-token blocks)."""
        t = self._u32(tokens)
        out = np.empty(1, np.uint32)
        fn = lib.mx_engine_prefill_chunked if chunked else lib.mx_engine_prefill
        check(fn(self.h, slot, t.ctypes.data, len(t), out.ctypes.data))
        return int(out[0])

    def verify(self, slot, tokens) -> np.ndarray:
        t = self._u32(tokens)
        out = np.empty(len(t), np.uint32)
        check(lib.mx_engine_verify(self.h, slot, t.ctypes.data, len(t), out.ctypes.data))
        return out

    def commit(self, slot, keep):
        check(lib.mx_engine_commit(self.h, slot, keep))

    def generate(self, slot, prompt, max_tokens, depth=0):
        """Greedy generation from an empty slot (mx_engine_generate): returns
        (tokens, {"rounds", "drafted", "accepted", "drafts"})."""
        t = self._u32(prompt)
        out = np.empty(max_tokens, np.uint32)
        n = C.c_int32(0)
        st = GenerateStatsC()
        drafts = np.empty(max(max_tokens * depth, 1), np.uint32)
        check(lib.mx_engine_generate(self.h, slot, t.ctypes.data, len(t), max_tokens, depth,
                                     out.ctypes.data, C.byref(n), C.byref(st), drafts.ctypes.data))
        return out[:n.value].copy(), {"rounds": st.rounds, "drafted": st.drafted,
                                      "accepted": st.accepted,
                                      "drafts": drafts[:st.drafted].copy()}

    def reset(self, slot):
        check(lib.mx_engine_reset_slot(self.h, slot))

    def clone(self, src, dst):
        check(lib.mx_engine_clone_slot(self.h, src, dst))

    def fill_slot(self, slot, length, seed=1):
        check(lib.mx_engine_fill_slot(self.h, slot, length, seed))

    def offset(self, slot) -> int:
        return lib.mx_engine_offset(self.h, slot)

    def slot_failed(self, slot) -> bool:
        """mx_engine_slot_failed: a failed step left this slot's caches partly updated."""
        return lib.mx_engine_slot_failed(self.h, slot) == 1

    def inject_failure(self, after_layers):
        """mx_engine_inject_failure (test hook): the next step stops with
        MX_EHIP after launching `after_layers` layers (eager mode)."""
        check(lib.mx_engine_inject_failure(self.h, after_layers))

    def profile_step(self, slots, tokens):
        """One eager decode step with per-layer expert-kernel timing."""
        s = np.ascontiguousarray(slots, np.int32)
        t = self._u32(tokens)
        out = np.empty(len(s), np.uint32)
        prof = StepProfileC()
        check(lib.mx_engine_profile_step(self.h, s.ctypes.data, t.ctypes.data, len(s),
                                         out.ctypes.data, C.byref(prof)))
        return out, {f: getattr(prof, f) for f, _ in StepProfileC._fields_}

    def profile_verify(self, slot, tokens):
        """One eager verify block with per-layer expert-kernel timing; the
        profile's step_bytes are the block's algorithmic bytes."""
        t = self._u32(tokens)
        out = np.empty(len(t), np.uint32)
        prof = StepProfileC()
        check(lib.mx_engine_profile_verify(self.h, slot, t.ctypes.data, len(t), out.ctypes.data,
                                           C.byref(prof)))
        return out, {f: getattr(prof, f) for f, _ in StepProfileC._fields_}

    def draft_bytes(self, pos) -> float:
        """Algorithmic bytes of one MTP draft step at cache position pos."""
        b = C.c_double(0.0)
        check(lib.mx_engine_draft_bytes(self.h, pos, C.byref(b)))
        return b.value

    def time_experts(self, rows):
        """Expert kernels of all MoE layers back to back (totals and bytes)."""
        t = ExpertTimingC()
        check(lib.mx_engine_time_experts(self.h, rows, C.byref(t)))
        return {f: getattr(t, f) for f, _ in ExpertTimingC._fields_}

    # components for set_flags(exact_parts=...): run exact while the rest stays fast
    EX_HC, EX_GDN_PROJ, EX_GDN, EX_ATTN_PROJ, EX_ATTN, EX_MOE, EX_HEAD = 1, 2, 4, 8, 16, 32, 64

    def set_flags(self, logits=False, eager=False, exact=False, exact_parts=0,
                  chunked_generate=False):
        check(lib.mx_engine_set_flags(self.h, (1 if logits else 0) | (2 if eager else 0)
                                      | (4 if exact else 0) | (exact_parts << 3)
                                      | (1024 if chunked_generate else 0)))

    def read(self, what: str, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(lib.mx_engine_read(self.h, what.encode(), out.ctypes.data, out.nbytes))
        return out

    def tensor_bytes(self, name: str) -> int:
        p, n = C.c_void_p(), C.c_size_t()
        check(lib.mx_engine_tensor(self.h, name.encode(), C.byref(p), C.byref(n)))
        return n.value

    # numpy dtype of a checkpoint array -> MX_DT_*; uint16 arrays carry bf16 bits
    _DT = {np.dtype(np.uint32): MX_DT_U32, np.dtype(np.uint16): MX_DT_BF16,
           np.dtype(np.float16): MX_DT_F16, np.dtype(np.float32): MX_DT_F32}

    def load_tensor(self, name: str, array: np.ndarray, raise_on_error=True) -> int:
        """mx_engine_load_tensor of one MLX-named checkpoint array; returns the
        status (raises on error unless raise_on_error is False)."""
        a = np.ascontiguousarray(array)
        shape = (C.c_int64 * a.ndim)(*a.shape)
        rc = lib.mx_engine_load_tensor(self.h, name.encode(), self._DT[a.dtype], shape, a.ndim,
                                       a.ctypes.data, a.nbytes)
        if raise_on_error:
            check(rc)
        return rc

    def load_safetensors(self, path: str) -> int:
        """mx_engine_load_safetensors: every tensor of the file; returns the count."""
        n = C.c_int32()
        check(lib.mx_engine_load_safetensors(self.h, os.fspath(path).encode(), C.byref(n)))
        return n.value


class Scheduler:
    """Host handle of an mx_sched: the equal-offset serving loop over an Engine
    (engine=...) or over a backend given as Python callables (prefill(slot,
    tokens) -> next, decode(slots, tokens) -> nexts, clone(src, dst))."""

    def __init__(self, batch_size, slots, max_context, prefix_entries=0, prefix_tokens=0,
                 stop=(), engine=None, prefill=None, decode=None, clone=None):
        stop = list(stop)
        cfg = SchedConfigC(batch_size, slots, prefix_entries, prefix_tokens, max_context,
                           len(stop), (C.c_uint32 * 8)(*stop))
        h = C.c_void_p()
        self._keep = None
        if engine is not None:
            check(lib.mx_sched_create_for_engine(engine.h, C.byref(cfg), C.byref(h)))
        else:
            def pf(ctx, slot, toks, n, out):
                try:
                    out[0] = int(prefill(slot, [toks[i] for i in range(n)]))
                    return MX_OK
                except Exception:
                    return 1

            def dc(ctx, slots_p, toks, n, out):
                try:
                    nxt = decode([slots_p[i] for i in range(n)], [toks[i] for i in range(n)])
                    for i in range(n):
                        out[i] = int(nxt[i])
                    return MX_OK
                except Exception:
                    return 5

            def cl(ctx, src, dst):
                try:
                    clone(src, dst)
                    return MX_OK
                except Exception:
                    return 1

            be = SchedBackendC(None, SCHED_PREFILL(pf), SCHED_DECODE(dc), SCHED_CLONE(cl))
            self._keep = be
            check(lib.mx_sched_create(C.byref(cfg), C.byref(be), C.byref(h)))
        self.h = h.value
        self.batch_size = batch_size

    def submit(self, job, prompt, max_tokens, prefix_cache=True):
        p = np.ascontiguousarray(prompt, np.uint32)
        check(lib.mx_sched_submit(self.h, job, p.ctypes.data if len(p) else None, len(p),
                                  max_tokens, int(prefix_cache)))

    def cancel(self, job) -> bool:
        return lib.mx_sched_cancel(self.h, job) == MX_OK

    def step(self):
        cap = 4 * self.batch_size
        ev = (SchedEventC * cap)()
        n, rows = C.c_int32(), C.c_int32()
        check(lib.mx_sched_step(self.h, ev, cap, C.byref(n), C.byref(rows)))
        return [(e.job, e.token, e.kind, e.detail) for e in ev[: n.value]], rows.value

    def pending(self) -> int:
        return lib.mx_sched_pending(self.h)

    def cached(self) -> int:
        return lib.mx_sched_cached(self.h)

    def close(self):
        if self.h:
            lib.mx_sched_destroy(self.h)
            self.h = None

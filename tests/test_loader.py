"""Checkpoint loading on the CPU, against the reference's own end-to-end
fixture (tests/fixtures/hybrid, copied byte for byte into tests/golden/hybrid
by copy_hybrid_fixture.py: config.json and the safetensors tensor names,
dtypes and shapes):
  * the engine configuration from config.json (rust_mlx_amd.config_from_mlx);
  * where every fixture tensor goes (mx_checkpoint_target, the mapping that
    mx_engine_load_tensor applies): its shape matches the engine matrix's
    rows and packed / per-group widths, the rows of each fused engine matrix
    (GDN qkv | z | a | b, router | shared gate, HC down | inject, attention
    q | k | v) are covered exactly once, and only the modules the engine
    does not build (per-layer n-gram embeddings, the attention indexer) are
    refused.  The fixture's fp32 (unquantised) embedding maps to the
    embedding's codes and is refused at load time (codes must be U32)."""
import json
import os
import struct
from collections import defaultdict

import numpy as np

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture():
    d = os.path.join(HERE, "golden", "hybrid")
    with open(os.path.join(d, "config.json")) as f:
        config = json.load(f)
    with open(os.path.join(d, "model.safetensors"), "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
    header.pop("__metadata__", None)
    tensors = {k: {"dtype": v["dtype"], "shape": v["shape"]} for k, v in header.items()}
    return {"config": config, "tensors": tensors}


def test_config_from_the_reference_fixture(mx):
    cfg = mx.config_from_mlx(fixture()["config"], max_context=64, seed=5)
    want = dict(hidden=128, layers=4, attn_every=4, vocab=256, hc=4, hc_rank=32, gdn_hk=2,
                gdn_hv=4, gdn_dk=32, gdn_dv=32, conv_k=4, heads=4, kv_heads=2, head_dim=32,
                rotary_dim=8, rope_theta=1e7, rms_eps=1e-6, experts=8, top_k=2, moe_inter=64,
                shared_inter=64, bits=4, down_bits=4, embed_bits=4, head_bits=4, group_size=32)
    for k, v in want.items():
        assert cfg[k] == v, (k, cfg[k], v)
    assert cfg["max_context"] == 64 and cfg["seed"] == 5 and cfg["mtp"] == 0


def test_config_rejects_what_the_engine_cannot_build(mx):
    c = fixture()["config"]
    bad = json.loads(json.dumps(c))
    bad["text_config"]["layer_types"] = ["linear_attention", "full_attention",
                                         "linear_attention", "full_attention"][::-1]
    with pytest.raises(ValueError):
        mx.config_from_mlx(bad)
    bad = json.loads(json.dumps(c))
    del bad["quantization"]
    with pytest.raises(ValueError):
        mx.config_from_mlx(bad)


def test_per_module_widths_override_the_default(mx):
    c = json.loads(json.dumps(fixture()["config"]))
    c["quantization"]["language_model.lm_head"] = {"bits": 8, "group_size": 32}
    for m in ("switch_mlp.down_proj", "shared_expert.down_proj"):
        c["quantization"][f"language_model.model.layers.0.mlp.{m}"] = {"bits": 5, "group_size": 32}
    cfg = mx.config_from_mlx(c)
    assert cfg["head_bits"] == 8 and cfg["down_bits"] == 5 and cfg["embed_bits"] == 4
    w = cfg["layer_widths"]
    assert w[:8] == [4, 5, 4, 4, 4, 4, 4, 4] and not any(w[8:])


def _layer_modules(mx, i, kind):
    return [m for _, m in mx._layer_modules(f"language_model.model.layers.{i}", kind)]


def test_every_layer_width_comes_from_its_modules(mx):
    """Each layer's table entries come from its modules' entries; the table
    drives the engine's per-layer widths (mx_checkpoint_target reads it)."""
    c = json.loads(json.dumps(fixture()["config"]))
    q = c["quantization"]
    types = c["text_config"]["layer_types"]
    for m in _layer_modules(mx, 2, types[2]):
        q[m] = {"bits": 8 if "down_proj" not in m else 6, "group_size": 32}
    for m in _layer_modules(mx, 3, types[3]):
        if "down_proj" in m:
            q[m] = {"bits": 5, "group_size": 32}
    cfg = mx.config_from_mlx(c)
    assert cfg["layer_widths"][4:8] == [8, 6, 4, 5]
    rc, _, t = mx.checkpoint_target(cfg, "language_model.model.layers.2.linear_attn.in_proj_z.weight")
    assert rc == 0 and t["bits"] == 8
    rc, _, t = mx.checkpoint_target(cfg, "language_model.model.layers.2.mlp.switch_mlp.down_proj.scales")
    assert rc == 0 and t["bits"] == 6
    rc, _, t = mx.checkpoint_target(cfg, "language_model.model.layers.3.mlp.shared_expert.down_proj.weight")
    assert rc == 0 and t["bits"] == 5
    rc, _, t = mx.checkpoint_target(cfg, "language_model.model.layers.3.attn_hyper_connection.input_mix_weight_up.weight")
    assert rc == 0 and t["bits"] == 4


@pytest.mark.parametrize("case", ["fused-differ", "group-size", "mixer", "mode"])
def test_widths_the_engine_cannot_hold_are_refused_by_name(mx, case):
    c = json.loads(json.dumps(fixture()["config"]))
    q = c["quantization"]
    if case == "fused-differ":      # one module of the fused GDN input projection at 8 bits
        q["language_model.model.layers.1.linear_attn.in_proj_z"] = {"bits": 8, "group_size": 32}
        want = "in_proj_z"
    elif case == "group-size":
        q["language_model.model.layers.0.mlp.gate"] = {"bits": 4, "group_size": 64}
        want = "mlp.gate"
    elif case == "mixer":
        for m in ("input_mix_weight_down", "input_mix_weight_up"):
            q[f"language_model.model.hyper_connection_mixer.{m}"] = {"bits": 8, "group_size": 32}
        want = "hyper_connection_mixer"
    else:
        q["mode"] = "mxfp4"
        want = "mode"
    with pytest.raises(ValueError, match=want):
        mx.config_from_mlx(c)


def test_every_fixture_tensor_maps_at_its_own_shape(mx):
    fx = fixture()
    cfg = mx.config_from_mlx(fx["config"])
    gs = cfg["group_size"]
    covered = defaultdict(list)  # (engine tensor, part) -> row ranges
    refused = []
    for name, meta in fx["tensors"].items():
        rc, tensor, info = mx.checkpoint_target(cfg, name)
        if rc != mx.MX_OK:
            assert rc == mx.MX_EUNSUPPORTED, (name, rc)
            refused.append(name)
            continue
        shape = meta["shape"]
        count = int(np.prod(shape))
        if meta["dtype"] == "F32" and name.endswith("embed_tokens.weight"):
            continue  # unquantised: refused when loaded (the engine's embedding is quantised)
        if info["kind"] == 0:
            rows = count // shape[-1]
            assert rows == info["rows"], (name, rows, info)
            want = info["k"] * info["bits"] // 32 if info["part"] == 0 else info["k"] // gs
            assert shape[-1] == want, (name, shape, info)
            assert meta["dtype"] == "U32" or info["part"] != 0
            covered[(tensor, info["part"])].append((info["row0"], info["rows"], info["n"]))
        else:
            assert count == info["count"], (name, shape, info)
            if info["kind"] == 3:
                assert shape == [info["count"] // cfg["conv_k"], cfg["conv_k"], 1]
    assert all("ple." in n or ".indexer." in n for n in refused), refused
    assert len(refused) == 22
    for key, ranges in covered.items():
        n = ranges[0][2]
        hit = np.zeros(n, np.int64)
        for r0, rows, _ in ranges:
            hit[r0:r0 + rows] += 1
        assert (hit == 1).all(), (key, ranges)
    fused = {t for (t, _), r in covered.items() if len(r) > 1}
    assert {"layers.0.gdn.in", "layers.3.attn.in", "layers.0.moe.router", "layers.0.attn_hc.down",
            "layers.3.mlp_hc.down"} <= fused


def test_unknown_and_absent_modules_are_reported(mx):
    cfg = mx.config_from_mlx(fixture()["config"])
    assert mx.checkpoint_target(cfg, "language_model.model.layers.0.linear_attn.q_proj.weight")[0] \
        == mx.MX_EINVAL  # a GDN layer has no q_proj
    assert mx.checkpoint_target(cfg, "language_model.model.layers.9.mlp.gate.weight")[0] == mx.MX_EINVAL
    assert mx.checkpoint_target(cfg, "mtp.fc_hidden.weight")[0] == mx.MX_EUNSUPPORTED  # no mtp
    cfg["mtp"] = 1
    rc, t, info = mx.checkpoint_target(cfg, "mtp.layers.0.self_attn.q_proj.weight")
    assert rc == mx.MX_OK and t == "mtp.layer.attn.in" and info["row0"] == 0


# ---- whole files, checked without a device (mx_checkpoint_check) -----------
def _tiny_file(mx, tmp_path, widths=None, name="m.safetensors", **write_kw):
    from mlx_ckpt import synth_checkpoint, write_safetensors

    base = dict(mx.TINY, mtp=0)
    T, config = synth_checkpoint(base, 3, widths)
    cfg = mx.config_from_mlx(config, max_slots=2, max_context=64, seed=9)
    path = tmp_path / name
    n = write_safetensors(path, T, **write_kw)
    return cfg, T, path, n


def test_a_mixed_width_file_passes_every_check(mx, tmp_path):
    cfg, T, path, n = _tiny_file(mx, tmp_path, widths={0: (8, 6), 3: (5, 8)})
    assert cfg["layer_widths"][:8] == [8, 6, 4, 5, 4, 5, 5, 8]
    assert mx.checkpoint_check(cfg, path) == n
    # the same file under a configuration with other widths is refused by name
    other = dict(cfg, layer_widths=[4, 5] * 4)
    with pytest.raises(mx.MxError, match="layers.0.+8-bit codes, the engine's matrix is 4-bit"):
        mx.checkpoint_check(other, path)


def _edit(name_part, fn):
    def edit(header):
        for k, v in header.items():
            if name_part in k:
                fn(v)
                return
        raise AssertionError(name_part)
    return edit


@pytest.mark.parametrize("case,match", [
    ("zero-dim", "dim 0"),
    ("negative-dim", "dim -3"),
    ("huge-offset", "outside the file"),
    ("negative-begin", "outside the file"),
    ("end-before-begin", "outside the file"),
    ("truncated", "outside the file"),
    ("header-past-end", "not a safetensors file"),
    ("bad-header", "unreadable header"),
    ("bytes-mismatch", "byte count does not match"),
    ("dtype", "unsupported dtype"),
])
def test_malformed_files_are_refused_without_a_crash(mx, tmp_path, case, match):
    """Offsets, dims and header length are checked against the file before
    anything is read or allocated (a malformed checkpoint returns an error
    naming the tensor; it never aborts the process)."""
    edit = {
        "zero-dim": _edit("lm_head.scales", lambda v: v.__setitem__("shape", [0, 4])),
        "negative-dim": _edit("lm_head.scales", lambda v: v.__setitem__("shape", [-3, 4])),
        "huge-offset": _edit("lm_head.scales", lambda v: v.__setitem__("data_offsets",
                                                                        [0, 2**62])),
        "negative-begin": _edit("lm_head.scales", lambda v: v.__setitem__(
            "data_offsets", [-64, v["data_offsets"][1]])),
        "end-before-begin": _edit("lm_head.scales", lambda v: v.__setitem__(
            "data_offsets", [v["data_offsets"][1], v["data_offsets"][0]])),
        "bytes-mismatch": _edit("lm_head.scales", lambda v: v.__setitem__(
            "data_offsets", [v["data_offsets"][0], v["data_offsets"][1] - 2])),
        "dtype": _edit("lm_head.scales", lambda v: v.__setitem__("dtype", "I64")),
    }.get(case)
    cfg, T, path, n = _tiny_file(mx, tmp_path, header_edit=edit)
    raw = path.read_bytes()
    if case == "truncated":
        path.write_bytes(raw[:-100])
    elif case == "header-past-end":
        path.write_bytes(struct.pack("<Q", len(raw)) + raw[8:])
    elif case == "bad-header":
        hlen = struct.unpack("<Q", raw[:8])[0]
        path.write_bytes(raw[:8] + b"{" + b"x" * (hlen - 1) + raw[8 + hlen:])
    with pytest.raises(mx.MxError, match=match):
        mx.checkpoint_check(cfg, path)


def test_float_values_are_kept_exactly_or_refused(mx, tmp_path):
    """bf16 tensors of the engine (scales, biases, norm weights) take F32 /
    F16 values only when bf16 holds them exactly: a float32 scale that would
    round is refused with the tensor's name, never rounded silently."""
    name = "language_model.model.layers.0.mlp.switch_mlp.gate_proj.scales"
    cfg, T, path, n = _tiny_file(mx, tmp_path, dtypes={name: "F32"})
    assert mx.checkpoint_check(cfg, path) == n            # F32 holding bf16 values
    cfg, T, path, n = _tiny_file(mx, tmp_path, dtypes={name: "F16"}, name="f16.safetensors")
    T2 = dict(T)
    bad = T2[name].copy()
    bad.reshape(-1)[5] = np.float32(0.01234567)           # not a bf16 value
    T2[name] = bad
    from mlx_ckpt import write_safetensors

    p2 = tmp_path / "inexact.safetensors"
    write_safetensors(p2, T2, dtypes={name: "F32"})
    with pytest.raises(mx.MxError, match="gate_proj.scales: value 0.0123456698 at index 5 is not a bf16"):
        mx.checkpoint_check(cfg, p2)
    norm = "language_model.model.layers.0.linear_attn.norm.weight"
    T3 = dict(T)
    T3[norm] = T[norm] + np.float32(1e-4)
    p3 = tmp_path / "norm.safetensors"
    write_safetensors(p3, T3, dtypes={norm: "F32"})
    with pytest.raises(mx.MxError, match="norm.weight"):
        mx.checkpoint_check(cfg, p3)
    # fp32 engine tensors (A_log) take any float32 value
    a = "language_model.model.layers.0.linear_attn.A_log"
    T4 = dict(T)
    T4[a] = T[a] + np.float32(1e-6)
    p4 = tmp_path / "alog.safetensors"
    assert mx.checkpoint_check(cfg, p4 if write_safetensors(p4, T4) else p4) == n


def test_the_engine_takes_group_size_64_only(mx, tmp_path):
    """The reference also loads group sizes 32 and 128 (src/weights.rs:83-86);
    the engine's exact-integer kernels combine 64-value groups, so another
    group size is refused before anything is loaded (and the fixture, at
    group size 32 with an unquantised embedding, is refused)."""
    cfg, T, path, n = _tiny_file(mx, tmp_path)
    with pytest.raises(mx.MxError, match="group_size must be 64"):
        mx.checkpoint_check(dict(cfg, group_size=32), path)
    fx = mx.config_from_mlx(fixture()["config"])
    assert fx["group_size"] == 32
    with pytest.raises(mx.MxError):
        mx.checkpoint_check(fx, os.path.join(HERE, "golden", "hybrid", "model.safetensors"))

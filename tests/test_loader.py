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
    c["quantization"]["language_model.model.layers.0.mlp.switch_mlp.down_proj"] = {
        "bits": 5, "group_size": 32}
    cfg = mx.config_from_mlx(c)
    assert cfg["head_bits"] == 8 and cfg["down_bits"] == 5 and cfg["embed_bits"] == 4


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

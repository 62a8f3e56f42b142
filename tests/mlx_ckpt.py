"""Synthetic MLX-format checkpoints of the engine's model, for tests: tensors
under the reference's names (src/hybrid.rs:56-66, 130-142, 335-352, 529-567;
src/mtp.rs:39-70) in MLX's affine layout, a config.json with per-module
quantization entries (src/weights.rs:70-90), a .safetensors writer, and the
engine tensors the same names map to through mx_checkpoint_target (the
oracle's fetch)."""
import json
import struct

import numpy as np


def bf16(a):
    """float32 values rounded to bf16 (round to nearest even), as float32."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


def synth_checkpoint(cfg, seed, widths=None):
    """(tensors by MLX name, config.json) of a random model of the engine
    configuration cfg; float values are bf16.  widths: {layer: (bits,
    down_bits)} for layers (index cfg["layers"]: the MTP layer) whose
    modules are quantised at other widths than cfg's base ones; they appear
    as per-module quantization entries."""
    rng = np.random.default_rng(seed)
    widths = widths or {}
    H, hc, r, gs = cfg["hidden"], cfg["hc"], cfg["hc_rank"], cfg["group_size"]
    T = {}
    quant_over = {}

    def quant(p, n, k, bits, lead=(), gain=1.0, kscale=True):
        T[p + ".weight"] = rng.integers(0, 2**32, size=lead + (n, k * bits // 32),
                                        dtype=np.uint64).astype(np.uint32)
        s = gain * np.sqrt(12.0) / ((np.sqrt(k) if kscale else 1.0) * 2**bits)
        sc = bf16(s * rng.uniform(0.75, 1.25, size=lead + (n, k // gs)))
        T[p + ".scales"] = sc
        T[p + ".biases"] = bf16(-sc * (2**bits - 1) / 2 + sc * rng.normal(0, 0.1, size=sc.shape))
        if bits != cfg["bits"]:
            quant_over[p] = {"bits": bits, "group_size": gs}

    def vec(p, shape, mean, std):
        T[p] = bf16(mean + std * rng.normal(size=shape))

    def hcw(p, layer_bits, inject):
        vec(p + ".hc_norm.weight", (hc * H,), 0.0, 0.1)
        quant(p + ".input_mix_weight_down", r, hc * H, layer_bits, gain=2.0)
        quant(p + ".input_mix_weight_up", hc * H, r, layer_bits)
        if inject:
            quant(p + ".block_inject_weight", hc, hc * H, layer_bits, gain=2.0)

    def moe(p, bits, dbits):
        E, I, SI = cfg["experts"], cfg["moe_inter"], cfg["shared_inter"]
        quant(p + ".gate", E, H, bits, gain=3.0)
        quant(p + ".shared_expert_gate", 1, H, bits)
        quant(p + ".switch_mlp.gate_proj", I, H, bits, lead=(E,))
        quant(p + ".switch_mlp.up_proj", I, H, bits, lead=(E,))
        quant(p + ".switch_mlp.down_proj", H, I, dbits, lead=(E,))
        quant(p + ".shared_expert.gate_proj", SI, H, bits)
        quant(p + ".shared_expert.up_proj", SI, H, bits)
        quant(p + ".shared_expert.down_proj", H, SI, dbits)

    def attn(p, bits):
        hd = cfg["head_dim"]
        quant(p + ".q_proj", cfg["heads"] * 2 * hd, H, bits)
        quant(p + ".k_proj", cfg["kv_heads"] * hd, H, bits)
        quant(p + ".v_proj", cfg["kv_heads"] * hd, H, bits)
        quant(p + ".o_proj", H, cfg["heads"] * hd, bits)
        vec(p + ".q_norm.weight", (hd,), 0.0, 0.1)
        vec(p + ".k_norm.weight", (hd,), 0.0, 0.1)

    base = (cfg["bits"], cfg["down_bits"])
    lm = "language_model.model."
    quant("language_model.model.embed_tokens", cfg["vocab"], H, cfg["embed_bits"], kscale=False)
    quant("language_model.lm_head", cfg["vocab"], H, cfg["head_bits"])
    hcw(lm + "hyper_connection_mixer", cfg["bits"], False)
    hk, hv, dk, dv = cfg["gdn_hk"], cfg["gdn_hv"], cfg["gdn_dk"], cfg["gdn_dv"]
    types = []
    for i in range(cfg["layers"]):
        bits, dbits = widths.get(i, base)
        p = f"{lm}layers.{i}"
        full = i % cfg["attn_every"] == cfg["attn_every"] - 1
        types.append("full_attention" if full else "linear_attention")
        hcw(p + ".attn_hyper_connection", bits, True)
        hcw(p + ".mlp_hyper_connection", bits, True)
        if full:
            attn(p + ".self_attn", bits)
        else:
            g = p + ".linear_attn"
            cd = 2 * hk * dk + hv * dv
            quant(g + ".in_proj_qkv", cd, H, bits)
            quant(g + ".in_proj_z", hv * dv, H, bits)
            quant(g + ".in_proj_a", hv, H, bits)
            quant(g + ".in_proj_b", hv, H, bits)
            quant(g + ".out_proj", H, hv * dv, bits)
            T[g + ".conv1d.weight"] = bf16(rng.normal(0, 0.5, size=(cd, cfg["conv_k"], 1)))
            T[g + ".A_log"] = rng.uniform(-1.0, 1.0, size=(hv,)).astype(np.float32)
            T[g + ".dt_bias"] = bf16(rng.uniform(0.0, 1.0, size=(hv,)))
            vec(g + ".norm.weight", (dv,), 1.0, 0.1)
        moe(p + ".mlp", bits, dbits)
    if cfg.get("mtp"):
        bits, dbits = widths.get(cfg["layers"], base)
        p = "mtp.layers.0"
        hcw(p + ".attn_hyper_connection", bits, True)
        hcw(p + ".mlp_hyper_connection", bits, True)
        attn(p + ".self_attn", bits)
        moe(p + ".mlp", bits, dbits)
        vec("mtp.pre_fc_norm_embedding.weight", (H,), 0.0, 0.1)
        vec("mtp.pre_fc_norm_hidden.weight", (hc * H,), 0.0, 0.1)
        quant("mtp.fc_embedding", H, H, bits)
        quant("mtp.fc_hidden", H, H, bits)
        hcw("mtp.hyper_connection_mixer", bits, False)
    text = dict(hidden_size=H, num_hidden_layers=cfg["layers"], hc_count=hc, hc_lowrank=r,
                num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv_heads"],
                head_dim=cfg["head_dim"], linear_num_key_heads=hk, linear_num_value_heads=hv,
                linear_key_head_dim=dk, linear_value_head_dim=dv,
                linear_conv_kernel_dim=cfg["conv_k"], num_experts=cfg["experts"],
                num_experts_per_tok=cfg["top_k"], moe_intermediate_size=cfg["moe_inter"],
                shared_expert_intermediate_size=cfg["shared_inter"], rms_norm_eps=cfg["rms_eps"],
                vocab_size=cfg["vocab"], layer_types=types, ngram_size=3, eos_token_id=cfg["vocab"] - 1,
                rope_parameters=dict(rope_theta=cfg["rope_theta"],
                                     partial_rotary_factor=cfg["rotary_dim"] / cfg["head_dim"]))
    config = {"text_config": text,
              "quantization": dict(bits=cfg["bits"], group_size=gs, mode="affine", **quant_over)}
    return T, config


def engine_tensors(mx, cfg, T):
    """The engine's tensors (oracle fetch names) assembled from the MLX ones by
    mx_checkpoint_target."""
    out = {}
    gs = cfg["group_size"]
    u16 = lambda a: (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    for name, a in T.items():
        rc, tensor, t = mx.checkpoint_target(cfg, name)
        assert rc == 0, (name, rc)
        kind = t["kind"]
        if kind == 0:                                   # quantised rows
            a2 = a.reshape(-1, a.shape[-1])
            assert a2.shape[0] == t["rows"], (name, a2.shape, t)
            part = t["part"]
            suffix = (".codes", ".scales", ".biases")[part]
            width = t["k"] * t["bits"] // 32 if part == 0 else t["k"] // gs
            dt = np.uint32 if part == 0 else np.uint16
            buf = out.setdefault(tensor + suffix, np.zeros((t["n"], width), dt))
            assert a2.shape[1] == width, (name, a2.shape, width)
            buf[t["row0"]:t["row0"] + t["rows"]] = a2 if part == 0 else u16(a2)
        elif kind == 1:                                 # bf16 vector
            assert a.size == t["count"], name
            out[tensor] = u16(a.reshape(-1))
        elif kind == 2:                                 # fp32 vector
            out[tensor] = np.ascontiguousarray(a, np.float32).reshape(-1)
        else:                                           # conv [C, K, 1] -> [K][C]
            out[tensor] = np.ascontiguousarray(a[:, :, 0].T, np.float32)
    return out


def make_fetch(E):
    def fetch(name, dtype, shape):
        a = E[name]
        assert a.dtype == np.dtype(dtype) and a.size == int(np.prod(shape)), (name, a.shape, shape)
        return np.ascontiguousarray(a.reshape(shape))
    return fetch


def st_dtype(name, a):
    """The dtype an MLX checkpoint stores: packed codes U32, A_log F32, other
    float tensors BF16 (their values are bf16)."""
    if a.dtype == np.uint32:
        return "U32"
    return "F32" if name.endswith("A_log") else "BF16"


def write_safetensors(path, tensors, dtypes=None, header_edit=None):
    """A .safetensors file of named arrays (float32 arrays written as BF16,
    F16 or F32 per st_dtype / dtypes[name]); header_edit(header) may change
    the JSON header before it is written (malformed-file tests)."""
    header, blobs, off = {}, [], 0
    dtypes = dtypes or {}
    for name, a in tensors.items():
        dt = dtypes.get(name) or st_dtype(name, a)
        if dt == "BF16":
            raw = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
        elif dt == "F16":
            raw = np.ascontiguousarray(a, np.float16)
        elif dt == "F32":
            raw = np.ascontiguousarray(a, np.float32)
        else:
            raw = np.ascontiguousarray(a, np.uint32)
        header[name] = {"dtype": dt, "shape": list(raw.shape), "data_offsets": [off, off + raw.nbytes]}
        blobs.append(raw.tobytes())
        off += raw.nbytes
    if header_edit:
        header_edit(header)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for blob in blobs:
            f.write(blob)
    return len(tensors)

"""Float32 restatement of the reference's hybrid text model over MLX-named
checkpoint tensors.  TEST INFRASTRUCTURE ONLY: used by tests/ as the checker
of the oracle's model composition, never by the product.

It restates, in numpy float32 and in the reference's own tensor names:
  HybridModel::forward_hidden / forward      src/hybrid.rs:594-685
  grouped_norm, HyperConnection              src/hybrid.rs:39-104
  MoE::parts / forward_write (softmax, top-k, normalised scores, shared
    expert times sigmoid gate)               src/hybrid.rs:192-300
  Gdn::forward_reference, gdn_reference      src/hybrid.rs:369-495
  Qsa::forward, dense (nblocks <= budget/ratio) and sparse (indexer block
    scores, top budget/ratio blocks + causal tail)   src/qsa.rs:66-176
  Attention::forward_selection (gated: q|gate split, norm, text RoPE,
    causal SDPA, sigmoid output gate)        src/dense.rs:139-270
  text RoPE                                  src/rope.rs:8-28, kernels/text_rope.metal
  Ple::forward_embedding, NGramHasher::rows  src/ple.rs:63-123, src/ngram.rs:326-360
  Mtp::forward                               src/mtp.rs:72-127
  compiled graphs (silu, swiglu, decay, norm, activate, injection, mix)
                                             src/compiled.rs:7-81
  Linear / embedding (affine dequantise, then x @ W^T)
                                             src/weights.rs:70-90, 184-226

Pinned by the reference's end-to-end fixture tests/fixtures/hybrid (prefill
logits within 1e-4 and its greedy tokens, as src/bin/hybrid-parity.rs checks;
a copy lives under tests/golden/hybrid), including the decode steps after
the QSA indexer has switched to sparse block selection.
Mtp.forward has no fixture in the reference: parity unpinned (its
composition is restated from src/mtp.rs:72-127 and cross-checked against the
oracle's draft step only).
"""
from __future__ import annotations

import json
import os

import numpy as np

F32 = np.float32


# ---------------------------------------------------------------- weights --
def unpack_codes(words: np.ndarray, bits: int) -> np.ndarray:
    """MLX affine codes: value j of a row occupies bits [j*bits, j*bits+bits)
    of the row's little-endian bitstream (one u32 word after another)."""
    words = np.ascontiguousarray(words, dtype="<u4")
    lead = words.shape[:-1]
    raw = np.unpackbits(words.view(np.uint8).reshape(*lead, -1), axis=-1, bitorder="little")
    k = raw.shape[-1] // bits
    raw = raw[..., : k * bits].reshape(*lead, k, bits).astype(np.uint32)
    return (raw << np.arange(bits, dtype=np.uint32)).sum(axis=-1).astype(F32)


def dequantize(w, scales, biases, bits, gs) -> np.ndarray:
    """w = scale * q + bias per group of gs values (MLX affine mode)."""
    q = unpack_codes(w, bits)
    lead = q.shape[:-1]
    q = q.reshape(*lead, -1, gs)
    s = np.asarray(scales, F32)[..., None]
    b = np.asarray(biases, F32)[..., None] if biases is not None else 0
    return (q * s + b).astype(F32).reshape(*lead, -1)


class Weights:
    """Tensors by MLX name (float tensors as float32), plus config.json."""

    def __init__(self, tensors: dict, config: dict):
        self.t = tensors
        self.config = config

    @classmethod
    def load_dir(cls, path: str):
        from safetensors.numpy import load_file
        with open(os.path.join(path, "config.json")) as f:
            config = json.load(f)
        tensors = {}
        for name in sorted(os.listdir(path)):
            if name.endswith(".safetensors"):
                tensors.update(load_file(os.path.join(path, name)))
        return cls(tensors, config)

    def tensor(self, name):
        a = self.t[name]
        return a.astype(F32) if a.dtype.kind == "f" else a

    def has(self, name):
        return name in self.t

    def quantization(self, prefix):
        """src/weights.rs:70-90: per-module entry, else the global one."""
        if prefix + ".scales" not in self.t:
            return None
        q = self.config.get("quantization") or self.config.get("quantization_config")
        q = q.get(prefix, q)
        return int(q["bits"]), int(q["group_size"])

    def linear(self, prefix):
        """Dequantised float32 weight [.., n, k] and the optional additive bias."""
        w = self.t[prefix + ".weight"]
        q = self.quantization(prefix)
        if q is not None:
            b = self.t.get(prefix + ".biases")
            W = dequantize(w, self.tensor(prefix + ".scales"),
                           self.tensor(prefix + ".biases") if b is not None else None, *q)
        else:
            W = np.asarray(w, F32)
        bias = self.t.get(prefix + ".bias")
        return W, (None if bias is None else np.asarray(bias, F32))


def lin(x, Wb):
    W, b = Wb
    y = (x.astype(F32) @ W.T).astype(F32)
    return y if b is None else (y + b).astype(F32)


# ------------------------------------------------------------ elementwise --
def sigmoid(x):
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-x.astype(F32)))).astype(F32)


def silu(x):
    return (x * sigmoid(x)).astype(F32)


def norm(x, scale, eps):
    """compiled::norm: x * rsqrt(mean(x^2) + eps) * (scale + 1) over the last axis."""
    x = x.astype(F32)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + F32(eps))
    return (x * inv.astype(F32) * (scale.astype(F32) + 1.0)).astype(F32)


def rms_norm(x, w, eps):
    """fast::rms_norm: x * rsqrt(mean(x^2) + eps) * w."""
    x = x.astype(F32)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + F32(eps))
    return (x * inv.astype(F32) * w.astype(F32)).astype(F32)


def grouped_norm(x, scale, hc, eps):
    """src/hybrid.rs:39-44: norm over each of the hc streams of width d."""
    s = x.shape
    d = s[-1] // hc
    return norm(x.reshape(*s[:-1], hc, d), scale.reshape(hc, d), eps).reshape(s)


def softplus(x):
    return np.logaddexp(x.astype(F32), F32(0)).astype(F32)


# ------------------------------------------------------- hyper-connection --
class HyperConnection:
    def __init__(self, w: Weights, p, hc, eps, inject):
        self.scale = w.tensor(p + ".hc_norm.weight")
        self.down = w.linear(p + ".input_mix_weight_down")
        self.up = w.linear(p + ".input_mix_weight_up")
        self.inject = w.linear(p + ".block_inject_weight") if inject else None
        self.hc, self.eps = hc, eps

    def forward(self, x):
        """(mixed [.., d], inject [.., hc] or None): src/hybrid.rs:78-99."""
        hc = self.hc
        xn = grouped_norm(x, self.scale, hc, self.eps)
        lo = silu(lin(xn, self.down) / F32(hc))                       # activate
        p = lin(lo, self.up)
        s = x.shape
        mixed = np.mean(sigmoid(p).reshape(*s[:-1], hc, s[-1] // hc)
                        * xn.reshape(*s[:-1], hc, s[-1] // hc), axis=-2).astype(F32)  # mix
        inj = None
        if self.inject is not None:
            inj = (sigmoid(lin(xn, self.inject) / F32(hc)) * F32(2)).astype(F32)  # injection
        return mixed, inj

    def write(self, x, y, gate):
        """x[.., hc, d] + y[.., 1, d] * gate[.., hc, 1]: src/hybrid.rs:100-104."""
        s = x.shape
        hc = self.hc
        return (x.reshape(*s[:-1], hc, s[-1] // hc)
                + y[..., None, :] * gate[..., :, None]).astype(F32).reshape(s)


# -------------------------------------------------------------------- MoE --
class MoE:
    def __init__(self, w: Weights, p, top_k):
        self.router = w.linear(p + ".gate")
        self.gate = w.linear(p + ".switch_mlp.gate_proj")
        self.up = w.linear(p + ".switch_mlp.up_proj")
        self.down = w.linear(p + ".switch_mlp.down_proj")
        self.sgate = w.linear(p + ".shared_expert.gate_proj")
        self.sup = w.linear(p + ".shared_expert.up_proj")
        self.sdown = w.linear(p + ".shared_expert.down_proj")
        self.shared_gate = w.linear(p + ".shared_expert_gate")
        self.top_k = top_k
        self.last_ids = None

    def forward(self, x):
        """y + shared * sigmoid(shared gate): src/hybrid.rs:192-291 with the
        default policies (softmax, the top_k largest gates, scores divided by
        their sum)."""
        lead = x.shape[:-1]
        xr = x.reshape(-1, x.shape[-1])
        logits = lin(xr, self.router)
        g = np.exp(logits - logits.max(-1, keepdims=True)).astype(F32)
        g = (g / g.sum(-1, keepdims=True)).astype(F32)
        ids = np.argsort(-g, axis=-1, kind="stable")[:, : self.top_k]
        sc = np.take_along_axis(g, ids, -1)
        sc = (sc / sc.sum(-1, keepdims=True)).astype(F32)
        self.last_ids = ids
        y = np.zeros_like(xr)
        for r in range(xr.shape[0]):
            for j in range(self.top_k):
                e = ids[r, j]
                a = xr[r] @ self.gate[0][e].T
                u = xr[r] @ self.up[0][e].T
                y[r] += (silu(a) * u) @ self.down[0][e].T * sc[r, j]
        shared = lin(silu(lin(xr, self.sgate)) * lin(xr, self.sup), self.sdown)
        factor = sigmoid(lin(xr, self.shared_gate))
        return (y + shared * factor).astype(F32).reshape(*lead, -1)


# -------------------------------------------------------------------- GDN --
class Gdn:
    def __init__(self, w: Weights, p, c):
        self.qkv = w.linear(p + ".in_proj_qkv")
        self.z = w.linear(p + ".in_proj_z")
        self.a = w.linear(p + ".in_proj_a")
        self.b = w.linear(p + ".in_proj_b")
        self.out = w.linear(p + ".out_proj")
        self.conv = w.tensor(p + ".conv1d.weight")[:, :, 0]          # [C, K]
        self.alog = w.tensor(p + ".A_log")
        self.dt = w.tensor(p + ".dt_bias")
        self.normw = w.tensor(p + ".norm.weight")
        self.hk, self.hv = c["linear_num_key_heads"], c["linear_num_value_heads"]
        self.dk, self.dv = c["linear_key_head_dim"], c["linear_value_head_dim"]
        self.kernel, self.eps = c["linear_conv_kernel_dim"], c["rms_norm_eps"]

    def new_cache(self):
        cd = 2 * self.hk * self.dk + self.hv * self.dv
        return {"conv": np.zeros((self.kernel - 1, cd), F32),
                "state": np.zeros((self.hv, self.dv, self.dk), F32)}

    def forward(self, x, cache):
        """x [t, H] of one sequence: src/hybrid.rs:369-452."""
        t = x.shape[0]
        kd, vd = self.hk * self.dk, self.hv * self.dv
        qkv = lin(x, self.qkv)
        inp = np.concatenate([cache["conv"], qkv], 0)
        cache["conv"] = inp[inp.shape[0] - self.kernel + 1:].copy()
        K = self.kernel
        conv = np.stack([(inp[i:i + K] * self.conv.T).sum(0) for i in range(t)]).astype(F32)
        conv = silu(conv)
        q = conv[:, :kd].reshape(t, self.hk, self.dk)
        k = conv[:, kd:2 * kd].reshape(t, self.hk, self.dk)
        v = conv[:, 2 * kd:].reshape(t, self.hv, self.dv)
        eps = F32(1e-6)
        q = (q / np.sqrt((q * q).sum(-1, keepdims=True) + eps) * F32(self.dk ** -0.5)).astype(F32)
        k = (k / np.sqrt((k * k).sum(-1, keepdims=True) + eps)).astype(F32)
        beta = sigmoid(lin(x, self.b))
        g = np.exp(-np.exp(self.alog) * softplus(lin(x, self.a) + self.dt)).astype(F32)  # decay
        # gdn_reference (src/hybrid.rs:457-495): value head h reads key head h / (hv/hk)
        rep = self.hv // self.hk
        S = cache["state"]
        ys = np.empty((t, self.hv, self.dv), F32)
        for ti in range(t):
            for h in range(self.hv):
                kh, qh = k[ti, h // rep], q[ti, h // rep]
                S[h] = S[h] * g[ti, h]
                mem = S[h] @ kh
                delta = (v[ti, h] - mem) * beta[ti, h]
                S[h] = S[h] + delta[:, None] * kh[None, :]
                ys[ti, h] = S[h] @ qh
        z = lin(x, self.z).reshape(t, self.hv, self.dv)
        y = rms_norm(ys, self.normw, self.eps) * sigmoid(z)
        return lin(y.reshape(t, vd).astype(F32), self.out)


# -------------------------------------------------------------- attention --
def rope_text(x, rot, theta, offset, stride=1):
    """x [heads, t, d] at positions (offset + i) * stride, i < t
    (runtime_prepare::positions, src/runtime_prepare.rs:61-66); the first rot
    values rotate as two halves (src/rope.rs:8-57, kernels/text_rope.metal)."""
    half = rot // 2
    inv = (F32(1.0) / np.power(F32(theta), np.arange(0, rot, 2, dtype=F32) / F32(rot))).astype(F32)
    pos = (np.arange(offset, offset + x.shape[1]) * stride).astype(F32)
    ang = (pos[:, None] * inv[None, :]).astype(F32)
    c, s = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
    y = x.copy()
    a, b = x[..., :half], x[..., half:rot]
    y[..., :half] = a * c - b * s
    y[..., half:rot] = b * c + a * s
    return y.astype(F32)


class Attention:
    """Qsa in its dense regime around the gated Attention."""

    def __init__(self, w: Weights, p, c):
        self.q = w.linear(p + ".q_proj")
        self.k = w.linear(p + ".k_proj")
        self.v = w.linear(p + ".v_proj")
        self.o = w.linear(p + ".o_proj")
        self.qn = w.tensor(p + ".q_norm.weight")
        self.kn = w.tensor(p + ".k_norm.weight")
        self.heads, self.kvh, self.hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        rp = c.get("rope_parameters") or {}
        self.theta = float(rp.get("rope_theta", 1e7))
        self.rot = int(self.hd * float(rp.get("partial_rotary_factor", 0.25)))
        self.eps = c["rms_norm_eps"]
        self.budget = c.get("indexer_budget")
        self.ratio = c.get("indexer_compress_ratio")
        self.index = None
        if w.has(p + ".indexer.index_qk_proj.weight"):
            # Qsa::load (src/qsa.rs:35-64): the indexer's q|k projection and norms
            self.index = w.linear(p + ".indexer.index_qk_proj")
            self.iqs = w.tensor(p + ".indexer.q_layernorm.weight")
            self.iks = w.tensor(p + ".indexer.k_layernorm.weight")
            self.ih, self.idim = c["indexer_n_heads"], c["indexer_head_dim"]

    def new_cache(self):
        return {"k": np.zeros((self.kvh, 0, self.hd), F32),
                "v": np.zeros((self.kvh, 0, self.hd), F32), "offset": 0, "len": 0,
                "raw": None, "blocks": None}

    def index_mask(self, x, cache):
        """Qsa::forward's indexer (src/qsa.rs:66-176) for rows x [t, H] at the
        cache's offset: the boolean attention mask [t, L] over all L cached
        positions, or None while the regime is dense (nblocks <= budget /
        ratio: plain causal attention).  Raw keys (the projection's last head)
        accumulate every step; each complete block of `ratio` raw keys is
        averaged, normed and rotated at position block * ratio once; a query's
        block score is sum over indexer heads of relu(q . block) / sqrt(dim);
        a row attends to its top budget / ratio complete blocks plus its own
        incomplete tail (causal) once more than budget / ratio blocks are
        complete, else causally."""
        t, ratio, d = x.shape[0], self.ratio, self.idim
        offset = cache["offset"]
        qk = lin(x, self.index).reshape(t, self.ih + 1, d)
        raw = qk[:, self.ih]
        cache["raw"] = raw.copy() if cache["raw"] is None else np.concatenate([cache["raw"], raw], 0)
        raw = cache["raw"]
        L = raw.shape[0]
        nb, topk = L // ratio, self.budget // ratio
        if nb <= topk:
            return None
        q = norm(qk[:, :self.ih], self.iqs, self.eps).transpose(1, 0, 2)    # [ih, t, d]
        q = rope_text(q, self.rot, self.theta, offset)
        old = 0 if cache["blocks"] is None else cache["blocks"].shape[0]
        if nb > old:
            new = raw[old * ratio:nb * ratio].astype(F32).reshape(nb - old, ratio, d).mean(1)
            new = norm(new.astype(F32), self.iks, self.eps)
            new = rope_text(new[None], self.rot, self.theta, old, ratio)[0]
            cache["blocks"] = new if cache["blocks"] is None else np.concatenate([cache["blocks"], new], 0)
        blocks = cache["blocks"]
        scores = (np.maximum((q @ blocks.T).astype(F32), F32(0)).sum(0)
                  / F32(np.sqrt(F32(d)))).astype(F32)                          # [t, nb]
        ends = offset + 1 + np.arange(t)
        complete = ends // ratio
        valid = np.arange(nb)[None, :] < complete[:, None]
        scores = np.where(valid, scores, -np.inf)
        selected = np.argpartition(scores, -topk, axis=-1)[:, -topk:]
        chosen = np.zeros((t, nb), bool)
        np.put_along_axis(chosen, selected, True, axis=-1)
        token_blocks = np.minimum(np.arange(L) // ratio, nb - 1)
        ids = np.arange(L)[None, :]
        tail = ids >= (complete * ratio)[:, None]
        causal = ids < ends[:, None]
        sparse = (chosen[:, token_blocks] | tail) & causal
        return np.where((complete > topk)[:, None], sparse, causal)

    def forward(self, x, cache, rope_offset=None):
        t = x.shape[0]
        cache["len"] += t
        allowed = None
        if self.index is not None:
            allowed = self.index_mask(x, cache)
        elif self.budget and cache["len"] // self.ratio > self.budget // self.ratio:
            raise NotImplementedError("the sparse QSA regime needs the indexer's tensors")
        H, hd = self.heads, self.hd
        qg = lin(x, self.q).reshape(t, H, 2, hd)
        q, gate = qg[:, :, 0], qg[:, :, 1]
        k = lin(x, self.k).reshape(t, self.kvh, hd)
        v = lin(x, self.v).reshape(t, self.kvh, hd).transpose(1, 0, 2)
        q = norm(q, self.qn, self.eps).transpose(1, 0, 2)
        k = norm(k, self.kn, self.eps).transpose(1, 0, 2)
        off = cache["offset"] if rope_offset is None else rope_offset
        q = rope_text(q, self.rot, self.theta, off)
        k = rope_text(k, self.rot, self.theta, off)
        cache["k"] = np.concatenate([cache["k"], k], 1)
        cache["v"] = np.concatenate([cache["v"], v], 1)
        old = cache["offset"]
        cache["offset"] += t
        Kc, Vc = cache["k"], cache["v"]
        rep = H // self.kvh
        out = np.empty((t, H, hd), F32)
        for h in range(H):
            sc = (q[h] @ Kc[h // rep].T * F32(hd ** -0.5)).astype(F32)   # [t, L]
            L = Kc.shape[1]
            if allowed is None:
                allowed = np.arange(L)[None, :] <= (old + np.arange(t))[:, None]
            sc = np.where(allowed, sc, -np.inf)
            p = np.exp(sc - sc.max(-1, keepdims=True))
            p = (p / p.sum(-1, keepdims=True)).astype(F32)
            out[:, h] = p @ Vc[h // rep]
        y = out.reshape(t, H * hd) * sigmoid(gate.reshape(t, H * hd))
        return lin(y.astype(F32), self.o)


# -------------------------------------------------------------------- PLE --
class Ple:
    def __init__(self, w: Weights, p, c, eos):
        self.key = w.linear(p + ".key_proj")
        self.value = w.linear(p + ".value_proj")
        self.nk = w.tensor(p + ".norm_key.weight")
        self.nq = w.tensor(p + ".norm_query.weight")
        self.nc = w.tensor(p + ".norm_conv.weight")
        self.conv = w.tensor(p + ".conv1d.weight")[:, :, 0]          # [D, K]
        ep = p + ".ple_embedding"
        shards = []
        i = 0
        while w.has(f"{ep}.ngram_embedding.shards.{i}.weight"):
            pre = f"{ep}.ngram_embedding.shards.{i}"
            q = w.quantization(pre)
            if q is None:
                shards.append(w.tensor(pre + ".weight"))
            else:
                shards.append(dequantize(w.t[pre + ".weight"], w.tensor(pre + ".scales"),
                                         w.tensor(pre + ".biases"), *q))
            i += 1
        self.table = np.concatenate(shards, 0).astype(F32)
        sc = f"{ep}.ngram_embedding.weight_scale"
        self.table_scale = w.tensor(sc) if w.has(sc) else None
        self.mult = [int(v) for v in w.t[ep + ".layer_multipliers"]]
        self.offsets = [int(v) for v in w.t[ep + ".ngram_heads_offsets"]]
        self.sizes = [int(v) for v in w.t[ep + ".ngram_heads_vocab_sizes"]]
        self.ngram, self.heads, self.eos = c["ngram_size"], c["heads_per_ngram"], eos
        self.hc, self.hidden, self.eps = c["hc_count"], c["hidden_size"], c["rms_norm_eps"]
        self.kernel, self.dilation = c["ple_conv_kernel_size"], c["ngram_size"]
        self.embed = c["ple_embed_dim"]

    def rows(self, tokens, history):
        """NGramHasher::rows (src/ngram.rs:326-360): n-gram contexts cut at
        the first end-of-sequence token, u64 wrapping multiply/xor mixing."""
        M = (1 << 64) - 1
        stream = list(history) + list(tokens)
        out = []
        for t in range(len(history), len(stream)):
            ctx = [stream[t]]
            cut = False
            for ago in range(1, self.ngram):
                raw = stream[t - ago] if t - ago >= 0 else None
                cut = cut or raw is None or raw == self.eos
                ctx.append(self.eos if cut else raw)
            mixed = (ctx[0] * (self.mult[0] & M)) & M
            for n in range(2, self.ngram + 1):
                mixed ^= (ctx[n - 1] * (self.mult[n - 1] & M)) & M
                for head in range(self.heads):
                    h = (n - 2) * self.heads + head
                    out.append(mixed % self.sizes[h] + self.offsets[h])
        return out

    def new_cache(self):
        return {"conv": np.zeros(((self.kernel - 1) * self.dilation, self.hc * self.hidden), F32)}

    def forward(self, x, tokens, history, cache):
        """src/ple.rs:63-123 on x [t, hc*H]."""
        t = x.shape[0]
        emb = self.table[np.asarray(self.rows(tokens, history), np.int64)].reshape(t, self.embed)
        if self.table_scale is not None:
            emb = (emb * self.table_scale).astype(F32)
        hc, H = self.hc, self.hidden
        key = grouped_norm(lin(emb, self.key), self.nk, hc, self.eps).reshape(t, hc, H)
        query = grouped_norm(x, self.nq, hc, self.eps).reshape(t, hc, H)
        gate = ((key * query).sum(-1, keepdims=True) / F32(np.sqrt(F32(H)))).astype(F32)
        gate = (np.sign(gate) * np.sqrt(np.maximum(np.abs(gate), F32(1e-6)))).astype(F32)
        gated = (sigmoid(gate) * lin(emb, self.value)[:, None, :]).reshape(t, hc * H).astype(F32)
        normed = grouped_norm(gated, self.nc, hc, self.eps)
        hist = (self.kernel - 1) * self.dilation
        inp = np.concatenate([cache["conv"], normed], 0)
        cache["conv"] = inp[inp.shape[0] - hist:].copy()
        conv = np.stack([sum(inp[i + j * self.dilation] * self.conv[:, j] for j in range(self.kernel))
                         for i in range(t)]).astype(F32)
        return (x + (gated + silu(conv))).astype(F32)


# ------------------------------------------------------------------ model --
class HybridModel:
    def __init__(self, w: Weights, prefix="language_model."):
        c = w.config.get("text_config", w.config)
        self.c, self.w = c, w
        hc, eps = c["hc_count"], c["rms_norm_eps"]
        self.hc, self.H = hc, c["hidden_size"]
        mp = prefix + "model."
        self.embedding = w.linear(mp + "embed_tokens")
        self.head = w.linear(prefix + "lm_head")
        self.mixer = HyperConnection(w, mp + "hyper_connection_mixer", hc, eps, False)
        eos = int(c.get("eos_token_id", 248044))
        self.layers, self.ple = [], []
        for i, kind in enumerate(c["layer_types"]):
            p = f"{mp}layers.{i}"
            L = {"attn_hc": HyperConnection(w, p + ".attn_hyper_connection", hc, eps, True),
                 "mlp_hc": HyperConnection(w, p + ".mlp_hyper_connection", hc, eps, True),
                 "moe": MoE(w, p + ".mlp", c["num_experts_per_tok"])}
            L["mixer"] = (Gdn(w, p + ".linear_attn", c) if kind == "linear_attention"
                          else Attention(w, p + ".self_attn", c))
            self.layers.append(L)
            self.ple.append(Ple(w, p + ".ple", c, eos) if w.has(p + ".ple.key_proj.weight") else None)
        self.reset()

    def reset(self):
        self.caches = [L["mixer"].new_cache() for L in self.layers]
        self.ple_caches = [p.new_cache() if p is not None else None for p in self.ple]
        self.history = []
        self.offset = 0

    def embed(self, tokens):
        W, _ = self.embedding
        return W[np.asarray(tokens, np.int64)]

    def forward_hidden(self, tokens):
        """(mixed [t, H], hidden streams [t, hc*H]) of one more chunk of
        tokens; keeps self.layer_in (each layer's input streams)."""
        assert len(tokens) > 0
        t = len(tokens)
        h = np.repeat(self.embed(tokens)[:, None, :], self.hc, axis=1).reshape(t, -1).astype(F32)
        self.layer_in = []
        self.routes = []
        for i, L in enumerate(self.layers):
            if self.ple[i] is not None:
                h = self.ple[i].forward(h, tokens, self.history, self.ple_caches[i])
            self.layer_in.append(h.copy())
            mixed, inj = L["attn_hc"].forward(h)
            branch = L["mixer"].forward(mixed, self.caches[i])
            h = L["attn_hc"].write(h, branch, inj)
            mixed, inj = L["mlp_hc"].forward(h)
            h = L["mlp_hc"].write(h, L["moe"].forward(mixed), inj)
            self.routes.append(L["moe"].last_ids)
        self.layer_in.append(h.copy())
        self.history = (self.history + list(tokens))[-(self.c["ngram_size"] - 1):]
        self.offset += t
        mixed = self.mixer.forward(h)[0]
        return mixed, h

    def forward(self, tokens):
        mixed, h = self.forward_hidden(tokens)
        return lin(mixed, self.head), h


class Mtp:
    """Mtp::forward (src/mtp.rs:72-127), parity unpinned (no reference fixture)."""

    def __init__(self, w: Weights, model: HybridModel):
        c = model.c
        hc, eps = c["hc_count"], c["rms_norm_eps"]
        p = "mtp.layers.0"
        self.norm_emb = w.tensor("mtp.pre_fc_norm_embedding.weight")
        self.norm_hid = w.tensor("mtp.pre_fc_norm_hidden.weight")
        self.fc_emb = w.linear("mtp.fc_embedding")
        self.fc_hid = w.linear("mtp.fc_hidden")
        self.attn = Attention(w, p + ".self_attn", c)
        self.attn_hc = HyperConnection(w, p + ".attn_hyper_connection", hc, eps, True)
        self.mlp_hc = HyperConnection(w, p + ".mlp_hyper_connection", hc, eps, True)
        self.moe = MoE(w, p + ".mlp", c["num_experts_per_tok"])
        self.mixer = HyperConnection(w, "mtp.hyper_connection_mixer", hc, eps, False)
        self.hc, self.H, self.eps = hc, c["hidden_size"], eps
        self.cache = self.attn.new_cache()

    def forward(self, embedding, previous_hidden, position):
        """embedding [t, H], previous_hidden [t, hc*H] -> (mixed [t, H], hidden)."""
        t = embedding.shape[0]
        e = lin(norm(embedding, self.norm_emb, self.eps), self.fc_emb)
        h = norm(previous_hidden, self.norm_hid, self.eps).reshape(t, self.hc, self.H)
        h = lin(h, self.fc_hid)
        h = (e[:, None, :] + h).reshape(t, self.hc * self.H).astype(F32)
        mixed, inj = self.attn_hc.forward(h)
        h = self.attn_hc.write(h, self.attn.forward(mixed, self.cache, rope_offset=position), inj)
        mixed, inj = self.mlp_hc.forward(h)
        h = self.mlp_hc.write(h, self.moe.forward(mixed), inj)
        return self.mixer.forward(h)[0], h

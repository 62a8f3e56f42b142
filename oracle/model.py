"""CPU restatement of the engine's model step (the checker for end-to-end
parity).  TEST INFRASTRUCTURE ONLY: used by tests/ and smoke(), never by the
product.

It follows HybridModel::forward_hidden (reference src/hybrid.rs:594-685) layer
by layer with the oracle's C primitives, in the same arithmetic order as the
engine's exact mode, so tokens, hidden states and caches agree bit for bit.
Every projection is the exact-integer affine projection (oracle/xq.c, the
engine's int8 matrix-core kernels): weights are viewed with mode XQ.
Weights are read from the engine under test (fetch(name, dtype, shape)); the
caches are the oracle's own numpy arrays.

The composition (which stream feeds which projection; injections, gates,
shared expert, caches, mixer; the draft layer) is checked against the float32
restatement oracle/hybrid.py -- itself pinned by the reference's end-to-end
fixture -- on one synthetic MLX checkpoint mapped through
mx_checkpoint_target (tests/test_oracle_composition.py).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import oracle as orc

_p = orc._p


def rope_table(max_ctx: int, rot: int, theta: float):
    """inv_freq = 1 / powf(theta, 2i/rot) in fp32 (reference src/rope.rs:20-24);
    angle = the fp32 product pos * inv_freq (kernels/text_rope.metal); cos/sin
    of that angle rounded to fp32 (libm, in C)."""
    half = rot // 2
    cs = np.empty((max_ctx, half), np.float32)
    sn = np.empty((max_ctx, half), np.float32)
    orc.lib.mxo_rope_table(max_ctx, rot, theta, _p(cs), _p(sn))
    return cs, sn


class Model:
    def __init__(self, cfg: dict, fetch, only_layers=None):
        """only_layers: load and run just these layer indices (a bounded CPU
        sample of a large model); None runs the whole stack."""
        self.c = c = dict(cfg)
        self.fetch = fetch
        self.mode = orc.XQ
        H, hc = c["hidden"], c["hc"]
        self.H, self.hc = H, hc
        self.cd = 2 * c["gdn_hk"] * 128 + c["gdn_hv"] * 128
        self.vd = c["gdn_hv"] * 128
        self.P = self.cd + self.vd + 2 * c["gdn_hv"]
        self.Q = c["heads"] * 2 * c["head_dim"] + 2 * c["kv_heads"] * c["head_dim"]
        self.attn = [(i % c["attn_every"]) == c["attn_every"] - 1 for i in range(c["layers"])]
        self.cache_index = []
        ng = na = 0
        for a in self.attn:
            self.cache_index.append(na if a else ng)
            na, ng = (na + 1, ng) if a else (na, ng + 1)
        self.n_gdn, self.n_attn = ng, na
        self._keep = []
        self.embed = self._qw("embed", c["vocab"], H, c["embed_bits"])
        self.head = self._qw("head", c["vocab"], H, c["head_bits"])
        self.mixer = self._hc("mixer", -1, False)
        self.layers = []
        self.layer_ids = list(range(c["layers"])) if only_layers is None else list(only_layers)
        for i in self.layer_ids:
            self.layers.append(self._load_layer(f"layers.{i}", i, self.attn[i]))
        # the MTP draft layer (src/mtp.rs:39-70): its tensors are drawn as layer
        # index `layers`; its KV plane follows the model's attention layers
        self.mtp = None
        if c.get("mtp"):
            m = c["layers"]
            bits = self.layer_bits(m)[0]
            self.mtp = {
                "layer": self._load_layer("mtp.layer", m, True),
                "norm_emb": fetch("mtp.norm_emb", np.uint16, (H,)),
                "norm_hid": fetch("mtp.norm_hidden", np.uint16, (hc * H,)),
                "fc_emb": self._qw("mtp.fc_emb", H, H, bits),
                "fc_hid": self._qw("mtp.fc_hidden", H, H, bits),
                "mixer": self._hc("mtp.mixer", m, False),
                "cache": self.n_attn,
            }
            self._keep += [self.mtp["norm_emb"], self.mtp["norm_hid"]]
        self.n_kv = self.n_attn + (1 if self.mtp is not None else 0)
        S = c["max_slots"]
        self.state = np.zeros((S * self.n_gdn, c["gdn_hv"], 128, 128), np.float32)
        self.conv = np.zeros((S * self.n_gdn, c["conv_k"] - 1, self.cd), np.uint16)
        self.kv_slot_stride = self.n_kv * c["kv_heads"] * c["max_context"] * c["head_dim"]
        self.k = np.zeros(S * self.kv_slot_stride, np.uint16)
        self.v = np.zeros(S * self.kv_slot_stride, np.uint16)
        self.offsets = [0] * S
        self.cos, self.sin = rope_table(c["max_context"], c["rotary_dim"], c["rope_theta"])
        self.hidden = None

    # ---- weights ----
    def layer_bits(self, i):
        """(projection bits, expert-down bits) of layer i: a checkpoint's width
        table entry (layer_widths, nonzero), else the base widths, or with
        mixed_bits a seeded draw from {4,5,6,8} (same rule as the engine)."""
        table = self.c.get("layer_widths") or []

        def width(w):
            if i >= 0 and 2 * i + w < len(table) and table[2 * i + w]:
                return int(table[2 * i + w])
            if not self.c.get("mixed_bits") or i < 0:
                return (self.c["bits"], self.c["down_bits"])[w]
            key = (self.c["seed"] ^ 0x5BD1E995) & (2**64 - 1)
            return (4, 5, 6, 8)[orc.lib.mxo_rng_u64(key, i * 2 + w) & 3]
        return width(0), width(1)

    def _load_layer(self, p, i, attn):
        c, H, fetch = self.c, self.H, self.fetch
        L = {"attn_hc": self._hc(p + ".attn_hc", i, True), "mlp_hc": self._hc(p + ".mlp_hc", i, True)}
        bits, dbits = self.layer_bits(i)
        if not attn:
            L["in"] = self._qw(p + ".gdn.in", self.P, H, bits)
            L["conv_w"] = fetch(p + ".gdn.conv_w", np.float32, (c["conv_k"], self.cd))
            L["a_log"] = fetch(p + ".gdn.a_log", np.float32, (c["gdn_hv"],))
            L["dt"] = fetch(p + ".gdn.dt_bias", np.uint16, (c["gdn_hv"],))
            L["norm"] = fetch(p + ".gdn.norm", np.uint16, (128,))
            L["out"] = self._qw(p + ".gdn.out", H, self.vd, bits)
        else:
            L["in"] = self._qw(p + ".attn.in", self.Q, H, bits)
            L["q_norm"] = fetch(p + ".attn.q_norm", np.uint16, (c["head_dim"],))
            L["k_norm"] = fetch(p + ".attn.k_norm", np.uint16, (c["head_dim"],))
            L["out"] = self._qw(p + ".attn.out", H, c["heads"] * c["head_dim"], bits)
        E, I, SI = c["experts"], c["moe_inter"], c["shared_inter"]
        L["router"] = self._qw(p + ".moe.router", E + 1, H, bits)
        L["gate"] = self._bank(p + ".moe.gate", E, I, H, bits)
        L["up"] = self._bank(p + ".moe.up", E, I, H, bits)
        L["down"] = self._bank(p + ".moe.down", E, H, I, dbits)
        L["sgate"] = self._qw(p + ".moe.shared_gate", SI, H, bits)
        L["sup"] = self._qw(p + ".moe.shared_up", SI, H, bits)
        L["sdown"] = self._qw(p + ".moe.shared_down", H, SI, dbits)
        return L

    def _qw(self, name, n, k, bits):
        gs = self.c["group_size"]
        codes = self.fetch(name + ".codes", np.uint32, (n, k * bits // 32))
        s = self.fetch(name + ".scales", np.uint16, (n, k // gs))
        b = self.fetch(name + ".biases", np.uint16, (n, k // gs))
        self._keep += [codes, s, b]
        return orc.qw(codes, s, b, n, k, bits, gs, self.mode)

    def _bank(self, name, E, n, k, bits):
        gs = self.c["group_size"]
        codes = self.fetch(name + ".codes", np.uint32, (E * n, k * bits // 32))
        s = self.fetch(name + ".scales", np.uint16, (E * n, k // gs))
        b = self.fetch(name + ".biases", np.uint16, (E * n, k // gs))
        self._keep += [codes, s, b]
        return orc.qbank(codes, s, b, E, n, k, bits, gs, self.mode)

    def _hc(self, p, layer, inject):
        c = self.c
        bits = self.layer_bits(layer)[0] if layer >= 0 else c["bits"]
        scale = self.fetch(p + ".scale", np.uint16, (c["hc"] * c["hidden"],))
        self._keep.append(scale)
        down = self._qw(p + ".down", c["hc_rank"] + (c["hc"] if inject else 0), c["hc"] * c["hidden"], bits)
        up = self._qw(p + ".up", c["hc"] * c["hidden"], c["hc_rank"], bits)
        return {"scale": scale, "down": down, "up": up, "inject": inject}

    # ---- pieces ----
    def _hc_forward(self, w, h, rows):
        c = self.c
        xn = np.empty_like(h)
        orc.lib.mxo_hc_norm(_p(h), _p(w["scale"]), rows, c["hc"], c["hidden"], c["rms_eps"], _p(xn))
        lo = np.empty((rows, c["hc_rank"]), np.uint16)
        inj = np.empty((rows, c["hc"]), np.uint16)
        orc.lib.mxo_hc_down(C.byref(w["down"]), _p(xn), rows, c["hc_rank"], c["hc"], _p(lo), _p(inj))
        mixed = np.empty((rows, c["hidden"]), np.uint16)
        orc.lib.mxo_hc_up_mix(C.byref(w["up"]), _p(lo), _p(xn), rows, c["hidden"], _p(mixed))
        return mixed, inj

    def _qmv(self, w, x):
        """bf16 projection of rows x by the weight struct w (its mode's arithmetic)."""
        x = np.ascontiguousarray(x, np.uint16)
        m = x.shape[0]
        if w.mode == orc.XQ:
            yf = np.empty((m, w.n), np.float32)
            orc.lib.mxo_xq(w.codes, w.scales, w.biases, w.n, w.k, w.bits, _p(x), m, _p(yf))
            return orc.f32_to_bf16(yf)
        y = np.empty((m, w.n), np.uint16)
        orc.lib.mxo_qmv(w.codes, w.scales, w.biases, w.n, w.k, w.bits, w.gs, _p(x), m, _p(y))
        return y

    def _run_layer(self, L, attn, ci, h, rows, slots_a, pos_a, gdn_slots, groups, t, history):
        """One layer (GDN or attention sublayer, then the MoE sublayer) on the
        hc streams h; ci: the layer's GDN or attention cache index."""
        c = self.c
        H, hc = self.H, self.hc
        mixed, inj = self._hc_forward(L["attn_hc"], h, rows)
        if not attn:
            gi = ci
            proj = self._qmv(L["in"], mixed)
            qkv = np.ascontiguousarray(proj[:, :self.cd])
            sl = gdn_slots + gi
            conv_out = np.empty((rows, self.cd), np.uint16)
            win = np.empty((groups, c["conv_k"] - 1 + t, self.cd), np.uint16) if history is not None else None
            orc.lib.mxo_gdn_conv(_p(qkv), self.cd, groups, t, _p(sl), _p(self.conv), _p(L["conv_w"]),
                                 self.cd, c["conv_k"], _p(conv_out), self.cd,
                                 _p(win) if win is not None else None)
            zab = np.ascontiguousarray(proj[:, self.cd:])
            zp = zab.ctypes.data
            hist = np.empty((rows, c["gdn_hv"], 128, 128), np.float32) if history is not None else None
            y = np.empty((rows, self.vd), np.uint16)
            orc.lib.mxo_gdn_recurrence(_p(conv_out), self.cd, zp, zp + 2 * self.vd,
                                       zp + 2 * (self.vd + c["gdn_hv"]), zab.shape[1], _p(L["a_log"]),
                                       _p(L["dt"]), _p(L["norm"]), c["rms_eps"], c["gdn_hk"],
                                       c["gdn_hv"], groups, t, _p(sl), _p(self.state),
                                       _p(hist) if hist is not None else None, _p(y))
            if history is not None:
                history.append((gi, hist, win))
            orc.lib.mxo_hc_write(C.byref(L["out"]), _p(y), rows, hc, _p(h), _p(inj))
        else:
            ai = ci
            qkv = self._qmv(L["in"], mixed)
            layer_off = ai * c["kv_heads"] * c["max_context"] * c["head_dim"]
            kview = self.k[layer_off:]
            vview = self.v[layer_off:]
            q = np.empty((rows, c["heads"] * c["head_dim"]), np.uint16)
            orc.lib.mxo_attn_prep(_p(qkv), self.Q, rows, _p(slots_a), _p(pos_a), _p(L["q_norm"]),
                                  _p(L["k_norm"]), c["rms_eps"], _p(self.cos), _p(self.sin),
                                  c["heads"], c["kv_heads"], c["head_dim"], c["rotary_dim"],
                                  c["max_context"], self.kv_slot_stride, _p(q), kview.ctypes.data,
                                  vview.ctypes.data)
            y = np.empty((rows, c["heads"] * c["head_dim"]), np.uint16)
            orc.lib.mxo_attention(_p(q), _p(qkv), self.Q, rows, _p(slots_a), _p(pos_a),
                                  kview.ctypes.data, vview.ctypes.data, c["heads"], c["kv_heads"],
                                  c["head_dim"], c["max_context"], self.kv_slot_stride, _p(y))
            orc.lib.mxo_hc_write(C.byref(L["out"]), _p(y), rows, hc, _p(h), _p(inj))
        mixed, inj = self._hc_forward(L["mlp_hc"], h, rows)
        logits = self._qmv(L["router"], mixed)
        self.last_router.append(logits.copy())
        E = c["experts"]
        ids, scores, factor = orc.moe_route(np.ascontiguousarray(logits[:, :E]),
                                            np.ascontiguousarray(logits[:, E]), c["top_k"])
        self.last_ids.append(ids.copy())
        pbuf = np.empty((rows, c["top_k"] + 1, H), np.uint16)
        orc.lib.mxo_moe_experts(_p(mixed), _p(ids), _p(scores), rows, c["top_k"], C.byref(L["gate"]),
                                C.byref(L["up"]), C.byref(L["down"]), C.byref(L["sgate"]),
                                C.byref(L["sup"]), C.byref(L["sdown"]), _p(pbuf))
        routed = orc.moe_reduce(pbuf, c["top_k"])
        shared = np.ascontiguousarray(pbuf[:, c["top_k"], :])
        h = orc.moe_hc_epilogue(routed, shared, factor, h, inj, hc)
        return h

    def step(self, tokens, slots, pos, groups, t, history=None):
        """One engine step over rows (slot, position); GDN rows grouped as
        `groups` sequences of `t` tokens.  Returns greedy next tokens.  For
        inspection by tests, the step keeps each MoE layer's routing
        (last_ids), router logits (last_router) and each layer's input
        streams, then the final ones (layer_in, len(layers) + 1 entries)."""
        self.last_ids = []
        self.last_router = []
        self.layer_in = []
        c = self.c
        rows = len(tokens)
        H, hc = self.H, self.hc
        tok = np.ascontiguousarray(tokens, np.uint32)
        h = np.empty((rows, hc * H), np.uint16)
        orc.lib.mxo_embed(C.byref(self.embed), _p(tok), rows, hc, _p(h))
        slots_a = np.ascontiguousarray(slots, np.int32)
        pos_a = np.ascontiguousarray(pos, np.int32)
        gdn_slots = np.array([slots[g * t] * self.n_gdn for g in range(groups)], np.int32)
        for i, L in zip(self.layer_ids, self.layers):
            self.layer_in.append(h.copy())
            h = self._run_layer(L, self.attn[i], self.cache_index[i], h, rows, slots_a, pos_a,
                                gdn_slots, groups, t, history)
        self.layer_in.append(h.copy())
        self.hidden = h.copy()
        mixed, _ = self._hc_forward(self.mixer, h, rows)
        self.last_mixed = mixed
        return orc.head_argmax(self.head, mixed)

    def mtp_step(self, slot, tokens, pos0, prev):
        """Mtp::forward (src/mtp.rs:72-127) over rows of one slot: token r is the
        token after MTP position pos0 + r, prev the previous hidden streams
        [rows, hc*H].  Returns the draft tokens; self.mtp_hidden holds the new
        hidden streams.  Both norms are compiled::norm (src/compiled.rs:22-28)
        in the hyper-connection norm's order, over H and over all hc*H values."""
        c, m = self.c, self.mtp
        rows = len(tokens)
        self.last_ids = []
        self.last_router = []
        h = self.mtp_compose(tokens, prev)
        slots_a = np.full(rows, slot, np.int32)
        pos_a = np.arange(pos0, pos0 + rows, dtype=np.int32)
        gdn_slots = np.array([slot * self.n_gdn], np.int32)
        h = self._run_layer(m["layer"], True, m["cache"], h, rows, slots_a, pos_a, gdn_slots, 1,
                            rows, None)
        self.mtp_hidden = h.copy()
        mixed, _ = self._hc_forward(m["mixer"], h, rows)
        self.last_mixed = mixed
        return orc.head_argmax(self.head, mixed)

    def mtp_compose(self, tokens, prev):
        """The draft layer's input streams (src/mtp.rs:88-104): e =
        fc_embedding(norm(embedding)) over H; the previous hidden streams
        normalised together over all hc*H values, then fc_hidden on each
        stream; h[s] = bf16(e + f[s]).  Also kept as self.mtp_input."""
        c, m = self.c, self.mtp
        H, hc = self.H, self.hc
        rows = len(tokens)
        tok = np.ascontiguousarray(tokens, np.uint32)
        emb = np.empty((rows, H), np.uint16)
        orc.lib.mxo_embed(C.byref(self.embed), _p(tok), rows, 1, _p(emb))
        a = np.empty_like(emb)
        orc.lib.mxo_hc_norm(_p(emb), _p(m["norm_emb"]), rows, 1, H, c["rms_eps"], _p(a))
        e = self._qmv(m["fc_emb"], a)
        prev = np.ascontiguousarray(prev, np.uint16).reshape(rows, hc * H)
        hn = np.empty_like(prev)
        orc.lib.mxo_hc_norm(_p(prev), _p(m["norm_hid"]), rows, 1, hc * H, c["rms_eps"], _p(hn))
        f = self._qmv(m["fc_hid"], hn.reshape(rows * hc, H))
        s32 = orc.bf16_to_f32(e).astype(np.float32)[:, None, :] + \
            orc.bf16_to_f32(f).astype(np.float32).reshape(rows, hc, H)
        h = orc.f32_to_bf16(s32.astype(np.float32)).reshape(rows, hc * H)
        self.mtp_input = h.copy()
        return h

    def generate(self, slot, prompt, max_tokens, depth=0):
        """mx_engine_generate's contract (speculative::generate_prepared,
        src/speculative.rs:225-483, default policies): returns (tokens, stats)."""
        assert self.offsets[slot] == 0
        n = len(prompt)
        stats = {"rounds": 0, "drafted": 0, "accepted": 0, "drafts": []}
        bonus = seed = dh = None
        for a in range(0, n, 8):
            chunk = [int(x) for x in prompt[a:a + 8]]
            nxt = self.block(slot, chunk)
            bonus = int(nxt[-1])
            if depth > 0:
                toks = [int(prompt[a + r + 1]) if a + r + 1 < n else bonus for r in range(len(chunk))]
                d = self.mtp_step(slot, toks, a, self.hidden.copy())
                seed = int(d[-1])
                dh = self.mtp_hidden[-1:].copy()
        out = [bonus]
        if depth == 0:
            while len(out) < max_tokens:
                out.append(int(self.decode_rows([slot], [out[-1]])[0]))
            return out, stats
        mtp_len = n
        while len(out) < max_tokens:
            k = min(depth, max_tokens - len(out))
            drafted = [seed]
            base = mtp_len
            for i in range(1, k):
                d = self.mtp_step(slot, [drafted[i - 1]], base + i - 1, dh)
                drafted.append(int(d[0]))
                dh = self.mtp_hidden[-1:].copy()
            stats["drafts"] += drafted
            pred = [int(x) for x in self.verify(slot, [bonus] + drafted)]
            vh = self.hidden.copy()
            accepted = 0
            while accepted < k and drafted[accepted] == pred[accepted]:
                accepted += 1
            nxt = pred[accepted]
            emitted_now, ending = 0, False
            for i in range(accepted + 1):
                if len(out) == max_tokens:
                    ending = True
                    break
                out.append(drafted[i] if i < accepted else nxt)
                emitted_now += 1
            self.commit(slot, (min(emitted_now, accepted) + 1) if ending else accepted + 1)
            stats["rounds"] += 1
            stats["drafted"] += k
            stats["accepted"] += accepted
            if ending or len(out) == max_tokens:
                break
            bonus = nxt
            kept = min(accepted, k - 1)
            mtp_len = base + kept
            toks = drafted[kept:accepted] + [nxt]
            d = self.mtp_step(slot, toks, mtp_len, vh[kept:accepted + 1])
            seed = int(d[-1])
            dh = self.mtp_hidden[-1:].copy()
            mtp_len += len(toks)
        return out, stats

    # ---- engine-level operations (same contracts as the C ABI) ----
    def decode_rows(self, slots, tokens):
        pos = [self.offsets[s] for s in slots]
        out = self.step(tokens, slots, pos, len(slots), 1)
        for s in slots:
            self.offsets[s] += 1
        return out

    def block(self, slot, tokens, history=None):
        n = len(tokens)
        pos = [self.offsets[slot] + i for i in range(n)]
        out = self.step(tokens, [slot] * n, pos, 1, n, history)
        self.offsets[slot] += n
        return out

    def prefill(self, slot, tokens):
        nxt = None
        for i in range(0, len(tokens), 8):
            nxt = self.block(slot, tokens[i:i + 8])[-1]
        return nxt

    def verify(self, slot, tokens):
        self._snap = (slot, self.offsets[slot],
                      self.state[slot * self.n_gdn:(slot + 1) * self.n_gdn].copy(),
                      self.conv[slot * self.n_gdn:(slot + 1) * self.n_gdn].copy())
        self._hist = []
        return self.block(slot, tokens, self._hist)

    def commit(self, slot, keep):
        s0, base, st, cv = self._snap
        assert s0 == slot
        K = self.c["conv_k"]
        if keep == 0:
            self.state[slot * self.n_gdn:(slot + 1) * self.n_gdn] = st
            self.conv[slot * self.n_gdn:(slot + 1) * self.n_gdn] = cv
        else:
            for gi, hist, win in self._hist:
                self.state[slot * self.n_gdn + gi] = hist[keep - 1]
                self.conv[slot * self.n_gdn + gi] = win[0, keep:keep + K - 1]
        self.offsets[slot] = base + keep

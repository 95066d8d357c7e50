"""An independent float64 model of the Needle 3 step (crates/model/src/
session.rs:76-165), written from the reference's Rust with NumPy, for pinning
the oracle: it reads the archive itself (docs/format.md), dequantises every
codebook matrix to dense rows (levels times norms, then the normalised
Walsh-Hadamard matrix of scipy), and runs the step in float64 with exact
exponentials and products. It keeps the reference's quantisation points that
are model semantics: fake_quantise_int8 before every projection and after the
gated attention, and the per-head int8 queries, keys and values. It does not
model the integer products' per-group input codes, the integer levels or the
12-bit attention coefficients: those are arithmetic, and where the oracle's
float32 result and this model part is the size of that arithmetic's error."""
import struct

import numpy as np
from scipy.linalg import hadamard


def _parse(data: bytes):
    fields = struct.unpack_from("<26I", data, 0)
    names = ("tag", "tensor_count", "codebook_len", "kv_window", "kv_bits", "vocab", "out_vocab", "d_model",
             "num_heads", "num_kv_heads", "num_layers", "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n",
             "mhc_lanes", "sliding_window", "global_lo", "global_hi", "qkv_conv_taps", "engram_slots",
             "engram_sub_dim", "engram_tables", "engram_conv_taps", "engram_conv_dilation", "engram_seed_heads")
    g = dict(zip(names, fields))
    n_orders = struct.unpack_from("<I", data, 104)[0]
    g["orders"] = list(struct.unpack_from("<4I", data, 108))[:n_orders]
    n_sites = struct.unpack_from("<I", data, 124)[0]
    g["sites"] = list(struct.unpack_from("<16I", data, 128))[:n_sites]
    g["rope_theta"] = struct.unpack_from("<f", data, 192)[0]
    g["global_layers"] = g["global_lo"] | (g["global_hi"] << 32)
    codebook = np.frombuffer(data, np.float32, g["codebook_len"], 196).astype(np.float64)
    records = []
    base = 196 + 4 * g["codebook_len"]
    for i in range(g["tensor_count"]):
        kind, rank, _, s0, s1, s2, s3, off, nbytes, group, bits = struct.unpack_from("<BBH4IQQII", data, base + 44 * i)
        records.append(dict(kind=kind, shape=(s0, s1, s2, s3)[:rank], blob=data[off:off + nbytes], group=group,
                            bits=bits))
    return g, codebook, records


def _floats(r):
    return np.frombuffer(r["blob"], np.float16 if r["kind"] == 1 else np.float32).astype(np.float64)


def _levels(codebook, bits, group):
    if bits == 1:
        v = np.sqrt(2.0 / np.pi) / np.sqrt(group)
        return np.array([-v, v])
    if bits == 2:
        return codebook[0:4]
    if bits == 3:
        return codebook[4:12]
    if bits == 4:
        return codebook[12:28]
    v = 1.2240064 / np.sqrt(group)  # ternary crumbs: index 1 is +, 3 is -
    return np.array([0.0, v, 0.0, -v])


def _dense(r, codebook):
    rows, columns = r["shape"]
    group, bits = r["group"], r["bits"]
    ib = 2 if bits == 5 else bits
    padded = -(-columns // group) * group
    nbytes = rows * padded * ib // 8
    raw = np.frombuffer(r["blob"], np.uint8, nbytes)
    bitstream = np.unpackbits(raw, bitorder="little").reshape(rows, padded, ib)
    index = (bitstream * (1 << np.arange(ib))).sum(axis=2)
    norms = np.frombuffer(r["blob"], np.float16, rows * padded // group, nbytes).astype(np.float64)
    lv = np.asarray(_levels(codebook, bits, group), np.float64)[index]
    lv = lv * np.repeat(norms.reshape(rows, -1), group, axis=1)
    H = hadamard(group).astype(np.float64) / np.sqrt(group)
    w = (lv.reshape(rows, padded // group, group) @ H).reshape(rows, padded)
    return w[:, :columns]


def _fq(x):
    peak = np.max(np.abs(x))
    s = peak / 127.0 if peak > 0 else 1.0
    return np.clip(np.round(x / s), -128, 127) * s


def _codes(x):
    peak = np.max(np.abs(x))
    s = peak / 127.0 if peak > 0 else 1.0
    return np.clip(np.round(x / s), -128, 127), s


def _norm(x, gain):
    return (1.0 + gain) * x / np.sqrt(np.mean(x * x) + 1e-6)


def _unit(x):
    return x / np.sqrt(np.mean(x * x) + 1e-6)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _softmax(x):
    e = np.exp(x - np.max(x))
    return e / e.sum()


class Model:
    def __init__(self, data: bytes, active=None):
        g, cb, recs = _parse(data)
        self.g = g
        it = iter(recs)
        take = lambda: next(it)  # noqa: E731
        self.embedding = _dense(take(), cb)
        L, d = g["num_layers"], g["d_model"]
        self.layers = []
        for _ in range(L):
            y = dict(norm_in=_floats(take()), q=_dense(take(), cb), k=_dense(take(), cb), v=_dense(take(), cb))
            if g["qkv_conv_taps"]:
                y["taps"] = [_floats(take()).reshape(g["qkv_conv_taps"], -1) for _ in range(3)]
            y["q_norm"], y["k_norm"] = _floats(take()), _floats(take())
            y["gate"], y["out"] = _dense(take(), cb), _dense(take(), cb)
            y["post_norm"], y["attn_gate"], y["pre_hada"] = _floats(take()), _floats(take())[0], _floats(take())
            for n in ("d1", "d2", "b2", "d3", "d4"):
                y[n] = _floats(take())
            y["factors"] = [_floats(take()).reshape(32, 32) for _ in range(6)]
            y["cond_v"] = _floats(take()).reshape(d, -1)
            y["cond_u"] = _floats(take()).reshape(y["cond_v"].shape[1], -1)
            self.layers.append(y)
        lanes = g["mhc_lanes"]
        self.a_pre, self.a_post, self.a_res = _floats(take()), _floats(take()), _floats(take())
        self.b_pre = _floats(take()).reshape(L, lanes)
        self.b_post = _floats(take()).reshape(L, lanes)
        self.b_res = _floats(take()).reshape(L, lanes, lanes)
        self.phi = [_dense(take(), cb) for _ in range(3)]
        self.perms = [_floats(take()).astype(np.int64) for _ in range(2)]
        self.engrams = []
        for _ in g["sites"]:
            self.engrams.append(dict(tables=_dense(take(), cb), key=_dense(take(), cb), value=_dense(take(), cb),
                                     taps=_floats(take()).reshape(g["engram_conv_taps"], d)))
        self.final_norm = _floats(take())
        self.active = list(range(L)) if active is None else list(active)

    def session(self):
        return Session(self)


class Session:
    def __init__(self, m: Model):
        self.m = m
        g = m.g
        self.tokens = []
        self.keys = {l: [] for l in range(g["num_layers"])}    # [(codes [kv][64], scales [kv])]
        self.values = {l: [] for l in range(g["num_layers"])}
        self.raw = {l: [] for l in range(g["num_layers"])}     # newest first
        self.engram_raw = {s: [] for s in range(len(g["sites"]))}
        self.cells = None
        self.hidden = None

    def _indices(self, position):
        g = self.m.g
        hpo = g["engram_tables"] // max(len(g["orders"]), 1)
        stride = hpo if g["engram_seed_heads"] == 0 else g["engram_seed_heads"]
        out = []
        for o, order in enumerate(g["orders"]):
            for head in range(hpo):
                acc = (0x9E3779B9 * (o * stride + head + 1)) & 0xFFFFFFFF
                for back in range(order):
                    token = self.tokens[position - back] if position >= back else 0
                    acc = ((acc ^ token) * 0x01000193) & 0xFFFFFFFF
                acc ^= acc >> 15
                out.append((acc % g["engram_slots"], order))
        return out

    def push(self, token):
        m, g = self.m, self.m.g
        d, lanes = g["d_model"], g["mhc_lanes"]
        H, KV = g["num_heads"], g["num_kv_heads"]
        position = len(self.tokens)
        self.tokens.append(int(token))
        stream = np.tile(m.embedding[token] * np.sqrt(d), (lanes, 1))
        cells = [stream.mean(axis=0)]
        outputs = {}
        for s, site_layer in enumerate(g["sites"]):
            if site_layer not in m.active:
                continue
            e = m.engrams[s]
            sub = g["engram_sub_dim"]
            rows = [e["tables"][t * g["engram_slots"] + idx] if position + 1 >= order else np.zeros(sub)
                    for t, (idx, order) in enumerate(self._indices(position))]
            gathered = _fq(np.concatenate(rows))
            key, raw = e["key"] @ gathered, e["value"] @ gathered
            self.engram_raw[s].insert(0, raw)
            value = np.zeros(d)
            for tap in range(g["engram_conv_taps"]):
                back = tap * g["engram_conv_dilation"]
                if position >= back:
                    value += e["taps"][tap] * self.engram_raw[s][back]
            outputs[s] = (key, value)
        for slot, layer in enumerate(m.active):
            y = m.layers[layer]
            # lanes.rs:48-84
            normalised = _fq(_unit(stream.reshape(-1)))
            pre = m.phi[0][layer * lanes:(layer + 1) * lanes] @ normalised
            post = m.phi[1][layer * lanes:(layer + 1) * lanes] @ normalised
            res = m.phi[2][layer * lanes * lanes:(layer + 1) * lanes * lanes] @ normalised
            own = slot % lanes
            boost = np.where(np.arange(lanes) == own, 4.0, -4.0)
            gates = _sigmoid(m.a_pre[layer] * pre + m.b_pre[layer] + boost)
            inp = gates @ stream
            post = 2.0 * _sigmoid(m.a_post[layer] * post + m.b_post[layer] + np.where(np.arange(lanes) == own, 0.0, -4.0))
            r = (m.a_res[layer] * res + m.b_res[layer].reshape(-1)).reshape(lanes, lanes)
            r = np.exp(r - r.max(axis=1, keepdims=True))
            for _ in range(20):
                r /= r.sum(axis=1, keepdims=True)
                r /= r.sum(axis=0, keepdims=True)
            x = inp.copy()
            if layer in g["sites"]:
                s = g["sites"].index(layer)
                if s in outputs:
                    key, value = outputs[s]
                    x = x + _sigmoid(np.dot(_unit(x), _unit(key)) / np.sqrt(d)) * value
            # attention.rs:96-154
            hq = _fq(_norm(x, y["norm_in"]))
            q, k, v, gate = y["q"] @ hq, y["k"] @ hq, y["v"] @ hq, y["gate"] @ hq
            if g["qkv_conv_taps"]:
                self.raw[layer].insert(0, (q, k, v))
                del self.raw[layer][g["qkv_conv_taps"]:]
                mixed = []
                for which in range(3):
                    acc = np.zeros_like((q, k, v)[which])
                    for tap in range(min(g["qkv_conv_taps"], position + 1)):
                        acc += y["taps"][which][tap] * self.raw[layer][tap][which]
                    mixed.append(acc)
                q, k, v = mixed
            half = 32
            freq = 1.0 / g["rope_theta"] ** (2.0 * np.arange(half) / 64.0)
            ang = position * freq

            def rope(head):
                a, b = head[:half], head[half:]
                return np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)])

            qh = [_codes(rope(_norm(q[h * 64:(h + 1) * 64], y["q_norm"]))) for h in range(H)]
            kh = [_codes(rope(_norm(k[h * 64:(h + 1) * 64], y["k_norm"]))) for h in range(KV)]
            vh = [_codes(v[h * 64:(h + 1) * 64]) for h in range(KV)]
            self.keys[layer].append(kh)
            self.values[layer].append(vh)
            total = position + 1
            first = 0
            if g["sliding_window"] > 0 and not (g["global_layers"] >> layer) & 1:
                first = max(0, total - g["sliding_window"])
            attended = np.zeros(H * 64)
            for h in range(H):
                kvh = h // (H // KV)
                qc, qs = qh[h]
                scores = np.array([np.dot(qc, self.keys[layer][p][kvh][0]) * self.keys[layer][p][kvh][1]
                                   for p in range(first, total)]) * qs / 8.0
                w = _softmax(scores)
                vals = np.array([self.values[layer][p][kvh][0] * self.values[layer][p][kvh][1] for p in range(first, total)])
                attended[h * 64:(h + 1) * 64] = w @ vals
            attended = _fq(attended * _sigmoid(gate))
            a = _norm(y["out"] @ attended, y["post_norm"])
            x = x + _sigmoid(y["attn_gate"]) * a
            x = x + self._hadamard(y, _norm(x, y["pre_hada"]))
            delta = x - inp
            stream = r @ stream + post[:, None] * delta[None, :]
            cells.append(stream.mean(axis=0))
        self.cells = np.array(cells)
        self.hidden = _norm(stream.mean(axis=0), m.final_norm)

    def _hadamard(self, y, pre):
        m = self.m
        width = pre.size
        weights = _softmax(pre @ y["cond_v"])
        modulation = 1.0 + weights @ y["cond_u"]
        padded = np.zeros(1024)
        padded[:width] = pre

        def kron(x, left, right):
            return (left.T @ (x.reshape(32, 32) @ right)).reshape(-1)

        f = y["factors"]
        first = kron(padded * y["d1"], f[0], f[1])
        z = y["d2"] * modulation * first[m.perms[0]] + y["b2"]
        second = kron(z / (1.0 + np.exp(-z)), f[2], f[3])
        third = kron(second[m.perms[1]] * y["d3"], f[4], f[5])
        return (third * y["d4"])[:width]

    def logits(self):
        return self.m.embedding[:self.m.g["out_vocab"] or self.m.g["vocab"]] @ _fq(self.hidden)

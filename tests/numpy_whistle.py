"""An independent float64 NumPy model of the Whistle-style speech path.

Written from the reference's definitions (crates/whistle/src/stem.rs,
encoder.rs, cross.rs; crates/model/src/session.rs:76-148), not from the
oracle's code: float64 sums in NumPy's order, libm-exact exp in the softmax
and silu. The discrete parts of the model are kept: int8 per-row activation
quantisation before every product, int8 per-(frame, head) query/key/value codes
in the attention (encoder.rs:226-285, cross.rs:86-170), the fp16 self-attention
cache of the decoder.
"""
from __future__ import annotations

import numpy as np

from numpy_decoder import norm, product, quantise, rotary


def silu(x):
    return x / (1.0 + np.exp(-x))


def head_codes(h, gain=None, pos=None, theta=10000.0):
    if gain is not None:
        h = norm(h, gain, 1e-6)
    if pos is not None:
        h = rotary(h, pos, theta)
    q, s = quantise(h)
    return q, s


def int8_attend(qc, qs, kc, ks, vc, vs):
    """qc [hd]; kc, vc [frames][hd]; ks, vs [frames]; qs includes 1/sqrt(hd)."""
    scores = (kc.astype(np.float64) @ qc.astype(np.float64)) * ks * qs
    e = np.exp(scores - scores.max())
    w = e / e.sum()
    return (w * vs) @ vc.astype(np.float64)


def stem(cfg, w, mel):
    F, M, d = mel.shape[0], cfg["mels"], cfg["d_model"]
    pad = np.zeros((F + 2, M))
    pad[1:-1] = mel
    W1 = w["conv1"].astype(np.float64)  # [d][3][M]
    h1 = np.zeros((F, d))
    for k in range(3):
        h1 += pad[k:k + F] @ W1[:, k, :].T
    h1 = silu(h1)
    # second conv1d (d -> d, kernel 3, stride 2, pad 1) as an int8 product of the
    # three input frames of each output frame, quantised per row like any input
    T = (F - 1) // 2 + 1
    hp = np.zeros((F + 3, d))
    hp[1:F + 1] = h1
    cols = np.stack([hp[2 * t:2 * t + 3].reshape(-1) for t in range(T)])
    y = np.stack([product(*w["conv2"], cols[t]) for t in range(T)])
    return silu(y)


def gated_ffn(cfg, gate_up, down, gain, x):
    f = cfg["ffn"]
    gu = product(*gate_up, norm(x, gain, 1e-6))
    return x + product(*down, silu(gu[:f]) * gu[f:])


def encoder_layer(cfg, lw, x):
    T, d = x.shape
    H, hd = cfg["heads"], cfg["head_dim"]
    qkv = np.stack([product(*lw["qkv"], norm(x[t], lw["norm_attn"], 1e-6)) for t in range(T)])
    qc = np.zeros((T, H, hd))
    kc = np.zeros((T, H, hd))
    vc = np.zeros((T, H, hd))
    qs = np.zeros((T, H))
    ks = np.zeros((T, H))
    vs = np.zeros((T, H))
    for t in range(T):
        for h in range(H):
            sl = slice(h * hd, (h + 1) * hd)
            qc[t, h], qs[t, h] = head_codes(qkv[t, sl], lw["q_norm"], t, cfg["rope_theta"])
            kc[t, h], ks[t, h] = head_codes(qkv[t, d:][sl], lw["k_norm"], t, cfg["rope_theta"])
            vc[t, h], vs[t, h] = head_codes(qkv[t, 2 * d:][sl])
    ctx = np.zeros((T, d))
    for t in range(T):
        for h in range(H):
            ctx[t, h * hd:(h + 1) * hd] = int8_attend(qc[t, h], qs[t, h] / np.sqrt(hd), kc[:, h], ks[:, h],
                                                      vc[:, h], vs[:, h])
    x = x + np.stack([product(*lw["out"], ctx[t]) for t in range(T)])
    return np.stack([gated_ffn(cfg, lw["gate_up"], lw["down"], lw["norm_ffn"], x[t]) for t in range(T)])


def position_table(T, d, gate):
    half = d // 2
    rate = -np.log(10000.0) / (half - 1)
    angle = np.arange(T)[:, None] * np.exp(rate * np.arange(half))[None, :]
    return np.concatenate([gate * np.sin(angle), gate * np.cos(angle)], axis=1)


def memory(cfg, w, encoded):
    T, d = encoded.shape
    H, hd = cfg["heads"], cfg["head_dim"]
    gate = 1.0 / (1.0 + np.exp(-w["position_gate"]))
    inp = encoded + position_table(T, d, gate)
    layers = []
    for lw in w["dec"]:
        kv = np.stack([product(*lw["cross_kv"], inp[t]) for t in range(T)])
        kc = np.zeros((T, H, hd))
        vc = np.zeros((T, H, hd))
        ks = np.zeros((T, H))
        vs = np.zeros((T, H))
        for t in range(T):
            for h in range(H):
                sl = slice(h * hd, (h + 1) * hd)
                kc[t, h], ks[t, h] = head_codes(kv[t, sl], lw["k_norm"])
                vc[t, h], vs[t, h] = head_codes(kv[t, d:][sl])
        layers.append((kc, ks, vc, vs))
    return layers


class Decoder:
    def __init__(self, cfg, w, mem, capacity):
        self.c, self.w, self.mem = cfg, w, mem
        L, H, hd = cfg["dec_layers"], cfg["heads"], cfg["head_dim"]
        self.K = np.zeros((L, H, capacity, hd), dtype=np.float16)
        self.V = np.zeros((L, H, capacity, hd), dtype=np.float16)
        self.length = 0

    def push(self, token):
        c, w = self.c, self.w
        d, H, hd, theta = c["d_model"], c["heads"], c["head_dim"], c["rope_theta"]
        pos = self.length
        ec, es = w["embedding"]
        x = ec[token].astype(np.float64) * np.repeat(es[token].astype(np.float64), 32) * np.sqrt(d)
        for l, lw in enumerate(w["dec"]):
            qkv = product(*lw["qkv"], norm(x, lw["norm_attn"], 1e-6))
            att = np.empty(d)
            for h in range(H):
                sl = slice(h * hd, (h + 1) * hd)
                self.K[l, h, pos] = rotary(qkv[d:][sl], pos, theta).astype(np.float16)
                self.V[l, h, pos] = qkv[2 * d:][sl].astype(np.float16)
                Kh = self.K[l, h, :pos + 1].astype(np.float64)
                Vh = self.V[l, h, :pos + 1].astype(np.float64)
                s = Kh @ rotary(qkv[sl], pos, theta) / np.sqrt(hd)
                p = np.exp(s - s.max())
                att[sl] = (p / p.sum()) @ Vh
            x = x + product(*lw["out"], att)
            # cross.rs:126-182 without the gate projection
            q = product(*lw["cross_q"], norm(x, lw["norm_cross"], 1e-6))
            kc, ks, vc, vs = self.mem[l]
            ctx = np.empty(d)
            for h in range(H):
                sl = slice(h * hd, (h + 1) * hd)
                qc, qsc = head_codes(q[sl], lw["q_norm"])
                ctx[sl] = int8_attend(qc, qsc / np.sqrt(hd), kc[:, h], ks[:, h], vc[:, h], vs[:, h])
            attended = norm(product(*lw["cross_out"], ctx), lw["post_norm"], 1e-6)
            x = x + (1.0 / (1.0 + np.exp(-lw["gate"]))) * attended
            x = gated_ffn(c, lw["gate_up"], lw["down"], lw["norm_ffn"], x)
        self.length = pos + 1
        hidden = norm(x, w["dec_norm"], 1e-6)
        return product(*w["embedding"], hidden)

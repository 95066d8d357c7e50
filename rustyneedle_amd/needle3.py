"""Needle 3 models: synthetic .cact archives in the canonical tensor order
(crates/cact/src/layout.rs:176-257) and the device model and session
(crates/model/src/model.rs, session.rs) over the C ABI.

There are no published Needle 3 weights here, so archives are synthetic: seeded
codebook indices and norms, float tensors drawn per name, permutations from a
seeded generator. The geometry presets name their sizes; NEEDLE3 follows the
reference's documented shape (d_model 768, 20 layers, four lanes, 32 x 32
Kronecker factors, a 1024-token window with four global layers, 8192 x 768
4-bit logits; docs/architecture.md)."""
from __future__ import annotations

import struct
from typing import Optional

import numpy as np

from . import cact
from . import synth_normal, synth_uniform, synthetic_codebook, synthetic_codebook_blob

# geometry field names follow the archive header (docs/format.md)
NEEDLE3 = dict(vocab=8192, out_vocab=8192, d_model=768, num_heads=12, num_kv_heads=4, num_layers=20, qk_head_dim=64,
               v_head_dim=64, max_seq_len=4096, hada_n=1024, mhc_lanes=4, sliding_window=1024,
               global_layers=(1 << 4) | (1 << 9) | (1 << 14) | (1 << 19), qkv_conv_taps=3, engram_slots=16384,
               engram_sub_dim=64, num_engram_tables=8, engram_conv_taps=4, engram_conv_dilation=1,
               engram_seed_heads=0, engram_orders=(2, 3), engram_sites=(1, 10), rope_theta=10000.0,
               heads=((1, 4, 4, 256), (2, 4, 4, 1)), group=128)

# a small model with every feature: two engram sites at different depths, a
# 16-token window with one global layer, conv taps, both head kinds
NEEDLE3_SMALL = dict(vocab=512, out_vocab=512, d_model=256, num_heads=4, num_kv_heads=2, num_layers=4, qk_head_dim=64,
                     v_head_dim=64, max_seq_len=512, hada_n=1024, mhc_lanes=4, sliding_window=16, global_layers=1 << 1,
                     qkv_conv_taps=3, engram_slots=256, engram_sub_dim=64, num_engram_tables=4, engram_conv_taps=3,
                     engram_conv_dilation=2, engram_seed_heads=0, engram_orders=(2, 3), engram_sites=(0, 2),
                     rope_theta=10000.0, heads=((1, 2, 3, 32), (2, 2, 3, 1)), group=128)

# bits of each matrix kind: 2-bit panels for the projections, 4-bit planes for
# the embedding and tables, a 3-bit (float path) head projection
BITS = dict(embedding=4, projection=2, lanes=2, tables=4, engram=2, probes=4, head_projection=3)

KIND_HALF, KIND_SINGLE, KIND_CODEBOOK, KIND_RAW = 1, 2, 3, 4


def synthetic_archive(geometry: dict, seed: int = 20261202, bits: Optional[dict] = None) -> bytes:
    """A .cact archive of the Needle 3 layout with seeded synthetic weights.
    geometry["heads"] lists (code, probes_per_layer, queries, projection_rows);
    bits (default BITS) gives the width of each matrix kind."""
    BITS = globals()["BITS"] if bits is None else bits
    g = dict(geometry)
    d, L, lanes, size = g["d_model"], g["num_layers"], g["mhc_lanes"], g["hada_n"]
    qk, vd, H, KV = g["qk_head_dim"], g["v_head_dim"], g["num_heads"], g["num_kv_heads"]
    group = g["group"]
    codebook = synthetic_codebook(group)
    rng = np.random.default_rng(seed)
    tensors = []

    def single(name, shape, sigma, centre=0.0):
        v = synth_normal(seed, name, sigma, (int(np.prod(shape)),)) + np.float32(centre)
        tensors.append((KIND_SINGLE, tuple(shape), v.astype(np.float32).tobytes(), 0, 0))

    def half(name, shape, sigma, centre=0.0):
        v = synth_normal(seed, name, sigma, (int(np.prod(shape)),)) + np.float32(centre)
        tensors.append((KIND_HALF, tuple(shape), v.astype(np.float16).tobytes(), 0, 0))

    def matrix(name, rows, columns, bits, grp=group):
        blob = synthetic_codebook_blob(rows, columns, grp, bits, seed=seed, name=name)
        tensors.append((KIND_CODEBOOK, (rows, columns), blob.tobytes(), grp, bits))

    matrix("embedding", g["vocab"], d, BITS["embedding"])
    for layer in range(L):
        p = f"layer{layer}."
        single(p + "norm_in", (d,), 0.1)
        matrix(p + "q", H * qk, d, BITS["projection"])
        matrix(p + "k", KV * qk, d, BITS["projection"])
        matrix(p + "v", KV * vd, d, BITS["projection"])
        if g["qkv_conv_taps"] > 0:
            for which, width in (("q", H * qk), ("k", KV * qk), ("v", KV * vd)):
                taps = synth_normal(seed, p + "taps_" + which, 0.2, (g["qkv_conv_taps"], width))
                taps[0] += np.float32(1.0)
                tensors.append((KIND_SINGLE, (g["qkv_conv_taps"], width), taps.astype(np.float32).tobytes(), 0, 0))
        half(p + "q_norm", (qk,), 0.1)
        half(p + "k_norm", (qk,), 0.1)
        matrix(p + "gate", H * vd, d, BITS["projection"])
        matrix(p + "out", d, H * vd, BITS["projection"])
        single(p + "post_norm", (d,), 0.1)
        single(p + "attn_gate", (1,), 0.5)
        single(p + "pre_hada", (d,), 0.1)
        # the 13 Hadamard tensors: d1 d2 b2 d3 d4, w1a w1b w2a w2b w3a w3b, cond_v cond_u
        single(p + "d1", (size,), 0.1, 1.0)
        single(p + "d2", (size,), 0.1, 1.0)
        single(p + "b2", (size,), 0.1)
        single(p + "d3", (size,), 0.1, 1.0)
        single(p + "d4", (size,), 0.1, 0.5)
        for f in ("w1a", "w1b", "w2a", "w2b", "w3a", "w3b"):
            single(p + f, (32, 32), float(1.0 / np.sqrt(32.0)))
        single(p + "cond_v", (d, 8), 0.05)
        single(p + "cond_u", (8, size), 0.2)
    # lanes (layout.rs:226-229): a_pre a_post a_res [L], b_pre b_post [L][lanes], b_res [L][lanes][lanes], phis
    single("lanes.a_pre", (L,), 0.2)
    single("lanes.a_post", (L,), 0.2)
    single("lanes.a_res", (L,), 0.2)
    single("lanes.b_pre", (L, lanes), 0.5)
    single("lanes.b_post", (L, lanes), 0.5)
    single("lanes.b_res", (L, lanes, lanes), 0.5)
    matrix("lanes.phi_pre", L * lanes, lanes * d, BITS["lanes"])
    matrix("lanes.phi_post", L * lanes, lanes * d, BITS["lanes"])
    matrix("lanes.phi_res", L * lanes * lanes, lanes * d, BITS["lanes"])
    for p in range(2):  # the Hadamard permutations, stored as floats
        perm = rng.permutation(size).astype(np.float32)
        tensors.append((KIND_SINGLE, (size,), perm.tobytes(), 0, 0))
    tables = g["num_engram_tables"]
    for site in range(len(g["engram_sites"])):
        p = f"engram{site}."
        matrix(p + "tables", tables * g["engram_slots"], g["engram_sub_dim"], BITS["tables"], grp=64)
        matrix(p + "key", d, tables * g["engram_sub_dim"], BITS["engram"])
        matrix(p + "value", d, tables * g["engram_sub_dim"], BITS["engram"])
        taps = synth_normal(seed, p + "taps", 0.2, (g["engram_conv_taps"], d))
        taps[0] += np.float32(1.0)
        tensors.append((KIND_SINGLE, (g["engram_conv_taps"], d), taps.astype(np.float32).tobytes(), 0, 0))
    single("final_norm", (d,), 0.1)
    heads = g.get("heads", ())
    if heads:
        codes = np.array([h[0] for h in heads], np.float16)
        tensors.append((KIND_HALF, (len(heads),), codes.tobytes(), 0, 0))
        for code, k, queries, out_rows in heads:
            p = f"head{code}."
            matrix(p + "probes", (L + 1) * k, d, BITS["probes"])
            single(p + "gain", ((L + 1) * k,), 0.1, 1.0)
            matrix(p + "query", queries, d, BITS["probes"])
            single(p + "row_bias", (queries, (L + 1) * k), 0.3)
            matrix(p + "proj", out_rows, queries * d, BITS["head_projection"])
            single(p + "bias", (out_rows,), 0.1)
            if code == 3:
                single(p + "calibration", (2,), 0.1)
    # the tokenizer blob (docs/format.md): no pieces
    tensors.append((KIND_RAW, (24,), struct.pack("<IIIIIBBH", 0, 0, 2, 1, 0, 1, 1, 0), 0, 0))
    fields = {k: g[k] for k in ("vocab", "out_vocab", "d_model", "num_heads", "num_kv_heads", "num_layers",
                                "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n", "mhc_lanes", "sliding_window",
                                "qkv_conv_taps", "engram_slots", "engram_sub_dim", "num_engram_tables",
                                "engram_conv_taps", "engram_conv_dilation", "engram_seed_heads")}
    fields["global_mask_lo"] = g["global_layers"] & 0xFFFFFFFF
    fields["global_mask_hi"] = g["global_layers"] >> 32
    return cact.write(tensors, codebook, rope_theta=g["rope_theta"], engram_orders=g["engram_orders"],
                      engram_sites=g["engram_sites"], **fields)


# ---- the device model and session ------------------------------------------------
from . import Archive, Choice, _ptr, check, lib  # noqa: E402

_p = __import__("ctypes").c_void_p
_C = __import__("ctypes")


class Model:
    """Model::open + with_depth (model.rs:50-78) on the device, from archive
    bytes or an open Archive."""

    def __init__(self, archive, depth: int = 0):
        self._archive = archive if isinstance(archive, Archive) else Archive(data=bytes(archive))
        h = _p()
        check(lib.rn_n3_model_open(self._archive.handle, depth, _C.byref(h)))
        self.handle = h.value
        g = self._archive.geometry()
        self.geometry = g
        n = _C.c_int()
        layers = (_C.c_int * max(1, g["num_layers"]))()
        check(lib.rn_n3_model_active_layers(self.handle, layers, _C.byref(n)))
        self.active = [layers[i] for i in range(n.value)]
        check(lib.rn_n3_model_output_vocab(self.handle, _C.byref(n)))
        self.output_vocab = n.value

    def session(self, capacity: int = 512) -> "Session":
        return Session(self, capacity)

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib.rn_n3_model_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Session:
    """Session (session.rs) on the device."""

    def __init__(self, model: Model, capacity: int):
        self.model = model
        h = _p()
        check(lib.rn_n3_session_create(model.handle, capacity, _C.byref(h)))
        self.handle = h.value
        self.capacity = capacity

    def push(self, token: int) -> None:
        check(lib.rn_n3_session_push(self.handle, int(token)))

    def feed(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, np.uint32)
        check(lib.rn_n3_session_feed(self.handle, _ptr(t), t.size))

    def stream(self) -> int:
        h = _p()
        check(lib.rn_n3_session_stream(self.handle, _C.byref(h)))
        return h.value

    def decode_greedy(self, first: int, steps: int) -> np.ndarray:
        ids = np.empty(steps, np.uint32)
        check(lib.rn_n3_session_decode_greedy(self.handle, int(first), steps, _ptr(ids)))
        return ids

    def clone(self) -> "Session":
        """#[derive(Clone)] on Session (session.rs:17): an independent copy."""
        h = _p()
        check(lib.rn_n3_session_clone(self.handle, _C.byref(h)))
        t = Session.__new__(Session)
        t.model, t.handle, t.capacity = self.model, h.value, self.capacity
        return t

    def run_turn(self, max_tokens: int, stops=(), window: int = 0):
        """Generator::run_turn's loop with no grammar (generator.rs:99-130):
        (ids, finished); window 0 takes the archive's max_seq_len."""
        ids = np.empty(max(1, max_tokens), np.uint32)
        st = np.ascontiguousarray(list(stops) or [0], np.uint32)
        n, fin = _C.c_int(), _C.c_int()
        check(lib.rn_n3_session_run_turn(self.handle, int(max_tokens), int(window), _ptr(st), len(stops), _ptr(ids),
                                         _C.byref(n), _C.byref(fin)))
        return ids[:n.value].copy(), bool(fin.value)

    def choose_allowed(self, allowed: np.ndarray):
        """generator.rs:104-116: (token, constrained, probability, mass) over this session's logits."""
        mask = np.ascontiguousarray(allowed, dtype=np.uint8)
        assert mask.shape == (self.model.output_vocab,)
        c = Choice()
        check(lib.rn_n3_session_choose_allowed(self.handle, _ptr(mask), _C.byref(c)))
        return int(c.token), bool(c.constrained), np.float32(c.probability), np.float32(c.mass)

    def __len__(self) -> int:
        n = _C.c_int()
        check(lib.rn_n3_session_length(self.handle, _C.byref(n)))
        return n.value

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.output_vocab, np.float32)
        check(lib.rn_n3_session_logits(self.handle, _ptr(out)))
        return out

    def hidden(self) -> np.ndarray:
        out = np.empty(self.model.geometry["d_model"], np.float32)
        check(lib.rn_n3_session_hidden(self.handle, _ptr(out)))
        return out

    def cells(self) -> np.ndarray:
        out = np.empty((len(self.model.active) + 1, self.model.geometry["d_model"]), np.float32)
        check(lib.rn_n3_session_cells(self.handle, _ptr(out)))
        return out

    def _head(self, fn, code: int, capacity: int) -> Optional[np.ndarray]:
        out = np.empty(capacity, np.float32)
        n = _C.c_int()
        check(fn(self.handle, code, _ptr(out), capacity, _C.byref(n)))
        return out[:n.value].copy() if n.value else None

    def head_output(self, code: int) -> Optional[np.ndarray]:
        return self._head(lib.rn_n3_session_head_output, code, 1 << 16)

    def pooled_readout(self, code: int) -> Optional[np.ndarray]:
        return self._head(lib.rn_n3_session_pooled_readout, code, 1 << 20)

    def cache(self, layer: int):
        g = self.model.geometry
        n, kv = len(self), g["num_kv_heads"]
        keys = np.empty((n, kv, 64), np.int8)
        values = np.empty((n, kv, 64), np.int8)
        ks = np.empty((kv, n), np.float32)
        vs = np.empty((kv, n), np.float32)
        check(lib.rn_n3_session_cache(self.handle, layer, _ptr(keys), _ptr(ks), _ptr(values), _ptr(vs)))
        return keys, ks, values, vs

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib.rn_n3_session_free(self.handle)
                self.handle = None
        except Exception:
            pass

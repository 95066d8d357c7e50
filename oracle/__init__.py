"""CPU oracle for the Needle token loop — test infrastructure, not the product.

A ctypes view of ``oracle/librn_oracle.so`` (built from ``rn_oracle.c`` by
``oracle/Makefile``). Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librn_oracle.so")

FORM_PANEL = 0
FORM_PLANE = 1


def build() -> None:
    """Compile the oracle with its Makefile (always rebuilds when sources changed)."""
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"oracle library missing: {LIB_PATH} (run oracle/Makefile)")
    return C.CDLL(LIB_PATH)


lib = _load()

_f = C.c_float
_i = C.c_int
_p = C.c_void_p

lib.ro_fast_exp.restype = _f
lib.ro_fast_exp.argtypes = [_f]
lib.ro_silu.restype = _f
lib.ro_silu.argtypes = [_f]
lib.ro_peak_magnitude.restype = _f
lib.ro_peak_magnitude.argtypes = [_p, _i]
lib.ro_int8_scale.restype = _f
lib.ro_int8_scale.argtypes = [_p, _i]
lib.ro_quantise_int8.restype = _f
lib.ro_quantise_int8.argtypes = [_p, _i, _p]
lib.ro_fake_quantise_int8.argtypes = [_p, _i]
lib.ro_sum_of_squares.restype = _f
lib.ro_sum_of_squares.argtypes = [_p, _i]
lib.ro_zero_centred_norm.argtypes = [_p, _p, _i, _p]
lib.ro_softmax_in_place.argtypes = [_p, _i]
lib.ro_rotary_frequencies.argtypes = [_i, _f, _p]
lib.ro_rotary_table.argtypes = [_i, _f, _i, _p, _p]
lib.ro_apply_rotary.argtypes = [_p, _i, _p, _p]
lib.ro_f32_to_f16.restype = C.c_uint16
lib.ro_f32_to_f16.argtypes = [_f]
lib.ro_f16_to_f32.restype = _f
lib.ro_f16_to_f32.argtypes = [C.c_uint16]
lib.ro_argmax.restype = C.c_uint32
lib.ro_argmax.argtypes = [_p, _i]
lib.ro_product.argtypes = [_i, _p, _p, _i, _i, _i, _p, _p, _i, _p, _p]
lib.ro_multiply.argtypes = [_i, _p, _p, _i, _i, _i, _p, _i, _p, _p, _p, _p]
lib.ro_attend_head.argtypes = [_p, _p, _p, _i, _i, _p]
lib.ro_set_threads.argtypes = [_i]
lib.ro_get_threads.restype = _i


class Config(C.Structure):
    _fields_ = [
        ("layers", _i), ("d_model", _i), ("heads", _i), ("head_dim", _i), ("ffn", _i),
        ("vocab", _i), ("group", _i), ("max_positions", _i),
        ("rope_theta", _f), ("norm_eps", _f),
    ]


class QMat(C.Structure):
    _fields_ = [("codes", _p), ("scales", _p)]


class Layer(C.Structure):
    _fields_ = [("qkv", QMat), ("out", QMat), ("gate_up", QMat), ("down", QMat),
                ("norm_attn", _p), ("norm_ffn", _p)]


class Model(C.Structure):
    _fields_ = [("embedding", QMat), ("norm_final", _p), ("layers", _p),
                ("rope_cos", _p), ("rope_sin", _p)]


class Session(C.Structure):
    _fields_ = [("keys", _p), ("values", _p), ("hidden", _p), ("capacity", _i), ("length", _i)]


lib.ro_embed.argtypes = [C.POINTER(Config), C.POINTER(Model), C.c_uint32, _p]
lib.ro_session_push.argtypes = [C.POINTER(Config), C.POINTER(Model), C.POINTER(Session), C.c_uint32]
lib.ro_session_prefill.argtypes = [C.POINTER(Config), C.POINTER(Model), C.POINTER(Session), _p, _i]
lib.ro_session_logits.argtypes = [C.POINTER(Config), C.POINTER(Model), C.POINTER(Session), _p]
lib.ro_greedy.argtypes = [C.POINTER(Config), C.POINTER(Model), C.POINTER(Session), C.c_uint32, _i, _p]


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib.ro_set_threads(int(n))


def fast_exp(v: float) -> float:
    return lib.ro_fast_exp(float(v))


lib.ro_libm_exp_array.restype = None
lib.ro_libm_exp_array.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]


def libm_exp_array(x: np.ndarray, sigmoid: bool = False) -> np.ndarray:
    """The C library's expf (f32::exp), or ops::sigmoid over it, elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib.ro_libm_exp_array(x.ctypes.data, y.ctypes.data, x.size, int(sigmoid))
    return y


lib.ro_libm_log_array.restype = None
lib.ro_libm_log_array.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]


def libm_log_array(x: np.ndarray) -> np.ndarray:
    """The C library's logf (f32::ln), elementwise."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib.ro_libm_log_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def silu(v: float) -> float:
    return lib.ro_silu(float(v))


def int8_scale(x) -> float:
    x = _f32(x)
    return lib.ro_int8_scale(_ptr(x), x.size)


def quantise_int8(x):
    x = _f32(x)
    codes = np.empty(x.size, dtype=np.int8)
    scale = lib.ro_quantise_int8(_ptr(x), x.size, _ptr(codes))
    return codes, np.float32(scale)


def fake_quantise_int8(x) -> np.ndarray:
    x = _f32(x).copy()
    lib.ro_fake_quantise_int8(_ptr(x), x.size)
    return x


def sum_of_squares(x) -> float:
    x = _f32(x)
    return lib.ro_sum_of_squares(_ptr(x), x.size)


def zero_centred_norm(x, gain) -> np.ndarray:
    x = _f32(x)
    gain = _f32(gain)
    out = np.empty_like(x)
    lib.ro_zero_centred_norm(_ptr(x), _ptr(gain), x.size, _ptr(out))
    return out


def softmax(v) -> np.ndarray:
    v = _f32(v).copy()
    lib.ro_softmax_in_place(_ptr(v), v.size)
    return v


def rotary_frequencies(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib.ro_rotary_frequencies(head_dim, theta, _ptr(out))
    return out


def rotary_table(head_dim: int, theta: float, positions: int):
    cos = np.empty((positions, head_dim // 2), dtype=np.float32)
    sin = np.empty_like(cos)
    lib.ro_rotary_table(head_dim, theta, positions, _ptr(cos), _ptr(sin))
    return cos, sin


def apply_rotary(head, cos_row, sin_row) -> np.ndarray:
    head = _f32(head).copy()
    cos_row, sin_row = _f32(cos_row), _f32(sin_row)
    lib.ro_apply_rotary(_ptr(head), head.size, _ptr(cos_row), _ptr(sin_row))
    return head


def f32_to_f16(v: float) -> int:
    return lib.ro_f32_to_f16(float(v))


def f16_to_f32(bits: int) -> float:
    return lib.ro_f16_to_f32(int(bits))


def argmax(values) -> int:
    values = _f32(values)
    return int(lib.ro_argmax(_ptr(values), values.size))


def product(form, W, sW, xq, sx, group=32, with_acc=False):
    """y[count][rows] (and acc[count][rows][groups]) from pre-quantised inputs."""
    W = np.ascontiguousarray(W, dtype=np.int8)
    sW = _f32(sW)
    xq = np.ascontiguousarray(np.atleast_2d(xq), dtype=np.int8)
    sx = _f32(np.atleast_1d(sx))
    rows, cols = W.shape
    count = xq.shape[0]
    y = np.empty((count, rows), dtype=np.float32)
    acc = np.empty((count, rows, cols // group), dtype=np.int32) if with_acc else None
    lib.ro_product(form, _ptr(W), _ptr(sW), rows, cols, group, _ptr(xq), _ptr(sx), count, _ptr(y),
                   _ptr(acc) if with_acc else None)
    return (y, acc) if with_acc else y


def multiply(form, W, sW, x, group=32, with_acc=False):
    """Quantise each input row (quantise_int8) and multiply: returns y, acc, codes, scales."""
    W = np.ascontiguousarray(W, dtype=np.int8)
    sW = _f32(sW)
    x = _f32(np.atleast_2d(x))
    rows, cols = W.shape
    count = x.shape[0]
    y = np.empty((count, rows), dtype=np.float32)
    acc = np.empty((count, rows, cols // group), dtype=np.int32) if with_acc else None
    codes = np.empty((count, cols), dtype=np.int8)
    scales = np.empty(count, dtype=np.float32)
    lib.ro_multiply(form, _ptr(W), _ptr(sW), rows, cols, group, _ptr(x), count, _ptr(y),
                    _ptr(acc) if with_acc else None, _ptr(codes), _ptr(scales))
    return y, acc, codes, scales


def attend_head(q, K, V) -> np.ndarray:
    """q: [hd] f32; K, V: [L][hd] float16 (or uint16 bits)."""
    q = _f32(q)
    K = np.ascontiguousarray(K).view(np.uint16)
    V = np.ascontiguousarray(V).view(np.uint16)
    L, hd = K.shape
    out = np.empty(hd, dtype=np.float32)
    lib.ro_attend_head(_ptr(q), _ptr(K), _ptr(V), hd, L, _ptr(out))
    return out


class OracleModel:
    """Holds numpy weights (the same host arrays handed to the GPU model) and the
    ctypes structs the oracle reads. `weights` is the dict produced by
    rustyneedle_amd.synthetic_weights (or any dict with the same keys)."""

    def __init__(self, config: dict, weights: dict):
        self.config = dict(config)
        c = self.config
        self.cfg = Config(c["layers"], c["d_model"], c["heads"], c["head_dim"], c["ffn"], c["vocab"],
                          c["group"], c["max_positions"], c["rope_theta"], c["norm_eps"])
        self.w = weights
        self.rope_cos, self.rope_sin = rotary_table(c["head_dim"], c["rope_theta"], c["max_positions"])
        layers = (Layer * c["layers"])()
        for l in range(c["layers"]):
            lw = weights["layers"][l]
            layers[l] = Layer(QMat(_ptr(lw["qkv"][0]), _ptr(lw["qkv"][1])),
                              QMat(_ptr(lw["out"][0]), _ptr(lw["out"][1])),
                              QMat(_ptr(lw["gate_up"][0]), _ptr(lw["gate_up"][1])),
                              QMat(_ptr(lw["down"][0]), _ptr(lw["down"][1])),
                              _ptr(lw["norm_attn"]), _ptr(lw["norm_ffn"]))
        self._layers = layers
        emb = weights["embedding"]
        self.model = Model(QMat(_ptr(emb[0]), _ptr(emb[1])), _ptr(weights["norm_final"]),
                           C.addressof(layers), _ptr(self.rope_cos), _ptr(self.rope_sin))

    def session(self, capacity: int) -> "OracleSession":
        return OracleSession(self, capacity)


class OracleSession:
    def __init__(self, model: OracleModel, capacity: int):
        c = model.config
        self.model = model
        shape = (c["layers"], c["heads"], capacity, c["head_dim"])
        self.keys = np.zeros(shape, dtype=np.uint16)
        self.values = np.zeros(shape, dtype=np.uint16)
        self.hidden = np.zeros(c["d_model"], dtype=np.float32)
        self.s = Session(_ptr(self.keys), _ptr(self.values), _ptr(self.hidden), capacity, 0)

    @property
    def length(self) -> int:
        return self.s.length

    def set_cache(self, keys: np.ndarray, values: np.ndarray) -> None:
        """keys/values: [layers][heads][length][hd] float16 or uint16 bits."""
        length = keys.shape[2]
        self.keys[:, :, :length] = np.asarray(keys).view(np.uint16)
        self.values[:, :, :length] = np.asarray(values).view(np.uint16)
        self.s.length = length

    def push(self, token: int) -> None:
        lib.ro_session_push(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), token)

    def feed(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lib.ro_session_prefill(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s),
                               _ptr(t), t.size)

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config["vocab"], dtype=np.float32)
        lib.ro_session_logits(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), _ptr(out))
        return out

    def greedy(self, first: int, steps: int) -> np.ndarray:
        ids = np.empty(steps, dtype=np.uint32)
        lib.ro_greedy(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), first, steps,
                      _ptr(ids))
        return ids


# ---- Whistle-style speech path (rn_whistle.c) ------------------------------------

class WConfig(C.Structure):
    _fields_ = [(n, _i) for n in ("mels", "frames", "d_model", "heads", "head_dim", "enc_layers", "dec_layers", "ffn",
                                  "vocab", "max_positions", "group")] + [("rope_theta", _f), ("norm_eps", _f)]


class WEncLayer(C.Structure):
    _fields_ = [("qkv", QMat), ("out", QMat), ("gate_up", QMat), ("down", QMat), ("norm_attn", _p),
                ("norm_ffn", _p), ("q_norm", _p), ("k_norm", _p)]


class WDecLayer(C.Structure):
    _fields_ = [("qkv", QMat), ("out", QMat), ("cross_q", QMat), ("cross_kv", QMat), ("cross_out", QMat),
                ("gate_up", QMat), ("down", QMat), ("norm_attn", _p), ("norm_cross", _p), ("post_norm", _p),
                ("norm_ffn", _p), ("q_norm", _p), ("k_norm", _p), ("cross_gain", _f)]


class WModel(C.Structure):
    _fields_ = [("conv1", _p), ("conv2", QMat), ("enc", _p), ("enc_norm", _p),
                ("cross_position", _p), ("embedding", QMat), ("dec", _p), ("dec_norm", _p), ("rope_cos", _p),
                ("rope_sin", _p)]


class WSession(C.Structure):
    _fields_ = [("keys", _p), ("values", _p), ("mem_k", _p), ("mem_ks", _p), ("mem_v", _p), ("mem_vs", _p),
                ("hidden", _p), ("capacity", _i), ("length", _i), ("frames", _i)]


_WC, _WM, _WS = C.POINTER(WConfig), C.POINTER(WModel), C.POINTER(WSession)
lib.ro_whistle_frames.restype = _i
lib.ro_whistle_frames.argtypes = [_WC]
lib.ro_sigmoid.restype = _f
lib.ro_sigmoid.argtypes = [_f]
lib.ro_whistle_position_table.argtypes = [_i, _i, _f, _p]
lib.ro_whistle_stem.argtypes = [_WC, _WM, _p, _p]
lib.ro_whistle_encoder_layer.argtypes = [_WC, _WM, _i, _p, _i]
lib.ro_whistle_encode.argtypes = [_WC, _WM, _p, _p]
lib.ro_whistle_memory.argtypes = [_WC, _WM, _p, _i, _p, _p, _p, _p]
lib.ro_int8_attend.argtypes = [_p, _f, _p, _p, _p, _p, _i, _i, _i, _i, _p]
lib.ro_whistle_push.argtypes = [_WC, _WM, _WS, C.c_uint32]
lib.ro_whistle_logits.argtypes = [_WC, _WM, _WS, _p]
lib.ro_whistle_greedy.argtypes = [_WC, _WM, _WS, C.c_uint32, _i, _p]


def sigmoid(v: float) -> float:
    return lib.ro_sigmoid(float(v))


def whistle_position_table(frames: int, d: int, gate: float) -> np.ndarray:
    out = np.empty((frames, d), dtype=np.float32)
    lib.ro_whistle_position_table(frames, d, float(gate), _ptr(out))
    return out


def int8_attend(qc, query_scale, kc, ks, vc, vs) -> np.ndarray:
    """One query head: qc [hd] int8; kc, vc [frames][hd] int8; ks, vs [frames]."""
    qc = np.ascontiguousarray(qc, dtype=np.int8)
    kc = np.ascontiguousarray(kc, dtype=np.int8)
    vc = np.ascontiguousarray(vc, dtype=np.int8)
    ks, vs = _f32(ks), _f32(vs)
    frames, hd = kc.shape
    out = np.empty(hd, dtype=np.float32)
    lib.ro_int8_attend(_ptr(qc), float(query_scale), _ptr(kc), _ptr(ks), _ptr(vc), _ptr(vs), frames, hd, hd, 1,
                       _ptr(out))
    return out


class OracleWhistle:
    """The Whistle-style model over the numpy weights of
    rustyneedle_amd.synthetic_whistle_weights (the same host arrays the GPU model
    uploads)."""

    def __init__(self, config: dict, weights: dict):
        self.config = c = dict(config)
        self.cfg = WConfig(*[c[n] for n in ("mels", "frames", "d_model", "heads", "head_dim", "enc_layers",
                                            "dec_layers", "ffn", "vocab", "max_positions", "group")],
                           c["rope_theta"], c["norm_eps"])
        self.w = weights
        self.frames = lib.ro_whistle_frames(C.byref(self.cfg))
        self.rope_cos, self.rope_sin = rotary_table(c["head_dim"], c["rope_theta"],
                                                    max(self.frames, c["max_positions"]))
        self.position = whistle_position_table(self.frames, c["d_model"], sigmoid(weights["position_gate"]))
        qm = lambda pair: QMat(_ptr(pair[0]), _ptr(pair[1]))
        enc = (WEncLayer * c["enc_layers"])()
        for l, lw in enumerate(weights["enc"]):
            enc[l] = WEncLayer(qm(lw["qkv"]), qm(lw["out"]), qm(lw["gate_up"]), qm(lw["down"]), _ptr(lw["norm_attn"]),
                               _ptr(lw["norm_ffn"]), _ptr(lw["q_norm"]), _ptr(lw["k_norm"]))
        dec = (WDecLayer * c["dec_layers"])()
        for l, lw in enumerate(weights["dec"]):
            dec[l] = WDecLayer(qm(lw["qkv"]), qm(lw["out"]), qm(lw["cross_q"]), qm(lw["cross_kv"]), qm(lw["cross_out"]),
                               qm(lw["gate_up"]), qm(lw["down"]), _ptr(lw["norm_attn"]), _ptr(lw["norm_cross"]),
                               _ptr(lw["post_norm"]), _ptr(lw["norm_ffn"]), _ptr(lw["q_norm"]), _ptr(lw["k_norm"]),
                               sigmoid(lw["gate"]))
        self._enc, self._dec = enc, dec
        self.model = WModel(_ptr(weights["conv1"]), qm(weights["conv2"]),
                            C.addressof(enc), _ptr(weights["enc_norm"]), _ptr(self.position), qm(weights["embedding"]),
                            C.addressof(dec), _ptr(weights["dec_norm"]), _ptr(self.rope_cos), _ptr(self.rope_sin))

    def stem(self, mel: np.ndarray) -> np.ndarray:
        mel = _f32(mel)
        out = np.empty((self.frames, self.config["d_model"]), dtype=np.float32)
        lib.ro_whistle_stem(C.byref(self.cfg), C.byref(self.model), _ptr(mel), _ptr(out))
        return out

    def encoder_layer(self, layer: int, x: np.ndarray) -> np.ndarray:
        x = _f32(x).copy()
        lib.ro_whistle_encoder_layer(C.byref(self.cfg), C.byref(self.model), layer, _ptr(x), x.shape[0])
        return x

    def encode(self, mel: np.ndarray) -> np.ndarray:
        mel = _f32(mel)
        out = np.empty((self.frames, self.config["d_model"]), dtype=np.float32)
        lib.ro_whistle_encode(C.byref(self.cfg), C.byref(self.model), _ptr(mel), _ptr(out))
        return out

    def memory(self, encoded: np.ndarray):
        encoded = _f32(encoded)
        c = self.config
        T = encoded.shape[0]
        shape = (c["dec_layers"], T, c["heads"], c["head_dim"])
        mk, mv = np.empty(shape, np.int8), np.empty(shape, np.int8)
        ks, vs = np.empty(shape[:3], np.float32), np.empty(shape[:3], np.float32)
        lib.ro_whistle_memory(C.byref(self.cfg), C.byref(self.model), _ptr(encoded), T, _ptr(mk), _ptr(ks), _ptr(mv),
                              _ptr(vs))
        return mk, ks, mv, vs

    def session(self, capacity: int, memory) -> "OracleWhistleSession":
        return OracleWhistleSession(self, capacity, memory)


class OracleWhistleSession:
    def __init__(self, model: OracleWhistle, capacity: int, memory):
        c = model.config
        self.model = model
        shape = (c["dec_layers"], c["heads"], capacity, c["head_dim"])
        self.keys = np.zeros(shape, dtype=np.uint16)
        self.values = np.zeros(shape, dtype=np.uint16)
        self.hidden = np.zeros(c["d_model"], dtype=np.float32)
        self.memory = tuple(np.ascontiguousarray(a) for a in memory)
        mk, ks, mv, vs = self.memory
        self.s = WSession(_ptr(self.keys), _ptr(self.values), _ptr(mk), _ptr(ks), _ptr(mv), _ptr(vs),
                          _ptr(self.hidden), capacity, 0, mk.shape[1])

    @property
    def length(self) -> int:
        return self.s.length

    def push(self, token: int) -> None:
        lib.ro_whistle_push(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), token)

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config["vocab"], dtype=np.float32)
        lib.ro_whistle_logits(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), _ptr(out))
        return out

    def greedy(self, first: int, steps: int) -> np.ndarray:
        ids = np.empty(steps, dtype=np.uint32)
        lib.ro_whistle_greedy(C.byref(self.model.cfg), C.byref(self.model.model), C.byref(self.s), first, steps,
                              _ptr(ids))
        return ids


# ---- codebook weight format (rn_codebook.c) ------------------------------------
lib.ro_walsh_transform.argtypes = [_p, _i]
lib.ro_codebook_prepare.argtypes = [_p, _i, _i, _i, _p]
lib.ro_codebook_levels.restype = _i
lib.ro_codebook_levels.argtypes = [_p, _i, _i, _p]
lib.ro_integer_levels.restype = _f
lib.ro_integer_levels.argtypes = [_p, _i, _p]
lib.ro_group_codes.argtypes = [_p, _i, _i, _p, _p]
lib.ro_codebook_product.argtypes = [_p, _p, _i, _i, _i, _i, _p, _f, _p, _p, _i, _p, _p]
lib.ro_codebook_dequantise_row.argtypes = [_p, _p, _i, _i, _i, _i, _p, _i, _p]
lib.ro_codebook_float_vector.argtypes = [_p, _p, _i, _i, _i, _i, _p, _p, _i, _p]
lib.ro_codebook_float_batch.argtypes = [_p, _p, _i, _i, _i, _i, _p, _p, _i, _p]


def walsh_transform(v) -> np.ndarray:
    v = _f32(v).copy()
    lib.ro_walsh_transform(_ptr(v), v.size)
    return v


def codebook_prepare(x, padded: int, group: int) -> np.ndarray:
    x = _f32(x)
    out = np.empty(padded, np.float32)
    lib.ro_codebook_prepare(_ptr(x), x.size, padded, group, _ptr(out))
    return out


def codebook_levels(codebook, bits: int, group: int):
    cb = _f32(codebook)
    levels = np.empty(16, np.float32)
    count = lib.ro_codebook_levels(_ptr(cb), bits, group, _ptr(levels))
    return levels, count


def integer_levels(levels, count: int):
    levels = _f32(levels)
    table = np.empty(16, np.int8)
    scale = lib.ro_integer_levels(_ptr(levels), count, _ptr(table))
    return table, np.float32(scale)


def group_codes(rotated, group: int):
    r = _f32(rotated)
    codes = np.empty(r.size, np.int8)
    scales = np.empty(r.size // group, np.float32)
    lib.ro_group_codes(_ptr(r), r.size, group, _ptr(codes), _ptr(scales))
    return codes, scales


class OracleCodebookMatrix:
    """A codebook-quantised matrix from its archive blob (packed indices, then
    fp16 norms), restating QuantisedMatrix's integer path."""

    def __init__(self, blob, rows: int, columns: int, group: int, bits: int, codebook):
        self.rows, self.columns, self.group, self.bits = rows, columns, group, bits
        self.padded = -(-columns // group) * group
        ib = 2 if bits == 5 else bits
        packed_len = rows * self.padded * ib // 8
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        self.packed = np.ascontiguousarray(blob[:packed_len])
        self.norms = np.ascontiguousarray(blob[packed_len:packed_len + rows * (self.padded // group) * 2]).view(np.uint16)
        self.levels, self.count = codebook_levels(codebook, bits, group)
        self.table, self.lscale = integer_levels(self.levels, self.count)

    def prepare(self, x) -> np.ndarray:
        return codebook_prepare(x, self.padded, self.group)

    def multiply_rotated(self, rotated, with_acc: bool = False):
        """rotated [count][padded] -> y [count][rows] (acc [count][rows][groups])."""
        rotated = _f32(rotated).reshape(-1, self.padded)
        count = rotated.shape[0]
        codes = np.empty(rotated.shape, np.int8)
        scales = np.empty((count, self.padded // self.group), np.float32)
        for t in range(count):
            codes[t], scales[t] = group_codes(rotated[t], self.group)
        y = np.empty((count, self.rows), np.float32)
        acc = np.empty((count, self.rows, self.padded // self.group), np.int32) if with_acc else None
        lib.ro_codebook_product(_ptr(self.packed), _ptr(self.norms), self.rows, self.padded, self.group, self.bits,
                                _ptr(self.table), float(self.lscale), _ptr(codes), _ptr(scales), count, _ptr(y),
                                _ptr(acc) if acc is not None else None)
        return (y, acc) if with_acc else y

    def multiply(self, x, with_acc: bool = False):
        """Unrotated inputs [count][columns]: prepare, then the product."""
        x = _f32(x).reshape(-1, self.columns)
        rotated = np.stack([self.prepare(row) for row in x])
        return self.multiply_rotated(rotated, with_acc)

    def multiply_float(self, rotated, batch: bool = False) -> np.ndarray:
        """The float path on rotated inputs [count][padded]: fill_rows_float
        (multiply_vector on x86-64, matrix.rs:427-440) or, with batch, the float
        tile of multiply_batch (matrix.rs:356-378)."""
        rotated = _f32(rotated).reshape(-1, self.padded)
        count = rotated.shape[0]
        y = np.empty((count, self.rows), np.float32)
        fn = lib.ro_codebook_float_batch if batch else lib.ro_codebook_float_vector
        fn(_ptr(self.packed), _ptr(self.norms), self.rows, self.padded, self.group, self.bits, _ptr(self.levels),
           _ptr(rotated), count, _ptr(y))
        return y

    def dequantise_row(self, row: int) -> np.ndarray:
        out = np.empty(self.columns, np.float32)
        lib.ro_codebook_dequantise_row(_ptr(self.packed), _ptr(self.norms), self.padded, self.columns, self.group,
                                       self.bits, _ptr(self.levels), row, _ptr(out))
        return out


# ---- grammar-constrained choice (rn_generate.c) ---------------------------------
lib.ro_argmax_allowed.restype = C.c_int32
lib.ro_argmax_allowed.argtypes = [_p, _p, _i]
lib.ro_allowed_statistics.argtypes = [_p, _p, _i, _i, C.POINTER(_f), C.POINTER(_f)]


def argmax_allowed(values, allowed) -> int:
    """generator.rs:147-155; -1 where the reference returns None."""
    v = _f32(values)
    a = np.ascontiguousarray(allowed, dtype=np.uint8)
    return int(lib.ro_argmax_allowed(_ptr(v), _ptr(a), v.size))


def allowed_statistics(logits, allowed, token: int):
    v = _f32(logits)
    a = np.ascontiguousarray(allowed, dtype=np.uint8)
    p, m = _f(), _f()
    lib.ro_allowed_statistics(_ptr(v), _ptr(a), v.size, token, C.byref(p), C.byref(m))
    return np.float32(p.value), np.float32(m.value)


def choose_allowed(logits, allowed):
    """generator.rs:99-117: argmax_allowed, else argmax; and the statistics of the choice."""
    token = argmax_allowed(logits, allowed)
    if token < 0:
        token = argmax(logits)
    return (token,) + allowed_statistics(logits, allowed, token)


# ---- speech front end (rn_frontend.c) -------------------------------------------
lib.ro_frontend_tables.argtypes = [_i, _i, _p, _p, _p]
lib.ro_power_spectrum.argtypes = [_p, _p, _i, _p, _p, _p]
lib.ro_log_mel.restype = _i
lib.ro_log_mel.argtypes = [_p, _i, _i, _i, _i, _i, _p, _p, C.POINTER(_i), C.POINTER(_f)]


def frontend_tables(fft_size: int, window: int):
    win, tc, ts = np.empty(window, np.float32), np.empty(fft_size // 2, np.float32), np.empty(fft_size // 2, np.float32)
    lib.ro_frontend_tables(fft_size, window, _ptr(win), _ptr(tc), _ptr(ts))
    return win, tc, ts


def power_spectrum(real, imaginary):
    re, im = _f32(real).copy(), _f32(imaginary).copy()
    _, tc, ts = frontend_tables(re.size, 2)
    out = np.empty(re.size // 2 + 1, np.float32)
    lib.ro_power_spectrum(_ptr(re), _ptr(im), re.size, _ptr(tc), _ptr(ts), _ptr(out))
    return out


def log_mel(samples, mels: int, fft_size: int, window: int, hop: int, mel_weights):
    """Frontend::log_mel: (features [frames][mels], valid, spread)."""
    x = _f32(samples)
    w = _f32(mel_weights)
    data = np.empty((x.size // hop + 1, mels), np.float32)
    valid, spread = _i(), _f()
    lib.ro_log_mel(_ptr(x) if x.size else None, x.size, mels, fft_size, window, hop, _ptr(w), _ptr(data),
                   C.byref(valid), C.byref(spread))
    return data, valid.value, np.float32(spread.value)


# ---- Kronecker apply (rn_hadamard.c) ----------------------------------------------
lib.ro_kronecker_apply_32.argtypes = [_p, _p, _p, _p]


def kronecker_apply_32(x, left, right) -> np.ndarray:
    """ops.rs:220-297: L^T . X . R for 32 x 32 factors, fused multiply-adds in index order."""
    x, left, right = _f32(x), _f32(left), _f32(right)
    out = np.empty(1024, np.float32)
    lib.ro_kronecker_apply_32(_ptr(x), _ptr(left), _ptr(right), _ptr(out))
    return out


# ---- lanes hyper-connection (rn_lanes.c) ------------------------------------------
lib.ro_unit_rms.argtypes = [_p, _i, _p]
lib.ro_sinkhorn.argtypes = [_p, _i, _i]
lib.ro_lanes_route_tail.argtypes = [_i, _i, _i, _i] + [_p] * 11
lib.ro_lanes_combine.argtypes = [_i, _i] + [_p] * 5


def unit_rms(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib.ro_unit_rms(_ptr(x), x.size, _ptr(out))
    return out


def sinkhorn(m, iterations: int = 20) -> np.ndarray:
    m = _f32(m).copy()
    lib.ro_sinkhorn(_ptr(m), int(round(m.size ** 0.5)), iterations)
    return m


def lanes_route(lanes, width, layer, slot, t, stream, phis):
    """lanes.rs:48-84 with the routing matrices as OracleCodebookMatrix (t: dict of the lane tensors)."""
    stream = _f32(stream).reshape(-1)
    normalised = fake_quantise_int8(unit_rms(stream))
    rotated = phis[0].prepare(normalised)
    pre = phis[0].multiply_rotated(rotated)[0][layer * lanes:(layer + 1) * lanes].copy()
    post = phis[1].multiply_rotated(rotated)[0][layer * lanes:(layer + 1) * lanes].copy()
    residual = phis[2].multiply_rotated(rotated)[0][layer * lanes * lanes:(layer + 1) * lanes * lanes].copy()
    a = {k: _f32(v) for k, v in t.items()}
    inp = np.empty(width, np.float32)
    lib.ro_lanes_route_tail(lanes, width, layer, slot, _ptr(a["a_pre"]), _ptr(a["a_post"]), _ptr(a["a_res"]),
                            _ptr(a["b_pre"]), _ptr(a["b_post"]), _ptr(a["b_res"]), _ptr(stream), _ptr(pre),
                            _ptr(post), _ptr(residual), _ptr(inp))
    return inp, post, residual.reshape(lanes, lanes)


def lanes_combine(lanes, width, post, residual, stream, delta) -> np.ndarray:
    post, residual, stream, delta = _f32(post), _f32(residual), _f32(stream), _f32(delta)
    out = np.empty((lanes, width), np.float32)
    lib.ro_lanes_combine(lanes, width, _ptr(post), _ptr(residual), _ptr(stream), _ptr(delta), _ptr(out))
    return out


# ---- Needle 3 (rn_needle3.c) ------------------------------------------------------
class N3Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "output_vocab", "d_model", "num_heads", "num_kv_heads", "num_layers",
                                        "qk_head_dim", "v_head_dim", "max_seq_len", "lanes", "sliding_window",
                                        "conv_taps", "hadamard_size")] + [
        ("global_layers", C.c_uint64), ("rope_theta", C.c_float)] + [
        (n, C.c_int) for n in ("engram_slots", "engram_sub_dim", "engram_tables", "engram_conv_taps",
                                "engram_dilation", "engram_seed_heads", "engram_order_count")] + [
        ("engram_orders", C.c_int * 4), ("engram_heads_per_order", C.c_int), ("engram_site_count", C.c_int),
        ("engram_sites", C.c_int * 16)]


lib.ro_n3_open.restype = C.c_int
lib.ro_n3_open.argtypes = [_p, C.c_size_t, C.c_int, C.POINTER(_p)]
lib.ro_n3_close.argtypes = [_p]
lib.ro_n3_config_of.restype = C.POINTER(N3Config)
lib.ro_n3_config_of.argtypes = [_p]
lib.ro_n3_active.restype = C.c_int
lib.ro_n3_active.argtypes = [_p, _p]
lib.ro_n3_session_new.restype = C.c_int
lib.ro_n3_session_new.argtypes = [_p, C.c_int, C.POINTER(_p)]
lib.ro_n3_session_free.argtypes = [_p]
lib.ro_n3_session_clone.restype = C.c_int
lib.ro_n3_session_clone.argtypes = [_p, C.POINTER(_p)]
lib.ro_n3_push.argtypes = [_p, C.c_uint32]
lib.ro_n3_feed.argtypes = [_p, _p, _i]
lib.ro_n3_logits.argtypes = [_p, _p]
lib.ro_n3_pooled_readout.restype = C.c_int
lib.ro_n3_pooled_readout.argtypes = [_p, C.c_int, _p]
lib.ro_n3_head_output.restype = C.c_int
lib.ro_n3_head_output.argtypes = [_p, C.c_int, _p]
lib.ro_n3_table_indices.argtypes = [C.POINTER(N3Config), _p, C.c_int, _p]
lib.ro_n3_attend_head.argtypes = [_p, _f, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p]


class N3Session(C.Structure):
    _fields_ = [("m", _p), ("length", C.c_int), ("capacity", C.c_int), ("tokens", _p), ("caches", _p),
                ("engram_history", _p), ("engram_count", _p), ("cos_tab", _p), ("sin_tab", _p), ("hidden", _p),
                ("cells", _p), ("peak", _p), ("total", _p), ("weighted", _p)]


class N3Cache(C.Structure):
    _fields_ = [("keys", _p), ("values", _p), ("key_scales", _p), ("value_scales", _p), ("history", _p),
                ("history_count", C.c_int), ("length", C.c_int)]


class OracleNeedle3:
    """Model::open + with_depth over archive bytes (crates/model/src/model.rs)."""

    def __init__(self, archive: bytes, depth: int = 0):
        self._bytes = np.frombuffer(archive, np.uint8).copy()
        h = _p()
        rc = lib.ro_n3_open(_ptr(self._bytes), self._bytes.size, depth, C.byref(h))
        if rc != 0:
            raise ValueError("depth outside the ladder" if rc == -2 else "malformed or unsupported archive")
        self.handle = h.value
        self.config = lib.ro_n3_config_of(self.handle).contents
        n = self.config.num_layers
        layers = (C.c_int * n)()
        count = lib.ro_n3_active(self.handle, layers)
        self.active = [layers[i] for i in range(count)]

    def session(self, capacity: int = 512) -> "OracleNeedle3Session":
        return OracleNeedle3Session(self, capacity)

    def __del__(self):
        if getattr(self, "handle", None):
            lib.ro_n3_close(self.handle)
            self.handle = None


class OracleNeedle3Session:
    """Session (session.rs): push / feed (feeding equals pushing in order: the
    batched prefill, prefill.rs:10-99, runs the same arithmetic per token),
    logits, hidden, cells, the probe heads, and the int8 caches."""

    def __init__(self, model: OracleNeedle3, capacity: int):
        self.model = model
        h = _p()
        lib.ro_n3_session_new(model.handle, capacity, C.byref(h))
        self.handle = h.value
        self.capacity = capacity

    def push(self, token: int) -> None:
        s = C.cast(self.handle, C.POINTER(N3Session)).contents
        if s.length >= self.capacity:
            raise ValueError("session is full")
        lib.ro_n3_push(self.handle, int(token))

    def feed(self, tokens) -> None:
        """Session::feed (session.rs:56-70): chunks of 128 as prefills (the
        projections and engram products through multiply_batch, which for 1-
        and 3-bit matrices is the float tile), a short last chunk pushed; with
        integer-path matrices equal to pushing every token."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).ravel())
        if len(self) + t.size > self.capacity:
            raise ValueError("session is full")
        if t.size:
            lib.ro_n3_feed(self.handle, _ptr(t), t.size)

    def greedy(self, first: int, steps: int) -> np.ndarray:
        """generator.rs:199-230 without grammar: push, logits, argmax (generator.rs:257-265)."""
        ids = np.empty(steps, np.uint32)
        token = int(first)
        for i in range(steps):
            self.push(token)
            token = argmax(self.logits())
            ids[i] = token
        return ids

    def clone(self) -> "OracleNeedle3Session":
        """#[derive(Clone)] on Session (session.rs:17)."""
        h = _p()
        if lib.ro_n3_session_clone(self.handle, C.byref(h)) != 0:
            raise MemoryError("clone failed")
        t = OracleNeedle3Session.__new__(OracleNeedle3Session)
        t.model, t.handle, t.capacity = self.model, h.value, self.capacity
        return t

    def run_turn(self, max_tokens: int, window: int, stops) -> tuple:
        """The loop of Generator::run_turn without a grammar (generator.rs:99-130):
        while n < max_tokens and len + 1 < window: next = argmax(logits);
        push(next); stop after pushing a token of `stops`. Returns (ids, finished)."""
        ids, finished = [], False
        stops = set(int(t) for t in stops)
        while len(ids) < max_tokens and len(self) + 1 < window:
            token = argmax(self.logits())
            ids.append(token)
            self.push(token)
            if token in stops:
                finished = True
                break
        return np.array(ids, np.uint32), finished

    def choose_allowed(self, allowed) -> tuple:
        """generator.rs:104-116 on this session's logits: (token, constrained,
        probability, mass), as rn_n3_session_choose_allowed returns them."""
        logits = self.logits()
        best = argmax_allowed(logits, allowed)
        token = best if best >= 0 else argmax(logits)
        probability, mass = allowed_statistics(logits, allowed, token)
        return token, int(best >= 0), probability, mass

    def __len__(self) -> int:
        return C.cast(self.handle, C.POINTER(N3Session)).contents.length

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config.output_vocab, np.float32)
        lib.ro_n3_logits(self.handle, _ptr(out))
        return out

    def hidden(self) -> np.ndarray:
        s = C.cast(self.handle, C.POINTER(N3Session)).contents
        d = self.model.config.d_model
        return np.ctypeslib.as_array(C.cast(s.hidden, C.POINTER(_f)), (d,)).copy()

    def cells(self) -> np.ndarray:
        s = C.cast(self.handle, C.POINTER(N3Session)).contents
        d = self.model.config.d_model
        n = len(self.model.active) + 1
        return np.ctypeslib.as_array(C.cast(s.cells, C.POINTER(_f)), (n, d)).copy()

    def head_output(self, code: int) -> Optional[np.ndarray]:
        out = np.empty(65536, np.float32)
        n = lib.ro_n3_head_output(self.handle, code, _ptr(out))
        return None if n < 0 else out[:n].copy()

    def pooled_readout(self, code: int) -> Optional[np.ndarray]:
        out = np.empty(1 << 20, np.float32)
        n = lib.ro_n3_pooled_readout(self.handle, code, _ptr(out))
        return None if n < 0 else out[:n].copy()

    def cache(self, layer: int):
        """keys [length][kv][qk] int8, key_scales [kv][length], values, value_scales."""
        c = self.model.config
        s = C.cast(self.handle, C.POINTER(N3Session)).contents
        k = C.cast(s.caches, C.POINTER(N3Cache))[layer]
        n = s.length
        cap = self.capacity
        keys = np.ctypeslib.as_array(C.cast(k.keys, C.POINTER(C.c_int8)), (cap, c.num_kv_heads, c.qk_head_dim))
        values = np.ctypeslib.as_array(C.cast(k.values, C.POINTER(C.c_int8)), (cap, c.num_kv_heads, c.v_head_dim))
        ks = np.ctypeslib.as_array(C.cast(k.key_scales, C.POINTER(_f)), (c.num_kv_heads, cap))
        vs = np.ctypeslib.as_array(C.cast(k.value_scales, C.POINTER(_f)), (c.num_kv_heads, cap))
        return keys[:n].copy(), ks[:, :n].copy(), values[:n].copy(), vs[:, :n].copy()

    def __del__(self):
        if getattr(self, "handle", None):
            lib.ro_n3_session_free(self.handle)
            self.handle = None


def n3_table_indices(config: N3Config, tokens, position: int) -> list:
    t = np.ascontiguousarray(tokens, np.uint32)
    n = config.engram_order_count * config.engram_heads_per_order
    out = np.empty(max(n, 1), np.int32)
    lib.ro_n3_table_indices(C.byref(config), _ptr(t), position, _ptr(out))
    return out[:n].tolist()


def n3_attend_head(query, query_scale, keys, key_scales, values, value_scales) -> np.ndarray:
    """kernels/src/attention.rs:53-80 over int8 keys [count][qk], values [count][vd]."""
    q = np.ascontiguousarray(query, np.int8)
    k = np.ascontiguousarray(keys, np.int8)
    v = np.ascontiguousarray(values, np.int8)
    ks, vs = _f32(key_scales), _f32(value_scales)
    count, qk = k.shape
    vd = v.shape[1]
    out = np.empty(vd, np.float32)
    lib.ro_n3_attend_head(_ptr(q), float(query_scale), _ptr(k), _ptr(ks), _ptr(v), _ptr(vs), count, qk, vd, qk, vd,
                          _ptr(out))
    return out


lib.ro_n3_hadamard_arrays.argtypes = [_i, _i] + [_p] * 11 + [_i, _p]


def n3_hadamard(t: dict, first_perm, second_perm, x) -> np.ndarray:
    """hadamard.rs:55-107: t holds d1 d2 b2 d3 d4 [size], factors [6][32][32],
    cond_v [width][rank], cond_u [rank][size]."""
    size = t["d1"].size
    rank = t["cond_u"].size // size
    a = {k: _f32(v) for k, v in t.items()}
    p1 = np.ascontiguousarray(first_perm, np.int32)
    p2 = np.ascontiguousarray(second_perm, np.int32)
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib.ro_n3_hadamard_arrays(size, rank, _ptr(a["d1"]), _ptr(a["d2"]), _ptr(a["b2"]), _ptr(a["d3"]), _ptr(a["d4"]),
                              _ptr(a["factors"]), _ptr(a["cond_v"]), _ptr(a["cond_u"]), _ptr(p1), _ptr(p2), _ptr(x),
                              x.size, _ptr(out))
    return out

"""rustyneedle_amd — the Needle token loop on MI355X (gfx950).

A thin Python view of ``librustyneedle_hip.so`` (the C ABI declared in
``include/rustyneedle.h``). Names mirror the reference's kernels / model API
(``QuantisedMatrix``, ``Model``, ``Session``) so that tests read like the
reference's own. Loading fails loudly when the HIP library has not been built:
there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librustyneedle_hip.so")

RN_OK = 0
RN_ERR_ARGUMENT = -1
RN_ERR_DEVICE = -2
RN_ERR_CAPACITY = -3
RN_ERR_STATE = -4
RN_ERR_MEMORY = -5

FORM_PANEL = 0
FORM_PLANE = 1

# Kernel kinds of rn_session_profile_step, in RN_PROFILE_* order.
PROFILE_KINDS = ("qkv_attention", "out", "gate_up", "down", "logits", "final")

# The decoder of the decode / prefill / batch workloads: 20 layers, d_model 512,
# 8 heads of 64, rotary base 10000, RMSNorm eps 1e-6, gated FFN 512->2048->512,
# int8 codes with one fp32 scale per 32 columns, tied int8 vocab 8192.
NEEDLE_DECODER = dict(layers=20, d_model=512, heads=8, head_dim=64, ffn=2048, vocab=8192, group=32,
                      max_positions=1024, rope_theta=10000.0, norm_eps=1e-6)
# The Whistle-style speech path: 80-bin log-mel input of 3000 frames, stem to
# d_model 384 over 1500 frames, 6 encoder layers, 4 decoder layers with
# cross-attention over the encoded frames, tied int8 vocab 8192.
WHISTLE = dict(mels=80, frames=3000, d_model=384, heads=6, head_dim=64, enc_layers=6, dec_layers=4, ffn=1536,
               vocab=8192, max_positions=64, group=32, rope_theta=10000.0, norm_eps=1e-6)
SEED = 20261201


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    return C.CDLL(LIB_PATH)


lib = _load()

_i, _f, _p, _u32, _u64, _sz = C.c_int, C.c_float, C.c_void_p, C.c_uint32, C.c_uint64, C.c_size_t


class Config(C.Structure):
    _fields_ = [("layers", _i), ("d_model", _i), ("heads", _i), ("head_dim", _i), ("ffn", _i),
                ("vocab", _i), ("group", _i), ("max_positions", _i), ("rope_theta", _f), ("norm_eps", _f)]


class QMatHost(C.Structure):
    _fields_ = [("codes", _p), ("scales", _p)]


class LayerHost(C.Structure):
    _fields_ = [("qkv", QMatHost), ("out", QMatHost), ("gate_up", QMatHost), ("down", QMatHost),
                ("norm_attn", _p), ("norm_ffn", _p)]


class WeightsHost(C.Structure):
    _fields_ = [("embedding", QMatHost), ("norm_final", _p), ("layers", _p)]


class Geometry(C.Structure):
    """rn_geometry: the .cact header (geometry.rs:10-37)."""
    _fields_ = [(n, C.c_uint32) for n in (
        "tensor_count", "codebook_len", "kv_window", "kv_bits", "vocab", "out_vocab", "d_model", "num_heads",
        "num_kv_heads", "num_layers", "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n", "mhc_lanes",
        "sliding_window")] + [("global_layers", C.c_uint64)] + [(n, C.c_uint32) for n in (
        "qkv_conv_taps", "engram_slots", "engram_sub_dim", "engram_tables", "engram_conv_taps",
        "engram_conv_dilation", "engram_seed_heads", "engram_order_count")] + [
        ("engram_orders", C.c_uint32 * 4), ("engram_site_count", C.c_uint32), ("engram_sites", C.c_uint32 * 16),
        ("rope_theta", C.c_float)]


class TensorRecord(C.Structure):
    """rn_tensor_record (record.rs:27-51)."""
    _fields_ = [("kind", C.c_int), ("rank", C.c_int), ("shape", C.c_uint32 * 4), ("offset", C.c_uint64),
                ("nbytes", C.c_uint64), ("group_size", C.c_uint32), ("bits", C.c_uint32)]


class Choice(C.Structure):
    """rn_choice: the constrained choice and its allowed_statistics (generator.rs:99-194)."""
    _fields_ = [("token", C.c_uint32), ("constrained", C.c_int32), ("probability", C.c_float), ("mass", C.c_float)]


class WhistleConfig(C.Structure):
    _fields_ = [(n, _i) for n in ("mels", "frames", "d_model", "heads", "head_dim", "enc_layers", "dec_layers", "ffn",
                                  "vocab", "max_positions", "group")] + [("rope_theta", _f), ("norm_eps", _f)]


class WhistleEncHost(C.Structure):
    _fields_ = [("qkv", QMatHost), ("out", QMatHost), ("gate_up", QMatHost), ("down", QMatHost),
                ("norm_attn", _p), ("norm_ffn", _p), ("q_norm", _p), ("k_norm", _p)]


class WhistleDecHost(C.Structure):
    _fields_ = [("qkv", QMatHost), ("out", QMatHost), ("cross_q", QMatHost), ("cross_kv", QMatHost),
                ("cross_out", QMatHost), ("gate_up", QMatHost), ("down", QMatHost), ("norm_attn", _p),
                ("norm_cross", _p), ("post_norm", _p), ("norm_ffn", _p), ("q_norm", _p), ("k_norm", _p),
                ("gate", _f)]


class WhistleWeightsHost(C.Structure):
    _fields_ = [("conv1", _p), ("conv2", QMatHost), ("enc", _p), ("enc_norm", _p), ("position_gate", _f),
                ("embedding", QMatHost), ("dec", _p), ("dec_norm", _p)]


# Every symbol of include/rustyneedle.h with its signature (restype int unless noted).
SIGNATURES = {
    "rn_last_error": (C.c_char_p, []),
    "rn_abi_version": (_i, []),
    "rn_device_count": (_i, [C.POINTER(_i)]),
    "rn_device_set": (_i, [_i]),
    "rn_malloc": (_i, [C.POINTER(_p), _sz]),
    "rn_free": (_i, [_p]),
    "rn_memcpy_htod": (_i, [_p, _p, _sz]),
    "rn_memcpy_dtoh": (_i, [_p, _p, _sz]),
    "rn_memcpy_dtod": (_i, [_p, _p, _sz]),
    "rn_stream_create": (_i, [C.POINTER(_p)]),
    "rn_stream_destroy": (_i, [_p]),
    "rn_stream_synchronize": (_i, [_p]),
    "rn_event_create": (_i, [C.POINTER(_p)]),
    "rn_event_destroy": (_i, [_p]),
    "rn_event_record": (_i, [_p, _p]),
    "rn_event_elapsed_ms": (_i, [_p, _p, C.POINTER(_f)]),
    "rn_matrix_create_i8": (_i, [_p, _p, _i, _i, _i, _i, C.POINTER(_p)]),
    "rn_matrix_free": (_i, [_p]),
    "rn_matrix_shape": (_i, [_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)]),
    "rn_matrix_multiply_vector": (_i, [_p, _p, _p, _p, _p]),
    "rn_matrix_multiply_vector_rows": (_i, [_p, _p, _p, _i, _p]),
    "rn_matrix_multiply_fused": (_i, [C.POINTER(_p), _i, _p, C.POINTER(_p), _p]),
    "rn_matrix_multiply_batch": (_i, [_p, _p, _i, _p, _p, _p]),
    "rn_matrix_multiply_batch_noalloc": (_i, [_p, _p, _i, _p, _p, _p]),
    "rn_matrix_dequantise_row": (_i, [_p, _i, _p]),
    "rn_matrix_multiply_vector_host": (_i, [_p, _p, _p]),
    "rn_matrix_multiply_vector_float": (_i, [_p, _p, _p, _p]),
    "rn_matrix_multiply_batch_float": (_i, [_p, _p, _i, _p, _p]),
    "rn_matrix_multiply_batch_host": (_i, [_p, _p, _i, _p]),
    "rn_matrix_prepare_host": (_i, [_p, _p, _i, _p]),
    "rn_matrix_create_codebook": (_i, [_p, _sz, _i, _i, _i, _i, _p, _i, C.POINTER(_p)]),
    "rn_matrix_padded_columns": (_i, [_p, C.POINTER(_i)]),
    "rn_matrix_prepare": (_i, [_p, _p, _i, _p, _p]),
    "rn_archive_open": (_i, [C.c_char_p, C.POINTER(_p)]),
    "rn_archive_from_memory": (_i, [_p, _sz, C.POINTER(_p)]),
    "rn_archive_close": (_i, [_p]),
    "rn_archive_geometry": (_i, [_p, C.POINTER(Geometry)]),
    "rn_archive_codebook": (_i, [_p, C.POINTER(C.POINTER(_f)), C.POINTER(_i)]),
    "rn_archive_record": (_i, [_p, _i, C.POINTER(TensorRecord)]),
    "rn_archive_tensor_bytes": (_i, [_p, _i, C.POINTER(C.POINTER(C.c_uint8)), C.POINTER(_sz)]),
    "rn_matrix_from_archive": (_i, [_p, _i, C.POINTER(_p)]),
    "rn_choose_allowed": (_i, [_p, _p, _i, _i, _p, _p]),
    "rn_kronecker_apply": (_i, [_p, _p, _i, _p, _i, _i, _p, _p]),
    "rn_ladder_order": (_i, [_i, _p]),
    "rn_ladder_select": (_i, [_i, _i, _p]),
    "rn_lanes_create": (_i, [_i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, C.POINTER(_p)]),
    "rn_lanes_free": (_i, [_p]),
    "rn_lanes_route": (_i, [_p, _i, _i, _p, _p, _p, _p, _p]),
    "rn_lanes_combine": (_i, [_p, _p, _p, _p, _p, _p, _p]),
    "rn_frontend_create": (_i, [_i, _i, _i, _i, _p, C.POINTER(_p)]),
    "rn_frontend_free": (_i, [_p]),
    "rn_frontend_log_mel": (_i, [_p, _p, _i, _p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_f)]),
    "rn_session_choose_allowed": (_i, [_p, _p, C.POINTER(Choice)]),
    "rn_quantise_int8": (_i, [_p, _i, _i, _p, _p, _p]),
    "rn_fast_exp": (_i, [_p, _p, _i, _p]),
    "rn_silu": (_i, [_p, _p, _i, _p]),
    "rn_libm_exp": (_i, [_p, _p, _i, _p]),
    "rn_sigmoid": (_i, [_p, _p, _i, _p]),
    "rn_libm_log": (_i, [_p, _p, _i, _p]),
    "rn_reciprocal": (_i, [_p, _p, _i, _p]),
    "rn_zero_centred_norm": (_i, [_p, _p, _i, _i, _p, _p]),
    "rn_attend_heads": (_i, [_p, _p, _p, _p, _i, _i, _i, _p, _p]),
    "rn_model_create": (_i, [C.POINTER(Config), C.POINTER(WeightsHost), C.POINTER(_p)]),
    "rn_model_create_synthetic": (_i, [C.POINTER(Config), _u64, C.POINTER(_p)]),
    "rn_model_free": (_i, [_p]),
    "rn_model_config": (_i, [_p, C.POINTER(Config)]),
    "rn_model_rotary_table": (_i, [_p, _p, _p]),
    "rn_session_create": (_i, [_p, _i, C.POINTER(_p)]),
    "rn_session_free": (_i, [_p]),
    "rn_session_clone": (_i, [_p, C.POINTER(_p)]),
    "rn_session_len": (_i, [_p, C.POINTER(_i)]),
    "rn_session_truncate": (_i, [_p, _i]),
    "rn_session_set_cache": (_i, [_p, _i, _p, _p]),
    "rn_session_get_cache": (_i, [_p, _i, _p, _p]),
    "rn_session_push": (_i, [_p, _u32]),
    "rn_session_feed": (_i, [_p, _p, _i]),
    "rn_session_hidden": (_i, [_p, _p]),
    "rn_session_logits": (_i, [_p, _p]),
    "rn_session_decode_greedy": (_i, [_p, _u32, _i, _p]),
    "rn_session_stream": (_i, [_p, C.POINTER(_p)]),
    "rn_session_profile_step": (_i, [_p, _u32, _i, _p, _p]),
    "rn_batch_create": (_i, [_p, _i, _i, C.POINTER(_p)]),
    "rn_batch_free": (_i, [_p]),
    "rn_batch_set_cache": (_i, [_p, _i, _i, _p, _p]),
    "rn_batch_decode_greedy": (_i, [_p, _p, _i, _p]),
    "rn_batch_stream": (_i, [_p, C.POINTER(_p)]),
    "rn_batch_truncate": (_i, [_p, _p]),
    "rn_batch_logits": (_i, [_p, _p]),
    "rn_batch_get_cache": (_i, [_p, _i, _i, _p, _p]),
    "rn_whistle_create_synthetic": (_i, [C.POINTER(WhistleConfig), _u64, C.POINTER(_p)]),
    "rn_whistle_create": (_i, [C.POINTER(WhistleConfig), C.POINTER(WhistleWeightsHost), C.POINTER(_p)]),
    "rn_whistle_free": (_i, [_p]),
    "rn_whistle_frames": (_i, [_p, C.POINTER(_i)]),
    "rn_whistle_tables": (_i, [_p, _p, _p]),
    "rn_whistle_stem": (_i, [_p, _p, _p]),
    "rn_whistle_encode": (_i, [_p, _p, _p]),
    "rn_whistle_encode_samples": (_i, [_p, _p, _p, _i, _p, _p]),
    "rn_whistle_memory": (_i, [_p, _p, _p, _p, _p]),
    "rn_whistle_reset": (_i, [_p]),
    "rn_whistle_push": (_i, [_p, _u32]),
    "rn_whistle_logits": (_i, [_p, _p]),
    "rn_whistle_decode_greedy": (_i, [_p, _u32, _i, _p]),
    "rn_whistle_stream": (_i, [_p, C.POINTER(_p)]),
    "rn_n3_model_open": (_i, [_p, _i, C.POINTER(_p)]),
    "rn_n3_model_free": (_i, [_p]),
    "rn_n3_model_active_layers": (_i, [_p, _p, C.POINTER(_i)]),
    "rn_n3_model_output_vocab": (_i, [_p, C.POINTER(_i)]),
    "rn_n3_session_create": (_i, [_p, _i, C.POINTER(_p)]),
    "rn_n3_session_free": (_i, [_p]),
    "rn_n3_session_push": (_i, [_p, _u32]),
    "rn_n3_session_feed": (_i, [_p, _p, _i]),
    "rn_n3_session_decode_greedy": (_i, [_p, _u32, _i, _p]),
    "rn_n3_session_clone": (_i, [_p, C.POINTER(_p)]),
    "rn_n3_session_run_turn": (_i, [_p, _i, _i, _p, _i, _p, C.POINTER(_i), C.POINTER(_i)]),
    "rn_n3_session_choose_allowed": (_i, [_p, _p, C.POINTER(Choice)]),
    "rn_n3_session_length": (_i, [_p, C.POINTER(_i)]),
    "rn_n3_session_logits": (_i, [_p, _p]),
    "rn_n3_session_hidden": (_i, [_p, _p]),
    "rn_n3_session_cells": (_i, [_p, _p]),
    "rn_n3_session_head_output": (_i, [_p, _i, _p, _i, C.POINTER(_i)]),
    "rn_n3_session_pooled_readout": (_i, [_p, _i, _p, _i, C.POINTER(_i)]),
    "rn_n3_session_cache": (_i, [_p, _i, _p, _p, _p, _p]),
    "rn_n3_session_stream": (_i, [_p, C.POINTER(_p)]),
    "rn_synth_codes": (_i, [_u64, C.c_char_p, _p, _sz]),
    "rn_synth_uniform": (_i, [_u64, C.c_char_p, _f, _f, _p, _sz]),
    "rn_synth_normal": (_i, [_u64, C.c_char_p, _f, _p, _sz]),
    "rn_synth_normal_f16": (_i, [_u64, C.c_char_p, _p, _sz]),
    "rn_synth_tokens": (_i, [_u64, C.c_char_p, _u32, _p, _sz]),
}

for _name, (_res, _args) in SIGNATURES.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


class RnError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def check(rc: int) -> None:
    if rc != RN_OK:
        raise RnError(rc, lib.rn_last_error().decode(errors="replace"))


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays handed to the C ABI must be contiguous"
    return a.ctypes.data


def device_count() -> int:
    n = _i(0)
    check(lib.rn_device_count(C.byref(n)))
    return n.value


# ---- device plumbing --------------------------------------------------------------

class DeviceBuffer:
    """Device memory owned by Python (rn_malloc/rn_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _p()
        check(lib.rn_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib.rn_memcpy_htod(self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib.rn_memcpy_dtoh(_ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib.rn_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if getattr(self, "ptr", None):
                lib.rn_free(self.ptr)
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _p()
        check(lib.rn_stream_create(C.byref(p)))
        self.handle = p.value

    def synchronize(self) -> None:
        check(lib.rn_stream_synchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib.rn_stream_destroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _p()
        check(lib.rn_event_create(C.byref(p)))
        self.handle = p.value

    def record(self, stream) -> None:
        check(lib.rn_event_record(self.handle, stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = _f(0)
        check(lib.rn_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib.rn_event_destroy(self.handle)
        except Exception:
            pass


# ---- kernels API ------------------------------------------------------------------

class QuantisedMatrix:
    """crates/kernels/src/matrix.rs:19-441 for int8 codes and fp32 per-32 scales."""

    def __init__(self, codes: np.ndarray, scales: np.ndarray, form: int = FORM_PANEL, group: int = 32):
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        rows, cols = codes.shape
        assert scales.shape == (rows, cols // group)
        h = _p()
        check(lib.rn_matrix_create_i8(_ptr(codes), _ptr(scales), rows, cols, group, form, C.byref(h)))
        self.handle = h.value
        self.rows, self.columns, self.group, self.form = rows, cols, group, form

    def multiply_vector(self, x_dev: int, y_dev: int, acc_dev: Optional[int] = None, stream=None) -> None:
        check(lib.rn_matrix_multiply_vector(self.handle, x_dev, y_dev, acc_dev, stream))

    def multiply_vector_rows(self, x_dev: int, y_dev: int, rows_per_block: int, stream=None) -> None:
        """The same product with the kernel instance of `rows_per_block` rows a block."""
        check(lib.rn_matrix_multiply_vector_rows(self.handle, x_dev, y_dev, int(rows_per_block), stream))

    def multiply_vector_host(self, x: np.ndarray, with_acc: bool = False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        assert x.shape == (self.columns,)
        xd = DeviceBuffer.from_array(x)
        yd = DeviceBuffer(4 * self.rows)
        ad = DeviceBuffer(4 * self.rows * (self.columns // self.group)) if with_acc else None
        self.multiply_vector(xd.ptr, yd.ptr, ad.ptr if ad else None)
        check(lib.rn_stream_synchronize(None))
        y = yd.download(np.float32, (self.rows,))
        if with_acc:
            return y, ad.download(np.int32, (self.rows, self.columns // self.group))
        return y

    def multiply_batch_host(self, x: np.ndarray, with_acc: bool = False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        count = x.shape[0]
        assert x.shape == (count, self.columns)
        xd = DeviceBuffer.from_array(x)
        yd = DeviceBuffer(4 * count * self.rows)
        ad = DeviceBuffer(4 * count * self.rows * (self.columns // self.group)) if with_acc else None
        check(lib.rn_matrix_multiply_batch(self.handle, xd.ptr, count, yd.ptr, ad.ptr if ad else None, None))
        check(lib.rn_stream_synchronize(None))
        y = yd.download(np.float32, (count, self.rows))
        if with_acc:
            return y, ad.download(np.int32, (count, self.rows, self.columns // self.group))
        return y

    def dequantise_row(self, row: int) -> np.ndarray:
        out = np.empty(self.columns, dtype=np.float32)
        check(lib.rn_matrix_dequantise_row(self.handle, row, _ptr(out)))
        return out

    def __del__(self):
        try:
            if self.handle:
                lib.rn_matrix_free(self.handle)
        except Exception:
            pass


class CodebookMatrix:
    """QuantisedMatrix (crates/kernels/src/matrix.rs:19-441) over a codebook-quantised
    record: the archive blob (packed indices LSB first, then fp16 group norms), the
    archive's 28 codebook levels, bits 2, 4 or 5 (ternary)."""

    def __init__(self, blob: np.ndarray, rows: int, columns: int, group: int, bits: int, codebook: np.ndarray):
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        codebook = np.ascontiguousarray(codebook, dtype=np.float32)
        h = _p()
        check(lib.rn_matrix_create_codebook(_ptr(blob), blob.size, rows, columns, group, bits, _ptr(codebook),
                                            codebook.size, C.byref(h)))
        self._adopt(h.value, rows, columns, group, bits)

    @classmethod
    def from_handle(cls, handle: int, rows: int, columns: int, group: int, bits: int) -> "CodebookMatrix":
        m = cls.__new__(cls)
        m._adopt(handle, rows, columns, group, bits)
        return m

    def _adopt(self, handle: int, rows: int, columns: int, group: int, bits: int) -> None:
        self.handle = handle
        self.rows, self.columns, self.group, self.bits = rows, columns, group, bits
        padded = _i()
        check(lib.rn_matrix_padded_columns(self.handle, C.byref(padded)))
        self.padded = padded.value
        self.groups = self.padded // group

    def prepare(self, x_dev: int, count: int, rotated_dev: int, stream=None) -> None:
        check(lib.rn_matrix_prepare(self.handle, x_dev, count, rotated_dev, stream))

    def prepare_host(self, x: np.ndarray) -> np.ndarray:
        """QuantisedMatrix::prepare(_batch) (matrix.rs:123-138): [count][columns] -> [count][padded]."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.columns)
        xd = DeviceBuffer.from_array(x)
        rd = DeviceBuffer(4 * x.shape[0] * self.padded)
        self.prepare(xd.ptr, x.shape[0], rd.ptr)
        check(lib.rn_stream_synchronize(None))
        return rd.download(np.float32, (x.shape[0], self.padded))

    def multiply_batch_host(self, rotated: np.ndarray, with_acc: bool = False):
        """multiply_vector (one row) or multiply_batch over rotated inputs [count][padded]."""
        rotated = np.ascontiguousarray(rotated, dtype=np.float32).reshape(-1, self.padded)
        count = rotated.shape[0]
        xd = DeviceBuffer.from_array(rotated)
        yd = DeviceBuffer(4 * count * self.rows)
        ad = DeviceBuffer(4 * count * self.rows * self.groups) if with_acc else None
        if count == 1:
            check(lib.rn_matrix_multiply_vector(self.handle, xd.ptr, yd.ptr, ad.ptr if ad else None, None))
        else:
            check(lib.rn_matrix_multiply_batch(self.handle, xd.ptr, count, yd.ptr, ad.ptr if ad else None, None))
        check(lib.rn_stream_synchronize(None))
        y = yd.download(np.float32, (count, self.rows))
        if with_acc:
            return y, ad.download(np.int32, (count, self.rows, self.groups))
        return y

    def multiply_float_host(self, rotated: np.ndarray, batch: bool = False) -> np.ndarray:
        """The float path on rotated inputs [count][padded]: fill_rows_float, or
        with batch multiply_batch's float tile (matrix.rs:356-440)."""
        rotated = np.ascontiguousarray(rotated, dtype=np.float32).reshape(-1, self.padded)
        count = rotated.shape[0]
        xd = DeviceBuffer.from_array(rotated)
        yd = DeviceBuffer(4 * count * self.rows)
        if batch:
            check(lib.rn_matrix_multiply_batch_float(self.handle, xd.ptr, count, yd.ptr, None))
        else:
            for t in range(count):
                check(lib.rn_matrix_multiply_vector_float(self.handle, xd.ptr + 4 * t * self.padded,
                                                          yd.ptr + 4 * t * self.rows, None))
        check(lib.rn_stream_synchronize(None))
        return yd.download(np.float32, (count, self.rows))

    def dequantise_row(self, row: int) -> np.ndarray:
        out = np.empty(self.columns, dtype=np.float32)
        check(lib.rn_matrix_dequantise_row(self.handle, row, _ptr(out)))
        return out

    def __del__(self):
        try:
            if self.handle:
                lib.rn_matrix_free(self.handle)
        except Exception:
            pass


class Archive:
    """cact::Archive (crates/cact/src/archive.rs): a memory-mapped .cact file."""

    def __init__(self, path: Optional[str] = None, data: Optional[bytes] = None):
        h = _p()
        if data is not None:
            buf = np.frombuffer(data, dtype=np.uint8)
            check(lib.rn_archive_from_memory(_ptr(buf) if buf.size else None, buf.size, C.byref(h)))
        else:
            check(lib.rn_archive_open(os.fsencode(path), C.byref(h)))
        self.handle = h.value

    def geometry(self) -> dict:
        g = Geometry()
        check(lib.rn_archive_geometry(self.handle, C.byref(g)))
        out = {name: getattr(g, name) for name, _ in Geometry._fields_}
        out["engram_orders"] = list(g.engram_orders)[:g.engram_order_count]
        out["engram_sites"] = list(g.engram_sites)[:g.engram_site_count]
        return out

    def codebook(self) -> np.ndarray:
        ptr, n = C.POINTER(_f)(), _i()
        check(lib.rn_archive_codebook(self.handle, C.byref(ptr), C.byref(n)))
        return np.ctypeslib.as_array(ptr, (n.value,)).copy() if n.value else np.zeros(0, np.float32)

    def record(self, index: int) -> dict:
        r = TensorRecord()
        check(lib.rn_archive_record(self.handle, index, C.byref(r)))
        return dict(kind=r.kind, shape=list(r.shape)[:r.rank], offset=r.offset, nbytes=r.nbytes,
                    group_size=r.group_size, bits=r.bits)

    def tensor_bytes(self, index: int) -> np.ndarray:
        ptr, n = C.POINTER(C.c_uint8)(), _sz()
        check(lib.rn_archive_tensor_bytes(self.handle, index, C.byref(ptr), C.byref(n)))
        return np.ctypeslib.as_array(ptr, (n.value,)).copy() if n.value else np.zeros(0, np.uint8)

    def matrix(self, index: int) -> "CodebookMatrix":
        """QuantisedMatrix::from_archive (matrix.rs:35-40)."""
        h = _p()
        check(lib.rn_matrix_from_archive(self.handle, index, C.byref(h)))
        r = self.record(index)
        return CodebookMatrix.from_handle(h.value, r["shape"][0], r["shape"][1] if len(r["shape"]) > 1 else 1,
                                          r["group_size"], r["bits"])

    def __del__(self):
        try:
            if self.handle:
                lib.rn_archive_close(self.handle)
        except Exception:
            pass


# Lloyd-Max levels of a unit Gaussian for 2, 3 and 4 bits (ascending); divided by
# sqrt(group) they approximate the coordinates of a unit vector of that length.
_LLOYD_MAX = {
    2: [-1.5104, -0.4528, 0.4528, 1.5104],
    3: [-2.1520, -1.3439, -0.7560, -0.2451, 0.2451, 0.7560, 1.3439, 2.1520],
    4: [-2.7326, -2.0690, -1.6181, -1.2562, -0.9424, -0.6568, -0.3881, -0.1284,
        0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326],
}


def synthetic_codebook(group: int) -> np.ndarray:
    """28 archive levels (2-bit, 3-bit, 4-bit) for unit-sphere groups of `group`."""
    s = np.float32(1.0) / np.sqrt(np.float32(group))
    return np.concatenate([np.float32(_LLOYD_MAX[b]) * s for b in (2, 3, 4)]).astype(np.float32)


def synthetic_codebook_blob(rows: int, columns: int, group: int, bits: int, seed: int = SEED,
                            name: str = "codebook") -> np.ndarray:
    """A record blob of seeded random indices (every byte but 0x80) and fp16 norms in [0.5, 2)."""
    padded = -(-columns // group) * group
    ib = 2 if bits == 5 else bits
    packed = synth_codes(seed, name + ".packed", (rows * padded * ib // 8,)).view(np.uint8)
    norms = synth_uniform(seed, name + ".norms", 0.5, 2.0, (rows * (padded // group),)).astype(np.float16)
    return np.concatenate([packed, norms.view(np.uint8)])


def multiply_fused_host(matrices, x: np.ndarray):
    """QuantisedMatrix::multiply_fused (matrix.rs:167-193) on one shared input."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    xd = DeviceBuffer.from_array(x)
    outs = [DeviceBuffer(4 * m.rows) for m in matrices]
    hs = (_p * len(matrices))(*[m.handle for m in matrices])
    ys = (_p * len(matrices))(*[o.ptr for o in outs])
    check(lib.rn_matrix_multiply_fused(hs, len(matrices), xd.ptr, ys, None))
    check(lib.rn_stream_synchronize(None))
    return [o.download(np.float32, (m.rows,)) for o, m in zip(outs, matrices)]


def _elementwise(fn, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    xd = DeviceBuffer.from_array(x)
    yd = DeviceBuffer(x.nbytes)
    check(fn(xd.ptr, yd.ptr, x.size, None))
    check(lib.rn_stream_synchronize(None))
    return yd.download(np.float32, x.shape)


def fast_exp(x: np.ndarray) -> np.ndarray:
    return _elementwise(lib.rn_fast_exp, x)


def silu(x: np.ndarray) -> np.ndarray:
    return _elementwise(lib.rn_silu, x)


def libm_exp(x: np.ndarray) -> np.ndarray:
    """f32::exp (the C library's expf) on the device."""
    return _elementwise(lib.rn_libm_exp, x)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return _elementwise(lib.rn_sigmoid, x)


def libm_log(x: np.ndarray) -> np.ndarray:
    """f32::ln (the C library's logf) on the device."""
    return _elementwise(lib.rn_libm_log, x)


def reciprocal(x: np.ndarray) -> np.ndarray:
    """The fused step's reciprocal (v_rcp_f32 and one Newton step) on the device;
    the IEEE 1/x for x in [2^-126, 2^126)."""
    return _elementwise(lib.rn_reciprocal, x)


def quantise_int8(x: np.ndarray):
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    count, cols = x.shape
    xd = DeviceBuffer.from_array(x)
    cd = DeviceBuffer(count * cols)
    sd = DeviceBuffer(4 * count)
    check(lib.rn_quantise_int8(xd.ptr, count, cols, cd.ptr, sd.ptr, None))
    check(lib.rn_stream_synchronize(None))
    return cd.download(np.int8, (count, cols)), sd.download(np.float32, (count,))


def zero_centred_norm(x: np.ndarray, gain: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    count, n = x.shape
    xd = DeviceBuffer.from_array(x)
    gd = DeviceBuffer.from_array(np.ascontiguousarray(gain, dtype=np.float32))
    od = DeviceBuffer(x.nbytes)
    check(lib.rn_zero_centred_norm(xd.ptr, gd.ptr, count, n, od.ptr, None))
    check(lib.rn_stream_synchronize(None))
    return od.download(np.float32, (count, n))


def attend_heads(q: np.ndarray, K: np.ndarray, V: np.ndarray, lengths: np.ndarray) -> np.ndarray:
    """q [count][64] f32; K, V [count][stride][64] float16; lengths [count]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    K = np.ascontiguousarray(K, dtype=np.float16)
    V = np.ascontiguousarray(V, dtype=np.float16)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    count, stride, hd = K.shape
    bufs = [DeviceBuffer.from_array(a) for a in (q, K, V, lengths)]
    od = DeviceBuffer(4 * count * hd)
    check(lib.rn_attend_heads(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, count, stride, hd, od.ptr, None))
    check(lib.rn_stream_synchronize(None))
    return od.download(np.float32, (count, hd))


# ---- synthetic inputs ---------------------------------------------------------------

def synth_codes(seed: int, name: str, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.int8)
    check(lib.rn_synth_codes(seed, name.encode(), _ptr(out), out.size))
    return out


def synth_uniform(seed: int, name: str, lo: float, hi: float, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    check(lib.rn_synth_uniform(seed, name.encode(), lo, hi, _ptr(out), out.size))
    return out


def synth_normal(seed: int, name: str, sigma: float, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    check(lib.rn_synth_normal(seed, name.encode(), sigma, _ptr(out), out.size))
    return out


def synth_normal_f16(seed: int, name: str, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    check(lib.rn_synth_normal_f16(seed, name.encode(), _ptr(out), out.size))
    return out.view(np.float16)


def synth_tokens(seed: int, name: str, vocab: int, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint32)
    check(lib.rn_synth_tokens(seed, name.encode(), vocab, _ptr(out), out.size))
    return out


def synthetic_weights(config: dict, seed: int = SEED) -> dict:
    """The tensors rn_model_create_synthetic draws, by the same names: codes
    U{-127..127}, scales U[1e-3, 1e-2], zero-centred gains N(0, 0.1)."""
    d, f, vocab = config["d_model"], config["ffn"], config["vocab"]

    def q(name, rows, cols):
        return (synth_codes(seed, name + ".codes", (rows, cols)),
                synth_uniform(seed, name + ".scales", 1e-3, 1e-2, (rows, cols // 32)))

    layers = []
    for l in range(config["layers"]):
        p = f"layers.{l}."
        layers.append(dict(qkv=q(p + "qkv", 3 * d, d), out=q(p + "out", d, d),
                           gate_up=q(p + "gate_up", 2 * f, d), down=q(p + "down", d, f),
                           norm_attn=synth_normal(seed, p + "norm_attn", 0.1, (d,)),
                           norm_ffn=synth_normal(seed, p + "norm_ffn", 0.1, (d,))))
    return dict(layers=layers, embedding=q("embedding", vocab, d),
                norm_final=synth_normal(seed, "norm_final", 0.1, (d,)))


def synthetic_whistle_weights(config: dict, seed: int = SEED) -> dict:
    """The tensors rn_whistle_create_synthetic draws, by the same names: codes
    U{-127..127}, scales U[1e-3, 1e-2], gains N(0, 0.1), the fp32 first stem
    convolution N(0, 1/sqrt(fan-in)), the position and layer gates N(0, 1)."""
    d, f, hd, M, V = config["d_model"], config["ffn"], config["head_dim"], config["mels"], config["vocab"]

    def q(name, rows, cols):
        return (synth_codes(seed, name + ".codes", (rows, cols)),
                synth_uniform(seed, name + ".scales", 1e-3, 1e-2, (rows, cols // 32)))

    def g(name, n):
        return synth_normal(seed, name, 0.1, (n,))

    enc = []
    for l in range(config["enc_layers"]):
        p = f"whistle.enc.{l}."
        enc.append(dict(qkv=q(p + "qkv", 3 * d, d), out=q(p + "out", d, d), gate_up=q(p + "gate_up", 2 * f, d),
                        down=q(p + "down", d, f), norm_attn=g(p + "norm_attn", d), norm_ffn=g(p + "norm_ffn", d),
                        q_norm=g(p + "q_norm", hd), k_norm=g(p + "k_norm", hd)))
    dec = []
    for l in range(config["dec_layers"]):
        p = f"whistle.dec.{l}."
        dec.append(dict(qkv=q(p + "qkv", 3 * d, d), out=q(p + "out", d, d), cross_q=q(p + "cross_q", d, d),
                        cross_kv=q(p + "cross_kv", 2 * d, d), cross_out=q(p + "cross_out", d, d),
                        gate_up=q(p + "gate_up", 2 * f, d), down=q(p + "down", d, f),
                        norm_attn=g(p + "norm_attn", d), norm_cross=g(p + "norm_cross", d),
                        post_norm=g(p + "post_norm", d), norm_ffn=g(p + "norm_ffn", d),
                        q_norm=g(p + "q_norm", hd), k_norm=g(p + "k_norm", hd),
                        gate=float(synth_normal(seed, p + "gate", 1.0, (1,))[0])))
    conv_sigma = float(np.float32(1.0) / np.sqrt(np.float32(3 * M)))
    return dict(conv1=synth_normal(seed, "whistle.conv1", conv_sigma, (d, 3, M)),
                conv2=q("whistle.conv2", d, 3 * d), enc=enc, enc_norm=g("whistle.enc_norm", d),
                position_gate=float(synth_normal(seed, "whistle.position_gate", 1.0, (1,))[0]),
                embedding=q("whistle.embedding", V, d), dec=dec, dec_norm=g("whistle.dec_norm", d))


def synthetic_mel(config: dict, name: str = "whistle.mel", seed: int = SEED) -> np.ndarray:
    """N(0, 1) log-mel input [frames][mels]."""
    return synth_normal(seed, name, 1.0, (config["frames"], config["mels"]))


def synthetic_cache(config: dict, length: int, name: str, seed: int = SEED):
    """N(0,1) fp16 keys and values [layers][heads][length][head_dim]."""
    shape = (config["layers"], config["heads"], length, config["head_dim"])
    return synth_normal_f16(seed, name + ".k", shape), synth_normal_f16(seed, name + ".v", shape)


# ---- model API ----------------------------------------------------------------------

def _config_struct(config: dict) -> Config:
    return Config(config["layers"], config["d_model"], config["heads"], config["head_dim"], config["ffn"],
                  config["vocab"], config["group"], config["max_positions"], config["rope_theta"],
                  config["norm_eps"])


class Model:
    """Model::open / Model::build (crates/model/src/model.rs:51-74)."""

    def __init__(self, config: dict, weights: Optional[dict] = None, seed: Optional[int] = None):
        self.config = dict(config)
        self._cfg = _config_struct(self.config)
        h = _p()
        if weights is None:
            check(lib.rn_model_create_synthetic(C.byref(self._cfg), SEED if seed is None else seed, C.byref(h)))
        else:
            layers = (LayerHost * self.config["layers"])()
            keep = []
            for l, lw in enumerate(weights["layers"]):
                arrs = {k: (np.ascontiguousarray(v[0]), np.ascontiguousarray(v[1])) if isinstance(v, tuple)
                        else np.ascontiguousarray(v) for k, v in lw.items()}
                keep.append(arrs)
                layers[l] = LayerHost(QMatHost(_ptr(arrs["qkv"][0]), _ptr(arrs["qkv"][1])),
                                      QMatHost(_ptr(arrs["out"][0]), _ptr(arrs["out"][1])),
                                      QMatHost(_ptr(arrs["gate_up"][0]), _ptr(arrs["gate_up"][1])),
                                      QMatHost(_ptr(arrs["down"][0]), _ptr(arrs["down"][1])),
                                      _ptr(arrs["norm_attn"]), _ptr(arrs["norm_ffn"]))
            emb = (np.ascontiguousarray(weights["embedding"][0]), np.ascontiguousarray(weights["embedding"][1]))
            nf = np.ascontiguousarray(weights["norm_final"])
            w = WeightsHost(QMatHost(_ptr(emb[0]), _ptr(emb[1])), _ptr(nf), C.addressof(layers))
            check(lib.rn_model_create(C.byref(self._cfg), C.byref(w), C.byref(h)))
        self.handle = h.value

    def rotary_table(self):
        c = self.config
        cos = np.empty((c["max_positions"], c["head_dim"] // 2), dtype=np.float32)
        sin = np.empty_like(cos)
        check(lib.rn_model_rotary_table(self.handle, _ptr(cos), _ptr(sin)))
        return cos, sin

    def session(self, capacity: int) -> "Session":
        return Session(self, capacity)

    def __del__(self):
        try:
            if self.handle:
                lib.rn_model_free(self.handle)
        except Exception:
            pass


class Session:
    """Session (crates/model/src/session.rs:17-177) with a device KV cache."""

    def __init__(self, model: Model, capacity: int, _handle: Optional[int] = None):
        self.model = model
        self.capacity = capacity
        if _handle is None:
            h = _p()
            check(lib.rn_session_create(model.handle, capacity, C.byref(h)))
            _handle = h.value
        self.handle = _handle

    def __len__(self) -> int:
        n = _i(0)
        check(lib.rn_session_len(self.handle, C.byref(n)))
        return n.value

    def truncate(self, length: int) -> None:
        check(lib.rn_session_truncate(self.handle, length))

    def clone(self) -> "Session":
        h = _p()
        check(lib.rn_session_clone(self.handle, C.byref(h)))
        return Session(self.model, self.capacity, h.value)

    def set_cache(self, keys: np.ndarray, values: np.ndarray) -> None:
        keys = np.ascontiguousarray(keys).view(np.uint16)
        values = np.ascontiguousarray(values).view(np.uint16)
        check(lib.rn_session_set_cache(self.handle, keys.shape[2], _ptr(keys), _ptr(values)))

    def get_cache(self, length: Optional[int] = None):
        c = self.model.config
        length = len(self) if length is None else length
        shape = (c["layers"], c["heads"], length, c["head_dim"])
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        check(lib.rn_session_get_cache(self.handle, length, _ptr(k), _ptr(v)))
        return k.view(np.float16), v.view(np.float16)

    def push(self, token: int) -> None:
        check(lib.rn_session_push(self.handle, int(token)))

    def feed(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        check(lib.rn_session_feed(self.handle, _ptr(t), t.size))

    def hidden(self) -> np.ndarray:
        out = np.empty(self.model.config["d_model"], dtype=np.float32)
        check(lib.rn_session_hidden(self.handle, _ptr(out)))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.config["vocab"], dtype=np.float32)
        check(lib.rn_session_logits(self.handle, _ptr(out)))
        return out

    def choose_allowed(self, allowed: np.ndarray):
        """generator.rs:99-117: (token, constrained, probability, mass) over this step's logits."""
        mask = np.ascontiguousarray(allowed, dtype=np.uint8)
        assert mask.shape == (self.model.config["vocab"],)
        c = Choice()
        check(lib.rn_session_choose_allowed(self.handle, _ptr(mask), C.byref(c)))
        return int(c.token), bool(c.constrained), np.float32(c.probability), np.float32(c.mass)

    def decode_greedy(self, first: int, steps: int) -> np.ndarray:
        ids = np.empty(steps, dtype=np.uint32)
        check(lib.rn_session_decode_greedy(self.handle, int(first), steps, _ptr(ids)))
        return ids

    def stream(self) -> int:
        p = _p()
        check(lib.rn_session_stream(self.handle, C.byref(p)))
        return p.value

    def profile_step(self, first: int, steps: int) -> dict:
        """Average microseconds per launch and launches per step of each kernel
        kind of the greedy decode step (HIP events after every kernel)."""
        us = np.zeros(len(PROFILE_KINDS), dtype=np.float32)
        count = np.zeros(len(PROFILE_KINDS), dtype=np.int32)
        check(lib.rn_session_profile_step(self.handle, int(first), steps, _ptr(us), _ptr(count)))
        return {k: dict(us=float(us[i]), per_step=int(count[i])) for i, k in enumerate(PROFILE_KINDS)}

    def __del__(self):
        try:
            if self.handle:
                lib.rn_session_free(self.handle)
        except Exception:
            pass


class Batch:
    """`count` independent sequences decoded together (M=count MFMA products)."""

    def __init__(self, model: Model, count: int, capacity: int):
        self.model = model
        self.count = count
        h = _p()
        check(lib.rn_batch_create(model.handle, count, capacity, C.byref(h)))
        self.handle = h.value

    def set_cache(self, sequence: int, keys: np.ndarray, values: np.ndarray) -> None:
        keys = np.ascontiguousarray(keys).view(np.uint16)
        values = np.ascontiguousarray(values).view(np.uint16)
        check(lib.rn_batch_set_cache(self.handle, sequence, keys.shape[2], _ptr(keys), _ptr(values)))

    def decode_greedy(self, first, steps: int) -> np.ndarray:
        first = np.ascontiguousarray(first, dtype=np.uint32)
        assert first.size == self.count
        ids = np.empty((self.count, steps), dtype=np.uint32)
        check(lib.rn_batch_decode_greedy(self.handle, _ptr(first), steps, _ptr(ids)))
        return ids

    def truncate(self, lengths) -> None:
        lengths = np.ascontiguousarray(lengths, dtype=np.int32)
        assert lengths.size == self.count
        check(lib.rn_batch_truncate(self.handle, _ptr(lengths)))

    def logits(self) -> np.ndarray:
        """The last decoded step's logits of every sequence, [count][vocab]."""
        out = np.empty((self.count, self.model.config["vocab"]), dtype=np.float32)
        check(lib.rn_batch_logits(self.handle, _ptr(out)))
        return out

    def get_cache(self, sequence: int, length: int):
        c = self.model.config
        shape = (c["layers"], c["heads"], length, c["head_dim"])
        k = np.empty(shape, dtype=np.uint16)
        v = np.empty(shape, dtype=np.uint16)
        check(lib.rn_batch_get_cache(self.handle, sequence, length, _ptr(k), _ptr(v)))
        return k.view(np.float16), v.view(np.float16)

    def stream(self) -> int:
        p = _p()
        check(lib.rn_batch_stream(self.handle, C.byref(p)))
        return p.value

    def __del__(self):
        try:
            if self.handle:
                lib.rn_batch_free(self.handle)
        except Exception:
            pass


# ---- Whistle-style speech path ---------------------------------------------------

class Whistle:
    """crates/whistle Whistle (lib.rs:77-312): the model, its encoder work buffers
    and one decoder session on the device, from host weights (the dict of
    synthetic_whistle_weights) or drawn on the library side from `seed`."""

    def __init__(self, config: dict, seed: int = SEED, weights: Optional[dict] = None):
        self.config = c = dict(config)
        self._cfg = WhistleConfig(*[c[n] for n in ("mels", "frames", "d_model", "heads", "head_dim", "enc_layers",
                                                   "dec_layers", "ffn", "vocab", "max_positions", "group")],
                                  c["rope_theta"], c["norm_eps"])
        h = _p()
        if weights is None:
            check(lib.rn_whistle_create_synthetic(C.byref(self._cfg), seed, C.byref(h)))
        else:
            qm = lambda pair: QMatHost(_ptr(pair[0]), _ptr(pair[1]))
            enc = (WhistleEncHost * c["enc_layers"])()
            for l, lw in enumerate(weights["enc"]):
                enc[l] = WhistleEncHost(qm(lw["qkv"]), qm(lw["out"]), qm(lw["gate_up"]), qm(lw["down"]),
                                        _ptr(lw["norm_attn"]), _ptr(lw["norm_ffn"]), _ptr(lw["q_norm"]),
                                        _ptr(lw["k_norm"]))
            dec = (WhistleDecHost * c["dec_layers"])()
            for l, lw in enumerate(weights["dec"]):
                dec[l] = WhistleDecHost(qm(lw["qkv"]), qm(lw["out"]), qm(lw["cross_q"]), qm(lw["cross_kv"]),
                                        qm(lw["cross_out"]), qm(lw["gate_up"]), qm(lw["down"]), _ptr(lw["norm_attn"]),
                                        _ptr(lw["norm_cross"]), _ptr(lw["post_norm"]), _ptr(lw["norm_ffn"]),
                                        _ptr(lw["q_norm"]), _ptr(lw["k_norm"]), float(lw["gate"]))
            wh = WhistleWeightsHost(_ptr(weights["conv1"]), qm(weights["conv2"]), C.addressof(enc),
                                    _ptr(weights["enc_norm"]), float(weights["position_gate"]),
                                    qm(weights["embedding"]), C.addressof(dec), _ptr(weights["dec_norm"]))
            check(lib.rn_whistle_create(C.byref(self._cfg), C.byref(wh), C.byref(h)))
        self.handle = h.value
        n = _i()
        check(lib.rn_whistle_frames(self.handle, C.byref(n)))
        self.frames = n.value

    def tables(self):
        pos = np.empty((self.frames, self.config["d_model"]), np.float32)
        gains = np.empty(self.config["dec_layers"], np.float32)
        check(lib.rn_whistle_tables(self.handle, _ptr(pos), _ptr(gains)))
        return pos, gains

    def stem(self, mel: np.ndarray) -> np.ndarray:
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        assert mel.shape == (self.config["frames"], self.config["mels"])
        out = np.empty((self.frames, self.config["d_model"]), np.float32)
        check(lib.rn_whistle_stem(self.handle, _ptr(mel), _ptr(out)))
        return out

    def encode(self, mel: np.ndarray, copy_out: bool = True):
        mel = np.ascontiguousarray(mel, dtype=np.float32)
        assert mel.shape == (self.config["frames"], self.config["mels"])
        out = np.empty((self.frames, self.config["d_model"]), np.float32) if copy_out else None
        check(lib.rn_whistle_encode(self.handle, _ptr(mel), _ptr(out) if copy_out else None))
        return out

    def encode_samples(self, frontend: "Frontend", samples: np.ndarray, copy_out: bool = True):
        """Whistle::encode from samples: the log-mel features stay on the device."""
        x = np.ascontiguousarray(samples, dtype=np.float32)
        out = np.empty((self.frames, self.config["d_model"]), np.float32) if copy_out else None
        spread = C.c_float()
        check(lib.rn_whistle_encode_samples(self.handle, frontend.handle, _ptr(x) if x.size else None, x.size,
                                            _ptr(out) if copy_out else None, C.byref(spread)))
        return out, np.float32(spread.value)

    def memory(self):
        c = self.config
        shape = (c["dec_layers"], self.frames, c["heads"], c["head_dim"])
        mk, mv = np.empty(shape, np.int8), np.empty(shape, np.int8)
        ks, vs = np.empty(shape[:3], np.float32), np.empty(shape[:3], np.float32)
        check(lib.rn_whistle_memory(self.handle, _ptr(mk), _ptr(ks), _ptr(mv), _ptr(vs)))
        return mk, ks, mv, vs

    def reset(self) -> None:
        check(lib.rn_whistle_reset(self.handle))

    def push(self, token: int) -> None:
        check(lib.rn_whistle_push(self.handle, int(token)))

    def logits(self) -> np.ndarray:
        out = np.empty(self.config["vocab"], np.float32)
        check(lib.rn_whistle_logits(self.handle, _ptr(out)))
        return out

    def decode_greedy(self, first: int, steps: int) -> np.ndarray:
        ids = np.empty(steps, np.uint32)
        check(lib.rn_whistle_decode_greedy(self.handle, int(first), int(steps), _ptr(ids)))
        return ids

    def stream(self) -> int:
        s = _p()
        check(lib.rn_whistle_stream(self.handle, C.byref(s)))
        return s.value

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib.rn_whistle_free(self.handle)
                self.handle = None
        except Exception:
            pass


def choose_allowed(logits: np.ndarray, allowed: np.ndarray, token: int = -1):
    """rn_choose_allowed on host arrays: (token, constrained, probability, mass)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    mask = np.ascontiguousarray(allowed, dtype=np.uint8)
    ld, md, od = DeviceBuffer.from_array(logits), DeviceBuffer.from_array(mask), DeviceBuffer(C.sizeof(Choice))
    check(lib.rn_choose_allowed(ld.ptr, md.ptr, logits.size, token, od.ptr, None))
    check(lib.rn_stream_synchronize(None))
    raw = od.download(np.uint8, (C.sizeof(Choice),))
    c = Choice.from_buffer_copy(raw.tobytes())
    return int(c.token), bool(c.constrained), np.float32(c.probability), np.float32(c.mass)


class Frontend:
    """crates/whistle/src/frontend.rs: the log-mel front end on the device."""

    def __init__(self, mels: int, fft_size: int, window: int, hop: int, mel_weights: np.ndarray):
        w = np.ascontiguousarray(mel_weights, dtype=np.float32)
        assert w.shape == (fft_size // 2 + 1, mels)
        h = _p()
        check(lib.rn_frontend_create(mels, fft_size, window, hop, _ptr(w), C.byref(h)))
        self.handle = h.value
        self.mels, self.hop = mels, hop

    def log_mel(self, samples: np.ndarray):
        """Frontend::log_mel: (features [frames][mels], valid, spread)."""
        x = np.ascontiguousarray(samples, dtype=np.float32)
        out = np.empty((x.size // self.hop + 1, self.mels), np.float32)
        frames, valid, spread = _i(), _i(), _f()
        check(lib.rn_frontend_log_mel(self.handle, _ptr(x) if x.size else None, x.size, _ptr(out), C.byref(frames),
                                      C.byref(valid), C.byref(spread)))
        return out, valid.value, np.float32(spread.value)

    def __del__(self):
        try:
            if self.handle:
                lib.rn_frontend_free(self.handle)
        except Exception:
            pass


def synthetic_mel_filters(mels: int, fft_size: int, sample_rate: int = 16000) -> np.ndarray:
    """Triangular mel filters [fft_size/2 + 1][mels] on the HTK mel scale (a
    stand-in for the archive's filterbank)."""
    bins = fft_size // 2 + 1
    hz = np.linspace(0, sample_rate / 2, bins)
    mel = lambda f: 2595.0 * np.log10(1.0 + f / 700.0)
    edges = 700.0 * (10 ** (np.linspace(mel(0.0), mel(sample_rate / 2), mels + 2) / 2595.0) - 1.0)
    w = np.zeros((bins, mels))
    for m in range(mels):
        lo, c, hi = edges[m], edges[m + 1], edges[m + 2]
        w[:, m] = np.maximum(0.0, np.minimum((hz - lo) / (c - lo), (hi - hz) / (hi - c)))
    return w.astype(np.float32)


def kronecker_apply(x: np.ndarray, left: np.ndarray, right: np.ndarray) -> np.ndarray:
    """ops::kronecker_apply for 32 x 32 factors over inputs [count][1024]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 1024)
    xd, ld, rd = (DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32)) for a in (x, left, right))
    od = DeviceBuffer(4 * x.size)
    check(lib.rn_kronecker_apply(xd.ptr, ld.ptr, 32, rd.ptr, 32, x.shape[0], od.ptr, None))
    check(lib.rn_stream_synchronize(None))
    return od.download(np.float32, x.shape)


class Lanes:
    """LaneWeights (crates/model/src/lanes.rs) over three CodebookMatrix routing matrices."""

    def __init__(self, lanes: int, width: int, layers: int, a_pre, a_post, a_res, b_pre, b_post, b_res,
                 phi_pre: "CodebookMatrix", phi_post: "CodebookMatrix", phi_res: "CodebookMatrix"):
        arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (a_pre, a_post, a_res, b_pre, b_post, b_res)]
        h = _p()
        check(lib.rn_lanes_create(lanes, width, layers, *[_ptr(a) for a in arrs], phi_pre.handle, phi_post.handle,
                                  phi_res.handle, C.byref(h)))
        self.handle = h.value
        self.lanes, self.width = lanes, width
        self._keep = (phi_pre, phi_post, phi_res)

    def route(self, layer: int, slot: int, stream: np.ndarray):
        """(input [width], post [lanes], residual [lanes][lanes])."""
        x = np.ascontiguousarray(stream, dtype=np.float32).reshape(-1)
        xd = DeviceBuffer.from_array(x)
        ind, pd, rd = DeviceBuffer(4 * self.width), DeviceBuffer(4 * self.lanes), DeviceBuffer(4 * self.lanes ** 2)
        check(lib.rn_lanes_route(self.handle, layer, slot, xd.ptr, ind.ptr, pd.ptr, rd.ptr, None))
        check(lib.rn_stream_synchronize(None))
        return (ind.download(np.float32, (self.width,)), pd.download(np.float32, (self.lanes,)),
                rd.download(np.float32, (self.lanes, self.lanes)))

    def combine(self, post, residual, stream, delta) -> np.ndarray:
        bufs = [DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=np.float32)) for a in (post, residual, stream, delta)]
        nd = DeviceBuffer(4 * self.lanes * self.width)
        check(lib.rn_lanes_combine(self.handle, *[b.ptr for b in bufs], nd.ptr, None))
        check(lib.rn_stream_synchronize(None))
        return nd.download(np.float32, (self.lanes, self.width))

    def __del__(self):
        try:
            if self.handle:
                lib.rn_lanes_free(self.handle)
        except Exception:
            pass


def ladder_order(layers: int) -> list:
    """ladder::order (crates/model/src/ladder.rs:1-20)."""
    out = np.empty(max(layers, 1), np.int32)
    check(lib.rn_ladder_order(layers, _ptr(out)))
    return out[:layers].tolist()


def ladder_select(layers: int, depth: int):
    """ladder::select (ladder.rs:22-29); None where the reference returns None."""
    out = np.empty(max(depth, 1), np.int32)
    rc = lib.rn_ladder_select(layers, depth, _ptr(out))
    return None if rc == RN_ERR_ARGUMENT else out[:depth].tolist()

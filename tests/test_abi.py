"""The C-ABI library loads, exports every declared entry point, and its host-only
logic (argument checks, seeded generators) behaves — no device needed."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import rustyneedle_amd as rn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rustyneedle.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rn_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    syms = declared_symbols()
    assert len(syms) > 40
    raw = C.CDLL(rn.LIB_PATH)
    for s in syms:
        assert hasattr(raw, s), f"{s} declared in include/rustyneedle.h but not exported"
        assert s in rn.SIGNATURES, f"{s} has no Python binding"
    assert set(rn.SIGNATURES) == set(syms)


def test_abi_version():
    assert rn.lib.rn_abi_version() == 1


def test_argument_errors_need_no_device():
    h = C.c_void_p()
    codes = np.zeros((4, 512), np.int8)
    scales = np.zeros((4, 16), np.float32)
    rc = rn.lib.rn_matrix_create_i8(codes.ctypes.data, scales.ctypes.data, 4, 500, 32, 0, C.byref(h))
    assert rc == rn.RN_ERR_ARGUMENT and b"columns" in rn.lib.rn_last_error()
    rc = rn.lib.rn_matrix_create_i8(codes.ctypes.data, scales.ctypes.data, 4, 512, 16, 0, C.byref(h))
    assert rc == rn.RN_ERR_ARGUMENT and b"group" in rn.lib.rn_last_error()
    cfg = dict(rn.NEEDLE_DECODER)
    cfg["d_model"] = 768
    rc = rn.lib.rn_model_create_synthetic(C.byref(rn._config_struct(cfg)), 1, C.byref(h))
    assert rc == rn.RN_ERR_ARGUMENT and b"d_model" in rn.lib.rn_last_error()
    cfg = dict(rn.NEEDLE_DECODER)
    cfg["norm_eps"] = 1e-5
    rc = rn.lib.rn_model_create_synthetic(C.byref(rn._config_struct(cfg)), 1, C.byref(h))
    assert rc == rn.RN_ERR_ARGUMENT


# ---- seeded generators: an independent numpy SplitMix64 ----------------------------------

M64 = (1 << 64) - 1


def fnv1a(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & M64
    return h


def splitmix(seed: int, name: str, n: int):
    s = seed ^ fnv1a(name)
    out = []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_published_vector():
    """Vigna's splitmix64.c from state 0: first output 0xE220A8397B1DCDAF."""
    z = splitmix(0, "", 1)[0]  # fnv1a("") ^ 0 is the offset basis, so undo it:
    s = 0
    s = (s + 0x9E3779B97F4A7C15) & M64
    z = ((s ^ (s >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    assert z ^ (z >> 31) == 0xE220A8397B1DCDAF


def test_synth_codes_and_tokens_match_numpy_restatement():
    zs = splitmix(20261201, "layers.3.qkv.codes", 1000)
    codes = rn.synth_codes(20261201, "layers.3.qkv.codes", (1000,))
    assert codes.tolist() == [(((z >> 32) * 255) >> 32) - 127 for z in zs]
    assert codes.min() >= -127 and codes.max() <= 127
    zs = splitmix(5, "t", 500)
    assert rn.synth_tokens(5, "t", 8192, 500).tolist() == [((z >> 32) * 8192) >> 32 for z in zs]


def test_synth_uniform_and_normal_match_numpy_restatement():
    zs = splitmix(9, "s", 256)
    u = rn.synth_uniform(9, "s", 1e-3, 1e-2, (256,))
    lo, hi = float(np.float32(1e-3)), float(np.float32(1e-2))  # the C entry point takes float bounds
    ref = np.array([lo + (hi - lo) * ((z >> 40) / 16777216.0) for z in zs]).astype(np.float32)
    assert np.array_equal(u, ref)
    assert u.min() >= 1e-3 and u.max() <= 1e-2
    zs = splitmix(9, "n", 2000)
    nrm = rn.synth_normal(9, "n", 1.0, (1000,))
    u1 = (np.array([z >> 40 for z in zs[0::2]], np.float64) + 1.0) / 16777216.0
    u2 = np.array([z >> 40 for z in zs[1::2]], np.float64) / 16777216.0
    ref = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)
    assert np.max(np.abs(nrm - ref)) < 1e-6
    assert abs(float(nrm.mean())) < 0.1 and abs(float(nrm.std()) - 1.0) < 0.1


def test_synth_streams_are_named_and_seeded():
    a = rn.synth_codes(1, "a", (64,))
    assert np.array_equal(a, rn.synth_codes(1, "a", (64,)))
    assert not np.array_equal(a, rn.synth_codes(2, "a", (64,)))
    assert not np.array_equal(a, rn.synth_codes(1, "b", (64,)))
    h = rn.synth_normal_f16(3, "h", (4096,))
    assert np.array_equal(h, rn.synth_normal(3, "h", 1.0, (4096,)).astype(np.float16))


def test_codebook_argument_errors_need_no_device():
    cb = rn.synthetic_codebook(128)
    blob = rn.synthetic_codebook_blob(4, 128, 128, 2)
    for bits, group, size, columns in ((6, 128, blob.size, 128), (0, 128, blob.size, 128), (3, 128, blob.size, 128),
                                       (2, 96, blob.size, 128),
                                       (2, 128, blob.size - 1, 128), (2, 128, blob.size, 50000)):
        with pytest.raises(rn.RnError):
            rn.CodebookMatrix(blob[:size], 4, columns, group, bits, cb)

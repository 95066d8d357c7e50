"""Writes .cact archives (crates/cact; docs/format.md): a 196-byte
header (48 u32 fields and the f32 rope_theta), the codebook levels, 44-byte
directory records (u8 kind, u8 rank, u16 pad, u32 shape[4], u64 offset,
u64 nbytes, u32 group_size, u32 bits) and 64-byte aligned blobs."""
import struct

import numpy as np

TAG = 0x05E12A84
HEADER_FIELDS = ("tensor_count", "codebook_len", "kv_window", "kv_bits", "vocab", "out_vocab", "d_model",
                 "num_heads", "num_kv_heads", "num_layers", "qk_head_dim", "v_head_dim", "max_seq_len", "hada_n",
                 "mhc_lanes", "sliding_window", "global_mask_lo", "global_mask_hi", "qkv_conv_taps", "engram_slots",
                 "engram_sub_dim", "num_engram_tables", "engram_conv_taps", "engram_conv_dilation",
                 "engram_seed_heads")


def write(tensors, codebook, rope_theta=10000.0, engram_orders=(), engram_sites=(), **fields) -> bytes:
    """tensors: list of (kind, shape, blob bytes, group_size, bits)."""
    values = dict.fromkeys(HEADER_FIELDS, 0)
    values.update(fields)
    values["tensor_count"] = len(tensors)
    values["codebook_len"] = len(codebook)
    orders = list(engram_orders) + [0] * (4 - len(engram_orders))
    sites = list(engram_sites) + [0] * (16 - len(engram_sites))
    header = struct.pack("<I", TAG) + struct.pack("<25I", *(values[k] for k in HEADER_FIELDS))
    header += struct.pack("<I4I", len(engram_orders), *orders) + struct.pack("<I16I", len(engram_sites), *sites)
    header += struct.pack("<f", rope_theta)
    assert len(header) == 196
    cb = np.asarray(codebook, np.float32).tobytes()
    start = len(header) + len(cb) + 44 * len(tensors)
    offset = (start + 63) // 64 * 64
    records, blobs = [], []
    for kind, shape, blob, group, bits in tensors:
        dims = list(shape) + [0] * (4 - len(shape))
        records.append(struct.pack("<BBH4IQQII", kind, len(shape), 0, *dims, offset, len(blob), group, bits))
        blobs.append((offset, bytes(blob)))
        offset = (offset + len(blob) + 63) // 64 * 64
    out = bytearray(offset)
    body = header + cb + b"".join(records)
    out[:len(body)] = body
    for off, blob in blobs:
        out[off:off + len(blob)] = blob
    return bytes(out)

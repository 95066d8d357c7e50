"""Benchmark of the Needle token loop on one MI355X.

Headline (`value`): batch-1 greedy decode tokens/s on the decode workload —
20 layers, d_model 512, 8 heads of 64, gated FFN 2048, int8 codes with fp32
per-32 scales, tied int8 vocab 8192, fp16 KV cache pre-filled to 256 positions
with N(0,1) values, 64 greedy tokens. One step = one 64-token greedy decode
from the 256-position context (the session is truncated back to 256 between
steps; the cache and weights stay resident in device memory).

Also reported: batch-64 decode tokens/s (64 sequences, ragged caches of 32..512
positions, 32 greedy tokens), prefill tokens/s (one 256-token sequence), the
single int8 matvec (2048 x 512) latency, a streaming int8 matvec over 512
distinct 2048 x 512 matrices in one launch (609 MB, more than the 256 MB
Infinity Cache: the HBM roofline of the product kernel), the speech path (encode
of a 3000-frame mel window through the stem and 6 encoder layers plus the cross
memory, then 48 greedy tokens of the 4-layer cross-attention decoder), the
codebook-format matvecs (2-bit and 4-bit streams larger than the Infinity Cache,
and the 2048 x 512 layer shape), the speech front end over 30 s of audio, and
the CPU oracle on the host cores as the baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
GEMV_UNIT_BYTES = 1_189_888    # one 2048x512 int8 matvec: W 1,048,576 + sW 131,072 + x 2,048 + y 8,192
DECODE_TOKENS = 64
CONTEXT = 256
KERNEL_NAMES = {
    "qkv_attention": "qkv_attend_kernel<512,norm> (norm + a head's q/k/v rows + rotary + fp16 append + attention; "
                     "layer 0 first reduces the previous logits' argmax keys and gathers the embedding row)",
    "out": "gemv_kernel<512,2,quant,residual,panel> (out)",
    "gate_up": "gemv_kernel<512,8,norm,silu,panel> (gate/up)",
    "down": "gemv_splitk_kernel<2048,2,panel> (down, four waves over the columns)",
    "logits": "gemv_kernel<512,8,norm,argmax,plane> (logits, block argmax keys, position advance)",
}
# Memory-side bytes per launch of each decode kernel, from two rocprofv3 --pmc
# passes (FETCH_SIZE, WRITE_SIZE) over this workload with direct launches; the
# KiB counts are scaled by what the counters read for a 256 MiB device copy
# (FETCH x2.000, WRITE x1.000). Recorded in profiles/decode_b1_needle20_traffic.md;
# they describe the kernels as built when measured and are re-measured with them.
PMC_TRAFFIC = {
    "qkv_attention": 1_833_616,  # 20-launch mean: 19 x 1,829,898 (layers 1-19) + 1,904,262 (layer 0)
    "out": 378_887,
    "gate_up": 2_493_441,
    "down": 1_338_368,
    "logits": 4_907_168,
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def time_events(rn, stream, fn, reps: int) -> float:
    """Average milliseconds of `fn` over `reps` calls, HIP events on `stream`."""
    a, b = rn.Event(), rn.Event()
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    return a.elapsed_ms(b) / reps


def bench_decode(rn, model, cfg, steps: int, warmup: int):
    keys, values = rn.synthetic_cache(cfg, CONTEXT, "decode")
    first = int(rn.synth_tokens(rn.SEED, "decode.first", cfg["vocab"], 1)[0])
    sess = model.session(CONTEXT + DECODE_TOKENS)
    sess.set_cache(keys, values)
    stream = sess.stream()

    def step():
        sess.truncate(CONTEXT)
        return sess.decode_greedy(first, DECODE_TOKENS)

    ref = None
    for _ in range(warmup):
        ref = step()
    rn.lib.rn_stream_synchronize(stream)
    start, stop = rn.Event(), rn.Event()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        ids = step()
        if ref is not None and not np.array_equal(ids, ref):
            raise RuntimeError("decode is not deterministic across steps")
        ref = ids
    stop.record(stream)
    ms = start.elapsed_ms(stop)
    wall = time.perf_counter() - t0
    return ms, wall, ref, (keys, values, first)


def decode_kernel_bytes(cfg, context: int, steps: int) -> dict:
    """Algorithmic HBM bytes per launch of each decode-step kernel kind: weights,
    scales, cache rows and vectors each read or written once."""
    d, f, v, h, hd = cfg["d_model"], cfg["ffn"], cfg["vocab"], cfg["heads"], cfg["head_dim"]
    q = lambda rows, cols: rows * cols + rows * (cols // 32) * 4   # codes + fp32 scales
    mean_cached = context + (steps - 1) / 2.0                        # cache rows read per attention launch
    blocks = (v + 7) // 8
    return {
        # W rows of every head, x, gains, K/V rows read, the new K/V row written, the output
        "qkv_attention": q(3 * d, d) + 4 * d + 4 * d + h * 2 * mean_cached * hd * 2 + h * 2 * hd * 2 + 4 * d,
        "out": q(d, d) + 4 * d + 2 * 4 * d,                           # W, attention in, residual read+write
        "gate_up": q(2 * f, d) + 4 * d + 4 * d + 4 * f,               # W, x, gains, silu(gate)*up out
        "down": q(d, f) + 4 * f + 2 * 4 * d,
        "logits": q(v, d) + 4 * d + 4 * d + 4 * v + 4 * d + 8 * blocks,
        "final": 8 * blocks + 4 * 4,
    }


def profile_decode(rn, model, cfg, cache, steps: int = DECODE_TOKENS):
    """Per-kernel average durations of the decode step (events after every kernel)."""
    keys, values, first = cache
    sess = model.session(CONTEXT + DECODE_TOKENS)
    sess.set_cache(keys, values)
    sess.profile_step(first, steps)  # warm-up
    sess.truncate(CONTEXT)
    prof = sess.profile_step(first, steps)
    prof = {k: p for k, p in prof.items() if p["per_step"] > 0}  # kinds the step launches
    # the roofline bytes assume the mean cache length of this run's positions
    nbytes = decode_kernel_bytes(cfg, CONTEXT, steps)
    for k, p in prof.items():
        p["bytes_per_launch"] = nbytes[k]
        p["gb_s"] = nbytes[k] / (p["us"] * 1e-6) / 1e9 if p["us"] > 0 else None
        p["us_per_token"] = p["us"] * p["per_step"]
    return prof


def bench_batch(rn, model, cfg, count: int = 64, steps: int = 32, reps: int = 2):
    lengths = (rn.synth_tokens(rn.SEED, "batch.lengths", 481, count) + 32).astype(np.int32)
    first = rn.synth_tokens(rn.SEED, "batch.first", cfg["vocab"], count)
    b = rn.Batch(model, count, int(lengths.max()) + steps)
    for i in range(count):
        k, v = rn.synthetic_cache(cfg, int(lengths[i]), f"batch.{i}")
        b.set_cache(i, k, v)
    stream = b.stream()
    b.decode_greedy(first, steps)  # warm-up
    times = []
    for _ in range(reps):
        b.truncate(lengths)
        t0 = rn.Event()
        t1 = rn.Event()
        t0.record(stream)
        b.decode_greedy(first, steps)
        t1.record(stream)
        times.append(t0.elapsed_ms(t1))
    ms = min(times)
    kv_bytes = int(40960 * (lengths.astype(np.int64) + steps // 2).sum())  # mean cache read per step
    return dict(tokens_per_s=count * steps / (ms / 1e3), ms_per_step=ms / steps, sequences=count, steps=steps,
                kv_bytes_per_step=kv_bytes)


def bench_prefill(rn, model, cfg, tokens: int = 256, reps: int = 5):
    ids = rn.synth_tokens(rn.SEED, "prefill.tokens", cfg["vocab"], tokens)
    s = model.session(tokens)
    s.feed(ids)  # warm-up (allocates the prefill scratch once)
    stream = s.stream()
    times = []
    for _ in range(reps):
        s.truncate(0)
        t0, t1 = rn.Event(), rn.Event()
        t0.record(stream)
        s.feed(ids)
        t1.record(stream)
        times.append(t0.elapsed_ms(t1))
    ms = min(times)
    return dict(tokens_per_s=tokens / (ms / 1e3), ms=ms, tokens=tokens,
                gemm_int8_ops=2 * tokens * 20 * (1536 * 512 + 512 * 512 + 4096 * 512 + 512 * 2048))


def bench_gemv(rn, rotations: int = 512):
    """The single 2048x512 int8 matvec and a stream over `rotations` distinct ones."""
    stream = rn.Stream()
    W = rn.synth_codes(rn.SEED, "gemv.codes", (2048, 512))
    sW = rn.synth_uniform(rn.SEED, "gemv.scales", 1e-3, 1e-2, (2048, 16))
    x = rn.synth_normal(rn.SEED, "gemv.x", 1.0, (512,))
    m = rn.QuantisedMatrix(W, sW)
    xd, yd = rn.DeviceBuffer.from_array(x), rn.DeviceBuffer(4 * 2048)
    call = lambda: m.multiply_vector(xd.ptr, yd.ptr, None, stream.handle)
    for _ in range(20):
        call()
    single_ms = time_events(rn, stream.handle, call, 2000)
    del m
    rows = 2048 * rotations
    Wr = rn.synth_codes(rn.SEED, "gemv.rotating.codes", (rows, 512))
    sWr = rn.synth_uniform(rn.SEED, "gemv.rotating.scales", 1e-3, 1e-2, (rows, 16))
    mr = rn.QuantisedMatrix(Wr, sWr)
    del Wr, sWr
    yr = rn.DeviceBuffer(4 * rows)
    # the stream: `rotations` distinct 2048 x 512 matrices one after another in
    # memory (609 MB, past the Infinity Cache), one launch of the kernel instance
    # the single 2048 x 512 product runs (8 rows a block), then of the 32-row
    # instance the library picks for a matrix this tall
    def stream_ms(rows_per_block):
        call = lambda: mr.multiply_vector_rows(xd.ptr, yr.ptr, rows_per_block, stream.handle)
        for _ in range(3):
            call()
        return time_events(rn, stream.handle, call, 20)
    rot_ms = stream_ms(8)
    rot32_ms = stream_ms(32)
    achieved = GEMV_UNIT_BYTES * rotations / (rot_ms / 1e3) / 1e9
    achieved32 = GEMV_UNIT_BYTES * rotations / (rot32_ms / 1e3) / 1e9
    return dict(single_us=single_ms * 1e3, single_gb_s=GEMV_UNIT_BYTES / (single_ms / 1e3) / 1e9,
                rotations=rotations, rotating_ms=rot_ms, rotating_gb_s=achieved,
                rotating_frac=achieved / HBM_PEAK_GBS, rotating_kernel="gemv_kernel<512,8,quant,store,panel>",
                rotating32_ms=rot32_ms, rotating32_gb_s=achieved32, rotating32_frac=achieved32 / HBM_PEAK_GBS)


def codebook_bytes(rows: int, columns: int, group: int, bits: int) -> int:
    """Algorithmic HBM bytes of one codebook matvec: indices, fp16 norms, the
    rotated input and the output."""
    padded = -(-columns // group) * group
    ib = 2 if bits == 5 else bits
    return rows * padded * ib // 8 + rows * (padded // group) * 2 + 4 * padded + 4 * rows


def bench_codebook(rn, shapes=((2, 128, 2048, 512), (2, 128, 2097152, 512), (4, 128, 1048576, 512),
                                (2, 128, 131072, 8192))):
    """Codebook-format matvecs (2-bit panel form, 4-bit plane form) on rotated
    inputs: the 2048 x 512 layer shape, and matrices of 264-272 MB (more than
    the 256 MB Infinity Cache) that stream from HBM."""
    stream = rn.Stream()
    out = {}
    for bits, group, rows, columns in shapes:
        cb = rn.synthetic_codebook(group)
        blob = rn.synthetic_codebook_blob(rows, columns, group, bits, name=f"bench.codebook.{bits}.{columns}")
        m = rn.CodebookMatrix(blob, rows, columns, group, bits, cb)
        del blob
        x = rn.synth_normal(rn.SEED, "bench.codebook.x", 1.0, (1, columns))
        xd = rn.DeviceBuffer.from_array(x)
        rd, yd = rn.DeviceBuffer(4 * m.padded), rn.DeviceBuffer(4 * rows)
        m.prepare(xd.ptr, 1, rd.ptr, stream.handle)
        call = lambda: rn.check(rn.lib.rn_matrix_multiply_vector(m.handle, rd.ptr, yd.ptr, None, stream.handle))
        for _ in range(3):
            call()
        n = 2000 if rows * columns <= (1 << 22) else 20
        ms = time_events(rn, stream.handle, call, n)
        nbytes = codebook_bytes(rows, columns, group, bits)
        gbs = nbytes / (ms / 1e3) / 1e9
        out[f"{bits}bit_{rows}x{columns}"] = dict(us=ms * 1e3, bytes=nbytes, gb_s=gbs, frac=gbs / HBM_PEAK_GBS)
        del m, xd, rd, yd
    out["float_path"] = bench_codebook_float(rn, stream)
    return out


def bench_codebook_float(rn, stream, rows: int = 2048, columns: int = 512, group: int = 128):
    """The float path (fill_rows_float, crates/kernels/src/matrix.rs:427-440): what
    the reference runs on x86-64 for every width, and everywhere for 1- and 3-bit
    matrices. The device kernel per width, and the oracle's restatement of it on
    one host core beside it (about 0.5 s of CPU work per width)."""
    import oracle
    out = {}
    for bits in (1, 2, 3, 4):
        cb = rn.synthetic_codebook(group)
        blob = rn.synthetic_codebook_blob(rows, columns, group, bits, name=f"bench.float.{bits}")
        m = rn.CodebookMatrix(blob, rows, columns, group, bits, cb)
        om = oracle.OracleCodebookMatrix(blob, rows, columns, group, bits, cb)
        x = rn.synth_normal(rn.SEED, "bench.float.x", 1.0, (1, m.padded))
        xd, yd = rn.DeviceBuffer.from_array(x), rn.DeviceBuffer(4 * rows)
        call = lambda: rn.check(rn.lib.rn_matrix_multiply_vector_float(m.handle, xd.ptr, yd.ptr, stream.handle))
        for _ in range(3):
            call()
        gpu_ms = time_events(rn, stream.handle, call, 200)
        oracle.set_threads(1)
        reps, spent = 0, 0.0
        ref = None
        while spent < 0.5 or reps < 3:
            t0 = time.perf_counter()
            ref = om.multiply_float(x)
            spent += time.perf_counter() - t0
            reps += 1
        same = np.array_equal(yd.download(np.float32, (1, rows)).view(np.uint32), ref.view(np.uint32))
        out[f"{bits}bit_{rows}x{columns}"] = dict(gpu_us=gpu_ms * 1e3, cpu_us=spent / reps * 1e6, cpu_cores=1,
                                                 cpu_kind="port", bit_identical=bool(same))
        del m, xd, yd
    return out


def bench_frontend(rn, seconds: int = 30, reps: int = 5):
    """The speech front end over a 30 s, 16 kHz input (3001 frames of 80 mels,
    FFT 512, window 400, hop 160): wall time of rn_frontend_log_mel including
    the sample upload and feature download (the kernels alone are in the trace)."""
    n = 16000 * seconds
    x = rn.synth_normal(rn.SEED, "bench.frontend", 0.1, (n,))
    f = rn.Frontend(80, 512, 400, 160, rn.synthetic_mel_filters(80, 512))
    f.log_mel(x)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        f.log_mel(x)
        times.append(time.perf_counter() - t0)
    return dict(samples=n, frames=n // 160 + 1, ms_with_transfers=min(times) * 1e3)


def bench_whistle(rn, reps: int = 3, steps: int = 48, with_cpu: bool = True):
    """The speech path: encode of a 3000-frame mel window (stem, 6 encoder
    layers over 1500 frames, the cross memory of 4 decoder layers), then a
    48-token greedy decode with cross-attention; HIP events on its stream."""
    cfg = dict(rn.WHISTLE)
    w = rn.Whistle(cfg)
    mel = rn.synthetic_mel(cfg)
    first = int(rn.synth_tokens(rn.SEED, "whistle.first", cfg["vocab"], 1)[0])
    stream = w.stream()
    w.encode(mel, copy_out=False)
    ref = w.decode_greedy(first, steps)
    enc_ms, dec_ms = [], []
    for _ in range(reps):
        t0, t1, t2 = rn.Event(), rn.Event(), rn.Event()
        t0.record(stream)
        w.encode(mel, copy_out=False)
        t1.record(stream)
        ids = w.decode_greedy(first, steps)
        t2.record(stream)
        if ids.tolist() != ref.tolist():
            raise RuntimeError("speech decode is not deterministic")
        enc_ms.append(t0.elapsed_ms(t1))
        dec_ms.append(t1.elapsed_ms(t2))
    T, d, f = w.frames, cfg["d_model"], cfg["ffn"]
    per_layer = 2 * T * (3 * d * d + d * d + 2 * f * d + d * f)
    # encoder layers, the stem's second convolution (im2col rows of 3 d) and the cross memory
    ops = cfg["enc_layers"] * per_layer + 2 * T * d * 3 * d + cfg["dec_layers"] * 2 * T * 2 * d * d
    out = dict(encode_ms=min(enc_ms), encode_int8_gops=ops / 1e9,
               decode_tokens_per_s=steps / (min(dec_ms) / 1e3), decode_ms_per_token=min(dec_ms) / steps,
               frames_in=cfg["frames"], encoder_frames=T, tokens=steps)
    if with_cpu:
        import oracle
        cores = os.cpu_count() or 1
        threads = max(1, min(cores - 1, 6))
        oracle.set_threads(threads)
        o = oracle.OracleWhistle(cfg, rn.synthetic_whistle_weights(cfg))
        t = time.perf_counter()
        encoded = o.encode(mel)
        mem = o.memory(encoded)
        cpu_enc = time.perf_counter() - t
        t = time.perf_counter()
        cpu_ids = o.session(cfg["max_positions"], mem).greedy(first, steps)
        cpu_dec = time.perf_counter() - t
        out["cpu"] = dict(encode_ms=cpu_enc * 1e3, decode_tokens_per_s=steps / cpu_dec, threads=threads,
                          kind="port", ids_match=cpu_ids.tolist() == ref.tolist())
    return out


def bench_needle3(rn, with_cpu: bool = True, context: int = 600, steps: int = 64):
    """The Needle 3 block (crates/model/src/session.rs) at its documented shape
    (d_model 768, 20 layers, 12 heads over 4 kv heads, four lanes, two engram
    sites, 32 x 32 Hadamard factors, 2-bit projections, 4-bit 8192 x 768
    logits) from a synthetic archive: a 600-token feed, then greedy decode
    (push, logits, argmax) at that context; a 4000-token feed; greedy decode
    after 1100 tokens (the reference bench's `decode --context 600`, `prefill
    --tokens 4000`); HIP events on the session's stream; the first pushes
    checked bit for bit against the oracle."""
    import oracle
    from rustyneedle_amd import needle3
    archive = needle3.synthetic_archive(needle3.NEEDLE3)
    model = needle3.Model(archive)
    prompt = rn.synth_tokens(rn.SEED, "needle3.prompt", needle3.NEEDLE3["vocab"], (context,))
    # bit identity with the oracle on the first pushes
    om = oracle.OracleNeedle3(archive)
    gs, os_ = model.session(16), om.session(16)
    identical = True
    for t in prompt[:4]:
        gs.push(int(t))
        os_.push(int(t))
        identical &= bool(np.array_equal(gs.hidden().view(np.uint32), os_.hidden().view(np.uint32)))
    s = model.session(context + steps + 8)
    stream = s.stream()
    t0, t1, t2, t3 = rn.Event(), rn.Event(), rn.Event(), rn.Event()
    t0.record(stream)
    s.feed(prompt)
    t1.record(stream)
    s.decode_greedy(int(prompt[-1]), 4)  # warm
    t2.record(stream)
    s.decode_greedy(int(prompt[-1]), steps)
    t3.record(stream)
    feed_ms, dec_ms = t0.elapsed_ms(t1), t2.elapsed_ms(t3)
    del s
    # the reference's other two figures: a 4000-token prefill, and decode at
    # 1100 tokens of context
    long_prompt = rn.synth_tokens(rn.SEED, "needle3.prompt4000", needle3.NEEDLE3["vocab"], (4000,))
    s = model.session(4000 + 8)
    stream = s.stream()
    t0.record(stream)
    s.feed(long_prompt)
    t1.record(stream)
    feed4000_ms = t0.elapsed_ms(t1)
    del s
    s = model.session(1100 + steps + 8)
    stream = s.stream()
    s.feed(long_prompt[:1100])
    s.decode_greedy(int(long_prompt[1099]), 4)
    t2.record(stream)
    s.decode_greedy(int(long_prompt[1099]), steps)
    t3.record(stream)
    dec1100_ms = t2.elapsed_ms(t3)
    del s
    out = dict(decode_tokens_per_s=steps / (dec_ms / 1e3), decode_ms_per_token=dec_ms / steps, context=context + 4,
               feed_tokens_per_s=context / (feed_ms / 1e3), feed_4000_tokens_per_s=4000 / (feed4000_ms / 1e3),
               feed_4000_ms=feed4000_ms, decode_1100_tokens_per_s=steps / (dec1100_ms / 1e3),
               layers=needle3.NEEDLE3["num_layers"], d_model=needle3.NEEDLE3["d_model"], bit_identical=identical,
               reference_published="decode about 830-860 tokens/s at 600 tokens of context, about 720 at 1100; "
                                   "prefill of 4000 tokens about 1800 tokens/s; on an Apple M1 Max "
                                   "(docs/architecture.md, Performance)")
    if with_cpu:
        # the reference's pool policy, min(cores - 1, 6) threads (pool.rs:48-52):
        # the oracle splits its row products over them; one thread beside it
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1
        threads = max(1, min(cores - 1, 6))

        def pushes(n_threads: int) -> float:
            oracle.set_threads(n_threads)
            cs = om.session(24)
            t = time.perf_counter()
            for tok in prompt[:16]:
                cs.push(int(tok))
            return (time.perf_counter() - t) / 16

        single = pushes(1)
        dt = pushes(threads)
        oracle.set_threads(1)
        out["cpu"] = dict(ms_per_push=dt * 1e3, tokens_per_s=1.0 / dt, cores=threads, kind="port",
                          single_thread_tokens_per_s=1.0 / single,
                          sample=f"16 pushes from an empty session, C oracle on {threads} threads "
                                 f"(row products split over them) of {cores} host cores")
    return out


def cpu_baseline(rn, cfg, cache, budget_s: float = 10.0):
    """The oracle (C restatement of the reference path) on the host cores, with
    the reference's thread policy min(cores - 1, 6) (crates/kernels/src/pool.rs:48-52)."""
    import oracle

    keys, values, first = cache
    cores = os.cpu_count() or 1
    threads = max(1, min(cores - 1, 6))
    om = oracle.OracleModel(cfg, rn.synthetic_weights(cfg))

    def run(n_threads: int, budget: float):
        """Median tokens/s of whole 64-token decodes repeated within `budget` seconds."""
        oracle.set_threads(n_threads)
        rates, ids, spent = [], None, 0.0
        while spent < budget or not rates:
            s = om.session(CONTEXT + DECODE_TOKENS)
            s.set_cache(keys, values)
            t0 = time.perf_counter()
            ids = s.greedy(first, DECODE_TOKENS)
            dt = time.perf_counter() - t0
            rates.append(DECODE_TOKENS / dt)
            spent += dt
        return float(np.median(rates)), len(rates), ids

    value, reps, ids = run(threads, budget_s)
    single, single_reps, _ = run(1, budget_s / 2)
    model_name = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model_name = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return dict(value=value, unit="tokens/s", cores=threads, kind="port", single_thread=single,
                cpu=model_name, host_cores=cores,
                sample=f"median of {reps} whole 64-token batch-1 greedy decodes from the 256-position context, "
                       f"C oracle (-O3, x86-64-v3, OpenMP) on {threads} threads of {cores} host cores "
                       f"({single_reps} decodes on 1 thread give single_thread)"), ids


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="decode only")
    ap.add_argument("--extras", default="gemv,prefill_256,decode_batch64,whistle,codebook,frontend,needle3",
                    help="comma-separated secondary measurements to run")
    ap.add_argument("--profile-steps", type=int, default=DECODE_TOKENS,
                    help="greedy steps timed kernel by kernel for the roofline")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the decode path is single-GPU by design",
              file=sys.stderr)
        return 2

    import rustyneedle_amd as rn

    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 20
        src, dst = rn.DeviceBuffer(n), rn.DeviceBuffer(n)
        rn.check(rn.lib.rn_memcpy_dtod(dst.ptr, src.ptr, n))
        log(f"bench: copied {args.copy_probe_mib} MiB device to device")
        del src, dst
    cfg = dict(rn.NEEDLE_DECODER)
    log("bench: building the synthetic 20-layer model on the device")
    model = rn.Model(cfg, seed=rn.SEED)
    log("bench: batch-1 decode")
    ms, wall, ids, cache = bench_decode(rn, model, cfg, args.steps, args.warmup)
    ms_per_step = ms / args.steps
    tok_s = DECODE_TOKENS * args.steps / (ms / 1e3)
    log("bench: per-kernel timing of the decode step")
    kernels = profile_decode(rn, model, cfg, cache, args.profile_steps)
    extra = {"decode_kernels": kernels}
    if not args.no_extra:
        wanted = {e.strip() for e in args.extras.split(",") if e.strip()}
        for name, fn in (("gemv", lambda: bench_gemv(rn)),
                         ("prefill_256", lambda: bench_prefill(rn, model, cfg)),
                         ("decode_batch64", lambda: bench_batch(rn, model, cfg)),
                         ("whistle", lambda: bench_whistle(rn, with_cpu=not args.no_cpu)),
                         ("codebook", lambda: bench_codebook(rn)),
                         ("frontend", lambda: bench_frontend(rn)),
                         ("needle3", lambda: bench_needle3(rn, with_cpu=not args.no_cpu))):
            if name not in wanted:
                continue
            log(f"bench: {name}")
            try:
                extra[name] = fn()
            except Exception as e:  # report, do not hide: the headline still prints
                extra[name] = {"error": repr(e)}
    base = None
    if not args.no_cpu:
        log("bench: CPU baseline (oracle on the host)")
        try:
            base, cpu_ids = cpu_baseline(rn, cfg, cache)
            if cpu_ids.tolist() != ids[:len(cpu_ids)].tolist():
                base["mismatch"] = "CPU greedy ids differ from the GPU's"
        except Exception as e:
            base = {"error": repr(e)}
    # the dominant kernel of the timed decode step: most microseconds per token
    dom_kind = max(kernels, key=lambda k: kernels[k]["us_per_token"])
    dom = kernels[dom_kind]
    roofline = dict(bound="hbm", kernel=KERNEL_NAMES[dom_kind], achieved=dom["gb_s"], peak=HBM_PEAK_GBS,
                    unit="GB/s", frac=dom["gb_s"] / HBM_PEAK_GBS, traffic=PMC_TRAFFIC.get(dom_kind),
                    bytes_per_launch=dom["bytes_per_launch"], avg_launch_us=dom["us"],
                    share_of_step=dom["us_per_token"] / (ms_per_step * 1e3 / DECODE_TOKENS))
    line = {
        "metric": "decode tokens/sec (batch 1, 64) + int8 GEMV GB/s and % HBM roofline",
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 products, f32 epilogue, fp16 KV",
        "data": "synthetic (seeded int8 weights, N(0,1) fp16 cache)",
        "config": {"workload": "Needle-style decoder decode, batch 1: 20 layers, d_model 512, 8x64 heads, "
                               "FFN 2048, vocab 8192, fp16 KV pre-filled to 256, 64 greedy tokens",
                   "tokens_per_step": DECODE_TOKENS, "context": CONTEXT, "wall_s": wall},
        "roofline": roofline,
        "cpu_baseline": base,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

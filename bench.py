"""Benchmark: codes/s of the 1.7B talker + code-predictor per-code loop at
batch 1 on one MI355X, with the achieved bandwidth of the kernel the loop
runs (k_engine, one cooperative launch per 16 codes), the stand-alone Q4 GEMV's, and the
oracle's codes/s on this host's CPU cores.

Workload (one "step" = one code = one frame of generate_speech's loop,
src/generate_new.rs:242-300): sample code 0 (top-k 50, T 0.8, repetition
penalty 1.05), 15 predictor passes (5 layers, argmax heads), the embedding
sum and one 28-layer talker step.  A 64-token random-embedding prompt is
prefilled first (untimed); EOS is ignored so every run produces exactly
--steps codes.  Weights are seeded random Q4 of the 1.7B shapes.

Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qora-tts-12hz-1.7b_amd")
sys.path.insert(0, PKG)
sys.path.insert(0, ROOT)

import qtts  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense binary16 MFMA
FP32_PEAK_TFLOPS = 157.3  # dense f32 MFMA
PROMPT = 64
# The loop the headline is quoted on: 500 codes after a 64-token prefill,
# cache lengths 65..564 (mean 314.5).  A shorter --steps run times a window
# of the same loop centred on that mean.  The talker-only loop (config 3)
# runs as many steps.
CONFIG_CODES = 500
CONFIG_STEPS = 500


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the benchmark needs (events, buffers), from
    the same libamdhip64 the library links."""

    def __init__(self):
        import ctypes as C

        self.C = C
        self.lib = C.CDLL("libamdhip64.so.7")

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def malloc(self, nbytes):
        p = self.C.c_void_p()
        self._ok(self.lib.hipMalloc(self.C.byref(p), self.C.c_size_t(nbytes)), "hipMalloc")
        return p.value

    def free(self, p):
        self.lib.hipFree(self.C.c_void_p(p))

    def h2d(self, dst, arr):
        self._ok(self.lib.hipMemcpy(self.C.c_void_p(dst), self.C.c_void_p(arr.ctypes.data),
                                    self.C.c_size_t(arr.nbytes), 1), "hipMemcpy")

    def event(self):
        e = self.C.c_void_p()
        self._ok(self.lib.hipEventCreate(self.C.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream):
        self._ok(self.lib.hipEventRecord(e, self.C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self._ok(self.lib.hipEventSynchronize(b), "hipEventSynchronize")
        ms = self.C.c_float()
        self._ok(self.lib.hipEventElapsedTime(self.C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value


def q4_bytes(k, n):
    """Bytes of a K x N Q4 weight: packed nibbles + one f16 scale per 32 columns."""
    return k * n // 2 + k * (n // 32) * 2


def _layer_bytes(c):
    """One layer's Q4 weights (q|k|v, o, gate|up, down) and f16 norm gammas."""
    qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim
    return (q4_bytes(c.hidden, qd + 2 * kd) + q4_bytes(qd, c.hidden) + q4_bytes(c.hidden, 2 * c.inter)
            + q4_bytes(c.inter, c.hidden) + 4 * c.hidden + 4 * c.head_dim)


def talker_step_bytes(tc, kv_len):
    """Algorithmic bytes of one talker decode step at a cache of kv_len rows:
    every layer weight once, the codec head, the final gamma, and the K/V rows
    read (kv_len + 1 positions, the new one included) -- 855,459,840 B at
    kv_len 256."""
    kv_row = tc.kv_heads * tc.head_dim * 4
    return (tc.layers * _layer_bytes(tc) + q4_bytes(tc.hidden, tc.vocab) + 2 * tc.hidden
            + tc.layers * 2 * kv_row * (kv_len + 1))


def frame_bytes(tc, pc, groups, kv_len):
    """Algorithmic bytes one engine launch (one code) moves: the talker step
    (above); the predictor's input projection in the first pass, 5 layers and
    one head per pass, less layer 0's q|k|v projection in the later passes;
    the rows each later pass reads from the per-code tables instead (its
    projected input and layer 0's q|k|v); and the predictor's K/V rows."""
    pred_pass = pc.layers * _layer_bytes(pc) + q4_bytes(pc.hidden, pc.vocab)
    p_qkv = pc.heads * pc.head_dim + 2 * pc.kv_heads * pc.head_dim
    pred_in = (q4_bytes(tc.hidden, pc.hidden) + (groups - 1) * 4 * (pc.hidden + p_qkv)
               - (groups - 1) * q4_bytes(pc.hidden, p_qkv))
    pred_kv = sum(pc.layers * 2 * pc.kv_heads * pc.head_dim * 4 * (g + 2) for g in range(groups))
    return talker_step_bytes(tc, kv_len) + groups * pred_pass + pred_in + pred_kv


def engine_roofline(frames, gpu_s, kv_len_mean):
    """k_engine, the kernel the loop runs (one cooperative launch runs up to
    16 codes, a grid barrier between them): algorithmic bytes per code over
    the average time per code from HIP events on the context's stream around
    the timed region (a launch of n codes moves n times the bytes in n times
    the time, so the ratio is the launch's)."""
    per = frame_bytes(qtts.TALKER_1P7B, qtts.PREDICTOR_1P7B, qtts.NUM_GROUPS, kv_len_mean)
    avg_s = gpu_s / frames
    achieved = per / avg_s / 1e9
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": read_traffic("k_engine_frame_counters.md", per="code"),
        "kernel": "k_engine (one cooperative launch per 16 codes; per code: sampler, 15 predictor passes, talker step)",
        "codes_per_launch": 16,
        "algorithmic_bytes_per_code": per,
        "avg_code_us": round(avg_s * 1e6, 2),
    }


def gemv_roofline(ctx, K=2048, N=12288, iters=256, copies=64, traffic_file=None, label=None):
    """Average duration of one stand-alone Q4 GEMV launch (qtts_gemv_device)
    of shape K -> N over `copies` distinct weights (a working set above the
    256 MB last-level cache from 2048 x 4096 up), timed with HIP events on
    the context's stream, the stream the kernels run on.  Algorithmic bytes
    per launch: K*N/2 nibble bytes + 2*K*N/32 scale bytes + 4K input + 4N
    output."""
    hip = Hip()
    ws = [qtts.DeviceQ4(ctx, qtts.Q4Weight.synthetic(99, f"roof.{K}.{N}.{i}", K, N)) for i in range(copies)]
    dx, dy = hip.malloc(4 * K), hip.malloc(4 * N)
    hip.h2d(dx, qtts.synth_normal_f32(99, "roof.x", K))
    for i in range(copies):
        ws[i].gemv_device(dx, dy)
    ctx.synchronize()
    start, end = hip.event(), hip.event()
    hip.record(start, ctx.stream)
    for i in range(iters):
        ws[i % copies].gemv_device(dx, dy)
    hip.record(end, ctx.stream)
    avg_s = hip.elapsed_ms(start, end) / 1e3 / iters
    hip.free(dx)
    hip.free(dy)
    for w in ws:
        w.close()
    algo_bytes = K * N // 2 + K * (N // 32) * 2 + 4 * K + 4 * N
    achieved = algo_bytes / avg_s / 1e9
    return {
        "shape": f"{K}->{N}",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": read_traffic(traffic_file, f"{K}x{N}") if traffic_file else None,
        "kernel": label or f"Q4 GEMV {K}->{N} (qtts_gemv_device, launch gaps included)",
        "algorithmic_bytes_per_launch": algo_bytes,
        "avg_launch_us": round(avg_s * 1e6, 3),
        "roofline_us": round(algo_bytes / (HBM_PEAK_GBS * 1e3), 3),
        "weights_rotated": copies,
    }


GEMV_PROFILE = "q4_gemv_shapes_counters.md"


def gemv_shapes(ctx):
    """The three isolated Q4 GEMV shapes (gate/up 2048->6144, down 6144->2048,
    fused q|k|v 2048->4096) and the fused gate|up launch the talker runs
    (2048->12288)."""
    out = [gemv_roofline(ctx, K, N, traffic_file=GEMV_PROFILE) for (K, N) in ((2048, 6144), (6144, 2048), (2048, 4096))]
    out.append(gemv_roofline(ctx, 2048, 12288, traffic_file=GEMV_PROFILE,
                             label="Q4 GEMV 2048->12288 (talker gate|up fused, qtts_gemv_device)"))
    return out


def copy_floor(ctx, sizes=(4743168, 7110656, 14213120), iters=256, copies=64):
    """Device-to-device copies that move as many HBM bytes per launch as the
    GEMV shapes (size / 2 read + size / 2 written), over `copies` buffer
    pairs, HIP events on the context's stream: the duration a plain copy
    kernel of that size needs, the fixed-cost floor a single launch of the
    GEMV sits above."""
    hip = Hip()
    out = []
    st = hip.C.c_void_p(ctx.stream)
    for size in sizes:
        half = size // 2
        bufs = [(hip.malloc(half), hip.malloc(half)) for _ in range(copies)]

        def cp(i):
            a, b = bufs[i % copies]
            hip._ok(hip.lib.hipMemcpyDtoDAsync(hip.C.c_void_p(b), hip.C.c_void_p(a), hip.C.c_size_t(half), st),
                    "hipMemcpyDtoDAsync")

        for i in range(copies):
            cp(i)
        ctx.synchronize()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, ctx.stream)
        for i in range(iters):
            cp(i)
        hip.record(e1, ctx.stream)
        s = hip.elapsed_ms(e0, e1) / 1e3 / iters
        for a, b in bufs:
            hip.free(a)
            hip.free(b)
        out.append({"bytes_moved": 2 * half, "avg_launch_us": round(s * 1e6, 3),
                    "GBps": round(2 * half / s / 1e9, 1), "frac": round(2 * half / s / 1e9 / HBM_PEAK_GBS, 4)})
    return out


def read_floor(ctx, sizes=(4743168, 7110656, 14213120), iters=256, copies=64):
    """One launch that only reads: qtts_stream_read_device (every 16-byte
    word once, one per thread, 256-thread blocks) over as many bytes as each
    GEMV shape streams, `copies` buffers rotated, HIP events on the context's
    stream.  The single-launch floor of streaming those bytes from HBM: a
    GEMV of that size cannot take less."""
    hip = Hip()
    lib = qtts.load_library()
    out = []
    for size in sizes:
        bufs = [hip.malloc(size) for _ in range(copies)]

        def rd(i):
            if lib.qtts_stream_read_device(hip.C.c_void_p(bufs[i % copies]), size, hip.C.c_void_p(ctx.stream)) != 0:
                raise RuntimeError("qtts_stream_read_device failed")

        for i in range(copies):
            rd(i)
        ctx.synchronize()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, ctx.stream)
        for i in range(iters):
            rd(i)
        hip.record(e1, ctx.stream)
        s = hip.elapsed_ms(e0, e1) / 1e3 / iters
        for b in bufs:
            hip.free(b)
        out.append({"bytes_read": size, "blocks": (size // 16 + 255) // 256, "avg_launch_us": round(s * 1e6, 3),
                    "GBps": round(size / s / 1e9, 1), "frac": round(size / s / 1e9 / HBM_PEAK_GBS, 4)})
    return out


def talker_step_measure(ctx, talker, steps=64, L=256):
    """A single talker decode step: 28 layers, KV pre-filled to L positions
    with N(0,1), one N(0,1) embedding per step at positions L, L+1, ...
    (qtts_forward_with_embedding, host input and output copies of 8 KB and
    20 KB included), HIP events on the context's stream.  Algorithmic bytes
    per step: every talker Q4 weight once, the codec head, the norm gammas
    and the K/V rows read (L+1 positions) and written."""
    c = talker.cfg
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    k = qtts.synth_normal_f32(3, "kv.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(3, "kv.v", int(np.prod(shape))).reshape(shape)
    kv = talker.new_kv(L + steps + 8)
    kv.load(k, v, L)
    emb = qtts.synth_normal_f32(3, "step.emb", c.hidden)
    talker.forward_with_embedding(emb, kv, L)  # program build, untimed
    hip = Hip()
    e0, e1 = hip.event(), hip.event()
    ctx.synchronize()
    hip.record(e0, ctx.stream)
    for i in range(steps):
        talker.forward_with_embedding(emb, kv, L + 1 + i)
    hip.record(e1, ctx.stream)
    s = hip.elapsed_ms(e0, e1) / 1e3 / steps
    kv.close()
    per = talker_step_bytes(qtts.TALKER_1P7B, L + (steps + 1) / 2.0)
    achieved = per / s / 1e9
    return {"kv_len": [L + 1, L + steps + 1], "steps": steps, "us_per_step": round(s * 1e6, 1),
            "timing": "HIP events around forward_with_embedding calls (host copies of the embedding and outputs "
                      "included)",
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": per}}


def mfma_gemm_roofline(ctx, rows=64, iters=128, copies=32):
    """The talker prefill's gate|up projection (K=2048 -> N=2*6144) for 64
    rows on the matrix cores (qtts_gemm: row split + k_gemm_mfma), averaged
    over `copies` distinct weights with HIP events on the context's stream.
    Algorithmic work is 2*M*K*N flops; the kernel issues three binary16
    MFMAs per product term (hi/lo operands) to stay at f32 accuracy."""
    K, N = 2048, 12288
    hip = Hip()
    ws = [qtts.DeviceQ4(ctx, qtts.Q4Weight.synthetic(98, f"mfma.{i}", K, N)) for i in range(copies)]
    dx, dy = hip.malloc(4 * K * rows), hip.malloc(4 * N * rows)
    hip.h2d(dx, qtts.synth_normal_f32(98, "mfma.x", K * rows))
    for i in range(copies):
        ws[i].gemm_device(dx, rows, dy)
    ctx.synchronize()
    start, end = hip.event(), hip.event()
    hip.record(start, ctx.stream)
    for i in range(iters):
        ws[i % copies].gemm_device(dx, rows, dy)
    hip.record(end, ctx.stream)
    avg_s = hip.elapsed_ms(start, end) / 1e3 / iters
    hip.free(dx)
    hip.free(dy)
    flops = 2.0 * rows * K * N
    achieved = flops / avg_s / 1e12
    return {
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": MFMA_F16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
        "kernel": "k_mfma_rows + k_gemm_mfma<2,8> (Q4 GEMM 64x2048 -> 12288, talker gate|up at prefill)",
        "weight_GBps": round((K * N // 2 + K * (N // 32) * 4) / avg_s / 1e9, 1),
        "avg_call_us": round(avg_s * 1e6, 2),
    }


def decoder_flops(c, frames):
    """Algorithmic multiply-adds x 2 of decode_to_audio at `frames` frames
    (projections, convolutions with their valid taps, attention)."""
    T, f = frames, 0
    ad = c.heads * c.head_dim
    f += 2 * T * c.codebook_dim * c.vq_dim * 2                       # two codebook projections
    f += 2 * T * c.vq_dim * c.latent * 3                             # pre-conv, kernel 3
    f += 2 * T * c.latent * c.hidden * 2                             # transformer in/out projections
    win = sum(min(t + 1, c.window) for t in range(T))
    f += c.layers * (2 * T * c.hidden * ad * 4 + 2 * T * c.hidden * c.inter * 3 + 2 * 2 * win * ad)
    L = T
    for s in c.upsample:
        f += 2 * c.latent * c.latent * L * s                          # transposed conv, kernel = stride
        L *= s
        inner = c.latent * c.convnext_mult
        f += 2 * L * (c.latent * c.convnext_kernel + 2 * c.latent * inner)
    f += 2 * c.latent * c.vocos_channels * 7 * L
    for (cin, cout, k, s) in c.vocos:
        f += 2 * cin * cout * k * L                                   # each input sample meets every tap once
        L *= s
        f += len(c.dilations) * 2 * L * (cout * cout * c.res_kernel + cout * cout)
    f += 2 * L * c.vocos[-1][1] * c.out_kernel
    return f


def decoder_measure(ctx, frames, cpu_frames=2, reps=3):
    """decode_to_audio of `frames` frames of the 1.7B decoder (random
    weights), codes and audio resident in HBM, HIP events on the context's
    stream; and the oracle's decode of a short sample on the host cores."""
    w = qtts.DecoderWeights(9)
    dec = qtts.SpeechDecoder(ctx, w)
    codes = w.synthetic_codes(12, frames)
    hip = Hip()
    n = dec.num_samples(frames)
    dc, da = hip.malloc(codes.nbytes), hip.malloc(4 * n)
    hip.h2d(dc, codes)
    dec.decode_to_audio_device(dc, frames, frames, da, n)  # warmup (work buffers)
    ctx.synchronize()
    start, end = hip.event(), hip.event()
    hip.record(start, ctx.stream)
    for _ in range(reps):
        dec.decode_to_audio_device(dc, frames, frames, da, n)
    hip.record(end, ctx.stream)
    avg_s = hip.elapsed_ms(start, end) / 1e3 / reps
    hip.free(dc)
    hip.free(da)
    flops = decoder_flops(w.cfg, frames)
    achieved = flops / avg_s / 1e12
    out = {
        "frames": frames, "samples": n, "ms": round(avg_s * 1e3, 2),
        "audio_seconds_per_second": round(n / 24000.0 / avg_s, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "algorithmic_flops": flops,
                     "issued_f16_TFLOPs": round(3 * achieved, 1),
                     "frac_of_f32_peak": round(achieved / FP32_PEAK_TFLOPS, 4),
                     "kernel": "whole decode (k_dec_conv_mfma dominant: every projection and convolution as "
                               "three binary16 MFMAs per f32 product term)"},
    }
    if cpu_frames:
        from oracle import oracle

        small = w.synthetic_codes(13, cpu_frames)
        t0 = time.perf_counter()
        oracle.decode_to_audio(w, small)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(cpu_frames * 1920 / 24000.0 / dt, 4), "unit": "audio s/s",
                               "cores": oracle.available_parallelism(), "kind": "port",
                               "sample": f"{cpu_frames} frames (C oracle, convolutions split over output channels "
                                         f"like the reference's threads)"}
    return out


def talker_only_measure(ctx, talker, prompt, steps=CONFIG_STEPS):
    """Config 3: the talker-only loop (the legacy feedback,
    codec_embedding[code0] as the next input, src/generate.rs:225-227) after
    a 64-token prefill, `steps` sampled steps (top-k 50, T 0.8, penalty 1.05,
    EOS ignored) at cache lengths 65..64+steps, HIP events on the context's
    stream around the loop.  Algorithmic bytes: talker_step_bytes at each
    step's cache length."""
    params = lambda n: qtts.loop_params(n, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False,
                                        talker_only=True)

    def run(n, seed, timed):
        kv = talker.new_kv(PROMPT + steps + 8)
        lh = talker.prefill_talker_raw(prompt, PROMPT, kv)
        lg = talker.apply_codec_head(lh)
        hip = Hip()
        e0, e1 = hip.event(), hip.event()
        ctx.synchronize()
        hip.record(e0, ctx.stream)
        codes = qtts.generate_codes(talker, None, kv, None, lh, lg, PROMPT, None, None, params(n), seed=seed)
        hip.record(e1, ctx.stream)
        s = hip.elapsed_ms(e0, e1) / 1e3
        kv.close()
        assert codes.shape[1] == n
        return s

    run(4, 3, False)  # program build, untimed
    s = run(steps, 7, True)
    tc = qtts.TALKER_1P7B
    total = sum(talker_step_bytes(tc, PROMPT + i) for i in range(steps))
    achieved = total / s / 1e9
    return {"steps": steps, "kv_len": [PROMPT + 1, PROMPT + steps], "codes_per_s": round(steps / s, 1),
            "ms_per_step": round(s * 1e3 / steps, 4),
            "timing": "HIP events around one qtts_generate_codes call (talker_only)",
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes": total}}


def cpu_side(tw, out, steps=16):
    """The oracle (the C restatement of the reference's CPU path, threads as
    the reference's gemv_q4 spawns them) on this host for the stand-alone
    measurements: each GEMV shape (5 calls), the config-2 talker step (2
    steps at a 256-row cache) and `steps` steps of the config-3 talker-only
    loop after the 64-token prefill."""
    from oracle import oracle

    threads = oracle.available_parallelism()
    for g in out.get("gemv", []):
        K, N = map(int, g["shape"].split("->"))
        w = qtts.Q4Weight.synthetic(99, f"roof.{K}.{N}.0", K, N)
        x = qtts.synth_normal_f32(99, "roof.x", K)
        oracle.gemv(x, w)
        t0 = time.perf_counter()
        for _ in range(5):
            oracle.gemv(x, w)
        g["cpu_us"] = round((time.perf_counter() - t0) / 5 * 1e6, 1)
        g["cpu_threads"] = threads
    ot = oracle.Talker(tw)
    c = tw.cfg
    if "talker_step" in out:
        L = out["talker_step"]["kv_len"][0] - 1
        shape = (c.layers, L, c.kv_heads, c.head_dim)
        k = qtts.synth_normal_f32(3, "kv.k", int(np.prod(shape))).reshape(shape)
        v = qtts.synth_normal_f32(3, "kv.v", int(np.prod(shape))).reshape(shape)
        okv = ot.new_kv(L + 4)
        okv.load(k, v, L)
        del k, v
        emb = qtts.synth_normal_f32(3, "step.emb", c.hidden)
        ot.forward_with_embedding(emb, okv, L)
        t0 = time.perf_counter()
        for i in range(2):
            ot.forward_with_embedding(emb, okv, L + 1 + i)
        out["talker_step"]["cpu_us"] = round((time.perf_counter() - t0) / 2 * 1e6, 1)
        out["talker_step"]["cpu_threads"] = threads
        del okv
    if "talker_only" in out:
        prompt = qtts.synth_normal_f32(2, "bench.prompt", PROMPT * c.hidden)
        okv = ot.new_kv(PROMPT + steps + 4)
        lh = ot.prefill_talker_raw(prompt, PROMPT, okv)
        lg = ot.apply_codec_head(lh)
        params = qtts.loop_params(steps, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False,
                                  talker_only=True)
        t0 = time.perf_counter()
        codes = oracle.generate_codes(ot, None, okv, None, lh, lg, PROMPT, None, None, params, seed=7)
        dt = time.perf_counter() - t0
        out["talker_only"]["cpu"] = {"codes_per_s": round(codes.shape[1] / dt, 3), "threads": threads,
                                     "sample": f"{codes.shape[1]} steps at KV {PROMPT + 1}..{PROMPT + codes.shape[1]}"}


def batch_measure(ctx, talker, pred, streams=16, kv_len=1064, frames=32):
    """The batched long-form case: `streams` independent loops in lockstep
    (qtts_generate_codes_batch), each prefilled to kv_len positions -- the
    mean cache length of 64-token prompts followed by 2000 codes -- then
    `frames` sampled frames; aggregate codes/s over the HIP-event-timed
    frames, and bytes per frame (every Q4 weight once for all streams plus
    each stream's K/V reads and appends)."""
    H = talker.cfg.hidden
    kvs, lhs, lgs = [], [], []
    for b in range(streams):
        x = qtts.synth_normal_f32(5, f"bench.batch.{b}", kv_len * H)
        kv = talker.new_kv(kv_len + frames + 8)
        lh = talker.prefill_talker_raw(x, kv_len, kv)
        kvs.append(kv)
        lhs.append(lh)
        lgs.append(talker.apply_codec_head(lh))
    text = qtts.synth_normal_f32(5, "bench.batch.text", streams * 8 * H, 0.0, 0.1).reshape(streams, 8, H)
    pad = qtts.synth_normal_f32(5, "bench.batch.pad", H, 0.0, 0.1)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    hip = Hip()
    ev0, ev1 = hip.event(), hip.event()
    ctx.synchronize()
    hip.record(ev0, ctx.stream)
    qtts.generate_codes_batch(talker, pred, kvs, np.stack(lhs), np.stack(lgs), [kv_len] * streams, text, pad, params,
                              list(range(streams)))
    hip.record(ev1, ctx.stream)
    ctx.synchronize()
    s = hip.elapsed_ms(ev0, ev1) / 1e3
    for kv in kvs:
        kv.close()
    weights = frame_bytes(qtts.TALKER_1P7B, qtts.PREDICTOR_1P7B, qtts.NUM_GROUPS, 0)
    kv_bytes = streams * 2 * 4 * qtts.TALKER_1P7B.layers * qtts.TALKER_1P7B.kv_heads * qtts.TALKER_1P7B.head_dim * (
        kv_len + frames / 2.0)
    per_frame = weights + kv_bytes
    achieved = per_frame * frames / s / 1e9
    return {"streams": streams, "kv_len": [kv_len, kv_len + frames], "frames": frames,
            "codes_per_s": round(streams * frames / s, 1), "ms_per_frame": round(s * 1e3 / frames, 3),
            "timing": "HIP events around qtts_generate_codes_batch (host copies of the prompt state included)",
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_frame": per_frame}}


def copy_calibration(ctx, nbytes=512 << 20):
    """One device-to-device copy of a known size: the plain copy kernel whose
    FETCH_SIZE / WRITE_SIZE counters calibrate the GEMV's."""
    hip = Hip()
    a, b = hip.malloc(nbytes), hip.malloc(nbytes)
    rc = hip.lib.hipMemcpyDtoD(hip.C.c_void_p(b), hip.C.c_void_p(a), hip.C.c_size_t(nbytes))
    hip._ok(rc, "hipMemcpyDtoD")
    hip._ok(hip.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")
    hip.free(a)
    hip.free(b)
    return nbytes


def read_traffic(name, key=None, per="launch"):
    """HBM bytes per launch (or per code) measured by the rocprofv3 counter
    runs (profiles/<name>), if present: the line `traffic_bytes_per_launch:`
    or, with a key, `traffic_bytes_per_launch[key]:`."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    tag = f"traffic_bytes_per_{per}" + (f"[{key}]" if key else "") + ":"
    for line in open(path):
        if line.startswith(tag):
            return int(float(line.split(":")[1]))
    return None


def host_info():
    """CPU model, the C library and the cores this process may run on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = "unknown"
    aff = sorted(os.sched_getaffinity(0))
    return {"cpu": model, "libc": libc, "affinity_cpus": len(aff),
            "affinity": f"{aff[0]}-{aff[-1]}" if aff else ""}


def cpu_baseline(tw, pw, gpu_kv, start, last_hidden, logits, text, pad, frames):
    """The oracle's frame loop on this host, from a copy of the GPU's cache at
    the timed window's first position."""
    from oracle import oracle

    ot, op = oracle.Talker(tw), oracle.CodePredictor(pw)
    okv = ot.new_kv(start + frames + 8)
    k, v = gpu_kv.store()
    okv.load(np.ascontiguousarray(k[:, :start]), np.ascontiguousarray(v[:, :start]), start)
    del k, v
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    t0 = time.perf_counter()
    codes = oracle.generate_codes(ot, op, okv, op.new_kv(), last_hidden, logits, start, text, pad, params, seed=42)
    dt = time.perf_counter() - t0
    threads = oracle.available_parallelism()
    info = host_info()
    return {
        "value": round(codes.shape[1] / dt, 4),
        "unit": "codes/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{codes.shape[1]} codes of the same loop at KV {start + 1}..{start + codes.shape[1]} "
                  f"(C oracle, -O3, no -march; talker GEMVs with k*n >= 4e6 split over {threads} threads as "
                  f"the reference's gemv_q4 spawns; the predictor single-threaded, as in the reference)",
        "host": info,
    }


def attention_only(ctx, talker, L, steps=8):
    """Multi-kernel talker steps (QTTS_ENGINE=ops) at a cache of L N(0,1)
    rows, so that the talker attention runs as its own launches (k_attn, one
    per layer): the command the attention kernel's counter and trace runs
    profile.  Prints the per-step time; algorithmic attention bytes per
    launch are the K and V rows read, 2 * rows * kv_heads * head_dim * 4,
    with rows = L + 1 .. L + steps (mean L + (steps + 1) / 2)."""
    os.environ["QTTS_ENGINE"] = "ops"
    c = talker.cfg
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    k = qtts.synth_normal_f32(3, "attn.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(3, "attn.v", int(np.prod(shape))).reshape(shape)
    kv = talker.new_kv(L + steps + 8)
    kv.load(k, v, L)
    del k, v
    emb = qtts.synth_normal_f32(3, "attn.emb", c.hidden)
    t0 = time.perf_counter()
    for i in range(steps):
        talker.forward_with_embedding(emb, kv, L + i)
    dt = (time.perf_counter() - t0) / steps
    per_launch = 2 * (L + (steps + 1) / 2.0) * c.kv_heads * c.head_dim * 4  # mean rows read: L + 4.5
    kv.close()
    return {"L": L, "steps": steps, "ms_per_step": round(dt * 1e3, 3), "attn_bytes_per_launch": per_launch}


ENGINE_OP_KINDS = {1: "GEMV", 2: "ATTN", 3: "COMB", 4: "AMAX", 5: "SAMP", 6: "EMB"}


def engine_trace_summary(path):
    """Critical-path attribution of the last k_engine launch in a
    QTTS_ENGINE_TRACE file ({nops, grid, kind[nops], ntasks[nops], u64
    stamps[nops][grid][10]}, slot 0 = a block's op start and slot 1 its op
    end on the 100 MHz wall clock).  Each op is charged the time by which it
    moves the end of the chain (its last block's end past every earlier op's
    end); ops before the embedding-sum op are the sampler and the 15
    predictor passes, ops after it the talker step."""
    data = open(path, "rb").read()
    off, last = 0, None
    while off < len(data):
        nops, grid = np.frombuffer(data, np.int32, 2, off)
        off += 8
        kinds = np.frombuffer(data, np.int32, nops, off)
        off += 4 * nops
        ntasks = np.frombuffer(data, np.int32, nops, off)
        off += 4 * nops
        st = np.frombuffer(data, np.uint64, nops * grid * 10, off).reshape(nops, grid, 10).astype(np.int64)
        off += 8 * nops * grid * 10
        last = (kinds, ntasks, st)
    kinds, ntasks, st = last
    valid = st[:, :, 0] > 0
    t0 = st[:, :, 0][valid].min()
    ends = np.array([st[i, valid[i], 1].max() if valid[i].any() else 0 for i in range(len(kinds))])
    emb = [i for i, k in enumerate(kinds) if k == 6]
    e = emb[0] if emb else len(kinds)
    groups, prev, sections = {}, t0, {"predictor": 0.0, "embedding sum": 0.0, "talker": 0.0}
    for i in range(len(kinds)):
        inc = (ends[i] - prev) * 0.01 if ends[i] > 0 else 0.0
        inc = max(inc, 0.0)
        prev = max(prev, ends[i])
        sec = "predictor" if i < e else ("embedding sum" if i == e else "talker")
        key = f"{sec} {ENGINE_OP_KINDS.get(int(kinds[i]), '?')} tasks={int(ntasks[i])}"
        n, tot = groups.get(key, (0, 0.0))
        groups[key] = (n + 1, tot + inc)
        sections[sec] += inc
    return {"ops": int(len(kinds)), "grid": int(st.shape[1]), "launch_us": round((ends.max() - t0) * 0.01, 1),
            "sections_us": {k: round(v, 1) for k, v in sections.items()},
            "by_op": {k: {"n": n, "us": round(t, 1), "us_per_op": round(t / n, 2)} for k, (n, t) in groups.items()}}


def engine_trace(ctx, talker, pred, path, codes=3):
    """Traces `codes` frames of the loop at cache lengths 315.. (the 500-code
    loop's mean, 314.5) after a 64-token prompt and 250 untimed codes."""
    hidden = talker.cfg.hidden
    prompt = qtts.synth_normal_f32(2, "bench.prompt", PROMPT * hidden)
    text = qtts.synth_normal_f32(2, "bench.text", 8 * hidden, 0.0, 0.1).reshape(8, hidden)
    pad = qtts.synth_normal_f32(2, "bench.pad", hidden, 0.0, 0.1)
    lead = 250
    kv = talker.new_kv(PROMPT + lead + codes + 8)
    lh = talker.prefill_talker_raw(prompt, PROMPT, kv)
    lg = talker.apply_codec_head(lh)
    pkv = pred.new_kv()
    params = lambda n: qtts.loop_params(n, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    qtts.generate_codes(talker, pred, kv, pkv, lh, lg, PROMPT, text, pad, params(lead), seed=40)
    if os.path.exists(path):
        os.remove(path)
    os.environ["QTTS_ENGINE_TRACE"] = path
    os.environ["QTTS_ENGINE_TRACE_FROM"] = "0"
    qtts.generate_codes(talker, pred, kv, pkv, lh, lg, PROMPT + lead, text, pad, params(codes), seed=42)
    del os.environ["QTTS_ENGINE_TRACE"]
    out = engine_trace_summary(path)
    out["kv_len"] = [PROMPT + lead + 1, PROMPT + lead + codes]
    kv.close()
    return out




def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=CONFIG_CODES)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-frames", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-roofline", action="store_true", help="skip the stand-alone timings")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the GEMV timings and the copy-kernel calibration (for counter runs)")
    ap.add_argument("--attention-only", type=int, default=0, metavar="L",
                    help="only multi-kernel talker steps at a cache of L rows (for attention counter runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 64-token talker prefill (10 timed calls) and its stand-alone gate|up GEMM "
                         "(for prefill kernel traces)")
    ap.add_argument("--batch-only", action="store_true",
                    help="only the 16-stream batched loop of the `batch` field (for batch kernel traces)")
    ap.add_argument("--decoder-only", type=int, default=0, metavar="FRAMES",
                    help="only the speech decoder's decode of FRAMES frames (for decoder kernel traces)")
    ap.add_argument("--engine-trace", default="", metavar="FILE",
                    help="only a per-op trace of 3 frames at cache lengths 315..317 (written to FILE) and its "
                         "critical-path summary")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the per-code loop at batch 1 is a serial "
              f"chain and independent streams shard with no collectives", file=sys.stderr)
        sys.exit(2)

    if args.roofline_only:
        ctx = qtts.Context(0)
        roof = gemv_shapes(ctx)
        floor = copy_floor(ctx)
        rfloor = read_floor(ctx)
        copied = copy_calibration(ctx)
        print(json.dumps({"gemv": roof, "copy_floor": floor, "read_floor": rfloor, "copy_bytes": copied}), flush=True)
        ctx.close()
        return

    if args.decoder_only:
        ctx = qtts.Context(0)
        print(json.dumps({"decoder": decoder_measure(ctx, args.decoder_only, cpu_frames=0)}), flush=True)
        ctx.close()
        return

    t0 = time.time()
    tw = qtts.TalkerWeights(1, qtts.TALKER_1P7B)
    pw = qtts.CodePredictorWeights(1, qtts.PREDICTOR_1P7B, talker_hidden=qtts.TALKER_1P7B.hidden)
    log(f"synthetic weights {time.time() - t0:.1f}s")
    ctx = qtts.Context(0)
    talker = qtts.Talker(ctx, tw)
    if args.attention_only:
        out = attention_only(ctx, talker, args.attention_only)
        print(json.dumps({"attention_only": out}), flush=True)
        ctx.close()
        return
    if args.prefill_only:
        hidden = tw.cfg.hidden
        prompt = qtts.synth_normal_f32(2, "bench.prompt", PROMPT * hidden)
        hip = Hip()
        ev0, ev1 = hip.event(), hip.event()
        def one_prefill():
            kv = talker.new_kv(2 * PROMPT)
            talker.prefill_talker_raw(prompt, PROMPT, kv)
            kv.close()

        for _ in range(2):
            one_prefill()
        ctx.synchronize()
        hip.record(ev0, ctx.stream)
        for _ in range(10):
            one_prefill()
        hip.record(ev1, ctx.stream)
        ctx.synchronize()
        pf_s = hip.elapsed_ms(ev0, ev1) / 1e3 / 10
        print(json.dumps({"prefill": {"tokens": PROMPT, "ms": round(pf_s * 1e3, 3),
                                      "timing": "HIP events around 10 prefill_talker_raw calls (cache creation "
                                                "included)", "gemm": mfma_gemm_roofline(ctx)}}), flush=True)
        ctx.close()
        return
    pred = qtts.CodePredictor(ctx, pw)
    log(f"uploaded {time.time() - t0:.1f}s")
    if args.batch_only:
        # a 2-frame call first makes the one-time matrix-core operand copies
        # and predictor tables, as the default run's earlier legs do
        batch_measure(ctx, talker, pred, frames=2)
        print(json.dumps({"batch": batch_measure(ctx, talker, pred)}), flush=True)
        ctx.close()
        return
    if args.engine_trace:
        print(json.dumps({"engine_trace": engine_trace(ctx, talker, pred, args.engine_trace)}), flush=True)
        ctx.close()
        return
    hidden = tw.cfg.hidden
    prompt = qtts.synth_normal_f32(2, "bench.prompt", PROMPT * hidden)
    text = qtts.synth_normal_f32(2, "bench.text", 8 * hidden, 0.0, 0.1).reshape(8, hidden)
    pad = qtts.synth_normal_f32(2, "bench.pad", hidden, 0.0, 0.1)
    # codes before the timed window (untimed, the same loop): the window's
    # mean cache length is the 500-code loop's, 314.5
    lead = max(0, int(round(PROMPT + 1 + (CONFIG_CODES - 1) / 2.0 - (args.steps - 1) / 2.0)) - (PROMPT + 1))
    cap = PROMPT + lead + max(args.steps, args.warmup) + 8

    def prefill():
        kv = talker.new_kv(cap)
        lh = talker.prefill_talker_raw(prompt, PROMPT, kv)
        return kv, lh, talker.apply_codec_head(lh)

    params = lambda n: qtts.loop_params(n, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    pkv = pred.new_kv()
    if args.warmup > 0:
        kv, lh, lg = prefill()
        qtts.generate_codes(talker, pred, kv, pkv, lh, lg, PROMPT, text, pad, params(args.warmup), seed=41)
        kv.close()
        log(f"warmup {args.warmup} codes done")
    kv, lh, lg = prefill()
    if lead:
        qtts.generate_codes(talker, pred, kv, pkv, lh, lg, PROMPT, text, pad, params(lead), seed=40)
    start = PROMPT + lead  # cache length before the first timed code
    assert len(kv) == start
    hip = Hip()
    ev0, ev1 = hip.event(), hip.event()
    ctx.synchronize()
    t1 = time.perf_counter()
    hip.record(ev0, ctx.stream)
    codes = qtts.generate_codes(talker, pred, kv, pkv, lh, lg, start, text, pad, params(args.steps), seed=42)
    hip.record(ev1, ctx.stream)
    ctx.synchronize()
    dt = time.perf_counter() - t1
    gpu_s = hip.elapsed_ms(ev0, ev1) / 1e3
    assert codes.shape == (16, args.steps), codes.shape
    cps = args.steps / dt
    log(f"{args.steps} codes (KV {start + 1}..{start + args.steps}) in {dt * 1e3:.1f} ms -> {cps:.1f} codes/s")

    out = {
        "metric": "codes/sec, 1.7B talker+predictor bs=1; Q4 GEMV HBM GB/s vs peak",
        "value": round(cps, 3),
        "unit": "codes/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "talker (28 layers, hidden 2048, 16/8 heads, SwiGLU 6144, vocab 3072) + code predictor "
                        "(5 layers, hidden 1024, 15 argmax heads of 2048) per code, Q4 g=32 weights, batch 1; "
                        "500-code loop after a 64-token prefill (KV 65..564)",
            "prompt_tokens": PROMPT,
            "kv_len": [start + 1, start + args.steps],
            "kv_len_mean": start + (args.steps + 1) / 2.0,
            "untimed_lead_codes": lead,
            "sampler": "top-k 50, temperature 0.8, repetition penalty 1.05",
        },
    }
    out["roofline"] = engine_roofline(args.steps, gpu_s, start + (args.steps - 1) / 2.0)
    log(f"roofline {out['roofline']}")
    if not args.no_roofline:
        out["gemv"] = gemv_shapes(ctx)
        for g in out["gemv"]:
            log(f"stand-alone gemv {g}")
        out["read_floor"] = read_floor(ctx)
        log(f"single-launch read floor {out['read_floor']}")
        out["talker_step"] = talker_step_measure(ctx, talker)
        log(f"talker step {out['talker_step']}")
        out["talker_only"] = talker_only_measure(ctx, talker, prompt)
        log(f"talker-only loop {out['talker_only']}")
        # the 64-token prompt prefill (matrix-core path), HIP events
        ctx.synchronize()
        hip.record(ev0, ctx.stream)
        for _ in range(5):
            prefill()[0].close()
        hip.record(ev1, ctx.stream)
        ctx.synchronize()
        pf_s = hip.elapsed_ms(ev0, ev1) / 1e3 / 5
        out["prefill"] = {"tokens": PROMPT, "ms": round(pf_s * 1e3, 3), "tokens_per_s": round(PROMPT / pf_s, 1),
                          "timing": "HIP events around 5 prefill_talker_raw calls, host copies included",
                          "gemm": mfma_gemm_roofline(ctx)}
        log(f"prefill {out['prefill']}")
        out["decoder"] = decoder_measure(ctx, CONFIG_CODES, cpu_frames=0 if args.no_cpu else 2)
        log(f"decoder {out['decoder']}")
        out["batch"] = batch_measure(ctx, talker, pred)
        log(f"batch {out['batch']}")
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(tw, pw, kv, start, lh, lg, text, pad, args.cpu_frames)
        log(f"cpu baseline {out['cpu_baseline']}")
        if not args.no_roofline:
            cpu_side(tw, out)
            log("cpu side: gemv " + str([g.get("cpu_us") for g in out["gemv"]]) +
                f" talker step {out['talker_step'].get('cpu_us')} us, talker-only {out['talker_only'].get('cpu')}")
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()

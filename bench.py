#!/usr/bin/env python3
"""Benchmark of the MI355X quantized decode hot path (one GPU).

Headline workload: the beam/ragged-batched int8 decode GEMV -- M = 3 packed
rows (beam width 3), K = 2048, N = 8192, int8 weights with one fp16 scale per
32-element group, activations quantized per row to int8 (absmax/127).  The
GEMV runs over enough distinct weight copies (>= 300 MB) that the 256 MB
Infinity Cache cannot hold them, so every launch streams its weights from
HBM; one step = one GEMV on each copy (a pass over that many layers).  The K
timed steps' launches are replayed as one HIP graph (no host launch overhead
in the timed region) and timed with HIP events on the stream the kernels run
on.

Printed: one JSON line with the metric, a roofline object for the GEMV
kernel (algorithmic bytes / average launch time vs 8 TB/s) and the CPU
baseline (a restatement of the reference CPU MatMulRows in the SIMD tier the
reference picks on the host, row-parallel over NEEDLE_THREADS = the physical
core count, on a bounded sample).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import needle_cs_amd as N  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA
METRIC = "int8 decode GEMV GB/s (% HBM peak); beam-3 batched decode tokens/sec"


PROFILE = os.path.join(ROOT, "profiles", "gemv_i8_decode_m3_k2048_n8192.txt")


def measured_traffic() -> int | None:
    """HBM bytes per launch of the headline GEMV kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (copy-kernel calibrated)."""
    try:
        with open(PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def gemv_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one int8/g32 GEMV: weights, fp16 scales, int8
    activations + fp32 row scales, fp32 outputs."""
    return n * k + n * (k // 32) * 2 + m * k + m * 4 + m * n * 4


class GemvCase:
    """Device-resident inputs of one GEMV shape: `copies` distinct weight
    matrices, one activation batch, one output buffer."""

    def __init__(self, m: int, k: int, n: int, seed: int, min_bytes: int = 300 << 20):
        self.m, self.k, self.n = m, k, n
        st = C.c_uint64(seed)
        per = n * k + n * (k // 32) * 2
        self.copies = max(2, -(-min_bytes // per))
        self.weights = []
        for _ in range(self.copies):
            w = N.synth_int8(st, n * k).reshape(n, k)
            s = N.synth_half_uniform(st, n * (k // 32), 0.002, 0.02).reshape(n, k // 32)
            self.weights.append(N.Weights.int8(w, s))
        self.host_w, self.host_s = w, s  # last copy, reused by the CPU baseline
        x = N.synth_normal(st, m * k).reshape(m, k)
        self.x = x
        dx = N.DeviceBuffer.from_array(x)
        self.dq = N.DeviceBuffer(m * k)
        self.ds = N.DeviceBuffer(m * 4)
        N.check(N.lib().nhip_quantize_rows_dev(dx.ptr, m, k, self.dq.ptr, self.ds.ptr, None))
        self.dy = N.DeviceBuffer(m * n * 4)
        self.bytes = gemv_bytes(m, k, n)

    def launch(self, i: int) -> None:
        w = self.weights[i % self.copies]
        N.check(N.lib().nhip_matmul_i8_dev(w.handle, self.dq.ptr, self.ds.ptr, self.m, self.dy.ptr, self.n, 0,
                                           self.n, None))

    def time(self, steps: int, warmup: int) -> float:
        """Average ms per launch over `steps` launches replayed as one graph,
        bracketed by two events on the launches' stream (after `warmup` eager
        launches and one untimed replay)."""
        for i in range(warmup):
            self.launch(i)
        N.check(N.lib().nhip_device_sync())
        with N.Graph.capture() as g:
            for i in range(steps):
                self.launch(i)
        g.launch()  # the first replay carries one-time costs
        N.check(N.lib().nhip_device_sync())
        start, stop = N.Event(), N.Event()
        start.record()
        g.launch()
        stop.record()
        ms = start.elapsed_ms(stop)
        N.check(N.lib().nhip_device_sync())
        g.close()
        return ms / steps

    def close(self) -> None:
        for w in self.weights:
            w.close()


class ReadCase:
    """The read ceiling of one launch: nhip_read_stream_dev over `nbytes`
    (the GEMV's weight and scale bytes) with the GEMV's access pattern,
    cycling as many distinct buffers as the GEMV cycles weight copies."""

    def __init__(self, nbytes: int, copies: int):
        self.nbytes = nbytes - nbytes % 16
        self.bufs = []
        for _ in range(copies):
            b = N.DeviceBuffer(self.nbytes)
            N.check(N.lib().nhip_memset(b.ptr, 0x5A, b.nbytes))
            self.bufs.append(b)
        self.sink = N.DeviceBuffer(-(-self.nbytes // 32768) * 4)

    def launch(self, i: int) -> None:
        b = self.bufs[i % len(self.bufs)]
        N.check(N.lib().nhip_read_stream_dev(b.ptr, self.nbytes, self.sink.ptr, None))

    time = GemvCase.time

    def close(self) -> None:
        for b in self.bufs:
            b.close()
        self.sink.close()


class Needle3Case:
    """Needle 3 attention inputs (nhip_needle3_attention_inputs_dev) for `rows`
    rows of one geometry: three-tap convolution over the slot history,
    ZeroCenteredRms, Rope and QuantizeInt8 into the queries and the KV cache.
    Rows of a slot are consecutive positions (a run per slot)."""

    def __init__(self, seed: int, rows: int, slots: int, heads: int = 16, kv: int = 16, qk: int = 64, vd: int = 64,
                 capacity: int = 256):
        st = C.c_uint64(seed)
        self.rows, self.g, self.slots, self.capacity = rows, (heads, kv, qk, vd), slots, capacity
        qw, kw, vw = heads * qk, kv * qk, kv * vd
        allw = qw + kw + vw
        D = N.DeviceBuffer.from_array
        f = lambda n, sc=1.0: N.synth_normal(st, n) * np.float32(sc)
        self.bufs = [D(f(rows * allw))]
        self.bufs += [D(f(3 * w, 0.5)) for w in (qw, kw, vw)]
        self.bufs += [D(f(qk, 0.1)), D(f(qk, 0.1))]
        ang = N.synth_uniform(st, capacity * qk // 2, 0.0, 6.28)
        self.bufs += [D(np.cos(ang).astype(np.float32)), D(np.sin(ang).astype(np.float32)), D(f(slots * 2 * allw))]
        per = -(-rows // slots)
        assert 100 + per < capacity
        slot = np.repeat(np.arange(slots, dtype=np.int32), per)[:rows]
        pos = np.concatenate([100 + np.arange(per, dtype=np.int32)] * slots)[:rows]
        self.bufs += [D(slot), D(pos)]
        self.bufs += [N.DeviceBuffer(rows * qw), N.DeviceBuffer(rows * heads * 4),
                      N.DeviceBuffer(slots * capacity * kw), N.DeviceBuffer(slots * capacity * kv * 4),
                      N.DeviceBuffer(slots * capacity * vw), N.DeviceBuffer(slots * capacity * kv * 4)]

    def launch(self, i: int) -> None:
        heads, kv, qk, vd = self.g
        b = [x.ptr for x in self.bufs]
        N.check(N.lib().nhip_needle3_attention_inputs_dev(
            b[0], self.rows, heads, kv, qk, vd, b[1], b[2], b[3], b[4], b[5], b[6], b[7], b[8], b[9], b[10],
            self.slots, self.capacity, b[11], b[12], b[13], b[14], b[15], b[16], None))

    time = GemvCase.time

    def close(self) -> None:
        for x in self.bufs:
            x.close()


class GemmCase(GemvCase):
    """Prefill int8 GEMM: M=512 tokens, K=2048, N=8192, per-token int8
    activations; `fused` selects the fused-epilogue entry point."""

    def __init__(self, m: int, k: int, n: int, seed: int, fused: bool):
        super().__init__(m, k, n, seed, min_bytes=64 << 20)
        self.fused = fused
        self.ops = 2 * m * n * k

    def launch(self, i: int) -> None:
        w = self.weights[i % self.copies]
        fn = N.lib().nhip_matmul_i8_fused_dev if self.fused else N.lib().nhip_matmul_i8_dev
        N.check(fn(w.handle, self.dq.ptr, self.ds.ptr, self.m, self.dy.ptr, self.n, 0, self.n, None))


class CqGemvCase(GemvCase):
    """Reference-native GEMV (the .cact weight format): 4- or 2-bit codebook
    indices (uniform bytes), a codebook of levels U(-1, 1) from the seeded
    stream with Codebook.Fill's bytes (round-half-even of level / ByteScale
    + 63, ByteScale = max |level| / 63), fp16 norms U(0.002, 0.02) per
    128-column group, and N(0,1) activations through the Hadamard prepare
    (nhip_prepare_dev) outside the timed region."""

    def __init__(self, m: int, k: int, n: int, bits: int, seed: int, min_bytes: int = 300 << 20):
        self.m, self.k, self.n, self.bits = m, k, n, bits
        st = C.c_uint64(seed)
        count = 16 if bits == 4 else 4
        book = N.Codebook()
        levels = N.synth_uniform(st, 16, -1.0, 1.0).astype(np.float32)
        bscale = np.float32(np.max(np.abs(levels[:count])) / np.float32(63.0))
        for i in range(16):
            book.levels[i] = float(levels[i])
        for i in range(32):
            book.bytes[i] = int(np.rint(levels[i % 16] / bscale)) + 63 if i % 16 < count else 0
        book.byte_scale = float(bscale)
        self.book = book
        per = n * k * bits // 8 + n * (k // 128) * 2
        self.copies = max(2, -(-min_bytes // per))
        self.weights = []
        for _ in range(self.copies):
            idx = N.synth_int8(st, n * k * bits // 8).view(np.uint8)
            norms = N.synth_half_uniform(st, n * (k // 128), 0.002, 0.02)
            self.weights.append(N.Weights.codebook(idx, norms, book, n, k, bits))
        self.stride = ((k // 128) + 7) // 8 * 8
        x = N.synth_normal(st, m * k)
        dx = N.DeviceBuffer.from_array(x)
        self.dv = N.DeviceBuffer(m * k)
        self.dsc = N.DeviceBuffer(m * self.stride * 4)
        self.doff = N.DeviceBuffer(m * self.stride * 4)
        N.check(N.lib().nhip_prepare_dev(dx.ptr, m, k, bits, self.dv.ptr, self.dsc.ptr, self.doff.ptr, self.stride,
                                         None))
        self.dy = N.DeviceBuffer(m * n * 4)
        self.bytes = per + m * k + 2 * m * self.stride * 4 + m * n * 4

    def launch(self, i: int) -> None:
        w = self.weights[i % self.copies]
        N.check(N.lib().nhip_matmul_cq_dev(w.handle, self.dv.ptr, self.dsc.ptr, self.doff.ptr, self.stride, self.m,
                                           self.dy.ptr, self.n, 0, self.n, None))


class BatchCase(CqGemvCase):
    """Quant.MatMulBatch at Needle 3's attention projections: Q, K, V and
    Gate (576, 96, 128, 768 rows x 768 columns, Cq2 codebook, g128 norms)
    sharing one prepared activation set; `copies` sets of the four weights
    are cycled past the MALL.  launch() runs the grouped launch
    (nhip_matmul_batch_dev); launch_separate() the four single-matrix
    launches it replaces."""

    ROWS = (576, 96, 128, 768)

    def __init__(self, m: int, seed: int, min_bytes: int = 300 << 20):
        k, bits = 768, 2
        super().__init__(m, k, self.ROWS[0], bits, seed, min_bytes=1)  # activations, codebook, one weight set
        st = C.c_uint64(seed + 1)
        per = sum(n * k * bits // 8 + n * (k // 128) * 2 for n in self.ROWS)
        self.copies = max(2, -(-min_bytes // per))
        for w in self.weights:
            w.close()
        self.sets = []
        for _ in range(self.copies):
            ws = []
            for n in self.ROWS:
                idx = N.synth_int8(st, n * k * bits // 8).view(np.uint8)
                norms = N.synth_half_uniform(st, n * (k // 128), 0.002, 0.02)
                ws.append(N.Weights.codebook(idx, norms, self.book, n, k, bits))
            self.sets.append(ws)
        self.weights = [w for ws in self.sets for w in ws]
        self.outs = [N.DeviceBuffer(m * n * 4) for n in self.ROWS]
        self.Y = (C.c_void_p * 4)(*[o.ptr for o in self.outs])
        self.L = (C.c_int32 * 4)(*self.ROWS)
        self.handles = [(C.c_void_p * 4)(*[w.handle for w in ws]) for ws in self.sets]
        self.bytes = per + m * k + 2 * m * self.stride * 4 + m * sum(self.ROWS) * 4
        self.separate = False

    def launch(self, i: int) -> None:
        if self.separate:
            for w, o, n in zip(self.sets[i % self.copies], self.outs, self.ROWS):
                N.check(N.lib().nhip_matmul_cq_dev(w.handle, self.dv.ptr, self.dsc.ptr, self.doff.ptr, self.stride,
                                                   self.m, o.ptr, n, 0, n, None))
            return
        N.check(N.lib().nhip_matmul_batch_dev(self.handles[i % self.copies], 4, self.dv.ptr, self.dsc.ptr,
                                              self.doff.ptr, self.stride, self.m, self.Y, self.L, None))


def batch_lines(args) -> list:
    """MatMulBatch at Needle 3's Q/K/V/Gate shapes: one grouped launch against
    the four launches it replaces."""
    out = []
    for m in (1, 3):
        case = BatchCase(m, seed=0x6006 + m)
        t = case.time(max(200, args.steps // 4), args.warmup)
        case.separate = True
        t4 = case.time(max(200, args.steps // 4), args.warmup)
        g = case.bytes / (t * 1e-3) / 1e9
        out.append({"workload": f"Needle 3 Q/K/V/Gate MatMulBatch, Cq2 K=768 rows 576+96+128+768, M={m}",
                    "us_per_launch": round(t * 1e3, 3), "GB/s": round(g, 1),
                    "frac_hbm_peak": round(g / HBM_PEAK_GBS, 4), "bytes_per_launch": case.bytes,
                    "us_four_separate_launches": round(t4 * 1e3, 3)})
        print(f"# MatMulBatch QKVG M={m}: {t * 1e3:.2f} us/launch ({g:.0f} GB/s); four launches {t4 * 1e3:.2f} us",
              file=sys.stderr, flush=True)
        case.close()
    return out


class AttnCase:
    """Ragged decode attention: 16 sequences, context lengths U[32, 2048]
    (seeded), 16 heads x 64 (qk 64, MHA), int8 KV cache quantized per
    (position, head) from N(0,1), scale 1/sqrt(64), fp32 output [16,16,64].
    `copies` pooled caches are cycled so that every launch reads HBM."""

    def __init__(self, seed: int, rows: int = 16, heads: int = 16, qk: int = 64, capacity: int = 2048,
                 copies: int = 4, max_chunks: int = 64):
        self.rows, self.heads, self.qk, self.capacity, self.max_chunks = rows, heads, qk, capacity, max_chunks
        st = C.c_uint64(seed)
        counts = []
        for _ in range(rows):
            u = N.synth_uniform(st, 1, 0.0, 1.0)[0]
            counts.append(32 + min(int(u * (2048 - 32 + 1)), 2048 - 32))
        self.counts = np.array(counts, dtype=np.int32)
        slots = rows
        per_pos = heads * qk + heads * 4 + heads * 64 + heads * 4
        n_k, n_v = slots * capacity * heads * qk, slots * capacity * heads * 64
        self.caches = []
        kf = N.DeviceBuffer.from_array(N.synth_normal(st, n_k))
        vf = N.DeviceBuffer.from_array(N.synth_normal(st, n_v))
        for c in range(copies):
            k, ks = N.DeviceBuffer(n_k), N.DeviceBuffer(n_k // qk * 4)
            v, vs = N.DeviceBuffer(n_v), N.DeviceBuffer(n_v // 64 * 4)
            if c == 0:
                N.check(N.lib().nhip_quantize_rows_dev(kf.ptr, n_k // qk, qk, k.ptr, ks.ptr, None))
                N.check(N.lib().nhip_quantize_rows_dev(vf.ptr, n_v // 64, 64, v.ptr, vs.ptr, None))
            else:
                for dst, src in zip((k, ks, v, vs), self.caches[0]):
                    N.check(N.lib().nhip_copy_dev(dst.ptr, src.ptr, src.nbytes, None))
            self.caches.append((k, ks, v, vs))
        kf.close()
        vf.close()
        qf = N.DeviceBuffer.from_array(N.synth_normal(st, rows * heads * qk))
        self.dq, self.dqs = N.DeviceBuffer(rows * heads * qk), N.DeviceBuffer(rows * heads * 4)
        N.check(N.lib().nhip_quantize_rows_dev(qf.ptr, rows * heads, qk, self.dq.ptr, self.dqs.ptr, None))
        self.slot = N.DeviceBuffer.from_array(np.arange(rows, dtype=np.int32))
        self.first = N.DeviceBuffer.from_array(np.zeros(rows, dtype=np.int32))
        self.count = N.DeviceBuffer.from_array(self.counts)
        self.ws = N.DeviceBuffer(N.lib().nhip_attention_decode_workspace(rows, heads, max_chunks))
        N.check(N.lib().nhip_attention_decode_workspace_init(self.ws.ptr, self.ws.nbytes, None))
        self.out = N.DeviceBuffer(rows * heads * 64 * 4)
        self.copies = copies
        self.bytes = int(self.counts.sum()) * per_pos + rows * heads * (qk + 4) + rows * heads * 64 * 4

    def launch(self, i: int) -> None:
        k, ks, v, vs = self.caches[i % self.copies]
        N.check(N.lib().nhip_attention_decode_dev(self.dq.ptr, self.dqs.ptr, self.rows, self.heads, self.heads,
                                                  self.qk, k.ptr, ks.ptr, v.ptr, vs.ptr, self.rows, self.capacity,
                                                  self.slot.ptr, self.first.ptr, self.count.ptr, self.max_chunks,
                                                  self.ws.ptr, self.ws.nbytes, self.out.ptr, None))

    time = GemvCase.time

    def close(self) -> None:
        for c in self.caches:
            for b in c:
                b.close()


def decode_loop(args, threads: int) -> dict:
    """Beam-3 batched decode on the 12-layer d1024 int8 decoder: prompt of
    128 seeded ids (prefill), then up to 64 new tokens with beam width 3.
    row-tokens/s = rows fed after the prompt / decode wall time (beams are
    rows); the CPU path runs the same search twice on `threads` host
    threads: in the oracle's scalar order (its token stream must equal the
    GPU's) and with every linear in the reference's SIMD tier (the timed
    baseline)."""
    from needle_cs_amd.decoder import CONFIG4, GpuDecoder, random_prompt, synthetic_model

    t0 = time.perf_counter()
    model = synthetic_model(CONFIG4, 0x5005)
    prompt = random_prompt(0x6006, 128, CONFIG4["vocab"])
    gen_s = time.perf_counter() - t0
    width, max_new, eos = 3, 64, 1
    gpu = GpuDecoder(model, slots=width, capacity=256, max_rows=128, max_chunks=args.decode_chunks)
    gpu.beam_search(prompt, width, max_new, eos)  # captures the per-row-count graphs
    runs = []
    for _ in range(3):
        toks, score, st = gpu.beam_search(prompt, width, max_new, eos)
        runs.append((st.decode_seconds, st.prefill_seconds, st.fed_rows, st.steps, toks, score))
    gpu.close()
    dec_s, pre_s, fed, steps, toks, score = min(runs, key=lambda r: r[0])
    weight_bytes = sum(lw[n].nbytes for lw in model["layers"] for n in ("wqkv", "sqkv", "wo", "so", "wgu", "sgu",
                                                                           "wd", "sd")) + model["wlm"].nbytes + \
        model["slm"].nbytes
    out = {"workload": "beam-3 decode, 12 layers d1024 16x64 SwiGLU 4096 vocab 32000, int8 g32; prompt 128, "
                       "64 new tokens",
           "row_tokens_per_s": round(fed / dec_s, 1), "seq_tokens_per_s": round(steps / dec_s, 1),
           "ms_per_step": round(dec_s / max(steps, 1) * 1e3, 4), "prefill_ms": round(pre_s * 1e3, 3),
           "steps": steps, "fed_rows": fed, "weight_bytes_per_step": weight_bytes,
           "weights_GBps_per_step": round(weight_bytes / (dec_s / max(steps, 1)) / 1e9, 1),
           "tokens": int(len(toks)), "model_gen_s": round(gen_s, 1)}
    print(f"# decode loop: {out['row_tokens_per_s']} row-tokens/s, {out['ms_per_step']} ms/step, "
          f"prefill {out['prefill_ms']} ms", file=sys.stderr, flush=True)
    if not args.no_cpu:
        from oracle import oracle as O  # the CPU path: checked token for token, and timed as the baseline

        # the oracle's canonical order (the checker of the GPU's token stream)
        cpu = O.CpuDecoder(model, slots=width, capacity=256, threads=threads, max_chunks=args.decode_chunks)
        ctoks, cscore, cfed = cpu.beam_search(prompt, width, max_new, eos)
        spre, sdec = float(cpu.seconds[0]), float(cpu.seconds[1])
        cpu.close()
        same = bool(np.array_equal(ctoks, toks) and np.float32(cscore) == np.float32(score))
        # the reference's SIMD tier for every linear (the timed baseline)
        tier = O.lib().or_simd_tier()
        cpu = O.CpuDecoder(model, slots=width, capacity=256, threads=threads, max_chunks=args.decode_chunks,
                           simd=tier)
        vtoks, vscore, vfed = cpu.beam_search(prompt, width, max_new, eos)
        cpre, cdec = float(cpu.seconds[0]), float(cpu.seconds[1])
        cpu.close()
        out["tokens_identical_to_cpu_path"] = same
        out["tokens_identical_to_simd_cpu_path"] = bool(np.array_equal(vtoks, toks))
        common = int(np.argmax(np.append(vtoks[:len(toks)] != toks[:len(vtoks)], True)))
        out["simd_cpu_path_matching_prefix"] = min(common, len(toks), len(vtoks))
        out["cpu_path"] = {"row_tokens_per_s": round(vfed / cdec, 2), "prefill_ms": round(cpre * 1e3, 1),
                           "threads": threads, "kind": "port", "tier": TIER_NAMES[tier],
                           "scalar_order_row_tokens_per_s": round(cfed / sdec, 2),
                           "sample": "the same prompt and 64-token beam-3 search on the host: every int8 linear in "
                                     f"the reference's {TIER_NAMES[tier]} tier (oracle/cpu_simd.c) row-parallel over "
                                     f"{threads} threads; the token stream is also checked against the oracle's "
                                     "scalar order, timed as scalar_order_row_tokens_per_s"}
        out["speedup_vs_cpu_path"] = round(out["row_tokens_per_s"] / out["cpu_path"]["row_tokens_per_s"], 1)
        print(f"# decode loop CPU path ({TIER_NAMES[tier]}): {out['cpu_path']['row_tokens_per_s']} row-tokens/s "
              f"(scalar order {out['cpu_path']['scalar_order_row_tokens_per_s']}); identical tokens: {same} "
              f"(SIMD path: {out['tokens_identical_to_simd_cpu_path']})", file=sys.stderr, flush=True)
    return out


def needle3_step_bytes(archive: bytes, geometry: dict) -> int:
    """Weight bytes one decode step reads: every codebook record but the
    engram tables (a few gathered rows), the tied embedding once for the head,
    and the dense records as the fp32 arrays they become on the device."""
    from needle_cs_amd.archive import parse
    _, _, _, recs = parse(archive)
    first_site = 1 + geometry["layers"] * 27 + 11  # Model.Open's record order
    tables = {first_site + 4 * s for s in range(len(geometry["sites"]))}
    total = 0
    for i, r in enumerate(recs):
        dtype, nbytes = r[0], r[8]
        if dtype == 3 and i not in tables:
            total += nbytes
        elif dtype in (1, 2):
            total += nbytes * (2 if dtype == 1 else 1)
    return total


def needle3_loop(args, threads: int) -> dict:
    """Batched greedy decode of three slots on a random-init archive of
    Needle 3's geometry (20 layers, hidden 768, 12/2 heads, 5 engram sites,
    vocab 8192) through the step API: a 64-token prompt per slot (63 fed with
    FeedSlot, the last in the first 3-row step), then 63 decode steps of 3
    rows with the head's ArgMax as the next tokens.  The CPU leg runs the
    oracle's engine in the engine's row order (the AVX2 tier's sums) on the
    same prompts for a bounded number of steps, its matmul rows, attention
    rows and MLP rows spread over `threads` host threads (each output is still
    one thread's sum): its tokens must match the GPU's, its step time is the
    port baseline."""
    from needle_cs_amd.archive import NEEDLE3, needle3_archive
    from needle_cs_amd.engine import BatchedEngine, Model

    g3 = NEEDLE3
    archive = needle3_archive(g3, 0x7007)
    slots, prompt_len, new = 3, 64, 64
    prompts = np.random.default_rng(0x7008).integers(0, g3["vocab"], (slots, prompt_len)).astype(np.int32)
    step_bytes = needle3_step_bytes(archive, g3)
    lanes = np.arange(slots, dtype=np.int32)
    with Model(archive) as model, BatchedEngine(model, context_length=prompt_len + new, chunk_size=64, slots=slots,
                                                max_chunks=8) as eng:
        def run():
            for s in range(slots):
                eng.reset_slot(s)
            t0 = time.perf_counter()
            for s in range(slots):
                eng.feed_slot(s, prompts[s, :-1], compute_logits=False)
            _, _, _, toks = eng.forward_batch(prompts[:, -1], lanes, lanes, logits=False, argmax=True)
            pre = time.perf_counter() - t0
            out = [toks]
            t1 = time.perf_counter()
            for _ in range(new - 1):
                _, _, _, toks = eng.forward_batch(toks, lanes, lanes, logits=False, argmax=True)
                out.append(toks)
            return pre, time.perf_counter() - t1, np.stack(out, 1)

        run()  # captures the step graphs
        pre, dec, toks = min((run() for _ in range(3)), key=lambda r: r[1])
        # the same loop with all 16 slots of a BatchedEngine busy: the step's
        # row kernels run side by side, so rows cost little more than one
        wide = 16
        wide_prompts = np.random.default_rng(0x7009).integers(0, g3["vocab"], (wide, prompt_len)).astype(np.int32)
        wlanes = np.arange(wide, dtype=np.int32)
        with BatchedEngine(model, context_length=prompt_len + new, chunk_size=64, slots=wide, max_chunks=8) as eng16:
            def run16():
                for s in range(wide):
                    eng16.reset_slot(s)
                for s in range(wide):
                    eng16.feed_slot(s, wide_prompts[s, :-1], compute_logits=False)
                _, _, _, t16 = eng16.forward_batch(wide_prompts[:, -1], wlanes, wlanes, logits=False, argmax=True)
                t1 = time.perf_counter()
                for _ in range(new - 1):
                    _, _, _, t16 = eng16.forward_batch(t16, wlanes, wlanes, logits=False, argmax=True)
                return time.perf_counter() - t1

            run16()
            dec16 = min(run16() for _ in range(3))
        # one sequence alone: the step's latency, the figure a single user waits per token
        with BatchedEngine(model, context_length=prompt_len + new, chunk_size=64, slots=1, max_chunks=8) as eng1:
            one = np.zeros(1, dtype=np.int32)

            def run1():
                eng1.reset_slot(0)
                eng1.feed_slot(0, prompts[0, :-1], compute_logits=False)
                _, _, _, t1 = eng1.forward_batch(prompts[:1, -1], one, one, logits=False, argmax=True)
                t0 = time.perf_counter()
                for _ in range(new - 1):
                    _, _, _, t1 = eng1.forward_batch(t1, one, one, logits=False, argmax=True)
                return time.perf_counter() - t0

            run1()
            dec1 = min(run1() for _ in range(3))
    steps = new - 1
    ms = dec / steps * 1e3
    out = {"workload": "greedy decode of 3 slots, Needle 3 geometry (20 layers, hidden 768, 12/2 heads x 48/64, "
                       "MLP 32x32, 5 engram sites, vocab 8192), random-init archive; prompt 64 per slot, 63 steps",
           "row_tokens_per_s": round(slots * steps / dec, 1), "ms_per_step": round(ms, 4),
           "prefill_ms": round(pre * 1e3, 2), "weight_bytes_per_step": step_bytes,
           "weights_GBps_per_step": round(step_bytes / (ms * 1e-3) / 1e9, 2),
           "frac_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 5),
           "slots16": {"row_tokens_per_s": round(wide * steps / dec16, 1),
                       "ms_per_step": round(dec16 / steps * 1e3, 4)},
           "slots1": {"row_tokens_per_s": round(steps / dec1, 1), "ms_per_step": round(dec1 / steps * 1e3, 4)}}
    print(f"# needle3 decode: {out['row_tokens_per_s']} row-tokens/s, {ms:.3f} ms/step, prefill {pre * 1e3:.1f} ms; "
          f"16 slots: {out['slots16']['row_tokens_per_s']} row-tokens/s, {out['slots16']['ms_per_step']} ms/step; "
          f"1 slot: {out['slots1']['ms_per_step']} ms/step",
          file=sys.stderr, flush=True)
    if not args.no_cpu:
        from oracle import needle3 as M
        from oracle import oracle as O

        check_steps = 12
        O.lib().or_n3_set_threads(threads)
        O.lib().or_n3_set_tier(1)  # the engine's row order: the AVX2 tier's sums
        cpu = M.OracleEngine(O, M.OracleModel(O, archive), slots=slots, capacity=prompt_len + new, max_chunks=8)
        for s in range(slots):
            cpu.step(prompts[s, :-1], [s] * (prompt_len - 1), [])
        lg = cpu.step(prompts[:, -1], lanes, lanes)
        ctoks = [np.argmax(lg, axis=1)]
        t0 = time.perf_counter()
        for _ in range(check_steps):
            lg = cpu.step(ctoks[-1].astype(np.int32), lanes, lanes)
            ctoks.append(np.argmax(lg, axis=1))
        cdec = time.perf_counter() - t0
        cpu.close()
        O.lib().or_n3_set_threads(1)
        O.lib().or_n3_set_tier(0)
        ctoks = np.stack(ctoks, 1)
        out["tokens_identical_to_cpu_path"] = bool(np.array_equal(ctoks, toks[:, :check_steps + 1]))
        out["cpu_path"] = {"row_tokens_per_s": round(slots * check_steps / cdec, 2),
                           "ms_per_step": round(cdec / check_steps * 1e3, 2), "threads": threads, "kind": "port",
                           "sample": f"the oracle's Needle 3 engine (oracle/needle3_model.c, AVX2-tier row order) on the same "
                                     f"prompts, matmul, attention and MLP rows over {threads} threads, "
                                     f"{check_steps} decode steps of 3 rows after the prefill; tokens compared over "
                                     f"those {check_steps + 1} per slot"}
        out["speedup_vs_cpu_path"] = round(out["row_tokens_per_s"] / out["cpu_path"]["row_tokens_per_s"], 1)
        print(f"# needle3 CPU path: {out['cpu_path']['row_tokens_per_s']} row-tokens/s; identical tokens: "
              f"{out['tokens_identical_to_cpu_path']}", file=sys.stderr, flush=True)
    return out


def physical_cores() -> int:
    """lscpu's distinct (core, socket) pairs: cores per socket x sockets."""
    try:
        import subprocess
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True).stdout
        cores = {tuple(line.split(",")) for line in out.splitlines() if line and not line.startswith("#")}
        return max(1, len(cores))
    except Exception:
        return max(1, (os.cpu_count() or 2) // 2)


def host_threads() -> int:
    """NEEDLE_THREADS when set, else the host's physical core count (the
    reference CLI's NEEDLE_THREADS setting for a whole host)."""
    return int(os.environ.get("NEEDLE_THREADS", "0")) or physical_cores()


TIER_NAMES = {0: "scalar", 1: "AVX2", 2: "AVX-VNNI"}


def cpu_baseline(case: GemvCase, budget_s: float) -> dict:
    """The reference CPU path's GEMV on the host cores, same shape: the SIMD
    tier Tiers.Best picks on this CPU (oracle/cpu_simd.c: Gemv.Tile4 / Tile2
    / Rows with the AVX-VNNI or AVX2 group dot), row-parallel as
    MatMulBatch.RunShard over the physical cores, bounded to about
    `budget_s` seconds; the scalar restatement of Scalar.MatMulRows is timed
    beside it on a shorter sample."""
    from oracle import oracle as O  # the checker's library, timed here as the CPU baseline

    threads = O.lib().or_baseline_start(host_threads())
    tier = O.lib().or_simd_tier()
    m, k, n = case.m, case.k, case.n
    st = C.c_uint64(0xC0FFEE)
    copies = 4
    ws = [N.synth_int8(st, n * k).reshape(n, k) for _ in range(copies)]
    ss = [N.synth_half_uniform(st, n * (k // 32), 0.002, 0.02).reshape(n, k // 32) for _ in range(copies)]
    q, qs = O.quantize_rows(case.x)
    y = np.zeros((m, n), dtype=np.float32)

    def sample(simd: bool, seconds: float):
        times = []
        t_end = time.perf_counter() + seconds
        i = 0
        while time.perf_counter() < t_end or i < 3:
            t0 = time.perf_counter()
            if simd:
                O.lib().or_baseline_simd_matmul_i8(tier, O.p(ws[i % copies]), O.p(ss[i % copies]), n, k, O.p(q),
                                                   O.p(qs), m, O.p(y), n, 0, n)
            else:
                O.lib().or_baseline_matmul_i8(O.p(ws[i % copies]), O.p(ss[i % copies]), n, k, 32, O.p(q), O.p(qs),
                                              m, O.p(y), n, 0, n)
            times.append(time.perf_counter() - t0)
            i += 1
        return times

    times = sample(True, budget_s)
    scalar = sample(False, max(1.0, budget_s / 5))
    O.lib().or_baseline_stop()
    med, smed = float(np.median(times)), float(np.median(scalar))
    return {"value": round(case.bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "tier": TIER_NAMES[tier], "physical_cores": physical_cores(),
            "scalar_port_GBps": round(case.bytes / smed / 1e9, 3),
            "sample": f"{len(times)} GEMVs M={m} K={k} N={n} cycling {copies} weight copies in {sum(times):.1f} s "
                      f"(median {med * 1e3:.3f} ms/GEMV); restatement of the reference's {TIER_NAMES[tier]} tier "
                      f"(Gemv.Tile2 + Rows, VnniDot / Avx2Dot), row-parallel over {threads} threads; the scalar "
                      f"MatMulRows restatement: median {smed * 1e3:.2f} ms/GEMV over {len(scalar)} GEMVs"}


def pmc_run(case: GemvCase, launches: int) -> int:
    """Eager launches for hardware-counter runs (one dispatch each): first a
    plain 64 MiB device-to-device copy kernel (nhip_copy_dev), whose
    FETCH_SIZE/WRITE_SIZE calibrate the counters, then `launches` headline
    GEMVs cycling the weight copies so that each reads its weights from HBM."""
    nbytes = 64 << 20
    src, dst = N.DeviceBuffer(nbytes), N.DeviceBuffer(nbytes)
    src.zero()
    for _ in range(3):
        N.check(N.lib().nhip_copy_dev(dst.ptr, src.ptr, nbytes, None))
    N.check(N.lib().nhip_device_sync())
    for i in range(launches):
        case.launch(i)
    N.check(N.lib().nhip_device_sync())
    print(f"# pmc run: 3 copies of {nbytes} B, {launches} GEMVs of {case.bytes} algorithmic bytes", file=sys.stderr)
    case.close()
    return 0


def codebook_lines(args) -> list:
    """The reference-native form of the GEMV configs: Cq4/Cq2 codebook
    weights, g128 norms, Hadamard-prepared activations."""
    out = []
    for bits, (m, k, n) in [(4, (1, 1024, 4096)), (4, (3, 2048, 8192)), (2, (3, 2048, 8192)), (4, (16, 2048, 8192)),
                            (2, (16, 2048, 8192))]:
        case = CqGemvCase(m, k, n, bits, seed=0x2800 + bits + m)
        t = case.time(max(200, args.steps // 2), args.warmup)
        g = case.bytes / (t * 1e-3) / 1e9
        out.append({"workload": f"Cq{bits} (reference-native codebook, g128) GEMV M={m} K={k} N={n}",
                    "us_per_launch": round(t * 1e3, 3), "GB/s": round(g, 1),
                    "frac_hbm_peak": round(g / HBM_PEAK_GBS, 4), "bytes_per_launch": case.bytes})
        print(f"# Cq{bits} GEMV M={m} K={k} N={n}: {t * 1e3:.2f} us/launch, {g:.0f} GB/s", file=sys.stderr,
              flush=True)
        case.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-decode-loop", action="store_true")
    ap.add_argument("--only", choices=["prefill", "attention", "decode_loop", "codebook", "batch", "needle3"],
                    help="run one secondary workload alone (for kernel tracing); prints no JSON line")
    ap.add_argument("--decode-chunks", type=int, default=64,
                    help="attention position-split cap of the decode loop (1: one chunk per row with the output quantize fused)")
    ap.add_argument("--pmc-run", type=int, default=0, metavar="LAUNCHES",
                    help="counter-collection mode: a 64 MiB device copy (the calibration kernel of known size), "
                         "then LAUNCHES eager headline GEMVs; prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU scaling is not part of this "
              "build", file=sys.stderr)
        return 2
    N.check(N.lib().nhip_init(0))
    print(f"# {N.lib().nhip_describe().decode()}", file=sys.stderr, flush=True)

    if args.only:
        threads = host_threads()
        if args.only == "decode_loop":
            print(json.dumps(decode_loop(args, threads)), file=sys.stderr)
        elif args.only == "needle3":
            print(json.dumps(needle3_loop(args, threads)), file=sys.stderr)
        elif args.only == "codebook":
            codebook_lines(args)
        elif args.only == "batch":
            batch_lines(args)
        elif args.only == "prefill":
            for fused in (True, False):
                case = GemmCase(512, 2048, 8192, seed=0x4004, fused=fused)
                t = case.time(max(50, args.steps // 20), max(5, args.warmup // 10))
                print(f"# prefill GEMM ({'fused' if fused else 'exact'}): {t * 1e3:.1f} us", file=sys.stderr)
                case.close()
        else:
            case = AttnCase(seed=0x3003)
            t = case.time(max(200, args.steps // 4), args.warmup)
            print(f"# attention: {t * 1e3:.2f} us/launch", file=sys.stderr)
            case.close()
        return 0
    main_case = GemvCase(3, 2048, 8192, seed=0x1001)
    if args.pmc_run:
        return pmc_run(main_case, args.pmc_run)
    # one step = one GEMV on each of the cycled weight matrices, like a
    # decode step's pass over that many layers; the launch time is the step
    # time over the launches, so it holds at the driver's 20 steps too
    per_step = main_case.copies
    ms = main_case.time(args.steps * per_step, args.warmup * per_step)
    gbs = main_case.bytes / (ms * 1e-3) / 1e9
    print(f"# headline GEMV M=3 K=2048 N=8192: {ms * 1e3:.2f} us/launch, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    rcase = ReadCase(main_case.bytes - (main_case.m * main_case.k + main_case.m * 4 + main_case.m * main_case.n * 4),
                     main_case.copies)
    rms = rcase.time(args.steps * per_step, args.warmup * per_step)
    rgbs = rcase.nbytes / (rms * 1e-3) / 1e9
    read_ceiling = {"workload": "pure read of the GEMV's weight and scale bytes, the GEMV's load pattern "
                                "(nhip_read_stream_dev), same copies cycled",
                    "bytes_per_launch": rcase.nbytes, "us_per_launch": round(rms * 1e3, 3), "GB/s": round(rgbs, 1),
                    "frac_hbm_peak": round(rgbs / HBM_PEAK_GBS, 4),
                    "gemv_frac_of_read_ceiling": round(rms / ms, 4)}
    print(f"# read ceiling {rcase.nbytes} B: {rms * 1e3:.2f} us/launch, {rgbs:.0f} GB/s", file=sys.stderr, flush=True)
    rcase.close()

    secondary = []
    if not args.no_secondary:
        for (m, k, n) in [(16, 2048, 8192), (3, 2048, 2048), (16, 2048, 2048), (1, 1024, 4096)]:
            case = GemvCase(m, k, n, seed=0x2000 + m + n)
            t = case.time(max(200, args.steps // 2), args.warmup)
            g = case.bytes / (t * 1e-3) / 1e9
            secondary.append({"workload": f"int8 GEMV M={m} K={k} N={n}", "us_per_launch": round(t * 1e3, 3),
                              "GB/s": round(g, 1), "frac_hbm_peak": round(g / HBM_PEAK_GBS, 4),
                              "bytes_per_launch": case.bytes})
            print(f"# GEMV M={m} K={k} N={n}: {t * 1e3:.2f} us/launch, {g:.0f} GB/s", file=sys.stderr, flush=True)
            case.close()
        secondary += codebook_lines(args)
        secondary += batch_lines(args)

    prefill = []
    if not args.no_secondary:
        for fused in (True, False):
            case = GemmCase(512, 2048, 8192, seed=0x4004, fused=fused)
            t = case.time(max(50, args.steps // 20), max(5, args.warmup // 10))
            tops = case.ops / (t * 1e-3) / 1e12
            prefill.append({"workload": "prefill int8 GEMM M=512 K=2048 N=8192 (%s epilogue)" %
                                        ("fused fma, 1e-4 RMS" if fused else "reference-order, bit-exact"),
                            "us_per_launch": round(t * 1e3, 2), "TOPS": round(tops, 1),
                            "frac_int8_mfma_peak": round(tops / INT8_PEAK_TOPS, 4)})
            print(f"# prefill GEMM ({'fused' if fused else 'exact'}): {t * 1e3:.1f} us, {tops:.0f} TOPS",
                  file=sys.stderr, flush=True)
            case.close()

    attention = None
    if not args.no_secondary:
        case = AttnCase(seed=0x3003)
        t = case.time(max(200, args.steps // 4), args.warmup)
        g = case.bytes / (t * 1e-3) / 1e9
        attention = {"workload": "ragged decode attention, 16 seqs ctx U[32,2048] (sum %d), 16 heads x 64, int8 KV"
                                 % int(case.counts.sum()),
                     "us_per_launch": round(t * 1e3, 3), "GB/s": round(g, 1), "frac_hbm_peak": round(g / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": case.bytes, "max_chunks": case.max_chunks}
        print(f"# attention: {t * 1e3:.2f} us/launch, {g:.0f} GB/s over {case.bytes} B", file=sys.stderr, flush=True)
        case.close()

    needle3 = []
    if not args.no_secondary:
        for rows, slots, what in ((3, 3, "one decode step of 3 rows in 3 slots"),
                                  (128, 1, "a 128-row prefill chunk of one slot")):
            case = Needle3Case(seed=0x5005 + rows, rows=rows, slots=slots)
            t = case.time(max(200, args.steps // 4), args.warmup)
            needle3.append({"workload": f"Needle 3 attention inputs, 16 heads x 64, {what}", "rows": rows,
                            "us_per_launch": round(t * 1e3, 3)})
            print(f"# needle3 attention inputs, {rows} rows: {t * 1e3:.2f} us/launch", file=sys.stderr, flush=True)
            case.close()

    threads = host_threads()
    loop = None
    if not args.no_decode_loop:
        loop = decode_loop(args, threads)

    n3 = None
    if not args.no_decode_loop:
        n3 = needle3_loop(args, threads)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(main_case, args.cpu_seconds)
        print(f"# cpu baseline ({cpu['tier']}): {cpu['value']} GB/s on {cpu['cores']} threads (scalar port "
              f"{cpu['scalar_port_GBps']} GB/s)", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms * per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded XorShift64: int8 U[-127,127] weights, fp16 U(0.002,0.02) group-32 scales, "
                "N(0,1) activations quantized per row)",
        "config": {"workload": "beam-batched int8 decode GEMV", "rows_M": 3, "K": 2048, "N": 8192,
                   "group": 32, "weight_copies_cycled": main_case.copies,
                   "launches_per_step": per_step, "bytes_per_launch": main_case.bytes,
                   "bytes_per_step": main_case.bytes * per_step},
        "timing": {"method": "a step is one GEMV on each of the cycled weight matrices (a pass over that many "
                             "layers); the K steps' launches are replayed as one graph between two HIP events on "
                             "their stream",
                   "us_per_launch": round(ms * 1e3, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "read_ceiling": read_ceiling,
        "secondary": secondary,
        "prefill": prefill,
        "attention": attention,
        "needle3_inputs": needle3,
        "decode_loop": loop,
        "needle3_decode": n3,
    }
    main_case.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

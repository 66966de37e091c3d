"""Benchmark of the KV-cache attention path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-graph] [--only decode|prefill|ragged|vision|gemv|gemm]

A step is one decode-attention op of config 2 (Llama-3-8B shape: 32 query
heads on 8 KV heads, hd 128, 4096 cached rows), through the C ABI: the
split-KV kernel appends the step's K, V row and attends all 4097 rows in
splits, and the merge kernel combines the splits. Steps rotate over `layers`
distinct KV states (>= 512 MiB together, as a real model's 32 layers are),
so K and V come from HBM, not the 256 MB Infinity Cache. Inputs are resident
in HBM before the timed region.

One JSON line on stdout: value = decode GB/s (algorithmic bytes / step time;
the K timed steps are captured into one HIP graph and the timed region is
its launch, so the kernels pace it, not Python's per-call dispatch; "extra"
has the same steps called one by one and their wall time), roofline of the
decode op (the same HIP-event time on the arena's stream),
the CPU oracle timed on this host, and the other configs' figures (prefill
TFLOP/s, ragged decode, ViT, quantized GEMV and GEMM) under "extra". --copy-bytes N adds one arena
copy of N bytes, the calibration dispatch for rocprofv3 --pmc FETCH_SIZE /
WRITE_SIZE runs.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from synapse_amd import capi  # noqa: E402
from synapse_amd import workloads as wl  # noqa: E402
from synapse_amd.capi import SYN_F16, SYN_F32, Arena, AttnDesc, SelfDesc, SeqDesc, check, lib  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, GB/s
# HBM bytes one config-2 decode step moves (split + merge kernels), from two
# rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by a copy of known
# size; profiles/decode_c2_pmc_traffic.md has the runs and the factors.
DECODE_TRAFFIC_BYTES = 18_196_480
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense f16 matrix, TFLOP/s
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 matrix, TOP/s


class Hip:
    """HIP events on the arena's stream, via the HIP runtime the library uses."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so")
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def events(self, n: int) -> list:
        out = []
        for _ in range(n):
            e = ctypes.c_void_p()
            assert self.rt.hipEventCreate(ctypes.byref(e)) == 0
            out.append(e)
        return out

    def record(self, ev, stream) -> None:
        assert self.rt.hipEventRecord(ev, stream) == 0

    def ms(self, a, b) -> float:
        assert self.rt.hipEventSynchronize(b) == 0
        t = ctypes.c_float()
        assert self.rt.hipEventElapsedTime(ctypes.byref(t), a, b) == 0
        return float(t.value)


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bench_decode(hip: Hip, cfg: wl.Decode, steps: int, warmup: int, layers: int, graph: bool = True):
    """Config 2: returns (ms_per_step, details).

    The timed region is exactly `steps` steps; step i runs on KV state
    (warmup + i) % layers, so the rotation continues past the warm-up's
    states and the timed steps read caches that are not the most recently
    touched. With graph (the default) the steps are captured beforehand into
    one HIP graph of 2 * steps kernel nodes, uploaded, and the timed region is
    that graph's one launch: the GPU runs the steps back to back, paced by
    the kernels, not by this process's per-call dispatch. Without it
    (profiler runs: rocprofv3's kernel trace once ended a process that
    captured graphs with a segmentation fault) the steps are called one by
    one through the C ABI. `details` has the per-call figures either way."""
    row = cfg.n_kv * cfg.head_dim
    max_ctx = cfg.ctx + 1
    state = capi.kv_state_bytes(max_ctx, cfg.n_kv, cfg.head_dim)
    qsz = cfg.n_heads * cfg.head_dim
    scratch_bytes = int(lib().syn_hip_attention_scratch_bytes(cfg.n_heads, cfg.n_kv, cfg.head_dim, max_ctx, 1))
    per_layer = state + capi.align(qsz * 4) * 2 + capi.align(row * 4) * 2 + 4096
    arena = Arena(layers * per_layer + scratch_bytes + (1 << 20))
    kc, vc, q, k, v = wl.decode_inputs(cfg)
    scratch = arena.alloc(scratch_bytes)
    descs = []
    for _ in range(layers):
        cache = capi.kv_state(arena, max_ctx, cfg.n_kv, cfg.head_dim)
        capi.upload_cache(arena, cache, kc, vc)
        d = AttnDesc(cache=cache, q_offset=arena.put(q), k_offset=arena.put(k), v_offset=arena.put(v),
                     out_offset=arena.alloc(qsz * 4), scratch_offset=scratch, scratch_bytes=scratch_bytes,
                     n_heads=cfg.n_heads, pos=cfg.ctx, n=1, scale=cfg.scale, q_dtype=SYN_F32, kv_dtype=SYN_F32)
        descs.append(d)
    arena.sync()
    stream = arena.stream
    L = lib()
    byref = [ctypes.byref(d) for d in descs]
    step = lambda i: check(L.syn_hip_attention(arena.handle, byref[i % layers]))  # noqa: E731
    t0, t1 = hip.events(2)

    # Per-call figures first (untimed as far as the headline goes): the same
    # steps called one by one from this Python loop, which the host's
    # dispatch can pace, and the spread of single bracketed calls.
    n_eager = max(steps, 2 * layers)
    for i in range(layers):
        step(i)
    arena.sync()
    hip.record(t0, stream)
    w0 = time.perf_counter()
    for i in range(n_eager):
        step(i)
    hip.record(t1, stream)
    eager_ms = hip.ms(t0, t1) / n_eager
    wall_ms = (time.perf_counter() - w0) * 1e3 / n_eager
    evs = hip.events(2 * n_eager)
    for i in range(n_eager):
        hip.record(evs[2 * i], stream)
        step(i)
        hip.record(evs[2 * i + 1], stream)
    kern = [hip.ms(evs[2 * i], evs[2 * i + 1]) for i in range(n_eager)]
    out = arena.download(descs[0].out_offset, (qsz,), np.float32)
    assert np.all(np.isfinite(out))

    det = {"eager_ms_per_step": eager_ms, "wall_ms_per_step": wall_ms, "kernel_ms_median": float(np.median(kern)),
           "timing": "HIP-graph launch of the timed steps" if graph else "steps called one by one"}
    if graph:
        warm = max(warmup, 1)  # (a graph needs a node: with W = 0 one step leads)
        with capi.HipGraph(arena, lambda: [step(i) for i in range(warm)]) as hw, \
                capi.HipGraph(arena, lambda: [step(warmup + i) for i in range(steps)]) as hg:
            hw.upload()
            hg.upload()
            hw.launch()
            arena.sync()
            # The warm-up steps run again right ahead of the start event, as a
            # graph: the GPU is busy with them while this process queues the
            # event and the timed graph, so the timed region holds the K steps
            # and not the host's launch latency (about 14 us before the first
            # kernel otherwise, 0.7 us per step at K = 20). The start event
            # is stream-ordered after the last warm-up kernel.
            hw.launch()
            hip.record(t0, stream)
            hg.launch()
            hip.record(t1, stream)
            step_ms = hip.ms(t0, t1) / steps
            arena.sync()
        out_g = arena.download(descs[warmup % layers].out_offset, (qsz,), np.float32)
        assert np.array_equal(out_g.view(np.uint32), out.view(np.uint32))
    else:
        for i in range(warmup):
            step(i)
        arena.sync()
        hip.record(t0, stream)
        for i in range(steps):
            step(warmup + i)
        hip.record(t1, stream)
        step_ms = hip.ms(t0, t1) / steps
    arena.close()
    return step_ms, det


def bench_decode_rope(hip: Hip, cfg: wl.Decode, steps: int, layers: int, graph: bool = True):
    """Config 2 with Llama 3's RoPE applied to the step's q and k: the layer's
    op_rope(q), op_rope(k) and op_attention as one syn_hip_attention_rope
    call (the split kernel rotates in LDS; 2 launches) against the three
    separate calls (4 launches). Same rotating KV states as bench_decode, and
    timed the same way: with graph, `steps` steps captured into one HIP graph
    whose launch is the timed region (a warm-up graph of the same steps runs
    right ahead of it); without, called one by one."""
    row = cfg.n_kv * cfg.head_dim
    max_ctx = cfg.ctx + 1
    qsz = cfg.n_heads * cfg.head_dim
    state = capi.kv_state_bytes(max_ctx, cfg.n_kv, cfg.head_dim)
    scratch_bytes = int(lib().syn_hip_attention_scratch_bytes(cfg.n_heads, cfg.n_kv, cfg.head_dim, max_ctx, 1))
    arena = Arena(layers * (state + 4 * capi.align(qsz * 4) + 4 * capi.align(row * 4)) + scratch_bytes + (1 << 20))
    kc, vc, q, k, v = wl.decode_inputs(cfg)
    scratch = arena.alloc(scratch_bytes)
    theta_scale = float(np.float32(cfg.theta) ** np.float32(-2.0 / cfg.head_dim))
    rope = dict(freq_factors_offset=capi.NO_OFFSET, theta_scale=theta_scale, mode=0, freq_scale=1.0,
                ext_factor=0.0, attn_factor=1.0, corr_low=0.0, corr_high=0.0)
    fused, separate = [], []
    for _ in range(layers):
        cache = capi.kv_state(arena, max_ctx, cfg.n_kv, cfg.head_dim)
        capi.upload_cache(arena, cache, kc, vc)
        q_off, k_off, v_off = arena.put(q), arena.put(k), arena.put(v)
        qr, kr, out = arena.alloc(qsz * 4), arena.alloc(row * 4), arena.alloc(qsz * 4)
        d = AttnDesc(cache=cache, q_offset=q_off, k_offset=k_off, v_offset=v_off, out_offset=out,
                     scratch_offset=scratch, scratch_bytes=scratch_bytes, n_heads=cfg.n_heads, pos=cfg.ctx, n=1,
                     scale=cfg.scale, q_dtype=SYN_F32, kv_dtype=SYN_F32)
        r = capi.AttnRopeDesc(q_out_offset=qr, k_out_offset=kr, temp_scale=0.0, temp_floor_len=0, **rope)
        fused.append((ctypes.byref(d), ctypes.byref(r)))
        rq = capi.RopeDesc(in_offset=q_off, out_offset=qr, n=1, size=qsz, head_dim=cfg.head_dim, pos=cfg.ctx, **rope)
        rk = capi.RopeDesc(in_offset=k_off, out_offset=kr, n=1, size=row, head_dim=cfg.head_dim, pos=cfg.ctx, **rope)
        d2 = AttnDesc(cache=cache, q_offset=qr, k_offset=kr, v_offset=v_off, out_offset=out,
                      scratch_offset=scratch, scratch_bytes=scratch_bytes, n_heads=cfg.n_heads, pos=cfg.ctx, n=1,
                      scale=cfg.scale, q_dtype=SYN_F32, kv_dtype=SYN_F32)
        separate.append((ctypes.byref(rq), ctypes.byref(rk), ctypes.byref(d2), d2))
    L = lib()
    stream = arena.stream

    def run_fused(i):
        check(L.syn_hip_attention_rope(arena.handle, *fused[i % layers]))

    def run_separate(i):
        rq, rk, d2, _ = separate[i % layers]
        check(L.syn_hip_rope(arena.handle, rq))
        check(L.syn_hip_rope(arena.handle, rk))
        check(L.syn_hip_attention(arena.handle, d2))

    result = {}
    for name, fn in (("fused_us", run_fused), ("separate_us", run_separate)):
        for i in range(2 * layers):
            fn(i)
        arena.sync()
        t0, t1 = hip.events(2)
        if graph:
            with capi.HipGraph(arena, lambda: [fn(i) for i in range(steps)]) as hg:
                hg.upload()
                hg.launch()
                arena.sync()
                hg.launch()
                hip.record(t0, stream)
                hg.launch()
                hip.record(t1, stream)
                arena.sync()
        else:
            hip.record(t0, stream)
            for i in range(steps):
                fn(i)
            hip.record(t1, stream)
        result[name] = round(hip.ms(t0, t1) / steps * 1e3, 3)
    out = arena.download(separate[0][3].out_offset, (qsz,), np.float32)
    assert np.all(np.isfinite(out))
    arena.close()
    result.update({"launches_fused": 2, "launches_separate": 4, "steps": steps,
                   "timing": "HIP-graph launch of the timed steps" if graph else "steps called one by one"})
    return result


def bench_prefill(hip: Hip, cfg: wl.Prefill, reps: int, graph: bool = True):
    """Config 3: the flash kernel alone (cache already appended) and the
    whole op (append + attend)."""
    qsz = cfg.n_heads * cfg.head_dim
    row = cfg.n_kv * cfg.head_dim
    arena = Arena(capi.kv_state_bytes(cfg.n, cfg.n_kv, cfg.head_dim) + cfg.n * (qsz * 6 + row * 4) + (8 << 20))
    q, k, v = wl.prefill_inputs(cfg)
    cache = capi.kv_state(arena, cfg.n, cfg.n_kv, cfg.head_dim)
    d = AttnDesc(cache=cache, q_offset=arena.put(q.astype(np.float16)), k_offset=arena.put(k.astype(np.float16)),
                 v_offset=arena.put(v.astype(np.float16)), out_offset=arena.alloc(cfg.n * qsz * 4),
                 scratch_offset=0, scratch_bytes=0, n_heads=cfg.n_heads, pos=0, n=cfg.n, scale=cfg.scale,
                 q_dtype=SYN_F16, kv_dtype=SYN_F16)
    L = lib()
    check(L.syn_hip_attention(arena.handle, ctypes.byref(d)))
    arena.sync()
    stream = arena.stream
    # Both timed back to back over the region, as the other configs are: a
    # pair of events around every launch adds each launch's dispatch to it.
    t0, t1 = hip.events(2)
    hip.record(t0, stream)
    for i in range(reps):
        check(L.syn_hip_attend(arena.handle, ctypes.byref(d)))
    hip.record(t1, stream)
    kern_ms = hip.ms(t0, t1) / reps
    t0, t1 = hip.events(2)
    hip.record(t0, stream)
    for i in range(reps):
        check(L.syn_hip_attention(arena.handle, ctypes.byref(d)))
    hip.record(t1, stream)
    op_ms = hip.ms(t0, t1) / reps
    # The append alone is shorter than a host call: replayed from a graph
    # (called one by one in profiling runs, where the host paces it).
    def appends():
        for i in range(reps):
            check(L.syn_hip_kv_append(arena.handle, ctypes.byref(cache), d.k_offset, d.v_offset, cfg.n, 0, SYN_F16))

    arena.sync()
    t0, t1 = hip.events(2)
    if graph:
        with capi.HipGraph(arena, appends) as hg:
            hg.upload()
            hg.launch()
            hip.record(t0, stream)
            hg.launch()
            hip.record(t1, stream)
            append_ms = hip.ms(t0, t1) / reps
            arena.sync()
    else:
        hip.record(t0, stream)
        appends()
        hip.record(t1, stream)
        append_ms = hip.ms(t0, t1) / reps
    arena.close()
    return kern_ms, op_ms, append_ms


def bench_prefill_rope(hip: Hip, cfg: wl.Prefill, reps: int):
    """Config 3 with Llama 3's RoPE on the run's q and k rows (f32, as op_rope
    takes them): one syn_hip_attention_rope call (the rotating append, then
    the prefill kernel: 2 launches) against the separate calls (rope q, rope
    k, then syn_hip_attention's append and prefill: 4 launches)."""
    qsz = cfg.n_heads * cfg.head_dim
    row = cfg.n_kv * cfg.head_dim
    arena = Arena(capi.kv_state_bytes(cfg.n, cfg.n_kv, cfg.head_dim) + cfg.n * (qsz * 12 + row * 16) + (8 << 20))
    q, k, v = wl.prefill_inputs(cfg)
    cache = capi.kv_state(arena, cfg.n, cfg.n_kv, cfg.head_dim)
    q_off, k_off, v_off = (arena.put(np.asarray(x, dtype=np.float32)) for x in (q, k, v))
    qr, kr, out = arena.alloc(cfg.n * qsz * 4), arena.alloc(cfg.n * row * 4), arena.alloc(cfg.n * qsz * 4)
    theta_scale = float(np.float32(cfg.theta) ** np.float32(-2.0 / cfg.head_dim))
    rope = dict(freq_factors_offset=capi.NO_OFFSET, theta_scale=theta_scale, mode=0, freq_scale=1.0,
                ext_factor=0.0, attn_factor=1.0, corr_low=0.0, corr_high=0.0)
    d = AttnDesc(cache=cache, q_offset=q_off, k_offset=k_off, v_offset=v_off, out_offset=out, scratch_offset=0,
                 scratch_bytes=0, n_heads=cfg.n_heads, pos=0, n=cfg.n, scale=cfg.scale, q_dtype=SYN_F32,
                 kv_dtype=SYN_F32)
    r = capi.AttnRopeDesc(q_out_offset=qr, k_out_offset=kr, temp_scale=0.0, temp_floor_len=0, **rope)
    rq = capi.RopeDesc(in_offset=q_off, out_offset=qr, n=cfg.n, size=qsz, head_dim=cfg.head_dim, pos=0, **rope)
    rk = capi.RopeDesc(in_offset=k_off, out_offset=kr, n=cfg.n, size=row, head_dim=cfg.head_dim, pos=0, **rope)
    d2 = AttnDesc(cache=cache, q_offset=qr, k_offset=kr, v_offset=v_off, out_offset=out, scratch_offset=0,
                  scratch_bytes=0, n_heads=cfg.n_heads, pos=0, n=cfg.n, scale=cfg.scale, q_dtype=SYN_F32,
                  kv_dtype=SYN_F32)
    L = lib()

    def run_fused():
        check(L.syn_hip_attention_rope(arena.handle, ctypes.byref(d), ctypes.byref(r)))

    def run_separate():
        check(L.syn_hip_rope(arena.handle, ctypes.byref(rq)))
        check(L.syn_hip_rope(arena.handle, ctypes.byref(rk)))
        check(L.syn_hip_attention(arena.handle, ctypes.byref(d2)))

    result = {}
    for name, fn in (("fused_us", run_fused), ("separate_us", run_separate)):
        fn()
        arena.sync()
        t0, t1 = hip.events(2)
        hip.record(t0, arena.stream)
        for _ in range(reps):
            fn()
        hip.record(t1, arena.stream)
        result[name] = round(hip.ms(t0, t1) / reps * 1e3, 2)
    assert np.all(np.isfinite(arena.download(out, (cfg.n, qsz), np.float32)))
    arena.close()
    result.update({"launches_fused": 2, "launches_separate": 4, "rows": "f32"})
    return result


def bench_ragged(hip: Hip, cfg: wl.Ragged, reps: int):
    lengths = [int(x) for x in cfg.lengths()]
    row = cfg.n_kv * cfg.head_dim
    qsz = cfg.n_heads * cfg.head_dim
    total = sum(capi.kv_state_bytes(L, cfg.n_kv, cfg.head_dim) for L in lengths)
    arena = Arena(total + cfg.n_seqs * qsz * 8 + (64 << 20))
    g = wl.rng(wl.SEED + 9)
    seqs = []
    for L in lengths:
        cache = capi.kv_state(arena, L, cfg.n_kv, cfg.head_dim)
        kc = wl.to_f16_bits(wl.normal(g, (L, row)))
        capi.upload_cache(arena, cache, kc, kc)
        seqs.append(SeqDesc(cache=cache, q_offset=arena.put(wl.normal(g, (qsz,))), out_offset=arena.alloc(qsz * 4),
                            pos=L - 1))
    arr = (SeqDesc * len(seqs))(*seqs)
    need = int(lib().syn_hip_attend_batch_scratch_bytes(arr, len(seqs), cfg.n_heads))
    scratch = arena.alloc(need)
    L_ = lib()
    call = lambda: check(L_.syn_hip_attend_batch(arena.handle, arr, len(seqs), cfg.n_heads, cfg.scale, SYN_F32,
                                                 scratch, need))
    call()
    arena.sync()
    t0, t1 = hip.events(2)
    hip.record(t0, arena.stream)
    for _ in range(reps):
        call()
    hip.record(t1, arena.stream)
    ms = hip.ms(t0, t1) / reps
    nbytes = sum(L * row * 2 * 2 for L in lengths) + cfg.n_seqs * qsz * 8
    arena.close()
    return ms, nbytes


def bench_vision(hip: Hip, cfg: wl.Vision, reps: int):
    """Config 5 over `sets` distinct copies of its inputs and outputs
    (>= 256 MB together, past the 256 MB Infinity Cache), launch i on copy
    i % sets, so each launch reads its Q, K, V from HBM and writes its
    output there. Returns (ms per launch, copies rotated)."""
    rows = cfg.batch * cfg.n
    size = cfg.n_heads * cfg.head_dim
    per_set = capi.align(rows * size * 2) * 3 + capi.align(rows * size * 4)
    sets = max(4, -(-(256 << 20) // per_set))
    arena = Arena(sets * per_set + (8 << 20))
    q, k, v = wl.vision_inputs(cfg)
    descs = []
    for _ in range(sets):
        descs.append(SelfDesc(q_offset=arena.put(q.astype(np.float16)), k_offset=arena.put(k.astype(np.float16)),
                              v_offset=arena.put(v.astype(np.float16)), out_offset=arena.alloc(rows * size * 4),
                              n=cfg.n, batch=cfg.batch, n_heads=cfg.n_heads, head_dim=cfg.head_dim,
                              scale=cfg.scale, in_dtype=SYN_F16))
    L = lib()
    for d in descs:
        check(L.syn_hip_self_attention(arena.handle, ctypes.byref(d)))
    arena.sync()
    t0, t1 = hip.events(2)
    hip.record(t0, arena.stream)
    for i in range(reps):
        check(L.syn_hip_self_attention(arena.handle, ctypes.byref(descs[i % sets])))
    hip.record(t1, arena.stream)
    ms = hip.ms(t0, t1) / reps
    arena.close()
    return ms, sets


# Quantized GEMV shapes of a Llama-3-8B Q4_K_M decode step (one token):
# (name, ggml type, rows, cols). ffn_gate/up are Q4_K, ffn_down Q6_K; Q8_0
# is the all-Q8_0 file's.
GEMV_SHAPES = [("ffn_up Q4_K", 12, 14336, 4096), ("ffn_down Q6_K", 14, 4096, 14336),
               ("ffn_up Q8_0", 8, 14336, 4096), ("attn_q Q4_K", 12, 4096, 4096)]
GEMV_BLOCK = {12: (256, 144), 14: (256, 210), 8: (32, 34)}


def bench_gemv(hip: Hip, reps: int):
    """syn_hip_matmul_q for one token (activation quantizer + GEMV) over
    distinct copies of each weight matrix (>= 320 MB together, past the
    Infinity Cache). Bytes = weights + x + quantized activations + out."""
    out = {}
    g = wl.rng(wl.SEED + 21)
    for name, t, rows, cols in GEMV_SHAPES:
        bs, ts = GEMV_BLOCK[t]
        wbytes = rows * (cols // bs) * ts
        copies = max(2, -(-(320 << 20) // wbytes))
        act_bytes = int(lib().syn_hip_matmul_q_act_bytes(t, 1, cols))
        arena = Arena(copies * capi.align(wbytes) + cols * 4 + act_bytes + rows * 4 + (4 << 20))
        raw = g.integers(0, 256, size=wbytes, dtype=np.uint8)
        w_offs = [arena.put(raw) for _ in range(copies)]
        x_off = arena.put(wl.normal(g, (cols,)))
        act_off = arena.alloc(act_bytes)
        out_off = arena.alloc(rows * 4)
        descs = [capi.MatmulQDesc(w_offset=o, x_offset=x_off, act_offset=act_off, bias_offset=capi.NO_OFFSET,
                                  out_offset=out_off, w_type=t, n=1, rows=rows, cols=cols) for o in w_offs]
        L = lib()
        for d in descs:
            check(L.syn_hip_matmul_q(arena.handle, ctypes.byref(d)))
        arena.sync()
        t0, t1 = hip.events(2)
        hip.record(t0, arena.stream)
        for i in range(reps):
            check(L.syn_hip_matmul_q(arena.handle, ctypes.byref(descs[i % copies])))
        hip.record(t1, arena.stream)
        ms = hip.ms(t0, t1) / reps
        arena.close()
        nbytes = wbytes + cols * 4 + 2 * act_bytes + rows * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"rows": rows, "cols": cols, "us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
                     "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
        log(f"gemv {name} {rows}x{cols}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
    return out


def bench_gemm(hip: Hip, reps: int, n: int = 512):
    """syn_hip_matmul_q for a prompt chunk of n activation rows (the int8
    matrix-core GEMM, activation quantizer included) on the Llama-3-8B
    shapes. TOP/s = 2 n rows cols / time."""
    out = {}
    g = wl.rng(wl.SEED + 23)
    for name, t, rows, cols in GEMV_SHAPES[:3]:
        bs, ts = GEMV_BLOCK[t]
        wbytes = rows * (cols // bs) * ts
        act_bytes = int(lib().syn_hip_matmul_q_act_bytes(t, n, cols))
        arena = Arena(capi.align(wbytes) + n * cols * 4 + act_bytes + n * rows * 4 + (4 << 20))
        w_off = arena.put(g.integers(0, 256, size=wbytes, dtype=np.uint8))
        x_off = arena.put(wl.normal(g, (n, cols)))
        act_off = arena.alloc(act_bytes)
        out_off = arena.alloc(n * rows * 4)
        d = capi.MatmulQDesc(w_offset=w_off, x_offset=x_off, act_offset=act_off, bias_offset=capi.NO_OFFSET,
                             out_offset=out_off, w_type=t, n=n, rows=rows, cols=cols)
        L = lib()
        check(L.syn_hip_matmul_q(arena.handle, ctypes.byref(d)))
        arena.sync()
        t0, t1 = hip.events(2)
        hip.record(t0, arena.stream)
        for _ in range(reps):
            check(L.syn_hip_matmul_q(arena.handle, ctypes.byref(d)))
        hip.record(t1, arena.stream)
        ms = hip.ms(t0, t1) / reps
        arena.close()
        tops = 2.0 * n * rows * cols / (ms * 1e-3) / 1e12
        out[name] = {"n": n, "rows": rows, "cols": cols, "us": round(ms * 1e3, 2), "tops": round(tops, 1),
                     "frac_of_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        log(f"gemm {name} n={n} {rows}x{cols}: {ms * 1e3:.1f} us, {tops:.0f} TOP/s")
    return out


# The box gives one GPU a share of 16 host CPUs, whatever os.cpu_count() says.
HOST_THREAD_SHARE = 16


def _oracle():
    sys.path.insert(0, str(ROOT / "oracle"))
    import binding as orc
    return orc


def _best_of(fn, budget_s: float, min_runs: int = 3):
    """Runs fn until budget_s has passed and at least min_runs times; the
    fastest run in seconds and the run count."""
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < min_runs:
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return min(times), len(times)


def _host_threads(cap: int) -> int:
    return max(1, min(cap, HOST_THREAD_SHARE, len(os.sched_getaffinity(0))))


def cpu_baseline(cfg: wl.Decode, budget_s: float):
    """The CPU oracle (oracle/liboracle.so, a port of the reference's
    attention()) timed on this host: full config-2 decode steps, threads over
    the 8 KV groups as the reference's session splits them
    (S/graph/session.hpp:360)."""
    orc = _oracle()
    kc, vc, q, k, v = wl.decode_inputs(cfg)
    ok_k, ok_v = orc.new_cache(cfg.ctx + 1, cfg.n_kv, cfg.head_dim)
    ok_k[: cfg.ctx], ok_v[: cfg.ctx] = kc, vc
    threads = _host_threads(cfg.n_kv)
    scores = np.zeros(orc.scratch_floats(cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.ctx + 1), np.float32)
    best, runs = _best_of(lambda: orc.attend_rows(q, cfg.ctx, ok_k, ok_v, cfg.n_heads, cfg.scale, threads=threads,
                                                  scores=scores), budget_s)
    return {"value": round(cfg.kv_bytes() / best / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{runs} config-2 decode steps (attend over 4097 cached rows, 32 heads), best of "
                      f"{runs}; oracle/liboracle.so, {threads} threads over KV groups, "
                      f"{os.cpu_count()} host CPUs visible",
            "ms_per_step": round(best * 1e3, 3)}


def cpu_prefill(cfg: wl.Prefill, budget_s: float):
    """Config 3 on the CPU oracle: the whole op (append 2048 rows, causal
    attention), threads over the KV groups (S/graph/session.hpp:360)."""
    orc = _oracle()
    q, k, v = wl.prefill_inputs(cfg)
    kc, vc = orc.new_cache(cfg.n, cfg.n_kv, cfg.head_dim)
    threads = _host_threads(cfg.n_kv)
    best, runs = _best_of(lambda: orc.attention_rows(q, k, v, 0, kc, vc, cfg.n_heads, cfg.scale, threads=threads),
                          budget_s)
    return {"tflops": round(cfg.flops() / best / 1e12, 4), "ms": round(best * 1e3, 2),
            "tokens_per_s": round(cfg.n / best, 1), "cores": threads, "kind": "port",
            "sample": f"whole config-3 op (append + attend, 2048 rows), best of {runs}; {threads} threads over "
                      f"KV groups"}


def cpu_ragged(cfg: wl.Ragged, budget_s: float):
    """Config 4 on the CPU oracle: each of the 16 sequences attends its own
    cache in turn, threads over its KV groups (S/graph/session.hpp:360). The
    inputs are bench_ragged's (same seed, K and V share one array)."""
    orc = _oracle()
    lengths = [int(x) for x in cfg.lengths()]
    row = cfg.n_kv * cfg.head_dim
    qsz = cfg.n_heads * cfg.head_dim
    g = wl.rng(wl.SEED + 9)
    seqs = []
    for L in lengths:
        kc = wl.to_f16_bits(wl.normal(g, (L, row)))
        seqs.append((kc, wl.normal(g, (1, qsz)), L))
    threads = _host_threads(cfg.n_kv)
    scores = np.zeros(orc.scratch_floats(cfg.n_heads, cfg.n_kv, cfg.head_dim, max(lengths)), np.float32)

    def batch():
        for kc, q, L in seqs:
            orc.attend_rows(q, L - 1, kc, kc, cfg.n_heads, cfg.scale, threads=threads, scores=scores)

    best, runs = _best_of(batch, budget_s)
    nbytes = sum(L * row * 2 * 2 for L in lengths) + cfg.n_seqs * qsz * 8
    return {"gbs": round(nbytes / best / 1e9, 3), "ms": round(best * 1e3, 2),
            "seqs_per_s": round(cfg.n_seqs / best, 1), "cores": threads, "kind": "port",
            "sample": f"all 16 sequences ({sum(lengths)} cached rows), best of {runs}; {threads} threads over "
                      f"KV groups"}


def cpu_vision(cfg: wl.Vision, budget_s: float):
    """Config 5 on the CPU oracle: the 32 images one after another, each
    split into head x 16 query blocks over the threads
    (S/graph/session.hpp:419-448)."""
    orc = _oracle()
    q, k, v = wl.vision_inputs(cfg)
    threads = _host_threads(cfg.n_heads * 16)
    n = cfg.n

    def batch():
        for b in range(cfg.batch):
            sl = slice(b * n, (b + 1) * n)
            orc.self_attention(q[sl], k[sl], v[sl], cfg.n_heads, cfg.scale, threads=threads)

    best, runs = _best_of(batch, budget_s)
    return {"tflops": round(cfg.flops() / best / 1e12, 4), "ms": round(best * 1e3, 2),
            "images_per_s": round(cfg.batch / best, 1), "cores": threads, "kind": "port",
            "sample": f"all 32 images, best of {runs}; {threads} threads over head x 16 query blocks"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--layers", type=int, default=40, help="distinct KV states rotated over (>= 32)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="no HIP graphs (profiling runs): decode steps and the append timing called one by one")
    ap.add_argument("--decode-only", action="store_true", help="same as --only decode")
    ap.add_argument("--only", choices=["decode", "prefill", "ragged", "vision", "gemv", "gemm"], default=None,
                    help="run one configuration (no JSON line unless it is decode)")
    ap.add_argument("--copy-bytes", type=int, default=0, help="one arena copy of this many bytes (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention path is built and measured on a single MI355X "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        return 2

    hip = Hip()
    only = "decode" if args.decode_only else args.only
    if args.copy_bytes:
        with Arena(2 * args.copy_bytes + 4096) as arena:
            check(lib().syn_hip_copy(arena.handle, args.copy_bytes, 0, args.copy_bytes))
            arena.sync()
        log(f"copy calibration: {args.copy_bytes} bytes")
    extra = {}
    if only in (None, "prefill"):
        p = wl.C3
        log(f"prefill {p.name}")
        kms, op_ms, app_ms = bench_prefill(hip, p, 50, graph=not args.no_graph)
        tf = p.flops() / (kms * 1e-3) / 1e12
        app_bytes = 2 * p.n * p.n_kv * p.head_dim * (2 + 2)  # K and V: binary16 rows in, cache rows out
        extra["prefill"] = {"kernel_us": round(kms * 1e3, 2), "tflops": round(tf, 1),
                            "frac_of_f16_peak": round(tf / MFMA_F16_PEAK_TFS, 4),
                            "op_us_with_append": round(op_ms * 1e3, 2),
                            "append_us": round(app_ms * 1e3, 2),
                            "append_gbs": round(app_bytes / (app_ms * 1e-3) / 1e9, 1),
                            "append_frac_of_hbm": round(app_bytes / (app_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                            "tokens_per_s": round(p.n / (op_ms * 1e-3), 0), "flops": p.flops()}
        extra["prefill_rope"] = bench_prefill_rope(hip, p, 20)
        log(f"prefill: {kms * 1e3:.1f} us, {tf:.0f} TFLOP/s; append {app_ms * 1e3:.2f} us; "
            f"with RoPE {extra['prefill_rope']}")
    if only in (None, "ragged"):
        r = wl.C4
        log(f"ragged {r.name}")
        rms, rbytes = bench_ragged(hip, r, 20)
        extra["ragged"] = {"us": round(rms * 1e3, 2), "gbs": round(rbytes / (rms * 1e-3) / 1e9, 1),
                           "frac_of_hbm": round(rbytes / (rms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": rbytes,
                           "seqs_per_s": round(r.n_seqs / (rms * 1e-3), 0)}
        log(f"ragged: {rms * 1e3:.1f} us, {extra['ragged']['gbs']:.0f} GB/s")
    if only in (None, "vision"):
        vcfg = wl.C5
        log(f"vision {vcfg.name}")
        vms, vsets = bench_vision(hip, vcfg, 48)
        vgbs = vcfg.bytes() / (vms * 1e-3) / 1e9
        vtf = vcfg.flops() / (vms * 1e-3) / 1e12
        extra["vision"] = {"us": round(vms * 1e3, 2), "tflops": round(vtf, 1),
                           "frac_of_f16_peak": round(vtf / MFMA_F16_PEAK_TFS, 4), "gbs": round(vgbs, 1),
                           "frac_of_hbm": round(vgbs / HBM_PEAK_GBS, 4), "bytes": vcfg.bytes(),
                           "input_sets_rotated": vsets, "images_per_s": round(vcfg.batch / (vms * 1e-3), 0)}
        log(f"vision: {vms * 1e3:.1f} us, {extra['vision']['tflops']:.0f} TFLOP/s")
    if only in (None, "gemv"):
        extra["gemv_q"] = bench_gemv(hip, 400)
    if only in (None, "gemm"):
        extra["gemm_q"] = bench_gemm(hip, 20)
    if only not in (None, "decode"):
        return 0

    cfg = wl.C2
    log(f"decode {cfg.name}: {args.steps} steps, {args.warmup} warmup, {args.layers} rotating KV states")
    step_ms, det = bench_decode(hip, cfg, args.steps, args.warmup, args.layers, graph=not args.no_graph)
    nbytes = cfg.kv_bytes()
    value = nbytes / (step_ms * 1e-3) / 1e9
    log(f"decode: {step_ms * 1e3:.2f} us/step -> {value:.0f} GB/s ({det['timing']}); called one by one: "
        f"{det['eager_ms_per_step'] * 1e3:.2f} us/step, wall {det['wall_ms_per_step'] * 1e3:.2f} us/step")
    extra["decode_rope"] = bench_decode_rope(hip, cfg, 400, args.layers, graph=not args.no_graph)
    log(f"decode with RoPE: {extra['decode_rope']}")
    extra.update({"decode_step_us": round(step_ms * 1e3, 3),
                  "decode_timing": det["timing"],
                  "decode_eager_step_us": round(det["eager_ms_per_step"] * 1e3, 3),
                  "decode_wall_us_per_step": round(det["wall_ms_per_step"] * 1e3, 3),
                  "decode_single_step_us_median": round(det["kernel_ms_median"] * 1e3, 3),
                  "decode_tokens_per_s_32_layers": round(1e3 / (step_ms * 32), 1),
                  "decode_kernels_per_step": 2})

    line = {
        "metric": "decode attn HBM GB/s (8B GQA, KV 4k) + prefill attn TFLOP/s; % roofline",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (seeded PCG64; K RoPE'd, theta 500000)",
        "config": {"workload": "config 2: Llama-3-8B decode attention, H=32, Hkv=8, hd=128, 4096 cached rows "
                               "+ 1 appended (append + attend per step)",
                   "kv_states_rotated": args.layers, "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": DECODE_TRAFFIC_BYTES,
                     "kernel": "decode op (split-KV kernel + merge kernel, 2 launches per step), HIP events "
                               "around the timed steps (" + det["timing"] + ")"},
        "cpu_baseline": None,
        "extra": extra,
    }
    if not args.no_cpu:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
        side = args.cpu_seconds / 4
        for key, fn, c in (("prefill", cpu_prefill, wl.C3), ("ragged", cpu_ragged, wl.C4),
                           ("vision", cpu_vision, wl.C5)):
            if key in extra:
                extra[key]["cpu"] = fn(c, side)
                log(f"cpu {key}: {extra[key]['cpu']}")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

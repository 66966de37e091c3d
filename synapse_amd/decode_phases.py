"""Phase timeline of one config-2 decode step, from the timing build's stamps.

    python -m synapse_amd.build --stamps
    python -m synapse_amd.decode_phases [--steps K] [--rope] [--out FILE]

Runs config 2 (Llama-3-8B heads, 4096 cached rows + the step's row) as the
bench does: K steps over 40 rotating KV states, replayed from one HIP graph,
on libsynapse_hip_stamps.so, whose decode kernels record s_memrealtime stamps
(100 MHz). The stamps of the graph's last step are then read: every wave of
the split kernel at its phase points, every merge block's entry and end, and
the previous step's merge blocks. With --rope each step is the fused
RoPE step (syn_hip_attention_rope: q and the step's K row rotated in the
split kernel, Llama 3's RoPE at theta 500000). Prints a markdown table of each phase's
spread over the waves, in microseconds after the step's first split-kernel
wave entered. The stamps perturb the kernels slightly (each is a scalar
memory read of the clock): the step is about 0.2 us longer than in the
library proper."""
from __future__ import annotations

import argparse
import ctypes
import sys

import numpy as np

from synapse_amd import capi
from synapse_amd import workloads as wl

# (stamp index, phase) in the order a wave passes them.
POINTS = [(0, "entry"), (9, "kernel arguments in registers"), (1, "K, V loads issued"),
          (10, "RoPE: cos/sin table built"), (11, "RoPE: q and the new row rotated"), (2, "q ready (LDS barrier)"), (3, "K landed, scores done"), (4, "softmax done"),
          (5, "V landed, P.V done"), (6, "partials in LDS"), (7, "after the LDS barrier"),
          (8, "stores issued (end)")]
BLOCKS, WAVES, MERGES = 512, 4, 64


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--rope", action="store_true", help="time the fused RoPE step (syn_hip_attention_rope)")
    ap.add_argument("--out", default=None, help="also write the table to this file")
    args = ap.parse_args(argv)
    stamps_lib = capi.ROOT / "libsynapse_hip_stamps.so"
    if not stamps_lib.exists():
        print(f"{stamps_lib} is missing: build it with `python -m synapse_amd.build --stamps`", file=sys.stderr)
        return 1
    capi.LIB_PATH = stamps_lib  # before the first library call
    L = capi.lib()
    u64p = ctypes.POINTER(ctypes.c_uint64)
    L.syn_hip_decode_stamps.argtypes = [u64p, u64p, u64p]
    L.syn_hip_decode_stamps.restype = ctypes.c_int

    cfg, layers = wl.C2, 40
    row, qsz, max_ctx = cfg.n_kv * cfg.head_dim, cfg.n_heads * cfg.head_dim, cfg.ctx + 1
    scratch_bytes = int(L.syn_hip_attention_scratch_bytes(cfg.n_heads, cfg.n_kv, cfg.head_dim, max_ctx, 1))
    per_layer = capi.kv_state_bytes(max_ctx, cfg.n_kv, cfg.head_dim) + 2 * capi.align(qsz * 4) + \
        2 * capi.align(row * 4) + 4096
    arena = capi.Arena(layers * (per_layer + 2 * capi.align(qsz * 4)) + scratch_bytes + (1 << 20))
    kc, vc, q, k, v = wl.decode_inputs(cfg)
    scratch = arena.alloc(scratch_bytes)
    descs = []
    for _ in range(layers):
        cache = capi.kv_state(arena, max_ctx, cfg.n_kv, cfg.head_dim)
        capi.upload_cache(arena, cache, kc, vc)
        descs.append(capi.AttnDesc(cache=cache, q_offset=arena.put(q), k_offset=arena.put(k),
                                   v_offset=arena.put(v), out_offset=arena.alloc(qsz * 4), scratch_offset=scratch,
                                   scratch_bytes=scratch_bytes, n_heads=cfg.n_heads, pos=cfg.ctx, n=1,
                                   scale=cfg.scale, q_dtype=capi.SYN_F32, kv_dtype=capi.SYN_F32))
    arena.sync()
    refs = [ctypes.byref(d) for d in descs]
    theta_scale = float(np.float32(cfg.theta) ** np.float32(-2.0 / cfg.head_dim))
    ropes = [capi.AttnRopeDesc(q_out_offset=arena.alloc(qsz * 4), k_out_offset=arena.alloc(qsz * 4),
                               freq_factors_offset=capi.NO_OFFSET, theta_scale=theta_scale, mode=0,
                               freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, corr_low=0.0, corr_high=0.0,
                               temp_scale=0.0, temp_floor_len=0) for _ in range(layers)]
    rrefs = [ctypes.byref(r) for r in ropes]

    def step(i):
        if args.rope:
            capi.check(L.syn_hip_attention_rope(arena.handle, refs[i % layers], rrefs[i % layers]))
        else:
            capi.check(L.syn_hip_attention(arena.handle, refs[i % layers]))

    with capi.HipGraph(arena, lambda: [step(i) for i in range(args.steps)]) as g:
        g.upload()
        g.launch()
        arena.sync()
        g.launch()
        arena.sync()
    split = np.zeros(BLOCKS * WAVES * len(POINTS), dtype=np.uint64)
    merge = np.zeros(MERGES * 2, dtype=np.uint64)
    prev = np.zeros(MERGES * 2, dtype=np.uint64)
    capi.check(L.syn_hip_decode_stamps(split.ctypes.data_as(u64p), merge.ctypes.data_as(u64p),
                                       prev.ctypes.data_as(u64p)))
    arena.close()

    split = split.reshape(BLOCKS, WAVES, len(POINTS)).astype(np.float64)
    merge, prev = merge.reshape(MERGES, 2).astype(np.float64), prev.reshape(MERGES, 2).astype(np.float64)
    used = split[:, 0, 0] > 0
    t0 = split[used][:, :, 0].min()
    us = lambda x: (x - t0) * 0.01  # noqa: E731  (100 MHz clock)
    lines = [f"config 2 decode step{' with fused RoPE' if args.rope else ''} (the last of {args.steps} graph-replayed "
             f"steps over {layers} KV states): "
             f"{int(used.sum())} split blocks x {WAVES} waves, {int((merge[:, 0] > 0).sum())} merge blocks; "
             "us after the first split wave's entry", "",
             "| phase | min | p10 | p50 | p90 | max |", "|---|---|---|---|---|---|"]

    def row_of(name, vals):
        v = np.sort(us(vals[vals > 0]))
        if v.size == 0:
            return
        q = lambda f: v[min(v.size - 1, int(f * v.size))]  # noqa: E731
        lines.append(f"| {name} | {v[0]:.2f} | {q(0.1):.2f} | {q(0.5):.2f} | {q(0.9):.2f} | {v[-1]:.2f} |")

    row_of("previous step: merge block entry", prev[:, 0])
    row_of("previous step: merge block end", prev[:, 1])
    for k, name in POINTS:
        row_of(f"split wave: {name}", split[used][:, :, k].reshape(-1))
    row_of("merge block entry", merge[:, 0])
    row_of("merge block end", merge[:, 1])
    pm = prev[:, 1][prev[:, 1] > 0]
    me = merge[:, 1][merge[:, 1] > 0]
    ends = split[used][:, :, 8].reshape(-1)
    ms = merge[:, 0][merge[:, 0] > 0]
    lines += ["", f"- previous merge's last end -> first split entry: {(t0 - pm.max()) * 0.01:.2f} us",
              f"- split kernel, first entry -> last wave end: {us(ends.max()):.2f} us",
              f"- last split wave end -> first merge entry: {(ms.min() - ends.max()) * 0.01:.2f} us",
              f"- merge kernel, first entry -> last end: {(me.max() - ms.min()) * 0.01:.2f} us",
              f"- step, previous merge's last end -> this merge's last end: {(me.max() - pm.max()) * 0.01:.2f} us"]
    text = "\n".join(lines)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())

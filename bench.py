"""Benchmark of the MI355X decoder hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--legs copy,c1,voices,c4,c2,codec,frames]

Default workload (c1): the isolated KV ring append + decode attention step --
B=64 independent sequences, 12 heads x 64, ring capacity 2048, bf16 KV
storage, one query per sequence per step, write positions U[1, 6144) from a
seed (about two thirds of the rings have wrapped).  A step is one layer's
append + attention for all 64 sequences; twelve layer rings are stepped in
turn (as a 12-layer decode does), so the 4.8 GB of KV never fits the 256 MB
last-level cache and the GB/s are HBM figures.  Every sequence advances one
position after each full pass over the twelve layers.

A step is one fused launch (k_attn_unit with the append): value = its
algorithmic bytes (live K/V window read once, q | k | v read, new K/V row and
the output written) / the launch's average duration, from HIP events around
the back-to-back timed launches on the stream they run on, inputs resident in
HBM.  Set-up fills every layer ring and reads each once (as a prefill's own
attention does); the start event is recorded behind the warm-up launches, so
the window holds exactly the timed launches.  The roofline object is the
same launch; `traffic` comes from the committed rocprofv3 PMC summary.  The two-launch path (append, then
attention) is timed beside it.  cpu_baseline = the C oracle (OpenMP) on a bounded sample
of the same workload on this host's cores.
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

METRIC = "decode frames/sec at B=1/64/256; KV-attn HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
D, H, HD, QKV = 768, 12, 64, 2304


PROFILE = os.path.join(ROOT, "profiles", "decode_attention_b64_c2048.md")


def profiled_traffic(key="traffic_bytes_per_launch_bf16"):
    """HBM bytes per decode-attention launch from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs scaled by a known-size copy), or
    None when the summary holds no such line."""
    try:
        for line in open(PROFILE):
            if line.startswith(key + ":"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def c1_positions(B=64, seed=20260101):
    g = np.random.default_rng(seed)
    return g.integers(1, 6144, size=B).astype(np.int32)


def attn_bytes(pos, C, e):
    """Algorithmic bytes of one decode-attention launch: every live K and V
    row once, q read (fp32) and the output written (fp32)."""
    valid = np.minimum(pos.astype(np.int64) + 1, C)
    return int(valid.sum()) * D * 2 * e + len(pos) * D * 4 * 2


def append_bytes(B, e):
    """q | k | v read (fp32), roped q written (fp32), K and V written (e bytes),
    the slot's position written (4 bytes)."""
    return B * (QKV * 4 + D * 4 + 2 * D * e + 4)


def fused_bytes(pos, C, e):
    """Algorithmic bytes of one fused append + attention launch: the fused
    q | k | v row read (fp32), the window's older live K and V rows read once,
    the new K and V row written, the output written (fp32)."""
    valid = np.minimum(pos.astype(np.int64) + 1, C)
    return int(valid.sum()) * D * 2 * e + len(pos) * (QKV + D) * 4


def prime_rings(ctx, L, B, pos0, max_pos):
    """Set-up, untimed: one read-only decode-attention pass over every layer
    ring at the last filled position pos0 - 1, as a decoder's prefill reads
    the rings it has just written in its own attention.  Without it the
    first read of each ring after the fill runs slower (per-dispatch kernel
    traces: C1 60.5 against 57.7 us, the last-filled ring 69.6 us), and a
    short timed window that opens on rings the warm-up has not reached
    measures that one-off cost instead of the decode loop's steady state."""
    import torch

    dev = torch.device("cuda")
    q = torch.zeros((B, D), device=dev)
    out = torch.empty((B, D), device=dev)
    p = torch.from_numpy((pos0 - 1).astype(np.int32)).to(dev)
    for layer in range(L):
        ctx.decode_attention_dev(layer, B, q.data_ptr(), p.data_ptr(), max_pos, out.data_ptr())
    torch.cuda.synchronize()


def timed_launches(stream, fn, first, lead, n):
    """Mean time of n back-to-back calls fn(first + lead), ..., from HIP
    events on the stream they run on.  The `lead` calls before them (the
    warm-up) are enqueued first and the start event is recorded behind
    them, so the window opens with the GPU already busy and holds exactly
    the n launches, not the idle gap of a launch issued to an idle GPU."""
    import torch

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    for i in range(lead):
        fn(first + i)
    t0.record(stream)
    for i in range(n):
        fn(first + lead + i)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1)


def run_c1(args, kv_name):
    """One step = one layer's ring append + decode attention for all 64
    sequences, as one fused launch (mb_append_attend_dev); twelve layer rings
    are stepped in turn and every sequence advances one position after each
    pass over the twelve.  The same steps through the two separate entry
    points (mb_ring_append_dev, then mb_decode_attention_dev) are timed beside
    it on a shorter run, and then the append alone (mb_ring_append_dev)."""
    import torch

    import mockbird_amd as mb

    B, C, L = 64, 2048, 12
    kv = mb.MB_KV_BF16 if kv_name == "bf16" else mb.MB_KV_F32
    e = 2 if kv == mb.MB_KV_BF16 else 4
    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=256, kv_dtype=kv)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    pos0 = c1_positions(B)
    start = np.maximum(0, pos0 - (C - 1)).astype(np.int32)
    nfill = (pos0 - start).astype(np.int32)
    tg = torch.Generator(device=dev)
    tg.manual_seed(7)
    chunk = 256
    for layer in range(L):
        for c0 in range(0, int(nfill.max()), chunk):
            qkv = torch.randn((B, chunk, QKV), generator=tg, device=dev)
            n = torch.from_numpy(np.clip(nfill - c0, 0, chunk).astype(np.int32)).to(dev)
            p0 = torch.from_numpy((start + c0).astype(np.int32)).to(dev)
            ctx.ring_write_rows_dev(layer, B, chunk, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), 0)
    torch.cuda.synchronize()
    unfused_steps = min(args.steps, 240)
    total = args.warmup + args.steps + 2 * (2 + unfused_steps)
    tokens = total // L + 2
    pos_all = torch.from_numpy((pos0[None, :] + np.arange(tokens)[:, None]).astype(np.int32)).to(dev)
    qkv_l = [torch.randn((B, QKV), generator=tg, device=dev) for _ in range(L)]
    q = torch.empty((B, D), device=dev)
    out = torch.empty((B, D), device=dev)
    max_pos = int(pos0.max()) + tokens

    def step(s):
        layer, tok = s % L, s // L
        ctx.append_attend_dev(layer, B, qkv_l[layer].data_ptr(), pos_all[tok].data_ptr(), max_pos,
                              out.data_ptr())

    def step_unfused(s):
        layer, tok = s % L, s // L
        p = pos_all[tok]
        ctx.ring_append_dev(layer, B, qkv_l[layer].data_ptr(), p.data_ptr(), q.data_ptr())
        ctx.decode_attention_dev(layer, B, q.data_ptr(), p.data_ptr(), max_pos, out.data_ptr())

    def step_append(s):
        layer, tok = s % L, s // L
        ctx.ring_append_dev(layer, B, qkv_l[layer].data_ptr(), pos_all[tok].data_ptr(), q.data_ptr())

    prime_rings(ctx, L, B, pos0, max_pos)
    ms_total = timed_launches(stream, step, 0, args.warmup, args.steps)
    ms_unfused = timed_launches(stream, step_unfused, args.warmup + args.steps, 2, unfused_steps)
    ms_append = timed_launches(stream, step_append, args.warmup + args.steps + 2 + unfused_steps, 2,
                               unfused_steps)
    # the same kernel at a prefill chunk's size (192 rows per voice; the ring
    # fills above use 256-row launches, so a trace tells the two apart),
    # where its bytes rather than its launch set the time; written at
    # positions past every step above, after them
    R, n_chunks = 192, 24
    qkv_c = torch.randn((B, R, QKV), generator=tg, device=dev)
    q_c = torch.empty((B, R, D), device=dev)
    p0_c = torch.from_numpy((pos0 + tokens).astype(np.int32)).to(dev)
    n_c = torch.full((B,), R, dtype=torch.int32, device=dev)

    def step_chunk(s):
        ctx.ring_write_rows_dev(s % L, B, R, qkv_c.data_ptr(), p0_c.data_ptr(), n_c.data_ptr(),
                                q_c.data_ptr())

    ms_chunk = timed_launches(stream, step_chunk, 0, 2, n_chunks)

    def mean_bytes(fn, first, n):
        tot = 0
        for i in range(n):
            tot += fn(pos0 + (first + i) // L)
        return tot / n

    b_fused = mean_bytes(lambda p: fused_bytes(p, C, e), args.warmup, args.steps)
    b_unfused = mean_bytes(lambda p: attn_bytes(p, C, e) + append_bytes(B, e),
                           args.warmup + args.steps + 2, unfused_steps)
    ms_step = ms_total / args.steps
    res = {
        "kv": kv_name,
        "ms_per_step": ms_step,
        "bytes_per_step": b_fused,
        "gbs": b_fused / (ms_step * 1e-3) / 1e9,
        "unfused_ms_per_step": ms_unfused / unfused_steps,
        "unfused_gbs": b_unfused / (ms_unfused / unfused_steps * 1e-3) / 1e9,
        "append_ms_per_step": ms_append / unfused_steps,
        "append_bytes_per_step": append_bytes(B, e),
        "append_gbs": append_bytes(B, e) / (ms_append / unfused_steps * 1e-3) / 1e9,
        "chunk_ms_per_launch": ms_chunk / n_chunks,
        "chunk_bytes_per_launch": append_bytes(B * R, e),
        "chunk_gbs": append_bytes(B * R, e) / (ms_chunk / n_chunks * 1e-3) / 1e9,
        "mean_valid": float(np.minimum(pos0 + (args.warmup + args.steps // 2) // L + 1, C).mean()),
    }
    ctx.close()
    return res


def run_fused(args, B, C, pos0, seed, workload):
    """Fused ring append + decode attention, bf16 KV, 12 layer rings stepped
    in turn.  Each ring holds positions max(0, pos0 - C) .. pos0 - 1 of every
    sequence (written through the rows append, so slots follow pos mod C); a
    step is one mb_append_attend_dev launch at the next position, timed back
    to back with HIP events on the stream the launches run on.  Every
    sequence advances one position after each pass over the twelve layers."""
    import torch

    import mockbird_amd as mb

    L = 12
    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=L, capacity=C, max_seqs=B, max_rows=128, kv_dtype=mb.MB_KV_BF16)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    start = np.maximum(0, pos0 - C).astype(np.int32)
    nfill = (pos0 - start).astype(np.int32)
    tg = torch.Generator(device=dev)
    tg.manual_seed(seed)
    chunk = 128
    for layer in range(L):
        for c0 in range(0, int(nfill.max()), chunk):
            qkv = torch.randn((B, chunk, QKV), generator=tg, device=dev)
            n = torch.from_numpy(np.clip(nfill - c0, 0, chunk).astype(np.int32)).to(dev)
            p0 = torch.from_numpy((start + c0).astype(np.int32)).to(dev)
            ctx.ring_write_rows_dev(layer, B, chunk, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), 0)
    torch.cuda.synchronize()
    steps, warmup = args.steps, args.warmup
    tokens = (warmup + steps) // L + 2
    pos_all = torch.from_numpy((pos0[None, :] + np.arange(tokens)[:, None]).astype(np.int32)).to(dev)
    qkv_l = [torch.randn((B, QKV), generator=tg, device=dev) for _ in range(L)]
    out = torch.empty((B, D), device=dev)
    max_pos = int(pos0.max()) + tokens

    def step(s):
        layer, tok = s % L, s // L
        ctx.append_attend_dev(layer, B, qkv_l[layer].data_ptr(), pos_all[tok].data_ptr(), max_pos,
                              out.data_ptr())

    prime_rings(ctx, L, B, pos0, max_pos)
    us = timed_launches(stream, step, 0, warmup, steps) * 1e3 / steps
    nbytes = np.mean([fused_bytes(pos0 + (warmup + i) // L, C, 2) for i in range(steps)])
    ctx.close()
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": workload, "avg_us": round(us, 2), "bytes_per_launch": int(nbytes),
            "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def voices_positions(B=256, frames_in=150, order="natural"):
    """The many-voice prompt lengths U[64, 400) (seed 33) plus `frames_in`
    decoded frames; `order` "desc" / "asc" sorts the voices by position (the
    same windows, dispatched longest or shortest first)."""
    g = np.random.default_rng(33)
    pos = (g.integers(64, 400, size=B) + frames_in).astype(np.int32)
    if order == "desc":
        return -np.sort(-pos)
    return np.sort(pos) if order == "asc" else pos


def run_voices_attention(args, B=256, C=1024):
    """The KV-attention kernel at the many-voice decode shape: 256 voices,
    ring capacity 1024; positions from voices_positions(), so the live windows
    span 214-549 slots and grow by one per pass over the layers."""
    pos0 = voices_positions(B, order=args.voice_order)
    if int(pos0.max()) + (args.warmup + args.steps) // 12 + 2 >= C:
        raise ValueError("positions exceed the ring")
    return run_fused(args, B, C, pos0, 11,
                     "fused ring append + decode attention, 256 voices, 12 x 64, ring 1024, "
                     "bf16 KV, windows 214-549 slots, 12 layer rings in turn")


def block_timeline(stamps, window):
    """Summary of one decode-attention launch's block stamps: rows of
    {start, end (100 MHz ticks), HW_ID, XCC_ID}, one per block, and each
    block's live window in slots."""
    st = stamps.astype(np.int64)
    window = np.asarray(window, np.float64)
    t0 = st[:, 0].min()
    start = (st[:, 0] - t0) * 0.01  # us
    end = (st[:, 1] - t0) * 0.01
    dur = end - start
    cu = st[:, 3] * 256 + ((st[:, 2] >> 8) & 0xFF)
    ucu, per_cu = np.unique(cu, return_counts=True)
    busy = np.array([dur[cu == c].sum() for c in ucu])
    busy_window = np.array([window[cu == c].sum() for c in ucu])
    # placement: the dispatcher's XCC for block b, and whether block b + 256
    # lands on block b's CU (a fixed round-robin over the CUs)
    b = np.arange(len(st))
    xcc_rr = float(np.mean(st[:, 3] == b % 8))
    same_256 = float(np.mean(cu[:-256] == cu[256:])) if len(st) > 256 else None
    pct = lambda a, qs: {str(q): round(float(np.percentile(a, q)), 2) for q in qs}
    hist = dict(zip(*np.unique(per_cu, return_counts=True)))
    # blocks running, and the window's K/V bytes read per microsecond (each
    # block's window x 64 dims x K,V x 2 bytes spread evenly over its
    # duration), in 4 us bins over the launch
    edges = np.arange(0.0, float(end.max()) + 4.0, 4.0)
    rate = window * HD * 2 * 2 / dur  # bytes per us
    flight, gbs_t = [], []
    for lo, hi in zip(edges[:-1], edges[1:]):
        overlap = np.clip(np.minimum(end, hi) - np.maximum(start, lo), 0.0, None)
        flight.append(round(float(overlap.sum() / (hi - lo)), 1))
        gbs_t.append(round(float((overlap * rate).sum() / (hi - lo) / 1e3), 1))
    return {"blocks": len(st), "span_us": round(float(end.max()), 2),
            "last_start_us": round(float(start.max()), 2),
            "block_us": pct(dur, (0, 10, 50, 90, 100)),
            "block_end_us": pct(end, (10, 50, 90, 99, 100)),
            "ns_per_window_slot": pct(dur / window * 1e3, (10, 50, 90)),
            "corr_block_us_window": (round(float(np.corrcoef(dur, window)[0, 1]), 3)
                                     if dur.std() > 0 and window.std() > 0 else None),
            "cus": int(len(ucu)), "blocks_per_cu": {str(k): int(v) for k, v in hist.items()},
            "cu_busy_us": pct(busy, (0, 50, 100)),
            "cu_window_slots": pct(busy_window, (0, 50, 100)),
            "xcc_is_block_mod_8": round(xcc_rr, 4),
            "cu_of_block_plus_256_same": None if same_256 is None else round(same_256, 4),
            "mean_blocks_in_flight_per_cu": round(float(busy.mean() / end.max()), 2),
            "bin_us": 4.0, "blocks_in_flight_by_bin": flight, "window_gbs_by_bin": gbs_t}


def run_timeline(args):
    """Per-block timeline of a fused decode-attention launch, run on the
    timeline build of the library (ring.hip under MB_BLOCK_TIMELINE, loaded
    through MB_HIP_LIB): the voices leg's shape (256 voices, ring 1024) or
    C1's (64 sequences, ring 2048, positions U[1, 6144)), bf16 KV.  Reads the
    last launch's stamps: each block's start and end (100 MHz counter) and the
    CU (XCC_ID, and HW_ID bits 8-15: CU, shader array and engine) that ran it.
    Reports the launch span, the spread of block starts, block durations and
    their correlation with the block's window, blocks, busy time and window
    slots per CU, and where the dispatcher placed the blocks;
    `--timeline-out` also saves the raw stamps and windows (.npz)."""
    import ctypes

    import mockbird_amd as mb

    lib = mb.load()
    if not hasattr(lib, "mb_probe_block_stamps"):
        raise SystemExit("the timeline leg needs the timeline build: python -m mockbird_amd.build, "
                         "then MB_HIP_LIB=mockbird_amd/libmockbird_hip_timeline.so")
    lib.mb_probe_block_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int]
    if args.timeline_shape == "c1":
        B, C = 64, 2048
        pos0 = c1_positions(B)
        run = run_fused(args, B, C, pos0, 17, "fused ring append + decode attention, 64 sequences, "
                        "12 x 64, ring 2048, bf16 KV, positions U[1,6144), 12 layer rings in turn")
    else:
        B, C = 256, 1024
        pos0 = voices_positions(B, order=args.voice_order)
        run = run_voices_attention(args, B, C)
    n = B * H
    raw = np.zeros(4 * n, np.uint64)
    if lib.mb_probe_block_stamps(raw.ctypes.data, n) != 0:
        raise RuntimeError("mb_probe_block_stamps failed")
    last = args.warmup + args.steps - 1  # the launch whose stamps survive
    window = np.repeat(np.minimum(pos0 + last // H + 1, C), H)
    if args.timeline_out:
        np.savez(args.timeline_out, stamps=raw.reshape(n, 4), window=window)
    return {"shape": args.timeline_shape, "launch": run, **block_timeline(raw.reshape(n, 4), window)}


def run_c4(args, B=32, C=4096):
    """The eviction-stress shape: 32 sequences, ring capacity 4096, every
    ring full and wrapping (positions from 4096 on, so each append evicts the
    position C older); every window is the full 4096 slots."""
    pos0 = np.full(B, C, np.int32)
    return run_fused(args, B, C, pos0, 13,
                     "fused ring append + decode attention after wrap, 32 sequences, 12 x 64, "
                     "ring 4096 (full windows, each append evicts), bf16 KV, 12 layer rings in turn")


def run_codec(args, B, kv_name, warm=216, frames=24):
    """The codec decoder at steady state: B voices, the real stage shapes
    (4/2/2/4 layers of d=256, windows 500/1696/2480/3248 positions), every
    ring full after `warm` frames (stage 2, the slowest, fills after 212).  One
    mb_codec_decode_dev call decodes `frames` frames; frames/s counts voice
    frames (B x frames / time).  The attention's algorithmic bytes per frame
    are every layer's full window of K and V read once per frame (the stage's
    positions attend to it in one pass) plus the frame's new K/V rows."""
    import torch

    import mockbird_amd as mb
    from mockbird_amd import synth

    kv = mb.MB_KV_BF16 if kv_name == "bf16" else mb.MB_KV_F32
    e = 2 if kv == mb.MB_KV_BF16 else 4
    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=1, capacity=16, max_seqs=1, max_rows=16)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    ctx.upload_all(synth.codec_weights(mb.CODEC_LAYERS, seed=21))
    ctx.codec_init(B, kv_dtype=kv)
    codes = torch.from_numpy(synth.codec_codes(22, warm + frames, B)).to(dev)
    chunk = 8
    pcm = torch.empty((B, 2, max(chunk, frames) * mb.CODEC_SAMPLES), device=dev)
    for f in range(0, warm, chunk):
        n = min(chunk, warm - f)
        ctx.codec_decode_dev(B, n, codes[f].data_ptr(), pcm.data_ptr())
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    ctx.codec_decode_dev(B, frames, codes[warm].data_ptr(), pcm.data_ptr())
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / frames
    ctx.close()
    window = sum(l * c for l, c in zip(mb.CODEC_LAYERS, mb.CODEC_CONTEXT))
    new_rows = sum(l * (4 << s) for s, l in enumerate(mb.CODEC_LAYERS))
    attn_bytes = B * (window + new_rows) * 256 * 2 * e
    return {"workload": f"codec decoder, {B} voices, rings full (4/2/2/4 layers, windows "
                        f"500/1696/2480/3248), {kv_name} rings, {frames} frames per call",
            "B": B, "kv": kv_name, "ms_per_frame": round(ms, 4),
            "voice_frames_per_sec": round(B / (ms * 1e-3), 1),
            "realtime_factor": round(B * 80.0 / ms, 1),
            "ring_bytes_per_frame": int(attn_bytes),
            "ring_gbs": round(attn_bytes / (ms * 1e-3) / 1e9, 1)}


def run_c2(args):
    """Causal prefill attention, B=16, S=512, 12 heads x 64, bf16 q/k/v with
    fp32 accumulation (bf16 MFMA), RoPE at pos = row, ring C=1024 from slot 0.
    Returns the attention launch's mean time over `reps` back-to-back
    launches between two events (as the other legs time their launches) and
    TFLOP/s (algorithmic FLOPs B*H*4*64*S(S+1)/2, causal half only), and
    beside it the mean of the same launch timed alone between two events of
    its own (`isolated_us`, which adds the launch's dispatch gap)."""
    import torch

    import mockbird_amd as mb

    B, S, C, reps = 16, 512, 1024, 50
    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=1, capacity=C, max_seqs=B, max_rows=S, kv_dtype=mb.MB_KV_BF16)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    tg = torch.Generator(device=dev)
    tg.manual_seed(2)
    qkv = torch.randn((B, S, QKV), generator=tg, device=dev).to(torch.bfloat16)
    p0 = torch.zeros(B, dtype=torch.int32, device=dev)
    n = torch.full((B,), S, dtype=torch.int32, device=dev)
    q = torch.empty((B, S, D), dtype=torch.bfloat16, device=dev)
    out = torch.empty((B, S, D), device=dev)
    ctx.ring_write_rows_dev(0, B, S, qkv.data_ptr(), p0.data_ptr(), n.data_ptr(), q.data_ptr(),
                            qkv_dtype=mb.MB_DT_BF16, q_dtype=mb.MB_DT_BF16)
    for _ in range(5):
        ctx.prefill_attention_dev(0, B, S, q.data_ptr(), p0.data_ptr(), n.data_ptr(), out.data_ptr(),
                                  q_dtype=mb.MB_DT_BF16)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        ctx.prefill_attention_dev(0, B, S, q.data_ptr(), p0.data_ptr(), n.data_ptr(), out.data_ptr(),
                                  q_dtype=mb.MB_DT_BF16)
        b.record(stream)
    torch.cuda.synchronize()
    iso = float(np.mean([a.elapsed_time(b) for a, b in evs]) * 1e3)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(reps):
        ctx.prefill_attention_dev(0, B, S, q.data_ptr(), p0.data_ptr(), n.data_ptr(), out.data_ptr(),
                                  q_dtype=mb.MB_DT_BF16)
    t1.record(stream)
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / reps
    flops = B * H * 4 * HD * S * (S + 1) / 2
    ctx.close()
    return {"workload": "causal prefill attention B=16 S=512 12x64 bf16 (fp32 acc)",
            "avg_us": round(us, 2), "isolated_us": round(iso, 2), "gflop": round(flops / 1e9, 3),
            "tflops": round(flops / (us * 1e-6) / 1e12, 1),
            "frac_bf16_peak": round(flops / (us * 1e-6) / 2.5e15, 4)}


def run_copy(nbytes=1 << 31, reps=10):
    """A plain device-to-device copy of `nbytes` (torch's copy kernel): the
    achievable HBM rate on this box, and the known-size kernel the HBM byte
    counters are calibrated against."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    dst.copy_(src)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        dst.copy_(src)
        b.record(stream)
    torch.cuda.synchronize()
    us = float(np.mean([a.elapsed_time(b) for a, b in evs]) * 1e3)
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "avg_us": round(us, 2),
            "gbs": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}


def run_read_ceiling(nbytes=4 << 30, reps=10):
    """The HBM read ceiling on this GPU, measured two ways: the probe kernel
    of libmb_probe.so streaming a 4 GiB buffer (16-byte non-temporal loads,
    each wave reading 256 KB front to back), and torch's sum over the same
    bytes as fp32.  Both are plain reads of data resident in HBM (4 GiB is 16x
    the last-level cache)."""
    import ctypes

    import torch

    import mockbird_amd as mb

    lib = ctypes.CDLL(os.path.join(os.path.dirname(mb.LIB_PATH), "libmb_probe.so"))
    lib.mbp_stream_read_bytes.argtypes = [ctypes.c_size_t]
    lib.mbp_stream_read_bytes.restype = ctypes.c_size_t
    lib.mbp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.mbp_stream_read.restype = ctypes.c_int
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    read = lib.mbp_stream_read_bytes(nbytes)
    sink = torch.zeros(read // (256 << 10), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(reps)]
        for a, b in evs:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
        return float(np.mean([a.elapsed_time(b) for a, b in evs]) * 1e3)

    def probe():
        rc = lib.mbp_stream_read(buf.data_ptr(), nbytes, stream.cuda_stream, sink.data_ptr())
        if rc != 0:
            raise RuntimeError(f"mbp_stream_read failed ({rc})")

    us_probe = timed(probe)
    us_sum = timed(lambda: buf.sum())
    del buf, sink
    torch.cuda.empty_cache()
    gp = read / (us_probe * 1e-6) / 1e9
    gs = nbytes / (us_sum * 1e-6) / 1e9
    return {"bytes": int(read), "stream_read_us": round(us_probe, 1), "stream_read_gbs": round(gp, 1),
            "stream_read_frac": round(gp / HBM_PEAK_GBS, 4), "torch_sum_us": round(us_sum, 1),
            "torch_sum_gbs": round(gs, 1), "torch_sum_frac": round(gs / HBM_PEAK_GBS, 4)}


FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X


def run_gemm(reps=60, sets=12):
    """The QKV (768 -> 2304) and output (768 -> 768) projections through
    mb_linear_dev (fp32 products and accumulation on MFMA, bias in the
    epilogue) at the prefill size of the causal-prefill configuration
    (M = 16 x 512 = 8192 rows) and at the 256-voice decode size (M = 256).
    `sets` weight copies are used in turn, as a 12-layer model reads a
    different layer's weights each time."""
    import torch

    import mockbird_amd as mb

    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=1, capacity=8, max_seqs=1, max_rows=8, vocab=16)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    out = []
    for M in (8192, 256):
        for name, N in (("qkv", QKV), ("o", D)):
            K = D
            a = torch.randn((M, K), generator=g, device=dev)
            ws = [torch.randn((K, N), generator=g, device=dev) * 0.02 for _ in range(sets)]
            bias = torch.randn(N, generator=g, device=dev) * 0.02
            c = torch.empty((M, N), device=dev)

            def call(i):
                ctx.linear_dev(M, N, K, a.data_ptr(), K, ws[i % sets].data_ptr(), bias.data_ptr(),
                               c.data_ptr(), N, mb.MB_EPI_STORE)

            for i in range(sets):
                call(i)
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for i in range(reps):
                call(i)
            t1.record(stream)
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) * 1e3 / reps
            flops = 2.0 * M * K * N
            tf = flops / (us * 1e-6) / 1e12
            out.append({"proj": name, "M": M, "K": K, "N": N, "avg_us": round(us, 2),
                        "gflop": round(flops / 1e9, 3), "tflops": round(tf, 1),
                        "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
            del a, ws, c
    # The projections as bf16-KV contexts run them, at the causal-prefill
    # configuration's 8192 rows and the 256-voice decode step's 256: split-bf16
    # products (mb_linear_split_dev, three bf16 MFMAs per fp32 product) on
    # weights split once by mb_split_weights_dev.  FLOPs are the fp32
    # product's 2 M N K; the matrix cores execute three times that.
    for M, name, N, K in [(m, *p) for m in (8192, 256) for p in (
            ("qkv", QKV, D), ("o", D, D), ("fc_in", 4 * D, D), ("fc_out", D, 4 * D))]:
        a = torch.randn((M, K), generator=g, device=dev)
        wxs = []
        for _ in range(sets):
            w = torch.randn((K, N), generator=g, device=dev) * 0.02
            wx = torch.empty(2 * K * N, dtype=torch.bfloat16, device=dev)
            ctx.split_weights_dev(w.data_ptr(), K, N, wx.data_ptr())
            wxs.append(wx)
            del w
        bias = torch.randn(N, generator=g, device=dev) * 0.02
        c = torch.empty((M, N), device=dev)

        def call_split(i):
            ctx.linear_split_dev(M, N, K, a.data_ptr(), K, wxs[i % sets].data_ptr(),
                                 bias.data_ptr(), c.data_ptr(), N, mb.MB_EPI_STORE)

        for i in range(sets):
            call_split(i)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(reps):
            call_split(i)
        t1.record(stream)
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / reps
        flops = 2.0 * M * K * N
        tf = flops / (us * 1e-6) / 1e12
        out.append({"proj": name, "M": M, "K": K, "N": N, "products": "split-bf16",
                    "avg_us": round(us, 2), "gflop": round(flops / 1e9, 3), "tflops": round(tf, 1),
                    "frac_bf16_mfma_peak": round(3 * tf / BF16_MFMA_PEAK_TFLOPS, 4),
                    "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
        del a, wxs, c
    ctx.close()
    return out


def frame_prompts(B, seed=33):
    """Voice-clone prompts with total lengths U[64, 400) (half code frames,
    the rest text ids), as the many-voice decode configuration draws them."""
    from mockbird_amd import synth

    g = np.random.default_rng(seed)
    lens = g.integers(64, 400, size=B)
    return [synth.prompt(1000 + b, n_frames=int(l) // 2, n_text=int(l) - 3 - int(l) // 2,
                         vocab=32000) for b, l in enumerate(lens)]


def run_frames(weights, B, frames, kv_name, warmup=3, weights_name="f32"):
    """Greedy decode frames/s: prefill the prompts (untimed), then time
    `frames` frames, each the 17-step local head (text decision + 16 codes with
    the repetition penalty) followed by the 12-layer global decode step of the
    frame row it produced.  Everything stays on the device (mb_decode_frames_dev:
    one graph launch per frame); positions advance one per frame.
    `weights_name` "bf16": the projection weights in bf16 storage
    (mb_set_weight_storage), the model's bf16 form."""
    import torch

    import mockbird_amd as mb
    from mockbird_amd import synth

    C = 1024
    kv = mb.MB_KV_BF16 if kv_name == "bf16" else mb.MB_KV_F32
    if B == 1:
        prompts = [synth.prompt(0, n_frames=150, n_text=128, vocab=32000)]
    else:
        prompts = frame_prompts(B)
    n = np.array([p.shape[0] for p in prompts], np.int32)
    ids = np.full((B, n.max(), 17), 1024, np.int32)
    for b, p in enumerate(prompts):
        ids[b, :n[b]] = p
    dev = torch.device("cuda")
    ctx = mb.Context(n_layers=12, capacity=C, max_seqs=B, max_rows=int(n.max()), kv_dtype=kv)
    ctx.upload_all(weights)
    if weights_name == "bf16":
        ctx.set_weight_storage(mb.MB_W_BF16)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    t_pf = time.perf_counter()
    h0 = ctx.prefill(ids, n)
    t_pf = time.perf_counter() - t_pf
    total = warmup + frames
    max_pos = int(n.max()) + total
    if max_pos >= C:
        raise ValueError("prompt + frames exceed the ring")
    h = torch.from_numpy(h0).to(dev)
    pos = torch.from_numpy(n.copy()).to(dev)
    codes = torch.empty((max(frames, warmup), B, 16), dtype=torch.int32, device=dev)
    cont = torch.empty((max(frames, warmup), B), dtype=torch.int32, device=dev)
    # warm-up frames into the same buffers: the first call captures the frame's
    # HIP graph and the timed call replays it
    ctx.decode_frames_dev(B, warmup, h.data_ptr(), pos.data_ptr(), max_pos, codes.data_ptr(),
                          cont.data_ptr())
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    ctx.decode_frames_dev(B, frames, h.data_ptr(), pos.data_ptr(), max_pos, codes.data_ptr(),
                          cont.data_ptr())
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    ok = bool(cont.all().item()) and bool(torch.isfinite(h).all().item())
    ctx.close()
    return {"B": B, "kv": kv_name, "weights": weights_name, "frames": frames,
            "ms_per_frame": round(ms / frames, 4),
            "frames_per_sec": round(B * frames / (ms * 1e-3), 1),
            "prompt_rows": [int(n.min()), int(n.max())], "prefill_s": round(t_pf, 3),
            "all_continued": ok}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_sample(B, seconds):
    """Append + attention steps of the oracle over the first B of the c1
    sequences (fp32 rings, C = 2048) until `seconds` have passed; the oracle
    parallelises over sequences, so B = 1 runs on one thread."""
    from oracle import oracle

    C = 2048
    pos = c1_positions(64)[:B]
    g = np.random.default_rng(5)
    ring = oracle.Ring(B, C)
    for b in range(B):
        lo = max(0, pos[b] - C + 1)
        for p in range(lo, pos[b]):
            ring.slot_pos[b, p % C] = p
    ring.K[:] = g.standard_normal(ring.K.shape, dtype=np.float32)
    ring.V[:] = g.standard_normal(ring.V.shape, dtype=np.float32)
    qkv = g.standard_normal((B, QKV), dtype=np.float32)
    nbytes, steps = 0, 0
    t0 = time.perf_counter()
    p = pos.copy()
    while time.perf_counter() - t0 < seconds:
        q = ring.append(qkv, p)
        ring.attend(q, p)
        nbytes += fused_bytes(p, C, 4)
        p = p + 1
        steps += 1
    return nbytes, steps, time.perf_counter() - t0


def cpu_baseline_c1(seconds=12.0):
    """The oracle (double-precision C, OpenMP over sequences) on a sample of the
    c1 workload: one sequence per host thread (at most the 64), fp32 rings,
    append + attention steps, repeated until `seconds` have passed; then the
    same on one sequence (one thread) for a third of the time."""
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    B = max(1, min(64, threads))
    nbytes, steps, dt = _cpu_sample(B, seconds)
    nb1, steps1, dt1 = _cpu_sample(1, seconds / 3)
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": B, "kind": "port",
            "sample": f"{steps} append+attention steps of {B} of the 64 sequences (fp32 rings, "
                      f"C=2048, OpenMP over sequences), {dt:.1f} s",
            "single_thread": {"value": nb1 / dt1 / 1e9, "unit": "GB/s",
                              "sample": f"{steps1} steps of sequence 0, {dt1:.1f} s"},
            "cpu_model": _cpu_model(), "nproc": os.cpu_count()}


def cpu_baseline_frames(weights, seconds=8.0):
    """Greedy decode frames/s of the oracle's fp32 build (liboracle_fp32.so:
    the same C restatement with fp32 accumulators, -O3 AVX2/FMA, OpenMP) on
    this host's cores: the stand-in for the reference's CPU path, ORT-wasm
    running the published graphs, which is not available offline.

    Each of three samples runs for a third of `seconds`.  B = 1: the
    single-stream prompt (281 rows) is prefilled (untimed), then frames --
    the 17-step local head with the repetition penalty, then the 12-layer
    decode step of the frame row -- run; the GEMMs split their columns over
    the threads.  B = 64 and B = 256: one frame for each of the voices at a
    time, the voices spread over the threads (each voice's GEMMs on one
    thread), on rings filled with 300 positions of placeholder K/V (the
    timing does not depend on their values)."""
    from mockbird_amd import synth
    from oracle import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    m = oracle.Model(weights, n_layers=12, vocab=32000, fp32=True)
    out = {"unit": "frames/s", "kind": "port", "cores": threads, "cpu_model": _cpu_model(),
           "nproc": os.cpu_count(),
           "what": "fp32 CPU restatement of the reference graph (stand-in for ORT-wasm, "
                   "unavailable offline)"}
    rows = synth.prompt(0, n_frames=150, n_text=128, vocab=32000)
    st = oracle.ModelState(m, 1, 1024)
    h = st.prefill_all(0, rows)[-1][None]
    pos = rows.shape[0]
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 3:
        codes, _, _ = st.local_frame(h)
        h = st.decode_step(synth.frame_row(codes[0])[None], [pos])
        pos += 1
        n += 1
    dt = time.perf_counter() - t0
    out["B1"] = {"value": round(n / dt, 2), "sample": f"{n} frames after a 281-row prefill, "
                 f"{dt:.1f} s, GEMM columns over {threads} threads"}
    del st
    P = 300
    g = np.random.default_rng(3)
    for B in (64, 256):
        st = oracle.ModelState(m, B, 1024, kv_bf16=False)
        st.K[:, :, :P] = 0.01
        st.V[:, :, :P] = 0.01
        st.slot_pos[:, :, :P] = np.arange(P, dtype=np.int32)
        h = g.standard_normal((B, D), dtype=np.float32)
        pos = np.full(B, P, np.int32)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 3:
            codes, _, _ = st.local_frame(h)
            h = st.decode_step(np.stack([synth.frame_row(c) for c in codes]), pos)
            pos = pos + 1
            n += 1
        dt = time.perf_counter() - t0
        out[f"B{B}"] = {"value": round(B * n / dt, 2), "sample": f"{n} frames of {B} voices at "
                        f"positions 300+, {dt:.1f} s, voices over {threads} threads"}
        del st
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1200)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--workload", default="c1", choices=["c1"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--kv", default="both", choices=["both", "bf16"])
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-frames", action="store_true")
    ap.add_argument("--legs", default="copy,ceiling,c1,voices,c4,c2,gemm,codec,frames",
                    help="comma list of copy (plain 2 GiB HBM copy), ceiling (HBM read "
                         "ceiling: a streaming read probe and torch's sum over 4 GiB), gemm "
                         "(QKV and O projections at M = 8192 and 256), c1 (append + decode "
                         "attention, 64 sequences, C=2048), voices (the same at 256 voices, "
                         "C=1024), timeline (per-block timeline of the voices launch; needs "
                         "the timeline build through MB_HIP_LIB), c4 (the same at 32 sequences, C=4096, wrapped), c2 "
                         "(prefill attention), codec (codec decoder frames/s at 64 and 256 "
                         "voices), frames (model decode frames/s); the JSON line needs c1")
    ap.add_argument("--voice-order", default="natural", choices=["natural", "desc", "asc"],
                    help="voice order of the voices and timeline legs (desc: longest window first)")
    ap.add_argument("--timeline-shape", default="voices", choices=["voices", "c1"],
                    help="launch shape of the timeline leg")
    ap.add_argument("--timeline-out", default=None, help="the timeline leg's raw stamps (.npz)")
    ap.add_argument("--frames-b", default="1,64,256", help="voice counts of the frames leg")
    ap.add_argument("--frames-weights", default="f32,bf16",
                    help="weight storage of the frames leg's runs (f32, bf16 or both)")
    ap.add_argument("--frames-n", type=int, default=0,
                    help="frames per voice count (default: 60 at B=1, 300 otherwise)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); sequences are "
              "independent, so N GPUs would each run this same workload on their own share.",
              file=sys.stderr)
        return 2
    legs = set(args.legs.split(","))
    if args.no_prefill:
        legs.discard("c2")
    if args.no_frames:
        legs.discard("frames")
    copy = run_copy() if "copy" in legs else None
    ceiling = run_read_ceiling() if "ceiling" in legs else None
    gemm = run_gemm() if "gemm" in legs else None
    voices = run_voices_attention(args) if "voices" in legs else None
    timeline = run_timeline(args) if "timeline" in legs else None
    c4 = run_c4(args) if "c4" in legs else None
    codec = ([run_codec(args, 64, "f32"), run_codec(args, 256, "bf16")]
             if "codec" in legs else None)
    c2 = run_c2(args) if "c2" in legs else None
    frames = None
    w = None
    if "frames" in legs or not args.no_cpu_baseline:
        from mockbird_amd import synth

        # random-init model with the benchmark's shapes; the assistant column of
        # the text head equals the audio_end column, so no voice ever stops
        w = synth.model_weights(n_layers=12, vocab=32000, seed=0)
        w["model.text_lm_head.weight"][:, 9] = w["model.text_lm_head.weight"][:, 7]
    frames_w16 = None
    if "frames" in legs:
        plan = {1: (60, "f32"), 64: (300, "bf16"), 256: (300, "bf16")}
        fw = args.frames_weights.split(",")
        if "f32" in fw:
            frames = [run_frames(w, b, args.frames_n or plan[b][0], plan[b][1])
                      for b in map(int, args.frames_b.split(","))]
        if "bf16" in fw:
            frames_w16 = [run_frames(w, b, args.frames_n or plan[b][0], plan[b][1],
                                     weights_name="bf16")
                          for b in map(int, args.frames_b.split(","))]
    if "c1" not in legs:
        print(json.dumps({"hbm_copy": copy, "hbm_read_ceiling": ceiling, "gemm": gemm,
                          "kv_attention_256_voices": voices, "timeline_256_voices": timeline,
                          "kv_attention_c4_wrapped": c4, "prefill_attention": c2,
                          "codec": codec, "frames_detail": frames,
                          "frames_detail_bf16_weights": frames_w16}), flush=True)
        return 0
    bf16 = run_c1(args, "bf16")
    f32 = run_c1(args, "f32") if args.kv == "both" else None
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_c1(args.cpu_seconds)
        cpu["frames_per_sec"] = cpu_baseline_frames(w, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(bf16["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(bf16["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "KV ring append + decode attention (isolated): B=64 sequences, 12 heads "
                        "x 64, ring capacity 2048, bf16 KV storage, write positions U[1,6144) "
                        "seed 20260101, one query per sequence per step, 12 layer rings in turn",
            "kv_dtype": "bf16", "B": 64, "capacity": 2048, "heads": 12, "head_dim": 64,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(bf16["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(bf16["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "kernel": "k_attn_unit (ring append fused into decode attention), one launch per step",
            "avg_us": round(bf16["ms_per_step"] * 1e3, 2),
            "bytes_per_launch": int(bf16["bytes_per_step"]),
        },
        "cpu_baseline": cpu,
        "two_launch_bf16": {"ms_per_step": round(bf16["unfused_ms_per_step"], 5),
                            "gbs": round(bf16["unfused_gbs"], 1)},
        "append_only_bf16": {
            "what": "the ring append alone (k_ring_write: q | k | v rows in, RoPE, K and V "
                    "into bf16 rings, roped q out)",
            "step": {"rows": "64 voices x 1 row (mb_ring_append_dev), launched back to back "
                             "from Python: the host's call rate, not the kernel, sets this",
                     "us_per_launch": round(bf16["append_ms_per_step"] * 1e3, 2),
                     "bytes_per_launch": bf16["append_bytes_per_step"],
                     "gbs": round(bf16["append_gbs"], 1)},
            "chunk": {"rows": "64 voices x 192 rows (mb_ring_write_rows_dev)",
                      "us_per_launch": round(bf16["chunk_ms_per_launch"] * 1e3, 2),
                      "bytes_per_launch": bf16["chunk_bytes_per_launch"],
                      "gbs": round(bf16["chunk_gbs"], 1),
                      "frac": round(bf16["chunk_gbs"] / HBM_PEAK_GBS, 4)}},
        "f32_kv": None if f32 is None else {
            "value": round(f32["gbs"], 2), "unit": "GB/s",
            "ms_per_step": round(f32["ms_per_step"], 5),
            "frac": round(f32["gbs"] / HBM_PEAK_GBS, 4),
            "two_launch_gbs": round(f32["unfused_gbs"], 1)},
        "hbm_copy": copy,
        "hbm_read_ceiling": ceiling,
        "gemm": gemm,
        "kv_attention_256_voices": voices,
        "timeline_256_voices": timeline,
        "kv_attention_c4_wrapped": c4,
        "prefill_attention": c2,
        "codec": codec,
        "frames_per_sec": None if frames is None else {f"B{r['B']}": r["frames_per_sec"] for r in frames},
        "frames_detail": frames,
        "frames_per_sec_bf16_weights": None if frames_w16 is None else {
            f"B{r['B']}": r["frames_per_sec"] for r in frames_w16},
        "frames_detail_bf16_weights": frames_w16,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

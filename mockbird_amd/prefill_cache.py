"""Dump and reload a prefilled voice's rings in the reference's prefill-cache file.

The reference's oracle caches its prefill so that work on the local head
restarts in seconds (tools/onnx-probe/ref-decode.mjs:327-372).  Its file is
little-endian and holds, for a prompt of S rows prefilled at positions
0 .. S-1:

    int32 S
    S x 768 float32   hidden rows after the final LayerNorm (the reader uses
                      only the last one, ref-decode.mjs:373)
    for each layer:   S x 768 float32 K rows (roped), then S x 768 float32 V rows

K and V rows are [head * 64 + dim], as mb_read_ring returns them.  `save`
writes that file from a context's rings (mb_read_ring) and `load` puts one
back into a context (mb_ring_reset, then mb_write_ring), so a file written
here is one the reference's oracle loads, and the other way round.  bf16
rings are widened exactly on save; loading fp32 rows into a bf16 ring rounds
them to nearest even, as the ring's own writes do.
"""
from __future__ import annotations

import numpy as np

D = 768


def file_bytes(S: int, n_layers: int) -> int:
    """Size of the file for S rows and n_layers layers (the reader's `need`)."""
    return 4 + S * 4 * D + n_layers * 2 * S * 4 * D


def save(path: str, ctx, seq: int, hidden: np.ndarray) -> int:
    """Write voice `seq`'s rings, positions 0 .. S-1 of every layer, with its
    hidden rows [S][768] to `path`.  Every layer's slots 0 .. S-1 must hold
    positions 0 .. S-1: the file has no room for any other arrangement.
    Returns S."""
    hidden = np.asarray(hidden, np.float32)
    if hidden.ndim != 2:
        raise ValueError(f"hidden must be [S][{D}], got shape {hidden.shape} "
                         "(save_last_row takes the last row alone)")
    return _write(path, ctx, seq, hidden.shape[0], hidden)


def save_last_row(path: str, ctx, seq: int, S: int, last: np.ndarray) -> int:
    """`save` for a caller that holds only the last row's hidden state (what
    mb_model_prefill returns): rows 0 .. S-2 are written as zeros."""
    last = np.asarray(last, np.float32).reshape(D)
    hidden = np.zeros((S, D), np.float32)
    hidden[S - 1] = last
    return _write(path, ctx, seq, S, hidden)


def _write(path, ctx, seq, S, hidden) -> int:
    if hidden.shape != (S, D):
        raise ValueError(f"hidden must be [S][{D}], got {hidden.shape}")
    if not 0 < S <= ctx.capacity:
        raise ValueError(f"S = {S} rows do not fit positions 0 .. S-1 of a {ctx.capacity}-slot ring")
    parts = [np.array([S], "<i4").tobytes(), hidden.astype("<f4").tobytes()]
    want = np.arange(S, dtype=np.int32)
    for layer in range(ctx.cfg.n_layers):
        k, v, sp = ctx.read_ring(layer, seq, 0, S)
        if not np.array_equal(sp, want):
            bad = int(np.flatnonzero(sp != want)[0])
            raise ValueError(f"layer {layer} slot {bad} holds position {int(sp[bad])}, not {bad}: "
                             "the cache file holds positions 0 .. S-1 only")
        parts += [k.astype("<f4").tobytes(), v.astype("<f4").tobytes()]
    with open(path, "wb") as fh:
        for p in parts:
            fh.write(p)
    return S


def read(path: str, n_layers: int):
    """Parse a cache file: (hidden [S][768], k [L][S][768], v [L][S][768])."""
    with open(path, "rb") as fh:
        buf = fh.read()
    if len(buf) < 4:
        raise ValueError(f"{path}: {len(buf)} bytes, too short for the row count")
    S = int(np.frombuffer(buf, "<i4", 1)[0])
    if S < 1:
        raise ValueError(f"{path}: row count {S}")
    need = file_bytes(S, n_layers)
    if len(buf) != need:
        raise ValueError(f"{path}: {len(buf)} bytes, {need} expected for {S} rows and "
                         f"{n_layers} layers")
    body = np.frombuffer(buf, "<f4", offset=4).reshape(1 + 2 * n_layers, S, D)
    hidden = np.array(body[0], np.float32)
    kv = body[1:].reshape(n_layers, 2, S, D)
    return hidden, np.array(kv[:, 0], np.float32), np.array(kv[:, 1], np.float32)


def load(path: str, ctx, seq: int) -> np.ndarray:
    """Empty voice `seq`'s rings and fill positions 0 .. S-1 of every layer
    from `path`; returns the hidden rows [S][768] (the last one is the
    state decoding continues from, at position S)."""
    hidden, k, v = read(path, ctx.cfg.n_layers)
    S = hidden.shape[0]
    if S > ctx.capacity:
        raise ValueError(f"{S} rows do not fit a {ctx.capacity}-slot ring")
    ctx.ring_reset([seq])
    pos = np.arange(S, dtype=np.int32)
    for layer in range(ctx.cfg.n_layers):
        ctx.write_ring(layer, seq, 0, k[layer], v[layer], pos)
    return hidden

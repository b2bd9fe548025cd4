"""Shared helpers for the parity tests: replay golden cases on any sample.h-shaped sampler."""
import zlib

import numpy as np


def f32_from_bits(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def replay(sampler, rows, params, seed, history, picks):
    """Configure, preload the history, pick `picks` times (row k % len(rows)); return the
    same summary the fixtures store."""
    sampler.config(*params, seed=seed)
    if history is not None and len(history):
        sampler.set_history(np.asarray(history, dtype=np.int32))
    ids = [int(sampler.pick(rows[k % len(rows)])) for k in range(picks)]
    h = np.asarray(sampler.history(), dtype=np.int32)
    return {"ids": ids, "rng_after": "%016x" % sampler.rng, "hist_len": int(len(h)),
            "hist_tail": [int(x) for x in h[-min(len(h), 8):]],
            "hist_crc": zlib.crc32(h.tobytes())}


def expect(case):
    return {k: case[k] for k in ("ids", "rng_after", "hist_len", "hist_tail", "hist_crc")}


def xorshift64_star(state):
    """sample.c:72-77 restated with Python integers (closed form, independent of C)."""
    m = (1 << 64) - 1
    x = state
    x ^= (x << 13) & m
    x ^= x >> 7
    x ^= (x << 17) & m
    return (x * 0x2545F4914F6CDD1D) & m, x

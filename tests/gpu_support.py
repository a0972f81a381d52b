"""Helpers shared by the GPU parity tests: oracle-side RoPE over many rows and the tolerance
checks the path is graded on (max-abs 1e-3 with f32 KV, normwise relative 2e-2 with f16 KV)."""

from __future__ import annotations

import numpy as np

from models_amd import synth
from oracle import oracle

F32_MAX_ABS = 1e-3   # north-star tolerance with f32 KV
F16_REL = 2e-2       # north-star tolerance with f16 KV: max|gpu - ref| <= 2e-2 * max|ref|


def rope_tables(positions, rotary_dim, theta, scale=1.0, factors=None):
    """Oracle RotaryTable factors for each position: arrays [n, pairs]."""
    cs, sn = [], []
    for p in positions:
        c, s = oracle.rotary_factors(rotary_dim, theta, scale, int(p), factors)
        cs.append(c)
        sn.append(s)
    return np.stack(cs), np.stack(sn)


def rope_rows(x, positions, heads, head_dim, rotary_dim, theta, neox, scale=1.0, factors=None,
              check_against_oracle=True):
    """Rotate x[n, heads*head_dim] with the oracle's factors. The rotation itself is evaluated
    in numpy float32 (two products and one add, each rounded, as the oracle's C does); a sample
    of rows is cross-checked against oracle.rope_apply bit for bit."""
    x = np.asarray(x, np.float32).reshape(len(positions), heads, head_dim)
    cs, sn = rope_tables(positions, rotary_dim, theta, scale, factors)
    pairs = rotary_dim // 2
    i = np.arange(pairs)
    first = i if neox else 2 * i
    second = i + pairs if neox else 2 * i + 1
    out = x.copy()
    c = cs[:, None, :]
    s = sn[:, None, :]
    x0 = x[:, :, first]
    x1 = x[:, :, second]
    out[:, :, first] = (x0 * c).astype(np.float32) - (x1 * s).astype(np.float32)
    out[:, :, second] = (x0 * s).astype(np.float32) + (x1 * c).astype(np.float32)
    if check_against_oracle:
        for r in sorted({0, len(positions) // 2, len(positions) - 1}):
            for h in sorted({0, heads - 1}):
                ref = oracle.rope_apply(x[r, h], cs[r], sn[r], neox)
                np.testing.assert_array_equal(out[r, h], ref)
    return out.reshape(len(positions), heads * head_dim)


def assert_f32_close(got, ref, what="", head_dim=None):
    """Max-abs error over every element (an element-wise bound needs no per-head scaling)."""
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))
    assert err <= F32_MAX_ABS, f"{what}: max abs error {err:.3e} > {F32_MAX_ABS}"
    return err


def assert_f16_close(got, ref, what="", head_dim=None):
    """Normwise relative error of every (row, head) output vector on its own: for each vector of
    head_dim elements, max|got - ref| / max|ref| <= 2e-2, and the worst ratio is returned. A wrong
    head whose values are small cannot hide behind another head's large ones."""
    assert head_dim is not None and head_dim > 0, "head_dim is required"
    ref = np.asarray(ref, np.float64).reshape(-1)
    got = np.asarray(got, np.float64).reshape(-1)
    assert got.size == ref.size and ref.size % head_dim == 0, (what, got.size, ref.size, head_dim)
    ref = ref.reshape(-1, head_dim)
    err = np.max(np.abs(got.reshape(-1, head_dim) - ref), axis=1)
    scale = np.max(np.abs(ref), axis=1)
    rel = np.where(scale > 0, err / np.where(scale > 0, scale, 1.0), err)
    rel = np.where(np.isnan(rel), np.inf, rel)
    worst = int(np.argmax(rel))
    assert rel[worst] <= F16_REL, (f"{what}: normwise relative error {rel[worst]:.3e} > {F16_REL} "
                                   f"at (row, head) vector {worst} of {rel.size}")
    return float(rel[worst])


def normal(seed, tag, shape):
    return synth.normal(seed, tag, shape)

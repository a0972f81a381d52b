"""Pins the oracle where the reference's tests leave it open: IEEE definitions, closed forms,
invariants and float64 brute force on small shapes. Each check is chosen so that a plausible slip
(dropped scale, wrong RoPE pair layout, off-by-one window, transposed operand) fails it."""

import math

import numpy as np
import pytest

from models_amd import synth


# ------------------------------------------------------------------ half precision

def test_f16_round_matches_ieee_rne_over_bit_patterns(oracle):
    # numpy's float32->float16 cast is IEEE round-to-nearest-even with overflow to inf.
    bits = np.arange(0, 1 << 32, 4093, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0x00000000, 0x80000000, 0x33000000, 0x33000001, 0x337fffff, 0x38800000,
                     0x387fe000, 0x387ff000, 0x477fe000, 0x477fefff, 0x477ff000, 0x7f800000,
                     0xff800000, 0x3eaaaaab, 0x3f800000, 0x3a000000, 0x3a001000, 0x3a003000],
                    dtype=np.uint32)
    x = np.concatenate([bits, edge]).view(np.float32)
    finite = ~np.isnan(x)
    ours = oracle.f16_round(x[finite])
    with np.errstate(over="ignore"):
        ref = x[finite].astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(ours.view(np.uint32), ref.view(np.uint32))
    nans = oracle.f16_round(x[~np.isnan(x) == False])  # noqa: E712
    assert np.all(np.isnan(nans))


def test_f16_round_one_third(oracle):
    # KvCacheTest.roundsThroughHalfPrecisionWhenTheReferenceModeIsEnabled (:281-291)
    third = np.float32(1.0) / np.float32(3.0)
    r = oracle.f16_round([third])[0]
    assert r != third and abs(r - third) < 1e-3


# ------------------------------------------------------------------ RoPE

def test_rotary_frequencies_closed_form(oracle):
    f = oracle.rotary_frequencies(128, 500000.0)
    expected = (1.0 / np.power(np.float64(500000.0), np.arange(64) * 2 / 128.0)).astype(np.float32)
    np.testing.assert_array_equal(f, expected)


@pytest.mark.parametrize("neox", [False, True])
def test_rope_identity_at_zero_and_norm_preserving(oracle, neox):
    x = synth.normal(1, "rope", (128,))
    c, s = oracle.rotary_factors(128, 10000.0, 1.0, 0)
    np.testing.assert_array_equal(oracle.rope_apply(x, c, s, neox), x)
    c, s = oracle.rotary_factors(128, 10000.0, 1.0, 777)
    y = oracle.rope_apply(x, c, s, neox)
    assert abs(np.linalg.norm(y.astype(np.float64)) - np.linalg.norm(x.astype(np.float64))) < 1e-4


@pytest.mark.parametrize("neox", [False, True])
def test_rope_table_equals_direct_and_float64_rotation(oracle, neox):
    # RotaryTableTest.cachedFactorsMatchDirectStandardAndNeoxRope (:43-59) generalised: the
    # table path equals the inline path bit for bit, and both match a float64 rotation of the
    # right coordinate pairs (interleaved vs split-half).
    d, pos, theta, scale = 64, 1234, 1000000.0, 0.25
    x = synth.normal(2, "rope2", (d,))
    c, s = oracle.rotary_factors(d, theta, scale, pos)
    a = oracle.rope_apply(x, c, s, neox)
    b = oracle.rope_direct(x, pos, d, theta, scale, neox)
    np.testing.assert_array_equal(a, b)
    half = d // 2
    i = np.arange(half)
    first = i if neox else 2 * i
    second = i + half if neox else 2 * i + 1
    ang = np.float32(np.float32(pos) * np.float32(scale)) * \
        (1.0 / np.power(np.float64(theta), 2 * i / d)).astype(np.float32)
    ang = ang.astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64.copy()
    ref[first] = x64[first] * np.cos(ang) - x64[second] * np.sin(ang)
    ref[second] = x64[first] * np.sin(ang) + x64[second] * np.cos(ang)
    np.testing.assert_allclose(a, ref, atol=2e-6, rtol=0)


def test_rope_batch_factors_address_by_token(oracle):
    # RotaryTableTest.batchFactorsArePreparedOnceAndAddressedByToken (:61-78)
    first = np.float32([1, 2, 3, 4])
    second = np.float32([5, 6, 7, 8])
    for pos, x in ((9, first), (10, second)):
        c, s = oracle.rotary_factors(4, 10000.0, 0.25, pos)
        np.testing.assert_array_equal(oracle.rope_apply(x, c, s, False),
                                      oracle.rope_direct(x, pos, 4, 10000.0, 0.25, False))


# ------------------------------------------------------------------ softmax

def test_softmax_matches_float64(oracle):
    for n in (1, 2, 17, 513):
        x = synth.normal(n, "softmax", (n,)) * 4
        y = oracle.softmax(x)
        x64 = x.astype(np.float64)
        ref = np.exp(x64 - x64.max())
        ref /= ref.sum()
        np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-9)


# ------------------------------------------------------------------ attention brute force

def _dense_gqa(q, keys, values, hq, hkv, dk, dv, scale):
    """float64 softmax(q K^T * scale) V per head over rows keys[L, hkv*dk]."""
    L = keys.shape[0]
    k = keys.reshape(L, hkv, dk).astype(np.float64)
    v = values.reshape(L, hkv, dv).astype(np.float64)
    qh = q.reshape(hq, dk).astype(np.float64)
    g = hq // hkv
    out = np.zeros((hq, dv))
    for h in range(hq):
        s = k[:, h // g, :] @ qh[h] * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, h // g, :]
    return out.reshape(-1)


@pytest.mark.parametrize("hq,hkv,dk,dv,L", [(4, 2, 8, 8, 1), (6, 2, 16, 8, 37), (8, 1, 32, 32, 200)])
def test_gqa_rows_matches_float64_brute_force(oracle, hq, hkv, dk, dv, L):
    q = synth.normal(3, "q", (hq * dk,))
    k = synth.normal(3, "k", (L, hkv * dk))
    v = synth.normal(3, "v", (L, hkv * dv))
    scale = np.float32(1.0 / math.sqrt(dk))
    out = oracle.gqa_rows(q, k, v, hq, hkv, dk, dv, float(scale))
    ref = _dense_gqa(q, k, v, hq, hkv, dk, dv, float(scale))
    np.testing.assert_allclose(out, ref, atol=2e-6, rtol=0)


def test_gqa_closed_forms(oracle):
    hq, hkv, d = 4, 2, 8
    # L = 1: output is the single V row of the head's group
    q = synth.normal(4, "q", (hq * d,))
    k = synth.normal(4, "k", (1, hkv * d))
    v = synth.normal(4, "v", (1, hkv * d))
    out = oracle.gqa_rows(q, k, v, hq, hkv, d, d, 0.35).reshape(hq, d)
    for h in range(hq):
        np.testing.assert_array_equal(out[h], v.reshape(hkv, d)[h // 2])
    # all keys equal -> uniform scores -> mean of the V rows
    L = 10
    k = np.tile(synth.normal(5, "k", (1, hkv * d)), (L, 1))
    v = synth.normal(5, "v", (L, hkv * d))
    out = oracle.gqa_rows(q, k, v, hq, hkv, d, d, 0.35).reshape(hq, d)
    mean = v.reshape(L, hkv, d).astype(np.float64).mean(axis=0)
    for h in range(hq):
        np.testing.assert_allclose(out[h], mean[h // 2], atol=1e-6)
    # one dominant key -> output is that key's V row
    k = np.zeros((L, hkv * d), np.float32)
    k[7] = 1.0
    qb = np.full(hq * d, 100.0, np.float32)
    out = oracle.gqa_rows(qb, k, v, hq, hkv, d, d, 1.0).reshape(hq, d)
    for h in range(hq):
        np.testing.assert_allclose(out[h], v.reshape(L, hkv, d)[7, h // 2], atol=1e-6)
    # equal q within a GQA group -> identical outputs
    q2 = np.tile(synth.normal(6, "q", (1, d)), (hq, 1)).reshape(-1)
    k = synth.normal(6, "k", (L, hkv * d))
    out = oracle.gqa_rows(q2, k, v, hq, hkv, d, d, 0.35).reshape(hq, d)
    np.testing.assert_array_equal(out[0], out[1])
    np.testing.assert_array_equal(out[2], out[3])


def test_windowed_gqa_equals_slice(oracle):
    from oracle.oracle import KvCache
    hq, hkv, d, n, w = 4, 2, 8, 40, 7
    cache = KvCache(1, 64, hkv * d, hkv * d)
    k = synth.normal(7, "k", (n, hkv * d))
    v = synth.normal(7, "v", (n, hkv * d))
    for p in range(n):
        cache.store(0, p, k[p], v[p])
    q = synth.normal(7, "q", (hq * d,))
    pos = n - 1
    out = cache.gqa(0, pos, q, hq, hkv, d, d, 0.5, window=w)
    first = pos - w + 1
    ref = oracle.gqa_rows(q, k[first:pos + 1], v[first:pos + 1], hq, hkv, d, d, 0.5)
    np.testing.assert_array_equal(out, ref)
    ref64 = _dense_gqa(q, k[first:pos + 1], v[first:pos + 1], hq, hkv, d, d, 0.5)
    np.testing.assert_allclose(out, ref64, atol=2e-6)


def test_prefill_equals_token_at_a_time(oracle):
    # LlamaForwardPassTest prefill == sequential forward (:462): the batched path stores every
    # row then attends per row, which must equal decoding the rows one at a time.
    from oracle.oracle import KvCache
    hq, hkv, d, n = 4, 2, 16, 21
    q = synth.normal(8, "q", (n, hq * d))
    k = synth.normal(8, "k", (n, hkv * d))
    v = synth.normal(8, "v", (n, hkv * d))
    a = KvCache(1, 64, hkv * d, hkv * d)
    out_a, _, _ = a.prefill_layer(0, 0, q, k, v, hq, hkv, d, d, 10000.0, 1.0, True, 0.25)
    b = KvCache(1, 64, hkv * d, hkv * d)
    rows = [b.decode_layer(0, p, q[p], k[p], v[p], hq, hkv, d, d, 10000.0, 1.0, True, 0.25)[0]
            for p in range(n)]
    np.testing.assert_array_equal(out_a, np.concatenate(rows))
    np.testing.assert_array_equal(a.key_buffer(), b.key_buffer())


def test_layered_gqa_ring_equals_linear(oracle):
    # Gemma4 computeAttention over a wrapped ring view equals the linear result on the same rows.
    from oracle.oracle import LayeredKvCache
    hq, hkv, d, n, w = 2, 1, 8, 29, 6
    ring = LayeredKvCache(64, [[hkv * d, hkv * d, 8]])
    lin = LayeredKvCache(64, [[hkv * d, hkv * d, 0]])
    k = synth.normal(9, "k", (n, hkv * d))
    v = synth.normal(9, "v", (n, hkv * d))
    for p in range(n):
        ring.store(0, p, k[p], v[p])
        lin.store(0, p, k[p], v[p])
    q = synth.normal(9, "q", (hq * d,))
    a = ring.gqa(0, n - 1, q, hq, hkv, d, 1.0, window=w)
    b = lin.gqa(0, n - 1, q, hq, hkv, d, 1.0, window=w)
    np.testing.assert_array_equal(a, b)
    assert len(ring.attention_view(0, n - w, n)) == 2  # the view really wraps


def test_batch_threads_match_single(oracle):
    hq, hkv, d = 6, 2, 16
    lens = [5, 33, 64]
    qs = [synth.normal(10, f"q{i}", (hq * d,)) for i in range(3)]
    ks = [synth.normal(10, f"k{i}", (n, hkv * d)) for i, n in enumerate(lens)]
    vs = [synth.normal(10, f"v{i}", (n, hkv * d)) for i, n in enumerate(lens)]
    one = oracle.gqa_rows_batch(qs, ks, vs, hq, hkv, d, d, 0.25, threads=1)
    many = oracle.gqa_rows_batch(qs, ks, vs, hq, hkv, d, d, 0.25, threads=4)
    for i in range(3):
        np.testing.assert_array_equal(one[i], many[i])
        np.testing.assert_array_equal(one[i], oracle.gqa_rows(qs[i], ks[i], vs[i], hq, hkv, d, d,
                                                              0.25))


def test_rms_norm_against_float64_and_in_place(oracle):
    # rms = sqrt(mean(x^2) + eps) computed in float64; the oracle's float sum and rounding stay
    # within a few ulp. A wrong divisor (d vs d-1), a missing eps or a missing weight fails this.
    rng = np.random.default_rng(5)
    for d in (2, 16, 64, 128, 256):
        x = rng.standard_normal(d).astype(np.float32) * 3
        w = rng.uniform(0.5, 1.5, d).astype(np.float32)
        eps = 1e-6
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps) * w
        got = oracle.rms_norm(x, w, eps)
        np.testing.assert_allclose(got, ref, rtol=4e-6, atol=0)
        heads = np.concatenate([x, 2 * x, np.zeros(d, np.float32)])
        out = oracle.qk_norm_heads(heads, 3, d, w, eps)
        np.testing.assert_array_equal(out[:d], got)  # in place (per head) == out of place
        np.testing.assert_allclose(out[d:2 * d], got, rtol=4e-6)  # scale invariance
        np.testing.assert_array_equal(out[2 * d:], np.zeros(d, np.float32))


def test_value_rms_norm_against_float64_and_rejections(oracle):
    # normalizeWithoutWeight: x / sqrt(mean(x^2) + eps) with no weight, computed in float64; the
    # oracle's float sum and its double reciprocal stay within a few ulp. A weight applied, a wrong
    # divisor or a missing eps fails this; eps <= 0 or non-finite is rejected as the reference's
    # IllegalArgumentException (gemma4/Gemma4Math.java:47-49).
    rng = np.random.default_rng(6)
    for d in (2, 16, 64, 128, 256):
        x = rng.standard_normal(d).astype(np.float32) * 3
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
        got = oracle.value_rms_norm(x, 1e-6)
        np.testing.assert_allclose(got, ref, rtol=4e-6, atol=0)
        heads = np.concatenate([x, 2 * x, np.zeros(d, np.float32)])
        out = oracle.value_rms_heads(heads, 3, d, 1e-6)
        np.testing.assert_array_equal(out[:d], got)
        np.testing.assert_allclose(out[d:2 * d], got, rtol=4e-6)  # scale invariance
        np.testing.assert_array_equal(out[2 * d:], np.zeros(d, np.float32))
    # A large eps dominates: x / sqrt(eps) for a small x.
    x = np.full(4, 1e-3, np.float32)
    np.testing.assert_allclose(oracle.value_rms_norm(x, 1.0), x / np.sqrt(1.0 + 1e-6), rtol=1e-6)
    for eps in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(oracle.OracleError):
            oracle.value_rms_norm(np.ones(4, np.float32), eps)

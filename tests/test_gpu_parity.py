"""GPU parity: the HIP path through the C ABI against the CPU oracle on identical seeded inputs.

Bars (from the path's contract): KV-cache contents, RoPE outputs, window bounds and positions are
bit-exact; attention outputs are within max-abs 1e-3 with f32 KV and normwise relative 2e-2 with
f16 KV (per (row, head) output vector). Configs C1-C5 are the five BASELINE workloads, each run at
its configured size against the oracle (C2's 16 x 128 layer-steps by oracle spot checks plus
size-independent properties: replay idempotence and bit-exact appended rows); reduced variants
exercise the host-buffer entry points and edge cases."""

import math
import sys

import numpy as np
import pytest

from gpu_support import (assert_f16_close, assert_f32_close, normal, rope_rows)
from models_amd import attention as A
from models_amd import synth
from oracle import oracle
from oracle.oracle import KvCache as OracleKv

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    lib = A.HipAttentionLibrary(0)
    yield lib
    lib.close()


# ------------------------------------------------------------------ KV cache semantics

def _pad(vec, width):
    out = np.zeros(width, np.float32)
    out[:len(vec)] = vec
    return out


def test_kv_cache_known_answers_on_device(hip, known_answers):
    """Replays backend-java's KvCacheTest cases (tests/golden) on the device cache. Head widths are
    padded to 16 (the device minimum); the observable semantics — stored values, null for
    unpopulated positions, slices, discardFrom, clear, range errors — must match exactly."""
    for case in known_answers["kv_cache"]:
        _say(f"kv case {case['name']}")
        layers, max_seq, kd, vd = case["ctor"]
        kv = hip.kv_cache(layers, max_seq, 1, 16, 16, half_precision=case.get("half_precision", False))
        try:
            def run(ops):
                for op in ops:
                    if op[0] == "store":
                        kv.store(op[1], op[2], _pad(op[3], 16), _pad(op[4], 16))
                    elif op[0] == "clear":
                        kv.clear()
                    elif op[0] == "discard":
                        kv.discard_from(op[1])
                    elif op[0] == "reserve":
                        pass  # device caches are allocated at max_seq_len up front

            def read_one(l, p, values):
                try:
                    k, v = kv.read(l, p, p + 1)
                except A.AttentionStatusError as e:
                    assert e.status == A.UNAVAILABLE, e
                    return None
                return (v if values else k)

            def check(exps):
                for e in exps:
                    kind = e[0]
                    if kind in ("key", "value"):
                        got = read_one(e[1], e[2], kind == "value")
                        if e[3] is None:
                            assert got is None, (case["name"], e)
                        else:
                            np.testing.assert_array_equal(got[:len(e[3])], np.float32(e[3]))
                            assert not np.any(got[len(e[3]):]), (case["name"], e)
                    elif kind in ("keyNotNull", "valueNotNull"):
                        assert read_one(e[1], e[2], kind == "valueNotNull") is not None
                    elif kind in ("keySlice", "valueSlice"):
                        if isinstance(e[4], str):
                            with pytest.raises(A.AttentionStatusError) as info:
                                kv.read(e[1], e[2], e[3])
                            assert info.value.status == A.UNAVAILABLE
                        else:
                            k, v = kv.read(e[1], e[2], e[3])
                            got = (k if kind == "keySlice" else v).reshape(e[3] - e[2], 16)
                            width = len(e[4]) // (e[3] - e[2])
                            np.testing.assert_array_equal(got[:, :width].reshape(-1), np.float32(e[4]))
                    elif kind == "storeError":
                        with pytest.raises(A.AttentionStatusError) as info:
                            kv.store(e[1], e[2], np.zeros(16), np.zeros(16))
                        assert info.value.status == A.OUT_OF_RANGE, e
            run(case["ops"])
            check(case["expect"])
            if "then_ops" in case:
                run(case["then_ops"])
                check(case["then_expect"])
        finally:
            kv.close()


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("neox", [False, True])
def test_append_rope_is_bit_exact(hip, half, neox):
    hq, hkv, d, n, theta, scale = 8, 2, 64, 40, 500000.0, 0.5
    rope = hip.rotary_table(d, theta, scale, max_positions=4096)
    kv = hip.kv_cache(2, 4096, hkv, d, d, half_precision=half)
    try:
        positions = np.array([0, 1, 2, 31, 32, 33, 1000, 4095] + list(range(100, 132)))[:n]
        q = normal(11, "q", (n, hq * d))
        k = normal(11, "k", (n, hkv * d))
        v = normal(11, "v", (n, hkv * d))
        layer = A.AttentionLayer(1, hq, neox=neox, rope=rope)
        qr = kv.append(layer, positions, q, k, v).reshape(n, hq * d)
        q_ref = rope_rows(q, positions, hq, d, d, theta, neox, scale)
        k_ref = rope_rows(k, positions, hkv, d, d, theta, neox, scale)
        np.testing.assert_array_equal(qr, q_ref)
        if half:
            k_ref = oracle.f16_round(k_ref)
            v = oracle.f16_round(v)
        for i, p in enumerate(positions):
            kk, vv = kv.read(1, int(p), int(p) + 1)
            np.testing.assert_array_equal(kk, k_ref[i])
            np.testing.assert_array_equal(vv, v[i])
        assert not kv.contains(0, int(positions[0]))
    finally:
        kv.close()
        rope.close()


def _qk_norm_rows(x, heads, d, weight, eps):
    """normalizeHead over every head of every row (LlamaForwardPass.java:1070-1083)."""
    if weight is None:
        return np.asarray(x, np.float32).copy()
    return np.stack([oracle.qk_norm_heads(row, heads, d, weight, eps) for row in x])


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("sides", ["both", "k_only"])
def test_append_qk_norm_is_bit_exact(hip, half, neox, sides):
    """QK-norm then RoPE in the append kernel: q_out and the K cache equal the oracle's sequential
    float sum of squares, double sqrt, reciprocal and two products, bit for bit. With only a k
    weight, q passes through unnormalised (an empty attn_q_norm array)."""
    hq, hkv, d, n, theta, eps = 8, 2, 128, 24, 1e6, 1e-6
    positions = np.array([0, 1, 7, 63, 64, 500, 1023] + list(range(200, 217)))[:n]
    q = normal(12, "qn/q", (n, hq * d)) * 3.0
    k = normal(12, "qn/k", (n, hkv * d)) * 0.25
    v = normal(12, "qn/v", (n, hkv * d))
    wq = None if sides == "k_only" else normal(12, "qn/wq", (d,)) + 1.0
    wk = normal(12, "qn/wk", (d,)) + 1.0
    rope = hip.rotary_table(d, theta, 1.0, max_positions=1024)
    kv = hip.kv_cache(1, 1024, hkv, d, d, half_precision=half)
    norm = hip.qk_norm(d, wq, wk, eps)
    try:
        layer = A.AttentionLayer(0, hq, neox=neox, rope=rope, qk_norm=norm)
        qr = kv.append(layer, positions, q, k, v).reshape(n, hq * d)
        q_ref = rope_rows(_qk_norm_rows(q, hq, d, wq, eps), positions, hq, d, d, theta, neox)
        k_ref = rope_rows(_qk_norm_rows(k, hkv, d, wk, eps), positions, hkv, d, d, theta, neox)
        np.testing.assert_array_equal(qr, q_ref)
        if half:
            k_ref = oracle.f16_round(k_ref)
            v = oracle.f16_round(v)
        for i, p in enumerate(positions):
            kk, vv = kv.read(0, int(p), int(p) + 1)
            np.testing.assert_array_equal(kk, k_ref[i])
            np.testing.assert_array_equal(vv, v[i])
    finally:
        norm.close()
        kv.close()
        rope.close()


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("sides", ["both", "k_only"])
def test_qk_norm_prefill_then_decode(hip, half, sides):
    """Qwen3-shaped layer with attn_q_norm / attn_k_norm (16 Q / 8 KV heads, d 128, NeoX theta 1e6):
    300 prior rows through the MFMA prefill, then 3 decode steps (one fused launch each: QK-norm,
    RoPE, append and attention). The oracle normalises q and k the same way before its own RoPE;
    with only a k weight, q passes through unnormalised."""
    hq, hkv, d, prior, steps, theta, eps = 16, 8, 128, 300, 3, 1e6, 1e-6
    n = prior + steps
    scale = A.default_scale(d)
    q = normal(13, "qnd/q", (n, hq * d))
    k = normal(13, "qnd/k", (n, hkv * d))
    v = normal(13, "qnd/v", (n, hkv * d))
    wq = None if sides == "k_only" else normal(13, "qnd/wq", (d,)) * 0.2 + 1.0
    wk = normal(13, "qnd/wk", (d,)) * 0.2 + 1.0
    qn = _qk_norm_rows(q, hq, d, wq, eps)
    kn = _qk_norm_rows(k, hkv, d, wk, eps)
    ref = OracleKv(1, 512, hkv * d, hkv * d, half_precision=half)
    ref_prefill, _, _ = ref.prefill_layer(0, 0, qn[:prior], kn[:prior], v[:prior], hq, hkv, d, d,
                                          theta, 1.0, True, scale)
    ref_dec = [ref.decode_layer(0, prior + s, qn[prior + s], kn[prior + s], v[prior + s], hq, hkv,
                                d, d, theta, 1.0, True, scale)[0] for s in range(steps)]
    rope = hip.rotary_table(d, theta, 1.0, max_positions=512)
    kv = hip.kv_cache(1, 512, hkv, d, d, half_precision=half)
    norm = hip.qk_norm(d, wq, wk, eps)
    close = assert_f16_close if half else assert_f32_close
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope, qk_norm=norm)
        got_prefill = kv.prefill(layer, 0, q[:prior], k[:prior], v[:prior])
        e = [close(got_prefill, ref_prefill, "QK-norm prefill", head_dim=d)]
        for s in range(steps):
            got = kv.decode(layer, [prior + s], q[prior + s], k[prior + s], v[prior + s])
            e.append(close(got, ref_dec[s], f"QK-norm decode step {s}", head_dim=d))
        _say(f"QK-norm half={half} errors " + " ".join(f"{x:.2e}" for x in e))
        np.testing.assert_array_equal(kv.key_slice(0, 0, n), ref.key_slice(0, 0, n))
    finally:
        norm.close()
        kv.close()
        rope.close()


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("d", [128, 256])
def test_gemma4_value_norm_prefill_then_decode(hip, half, d):
    """Gemma-4-shaped layer (Gemma4ForwardPass.executeLayer, gemma4/Gemma4ForwardPass.java:955-1006):
    q and k heads RMS-normalised with weights, every v head RMS-normalised without a weight
    (Gemma4Math.normalizeWithoutWeight), NeoX RoPE, scale 1.0; a layer without a value projection
    passes the raw keys as v (:966-968). 200 prior rows through the prefill, then 3 decode steps,
    against the oracle fed the host-normalised q, k and v; the stored K and V rows are the
    oracle's bit for bit."""
    hq, hkv, prior, steps, theta, eps = 8, 2, 200, 3, 1e6, 1e-6
    n = prior + steps
    close = assert_f16_close if half else assert_f32_close
    for k_as_v in (False, True):
        q = normal(14, f"g4/q{d}", (n, hq * d))
        k = normal(14, f"g4/k{d}", (n, hkv * d))
        v = k.copy() if k_as_v else normal(14, f"g4/v{d}", (n, hkv * d))
        wq = normal(14, f"g4/wq{d}", (d,)) * 0.2 + 1.0
        wk = normal(14, f"g4/wk{d}", (d,)) * 0.2 + 1.0
        qn = _qk_norm_rows(q, hq, d, wq, eps)
        kn = _qk_norm_rows(k, hkv, d, wk, eps)
        vn = np.stack([oracle.value_rms_heads(row, hkv, d, eps) for row in v])
        ref = OracleKv(1, 512, hkv * d, hkv * d, half_precision=half)
        ref_prefill, _, _ = ref.prefill_layer(0, 0, qn[:prior], kn[:prior], vn[:prior], hq, hkv,
                                              d, d, theta, 1.0, True, 1.0)
        ref_dec = [ref.decode_layer(0, prior + s, qn[prior + s], kn[prior + s], vn[prior + s], hq,
                                    hkv, d, d, theta, 1.0, True, 1.0)[0] for s in range(steps)]
        rope = hip.rotary_table(d, theta, 1.0, max_positions=512)
        kv = hip.kv_cache(1, 512, hkv, d, d, half_precision=half)
        norm = hip.qk_norm(d, wq, wk, eps, value_rms=True)
        try:
            layer = A.AttentionLayer(0, hq, neox=True, scale=1.0, rope=rope, qk_norm=norm)
            got_prefill = kv.prefill(layer, 0, q[:prior], k[:prior], v[:prior])
            e = [close(got_prefill, ref_prefill, f"Gemma-4 prefill d {d} k_as_v {k_as_v}", head_dim=d)]
            for s in range(steps):
                got = kv.decode(layer, [prior + s], q[prior + s], k[prior + s], v[prior + s])
                e.append(close(got, ref_dec[s], f"Gemma-4 decode d {d} step {s}", head_dim=d))
            _say(f"Gemma-4 d={d} half={half} k_as_v={k_as_v} errors " + " ".join(f"{x:.2e}" for x in e))
            np.testing.assert_array_equal(kv.key_slice(0, 0, n), ref.key_slice(0, 0, n))
            np.testing.assert_array_equal(kv.value_slice(0, 0, n), ref.value_slice(0, 0, n))
        finally:
            norm.close()
            kv.close()
            rope.close()


def test_value_norm_rejects_bad_shapes(hip):
    """normalizeWithoutWeight rejects eps <= 0 (gemma4/Gemma4Math.java:47-49); the value norm's
    head_dim must equal the cache's value_length."""
    with pytest.raises(A.AttentionStatusError) as info:
        hip.qk_norm(64, None, None, 0.0, value_rms=True)
    assert info.value.status == A.INVALID_SHAPE
    norm = hip.qk_norm(64, None, None, 1e-6, value_rms=True)
    kv = hip.kv_cache(1, 8, 1, 64, 128, half_precision=False)
    try:
        layer = A.AttentionLayer(0, 1, qk_norm=norm)
        with pytest.raises(A.AttentionStatusError) as info:
            kv.append(layer, [0], np.ones(64), np.ones(64), np.ones(128))
        assert info.value.status == A.INVALID_SHAPE
    finally:
        kv.close()
        norm.close()


def test_qk_norm_rejects_bad_weights(hip):
    with pytest.raises(ValueError):
        hip.qk_norm(64, np.ones(32), None)
    norm = hip.qk_norm(64, None, None)
    rope = hip.rotary_table(128, 1e4, 1.0, max_positions=8)
    kv = hip.kv_cache(1, 8, 1, 128, 128, half_precision=False)
    try:
        layer = A.AttentionLayer(0, 1, neox=True, rope=rope, qk_norm=norm)
        with pytest.raises(A.AttentionStatusError) as info:
            kv.append(layer, [0], np.ones(128), np.ones(128), np.ones(128))
        assert info.value.status == A.INVALID_SHAPE
    finally:
        kv.close()
        rope.close()
        norm.close()


def test_rope_gemma4_proportional_golden_on_device(hip, known_answers):
    case = known_answers["rope"][0]  # RotaryTableTest :80-91
    rope = hip.rotary_table(case["rotary_dim"], case["theta"], case["frequency_scale"],
                            max_positions=8, frequency_factors=case["factors"])
    kv = hip.kv_cache(1, 8, 1, 16, 16, half_precision=False)
    try:
        head = _pad(case["input"], 16)
        layer = A.AttentionLayer(0, 1, neox=True, rope=rope)
        qr = kv.append(layer, [case["position"]], head, head, np.zeros(16))
        for idx, value, tol in case["expect_close"]:
            assert abs(float(qr[idx]) - value) <= tol
        for idx, value in case["expect_exact"]:
            assert qr[idx] == np.float32(value)
        assert not np.any(qr[8:])
    finally:
        kv.close()
        rope.close()


# ------------------------------------------------------------------ C1: Qwen3-0.6B f32 decode

def test_c1_qwen3_decode_f32(hip):
    """16 Q heads, 8 KV heads, d 128, NeoX theta 1e6, f32 KV: 512 prior positions (causal prefill
    through the d-sliced prefill kernel on f32 matrix ops) then the decode step at position 512.
    Full size."""
    hq, hkv, d, prior, theta = 16, 8, 128, 512, 1e6
    scale = A.default_scale(d)
    q = normal(1, "c1/q", (prior + 1, hq * d))
    k = normal(1, "c1/k", (prior + 1, hkv * d))
    v = normal(1, "c1/v", (prior + 1, hkv * d))
    ref = OracleKv(1, 1024, hkv * d, hkv * d)
    ref_prefill, _, _ = ref.prefill_layer(0, 0, q[:prior], k[:prior], v[:prior], hq, hkv, d, d,
                                          theta, 1.0, True, scale)
    ref_out, _, _ = ref.decode_layer(0, prior, q[prior], k[prior], v[prior], hq, hkv, d, d, theta,
                                     1.0, True, scale)
    rope = hip.rotary_table(d, theta, 1.0, max_positions=1024)
    kv = hip.kv_cache(1, 1024, hkv, d, d, half_precision=False)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        got_prefill = kv.prefill(layer, 0, q[:prior], k[:prior], v[:prior])
        got = kv.decode(layer, [prior], q[prior], k[prior], v[prior])
        e1 = assert_f32_close(got_prefill, ref_prefill, "C1 prefill rows", head_dim=d)
        e2 = assert_f32_close(got, ref_out, "C1 decode", head_dim=d)
        _say(f"C1 max abs err prefill {e1:.2e} decode {e2:.2e}")
        np.testing.assert_array_equal(kv.key_slice(0, 0, prior + 1), ref.key_slice(0, 0, prior + 1))
        np.testing.assert_array_equal(kv.value_slice(0, 0, prior + 1),
                                      ref.value_slice(0, 0, prior + 1))
    finally:
        kv.close()
        rope.close()


# ------------------------------------------------------------------ C2: Llama-3.2-1B f16 decode

def test_c2_llama_decode_f16_reduced(hip):
    """32 Q heads, 8 KV heads, d 64, interleaved theta 5e5, f16 KV; 2 layers, 1000 prior
    positions (MFMA prefill), then 4 consecutive decode steps per layer."""
    hq, hkv, d, prior, steps, theta, layers = 32, 8, 64, 1000, 4, 5e5, 2
    scale = A.default_scale(d)
    n = prior + steps
    rope = hip.rotary_table(d, theta, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True)
    try:
        for l in range(layers):
            q = normal(2, f"c2/q{l}", (n, hq * d))
            k = normal(2, f"c2/k{l}", (n, hkv * d))
            v = normal(2, f"c2/v{l}", (n, hkv * d))
            ref = OracleKv(1, n, hkv * d, hkv * d, half_precision=True)
            k_rot = rope_rows(k, range(n), hkv, d, d, theta, False)
            for p in range(prior):
                ref.store(0, p, k_rot[p], v[p])
            layer = A.AttentionLayer(l, hq, neox=False, rope=rope)
            got_prefill = kv.prefill(layer, 0, q[:prior], k[:prior], v[:prior]).reshape(prior, -1)
            q_rot = rope_rows(q, range(n), hq, d, d, theta, False)
            for row in (0, 1, 31, 32, 500, prior - 1):
                want = ref.gqa(0, row, q_rot[row], hq, hkv, d, d, scale)
                assert_f16_close(got_prefill[row], want, f"C2 prefill row {row}", head_dim=d)
            for s in range(steps):
                p = prior + s
                got = kv.decode(layer, [p], q[p], k[p], v[p])
                want, _, _ = ref.decode_layer(0, p, q[p], k[p], v[p], hq, hkv, d, d, theta, 1.0,
                                              False, scale)
                rel = assert_f16_close(got, want, f"C2 layer {l} step {s}", head_dim=d)
            _say(f"C2 layer {l} last-step normwise rel err {rel:.2e}")
            np.testing.assert_array_equal(kv.key_slice(l, 0, n), ref.key_slice(0, 0, n))
            np.testing.assert_array_equal(kv.value_slice(l, 0, n), ref.value_slice(0, 0, n))
    finally:
        kv.close()
        rope.close()


# ------------------------------------------------------------------ C3: Llama-3.2-3B prefill

def test_c3_llama_prefill_f16_full(hip):
    """S 2048, 24 Q heads, 8 KV heads, d 128, interleaved theta 5e5, f16 Q/K/V, causal. Full
    size: the oracle runs per-row GQA over each causal prefix on 16 threads."""
    hq, hkv, d, S, theta = 24, 8, 128, 2048, 5e5
    scale = A.default_scale(d)
    q = oracle.f16_round(normal(3, "c3/q", (S, hq * d)))
    k = oracle.f16_round(normal(3, "c3/k", (S, hkv * d)))
    v = oracle.f16_round(normal(3, "c3/v", (S, hkv * d)))
    rope = hip.rotary_table(d, theta, 1.0, max_positions=S)
    kv = hip.kv_cache(1, S, hkv, d, d, half_precision=True)
    try:
        layer = A.AttentionLayer(0, hq, neox=False, rope=rope)
        got = kv.prefill(layer, 0, q, k, v).reshape(S, hq * d)
        k_ref = oracle.f16_round(rope_rows(k, range(S), hkv, d, d, theta, False))
        keys, values = kv.read(0, 0, S)
        np.testing.assert_array_equal(keys, k_ref.reshape(-1))
        np.testing.assert_array_equal(values, v.reshape(-1))
        q_rot = rope_rows(q, range(S), hq, d, d, theta, False)
        keys = keys.reshape(S, -1)
        values = values.reshape(S, -1)
        rows = list(range(S))
        outs = oracle.gqa_rows_batch([q_rot[r] for r in rows], [keys[:r + 1] for r in rows],
                                     [values[:r + 1] for r in rows], hq, hkv, d, d, scale,
                                     threads=16)
        rel = assert_f16_close(got, np.stack(outs), "C3 prefill", head_dim=d)
        _say(f"C3 normwise rel err {rel:.2e}")
    finally:
        kv.close()
        rope.close()


def test_prefill_chunked_and_windowed_matches_oracle(hip):
    """Chunked prefill (start > 0 attends to cached rows) and a sliding window through the MFMA
    kernel, against the oracle's prefill (computeBatchedAttention) on the same cache."""
    hq, hkv, d, theta, w = 6, 2, 64, 1e4, 48
    scale = A.default_scale(d)
    n1, n2 = 70, 93
    n = n1 + n2
    q = normal(4, "pc/q", (n, hq * d))
    k = normal(4, "pc/k", (n, hkv * d))
    v = normal(4, "pc/v", (n, hkv * d))
    rope = hip.rotary_table(d, theta, 1.0, max_positions=256)
    for window in (0, w):
        ref = OracleKv(1, 256, hkv * d, hkv * d, half_precision=True)
        r1, _, _ = ref.prefill_layer(0, 0, q[:n1], k[:n1], v[:n1], hq, hkv, d, d, theta, 1.0,
                                     True, scale, window=window)
        r2, _, _ = ref.prefill_layer(0, n1, q[n1:], k[n1:], v[n1:], hq, hkv, d, d, theta, 1.0,
                                     True, scale, window=window)
        kv = hip.kv_cache(1, 256, hkv, d, d, half_precision=True)
        try:
            layer = A.AttentionLayer(0, hq, sliding_window=window, neox=True, rope=rope)
            g1 = kv.prefill(layer, 0, q[:n1], k[:n1], v[:n1])
            g2 = kv.prefill(layer, n1, q[n1:], k[n1:], v[n1:])
            assert_f16_close(g1, r1, f"chunk 1 window {window}", head_dim=d)
            assert_f16_close(g2, r2, f"chunk 2 window {window}", head_dim=d)
        finally:
            kv.close()
    rope.close()


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_prefill_split_blocks_match_oracle(monkeypatch, d):
    """Row blocks whose kv range is split between two workgroups (the later to finish merges the
    two states, the other's stored device-coherent) against the oracle, for every split threshold
    (JMA_PREFILL_SPLIT_TILES: 0 never splits, 2 splits every block of two or more kv tiles, 32 the
    longest, -1 splits while the grid underfills the device), causal and windowed, a chunk start,
    a group of 3 (ragged stripes) and ragged tails."""
    hq, hkv, theta = 12, 4, 1e4
    scale = A.default_scale(d)
    n1, n2 = 150, 1061
    n, cap = n1 + n2, 1280
    q = normal(21, f"ps/q{d}", (n, hq * d))
    k = normal(21, f"ps/k{d}", (n, hkv * d))
    v = normal(21, f"ps/v{d}", (n, hkv * d))
    for window in (0, 700):
        ref = OracleKv(1, cap, hkv * d, hkv * d, half_precision=True)
        r1, _, _ = ref.prefill_layer(0, 0, q[:n1], k[:n1], v[:n1], hq, hkv, d, d, theta, 1.0,
                                     True, scale, window=window)
        r2, _, _ = ref.prefill_layer(0, n1, q[n1:], k[n1:], v[n1:], hq, hkv, d, d, theta, 1.0,
                                     True, scale, window=window)
        for split in ("0", "2", "32", "-1"):
            monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", split)
            lib = A.HipAttentionLibrary(0)
            try:
                rope = lib.rotary_table(d, theta, 1.0, max_positions=cap)
                kv = lib.kv_cache(1, cap, hkv, d, d, half_precision=True)
                layer = A.AttentionLayer(0, hq, sliding_window=window, neox=True, rope=rope)
                for rep in range(2):  # the second pass reuses the restored words and tickets
                    g1 = kv.prefill(layer, 0, q[:n1], k[:n1], v[:n1])
                    g2 = kv.prefill(layer, n1, q[n1:], k[n1:], v[n1:])
                    assert_f16_close(g1, r1, f"d {d} window {window} split {split} chunk 1", head_dim=d)
                    assert_f16_close(g2, r2, f"d {d} window {window} split {split} chunk 2", head_dim=d)
                kv.close()
                rope.close()
            finally:
                lib.close()
            _say(f"d {d} window {window} split {split} ok")


def test_gemma3_prefill_2048_automatic_split(hip):
    """A Gemma-3-shaped 2048-row prefill (4 Q / 1 KV heads, d 256, NeoX theta 1e6) under the
    automatic plan: row blocks hold 2 stripes of 8 rows x 4 heads, and the 34 longest (>= 48 kv
    tiles against an average of 16 per compute unit) have their kv range split between two
    workgroups that merge through the partial-word exchange. Every row against the oracle over
    the read-back cache; K bit-exact."""
    hq, hkv, d, S, theta = 4, 1, 256, 2048, 1e6
    scale = A.default_scale(d)
    q = normal(23, "g3p/q", (S, hq * d))
    k = normal(23, "g3p/k", (S, hkv * d))
    v = normal(23, "g3p/v", (S, hkv * d))
    rope = hip.rotary_table(d, theta, 1.0, max_positions=S)
    kv = hip.kv_cache(1, S, hkv, d, d, half_precision=True)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        got = kv.prefill(layer, 0, q, k, v).reshape(S, hq * d)
        got2 = kv.attend_causal(layer, 0, rope_rows(q, range(S), hq, d, d, theta, True)).reshape(S, -1)
        np.testing.assert_array_equal(got2, got)  # the exchange words and tickets were restored
        keys, values = kv.read(0, 0, S)
        keys, values = keys.reshape(S, -1), values.reshape(S, -1)
        np.testing.assert_array_equal(keys, oracle.f16_round(rope_rows(k, range(S), hkv, d, d,
                                                                        theta, True)))
        q_rot = rope_rows(q, range(S), hq, d, d, theta, True)
        outs = oracle.gqa_rows_batch([q_rot[r] for r in range(S)], [keys[:r + 1] for r in range(S)],
                                     [values[:r + 1] for r in range(S)], hq, hkv, d, d, scale,
                                     threads=16)
        rel = assert_f16_close(got, np.stack(outs), "Gemma-3 2048-row prefill", head_dim=d)
        _say(f"Gemma-3 2048-row prefill normwise rel err {rel:.2e}")
    finally:
        kv.close()
        rope.close()


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("which", ["k", "v"])
@pytest.mark.parametrize("window", [0, 20])
def test_prefill_ignores_rows_it_does_not_see(hip, window, which, d):
    _nonfinite_rows_case(hip, window, which, d)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("which", ["k", "v"])
def test_split_prefill_ignores_rows_it_does_not_see(monkeypatch, which, d):
    """The same with every row block of two or more kv tiles split between two workgroups
    (JMA_PREFILL_SPLIT_TILES=2): a half that repeats its pass still meets its partner."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    try:
        _nonfinite_rows_case(lib, 0, which, d)
    finally:
        lib.close()


def _nonfinite_rows_case(hip, window, which, d):
    """Positions a row does not see never reach its result, whatever the cache holds there: 48
    rows are appended with key (or value) row 45 (and, windowed, row 3) overflowing f16 to
    infinity, positions 40.. are discarded (the slots keep their contents), and rows 40..43 are
    prefilled again, then position 44 decoded. Their causal (and window) ranges exclude the
    infinite rows, which share kv tiles with rows they do see; the reference's results are
    finite."""
    hq, hkv, theta, cap = 8, 2, 1e4, 128
    scale = A.default_scale(d)
    q = normal(22, "nf/q", (48, hq * d))
    k = normal(22, "nf/k", (48, hkv * d))
    v = normal(22, "nf/v", (48, hkv * d))
    k_bad, v_bad = k.copy(), v.copy()
    bad = k_bad if which == "k" else v_bad
    bad[45] = 1e6
    if window:
        bad[3] = -1e6
    q2 = normal(22, "nf/q2", (4, hq * d))
    k2 = normal(22, "nf/k2", (4, hkv * d))
    v2 = normal(22, "nf/v2", (4, hkv * d))
    ref = OracleKv(1, cap, hkv * d, hkv * d, half_precision=True)
    ref.prefill_layer(0, 0, q[:40], k[:40], v[:40], hq, hkv, d, d, theta, 1.0, True, scale,
                      window=window)
    want, _, _ = ref.prefill_layer(0, 40, q2, k2, v2, hq, hkv, d, d, theta, 1.0, True, scale,
                                   window=window)
    rope = hip.rotary_table(d, theta, 1.0, max_positions=cap)
    kv = hip.kv_cache(1, cap, hkv, d, d, half_precision=True)
    try:
        layer = A.AttentionLayer(0, hq, sliding_window=window, neox=True, rope=rope)
        kv.append(layer, list(range(48)), q, k_bad, v_bad)
        stored = kv.key_slice(0, 45, 46) if which == "k" else kv.value_slice(0, 45, 46)
        assert not np.all(np.isfinite(stored))
        kv.discard_from(40)
        got = kv.prefill(layer, 40, q2, k2, v2)
        assert_f16_close(got, want, f"d {d} {which} window {window} prefill", head_dim=d)
        # and a decode step at 44, whose kv tile still holds the infinite row 45
        q3, k3, v3 = (normal(22, f"nf/{t}3", (hq * d if t == "q" else hkv * d,)) for t in "qkv")
        want3, _, _ = ref.decode_layer(0, 44, q3, k3, v3, hq, hkv, d, d, theta, 1.0, True, scale,
                                       window=window)
        got3 = kv.decode(layer, [44], q3, k3, v3)
        assert_f16_close(got3, want3, f"d {d} {which} window {window} decode", head_dim=d)
    finally:
        kv.close()
        rope.close()


# ------------------------------------------------------------------ C4: ragged batched decode

def test_c4_ragged_decode_reduced(hip):
    """64 sessions with KV lengths uniform on [256, 2048] (the full config draws up to 16384),
    12 Q heads, 2 KV heads, d 128, NeoX theta 1e6, f16 KV; one new token per session."""
    hq, hkv, d, theta, B = 12, 2, 128, 1e6, 64
    scale = A.default_scale(d)
    lens = [int(x) for x in synth.uniform_int(4, "c4/len", B, 256, 2048)]
    maxlen = max(lens) + 1
    rope = hip.rotary_table(d, theta, 1.0, max_positions=maxlen)
    kv = hip.kv_cache(1, maxlen, hkv, d, d, half_precision=True, sequences=B)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        for s, L in enumerate(lens):
            k = normal(4, f"c4/k{s}", (L, hkv * d))
            v = normal(4, f"c4/v{s}", (L, hkv * d))
            kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32), k, v,
                      sequences=np.full(L, s))
        qn = normal(4, "c4/qn", (B, hq * d))
        kn = normal(4, "c4/kn", (B, hkv * d))
        vn = normal(4, "c4/vn", (B, hkv * d))
        got = kv.decode(layer, lens, qn, kn, vn, sequences=np.arange(B)).reshape(B, -1)
        worst = 0.0
        for s, L in enumerate(lens):
            keys, values = kv.read(0, 0, L + 1, sequence=s)
            q_rot = rope_rows(qn[s:s + 1], [L], hq, d, d, theta, True, check_against_oracle=(s == 0))
            k_new = oracle.f16_round(rope_rows(kn[s:s + 1], [L], hkv, d, d, theta, True,
                                               check_against_oracle=False))
            np.testing.assert_array_equal(keys.reshape(L + 1, -1)[L], k_new[0])
            want = oracle.gqa_rows(q_rot[0], keys, values, hq, hkv, d, d, scale)
            worst = max(worst, assert_f16_close(got[s], want, f"C4 session {s} (L={L})", head_dim=d))
        _say(f"C4 worst normwise rel err {worst:.2e}")
    finally:
        kv.close()
        rope.close()


def test_c4_ragged_decode_full_size(hip):
    """BASELINE configs[3] at its configured size: 64 sessions whose KV lengths are the
    benchmark's draw (U[256, 16384], seed 4, 480k cached rows), 12 Q / 2 KV heads, d 128, NeoX
    theta 1e6, f16 KV, one new token per session in one fused decode launch (RoPE, append,
    split-K attention, cross-split reduction). Every session against the oracle's GQA over the
    read-back cache (attendIndependentSessions, llama/LlamaForwardPass.java:793-839); the appended
    rows bit-exact; the longest and shortest sessions' whole caches bit-exact."""
    from models_amd.hip_runtime import DeviceArray
    hq, hkv, d, theta, B = 12, 2, 128, 1e6, 64
    scale = A.default_scale(d)
    lens = [int(x) for x in synth.uniform_int(4, "bench/c4/len", B, 256, 16384)]
    maxlen = max(lens) + 1
    qd, kd = hq * d, hkv * d
    rope = hip.rotary_table(d, theta, 1.0, max_positions=maxlen)
    kv = hip.kv_cache(1, maxlen, hkv, d, d, half_precision=True, sequences=B)
    zq = DeviceArray(maxlen * qd)
    zq.zero()
    dk, dv = DeviceArray(maxlen * kd), DeviceArray(maxlen * kd)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        k_host = {}
        check_full = {int(np.argmax(lens)), int(np.argmin(lens))}
        for s, L in enumerate(lens):
            k = normal(4, f"c4full/k{s}", (L, kd))
            v = normal(4, f"c4full/v{s}", (L, kd))
            if s in check_full:
                k_host[s] = (k, v)
            dk.upload(k)
            dv.upload(v)
            kv.append_device(layer, np.full(L, s, np.uint32), np.arange(L), zq.ptr, L * qd,
                             dk.ptr, L * kd, dv.ptr, L * kd)
        hip.synchronize()
        _say(f"C4 full: {sum(lens)} rows cached")
        qn = normal(4, "c4full/qn", (B, qd))
        kn = normal(4, "c4full/kn", (B, kd))
        vn = normal(4, "c4full/vn", (B, kd))
        got = kv.decode(layer, lens, qn, kn, vn, sequences=np.arange(B)).reshape(B, -1)
        q_rot = rope_rows(qn, lens, hq, d, d, theta, True)
        k_new = oracle.f16_round(rope_rows(kn, lens, hkv, d, d, theta, True))
        qs, ks, vs = [], [], []
        for s, L in enumerate(lens):
            keys, values = kv.read(0, 0, L + 1, sequence=s)
            keys, values = keys.reshape(L + 1, kd), values.reshape(L + 1, kd)
            np.testing.assert_array_equal(keys[L], k_new[s])
            np.testing.assert_array_equal(values[L], oracle.f16_round(vn[s]))
            if s in check_full:
                k, v = k_host[s]
                k_ref = oracle.f16_round(rope_rows(k, range(L), hkv, d, d, theta, True,
                                                   check_against_oracle=False))
                np.testing.assert_array_equal(keys[:L], k_ref)
                np.testing.assert_array_equal(values[:L], oracle.f16_round(v))
            qs.append(q_rot[s])
            ks.append(keys)
            vs.append(values)
        outs = oracle.gqa_rows_batch(qs, ks, vs, hq, hkv, d, d, scale, threads=16)
        worst = 0.0
        for s, L in enumerate(lens):
            worst = max(worst, assert_f16_close(got[s], outs[s], f"C4 full session {s} (L={L})",
                                                head_dim=d))
        _say(f"C4 full worst normwise rel err {worst:.2e}")
    finally:
        for buf in (zq, dk, dv):
            buf.free()
        kv.close()
        rope.close()


# ------------------------------------------------------------------ C5: Gemma-3 SWA / global

@pytest.mark.parametrize("ring", [False, True])
def test_c5_gemma3_sliding_window_reduced(hip, ring):
    """4 Q heads, 1 KV head (MQA), d 256, 6 layers in the 5 sliding (window 512, theta 1e4) : 1
    global (theta 1e6) pattern, f16 KV, 1500 prior positions and 3 decode steps (the full config
    runs 26 layers at 32768). With ring=True the sliding layers keep a 544-slot ring
    (window + one 32-row chunk, LayeredKvCache RING retention)."""
    hq, hkv, d, prior, steps, layers, w = 4, 1, 256, 1500, 3, 6, 512
    scale = A.default_scale(d)
    n = prior + steps
    rope_swa = hip.rotary_table(d, 1e4, 1.0, max_positions=n)
    rope_glb = hip.rotary_table(d, 1e6, 1.0, max_positions=n)
    sliding = [A.uses_sliding_window(l, 6, w) for l in range(layers)]
    ring_caps = [544 if s else 0 for s in sliding] if ring else None
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True, ring_capacity=ring_caps)
    try:
        for l in range(layers):
            theta = 1e4 if sliding[l] else 1e6
            window = w if sliding[l] else 0
            layer = A.AttentionLayer(l, hq, sliding_window=window, neox=True,
                                     rope=rope_swa if sliding[l] else rope_glb)
            q = normal(5, f"c5/q{l}", (n, hq * d))
            k = normal(5, f"c5/k{l}", (n, hkv * d))
            v = normal(5, f"c5/v{l}", (n, hkv * d))
            ref = OracleKv(1, n, hkv * d, hkv * d, half_precision=True)
            k_rot = rope_rows(k, range(n), hkv, d, d, theta, True)
            for p in range(prior):
                ref.store(0, p, k_rot[p], v[p])
            # Fill the prior positions in chunks no longer than the ring can hold with the window.
            chunk = 32 if (ring and sliding[l]) else prior
            for start in range(0, prior, chunk):
                stop = min(prior, start + chunk)
                kv.prefill(layer, start, q[start:stop], k[start:stop], v[start:stop])
            for s in range(steps):
                p = prior + s
                got = kv.decode(layer, [p], q[p], k[p], v[p])
                want, _, _ = ref.decode_layer(0, p, q[p], k[p], v[p], hq, hkv, d, d, theta, 1.0,
                                              True, scale, window=window)
                rel = assert_f16_close(got, want, f"C5 layer {l} step {s}", head_dim=d)
            _say(f"C5 ring={ring} layer {l} ({'swa' if sliding[l] else 'global'}) rel {rel:.2e}")
            if ring and sliding[l]:
                assert not kv.contains(l, 0) and kv.contains(l, n - 1)
                assert kv.contains(l, n - 544) and not kv.contains(l, n - 545)
    finally:
        kv.close()
        rope_swa.close()
        rope_glb.close()


def test_c5_gemma3_long_context_full_size(hip):
    """BASELINE configs[4] at its configured size: 4 Q / 1 KV heads (MQA), d 256, NeoX RoPE
    (theta 1e4 on sliding layers, 1e6 on the global layers 5, 11, 17, 23), f16 KV, 26 layers in
    the 5 sliding (window 512) : 1 global pattern (LlamaConfig.usesSlidingWindow and
    attentionStartPosition, llama/LlamaConfig.java:157-162, 184-195), 32704 prior positions and
    the configured 64 decode steps (to position 32767, the cache's last). Sliding layers keep
    LayeredKvCache RING retention of 544 slots (window + one 32-row chunk) holding their last 512
    prior positions; the global layers hold all 32704 and run the wide split plans. Eight steps
    spread over the run (0, 9, ..., 63) check every layer against the oracle's GQA over the window
    read back from the device, with the appended rows bit-exact."""
    from models_amd.hip_runtime import DeviceArray
    hq, hkv, d, prior, steps, layers, w, ring = 4, 1, 256, 32704, 64, 26, 512, 544
    checked = list(range(0, steps, 9))
    assert len(checked) == 8 and checked[-1] == steps - 1
    scale = A.default_scale(d)
    n = prior + steps
    qd, kd = hq * d, hkv * d
    sliding = [A.uses_sliding_window(l, 6, w) for l in range(layers)]
    assert [l for l in range(layers) if not sliding[l]] == [5, 11, 17, 23]
    rope_swa = hip.rotary_table(d, 1e4, 1.0, max_positions=n)
    rope_glb = hip.rotary_table(d, 1e6, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True,
                      ring_capacity=[ring if sl else 0 for sl in sliding])
    zq = DeviceArray(prior * qd)
    zq.zero()
    dk, dv = DeviceArray(prior * kd), DeviceArray(prior * kd)
    try:
        lp = [A.AttentionLayer(l, hq, sliding_window=w if sliding[l] else 0, neox=True,
                               rope=rope_swa if sliding[l] else rope_glb) for l in range(layers)]
        for l in range(layers):
            first = prior - w if sliding[l] else 0
            rows = prior - first
            dk.upload(normal(5, f"c5full/k{l}", (rows, kd)))
            dv.upload(normal(5, f"c5full/v{l}", (rows, kd)))
            kv.append_device(lp[l], np.zeros(rows, np.uint32), np.arange(first, prior), zq.ptr,
                             rows * qd, dk.ptr, rows * kd, dv.ptr, rows * kd)
        hip.synchronize()
        _say("C5 full: caches filled")
        q = normal(5, "c5full/q", (layers, steps, qd))
        kn = normal(5, "c5full/kn", (layers, steps, kd))
        vn = normal(5, "c5full/vn", (layers, steps, kd))
        worst = {True: 0.0, False: 0.0}
        for st in range(steps):
            p = prior + st
            outs = [kv.decode(lp[l], [p], q[l, st], kn[l, st], vn[l, st]) for l in range(layers)]
            if st not in checked:
                continue
            qs, ks, vs = [], [], []
            for l in range(layers):
                theta = 1e4 if sliding[l] else 1e6
                first = A.attention_start_position(p, w if sliding[l] else 0)
                keys, values = kv.read(l, first, p + 1)
                keys, values = keys.reshape(-1, kd), values.reshape(-1, kd)
                k_new = oracle.f16_round(rope_rows(kn[l, st:st + 1], [p], hkv, d, d, theta, True,
                                                   check_against_oracle=(l < 6 and st == 0)))
                np.testing.assert_array_equal(keys[-1], k_new[0])
                np.testing.assert_array_equal(values[-1], oracle.f16_round(vn[l, st]))
                qs.append(rope_rows(q[l, st:st + 1], [p], hq, d, d, theta, True,
                                    check_against_oracle=(l < 6 and st == 0))[0])
                ks.append(keys)
                vs.append(values)
            want = oracle.gqa_rows_batch(qs, ks, vs, hq, hkv, d, d, scale, threads=16)
            for l in range(layers):
                rel = assert_f16_close(outs[l], want[l], f"C5 full layer {l} step {st}", head_dim=d)
                worst[sliding[l]] = max(worst[sliding[l]], rel)
            # the ring holds the last 544 positions stored (the 512 prior ones appended first,
            # then the decoded rows) and nothing older
            oldest = max(prior - w, p + 1 - ring)
            assert kv.contains(0, oldest) and not kv.contains(0, oldest - 1)
            _say(f"C5 full step {st}: 26 layers against the oracle")
        _say(f"C5 full worst normwise rel err: sliding {worst[True]:.2e}, global {worst[False]:.2e}")
    finally:
        for buf in (zq, dk, dv):
            buf.free()
        kv.close()
        rope_swa.close()
        rope_glb.close()


# ------------------------------------------------------------------ error paths

def test_error_paths_match_reference_exceptions(hip):
    hq, hkv, d = 4, 2, 32
    rope = hip.rotary_table(d, 1e4, 1.0, max_positions=64)
    kv = hip.kv_cache(2, 64, hkv, d, d, half_precision=True, ring_capacity=[0, 32])
    try:
        layer = A.AttentionLayer(0, hq, rope=rope)
        z = lambda *shape: np.zeros(shape, np.float32)  # noqa: E731
        kv.append(layer, [0, 1, 2, 3], normal(6, "q", (4, hq * d)), normal(6, "k", (4, hkv * d)),
                  normal(6, "v", (4, hkv * d)))
        # reading past the populated prefix: IllegalStateException -> UNAVAILABLE
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(layer, [5], z(hq * d))
        assert e.value.status == A.UNAVAILABLE
        # decode at 5 needs 4 populated
        with pytest.raises(A.AttentionStatusError) as e:
            kv.decode(layer, [5], z(hq * d), z(hkv * d), z(hkv * d))
        assert e.value.status == A.UNAVAILABLE
        # position beyond maxSeqLen: IllegalArgumentException -> OUT_OF_RANGE
        with pytest.raises(A.AttentionStatusError) as e:
            kv.decode(layer, [64], z(hq * d), z(hkv * d), z(hkv * d))
        assert e.value.status == A.OUT_OF_RANGE
        # layer out of range
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(A.AttentionLayer(2, hq, rope=rope), [0], z(hq * d))
        assert e.value.status == A.OUT_OF_RANGE
        # undersized buffer
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(layer, [3], z(hq * d - 1))
        assert e.value.status == A.BUFFER_TOO_SMALL
        # NaN query -> softmax rejects NaN scores -> NON_FINITE, and the context recovers
        bad = normal(6, "bad", (hq * d,))
        bad[5] = np.nan
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(layer, [3], bad)
        assert e.value.status == A.NON_FINITE
        ok = kv.attend(layer, [3], normal(6, "good", (hq * d,)))
        assert np.all(np.isfinite(ok))
        # discardFrom then read: the tail is gone
        kv.discard_from(2)
        assert kv.contains(0, 1) and not kv.contains(0, 2)
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(layer, [3], z(hq * d))
        assert e.value.status == A.UNAVAILABLE
        # ring layer: a window wider than the ring -> OUT_OF_RANGE (attentionView :185-191)
        ring_layer = A.AttentionLayer(1, hq, rope=rope)
        kv.append(ring_layer, list(range(40)), z(40, hq * d), normal(7, "k", (40, hkv * d)),
                  normal(7, "v", (40, hkv * d)))
        assert not kv.contains(1, 7) and kv.contains(1, 8)
        with pytest.raises(A.AttentionStatusError) as e:
            kv.attend(ring_layer, [39], z(hq * d))
        assert e.value.status == A.OUT_OF_RANGE
        windowed = A.AttentionLayer(1, hq, sliding_window=32, rope=rope)
        assert np.all(np.isfinite(kv.attend(windowed, [39], normal(7, "q", (hq * d,)))))
        # sessions of one batch must be distinct
        kv2 = hip.kv_cache(1, 64, hkv, d, d, sequences=2)
        try:
            with pytest.raises(A.AttentionStatusError) as e:
                kv2.decode(layer, [0, 1], z(2, hq * d), z(2, hkv * d), z(2, hkv * d),
                           sequences=[0, 0])
            assert e.value.status == A.INVALID_SHAPE
        finally:
            kv2.close()
    finally:
        kv.close()
        rope.close()


# ------------------------------------------------------------------ properties at full size

def test_c2_full_size_every_layer_step_and_properties(hip):
    """C2 at its full size (16 layers, 4096 prior positions, 128 steps) through the device-pointer
    entry points, as the benchmark runs it. Checks: every one of the 16 x 128 layer-steps against
    the oracle's GQA (groupedQueryAttention, llama/LlamaForwardPass.java:1543-1593) over the
    cache read back from the device, the 128 rows of a layer in one threaded oracle batch; a
    second replay after discard_from(4096) reproduces the outputs exactly (idempotence of the
    resident cache); every row the run appended, in every layer, equals the oracle's rotated,
    f16-rounded K and f16-rounded V."""
    from models_amd.hip_runtime import DeviceArray
    hq, hkv, d, prior, steps, layers, theta = 32, 8, 64, 4096, 128, 16, 5e5
    scale = A.default_scale(d)
    n = prior + steps
    rope = hip.rotary_table(d, theta, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True)
    qd, kd = hq * d, hkv * d
    zeros_q = DeviceArray(prior * qd)
    zeros_q.zero()
    dq = DeviceArray(layers * steps * qd)
    dk = DeviceArray(layers * n * kd)
    dv = DeviceArray(layers * n * kd)
    dout = DeviceArray(layers * steps * qd)
    try:
        q_host = normal(2, "c2full/q", (layers, steps, qd))
        dq.upload(q_host)
        k_host, v_host = [], []
        for l in range(layers):
            k_host.append(normal(2, f"c2full/k{l}", (n, kd)))
            v_host.append(normal(2, f"c2full/v{l}", (n, kd)))
            dk.upload(k_host[l], l * n * kd)
            dv.upload(v_host[l], l * n * kd)
        _say("C2 full: inputs uploaded")
        seqs = np.zeros(prior, np.uint32)
        for l in range(layers):
            layer = A.AttentionLayer(l, hq, neox=False, rope=rope)
            kv.append_device(layer, seqs, np.arange(prior), zeros_q.ptr, prior * qd,
                             dk.at(l * n * kd), prior * kd, dv.at(l * n * kd), prior * kd)
        hip.synchronize()
        layers_p = [A.AttentionLayer(l, hq, neox=False, rope=rope) for l in range(layers)]

        def run_steps():
            for s in range(steps):
                p = prior + s
                for l in range(layers):
                    kv.decode_device(layers_p[l], [0], [p], dq.at((l * steps + s) * qd), qd,
                                     dk.at((l * n + p) * kd), kd, dv.at((l * n + p) * kd), kd,
                                     dout.at((l * steps + s) * qd), qd)
            hip.synchronize()
            return dout.download().reshape(layers, steps, qd)

        first = run_steps()
        kv.discard_from(prior)
        second = run_steps()
        np.testing.assert_array_equal(first, second)
        _say("C2 full: replay identical")
        worst = 0.0
        for l in range(layers):
            keys, values = kv.read(l, 0, n)
            keys = np.ascontiguousarray(keys.reshape(n, -1))
            values = np.ascontiguousarray(values.reshape(n, -1))
            k_rot = oracle.f16_round(rope_rows(k_host[l][prior:], range(prior, n), hkv, d, d,
                                               theta, False, check_against_oracle=(l == 0)))
            np.testing.assert_array_equal(keys[prior:], k_rot)
            np.testing.assert_array_equal(values, oracle.f16_round(v_host[l]))
            q_rot = rope_rows(q_host[l], range(prior, n), hq, d, d, theta, False,
                              check_against_oracle=(l == 0))
            want = oracle.gqa_rows_batch([q_rot[s] for s in range(steps)],
                                         [keys[:prior + s + 1] for s in range(steps)],
                                         [values[:prior + s + 1] for s in range(steps)],
                                         hq, hkv, d, d, scale, threads=16)
            for s in range(steps):
                rel = assert_f16_close(first[l, s], want[s], f"C2 full layer {l} step {s}",
                                       head_dim=d)
                worst = max(worst, rel)
            _say(f"C2 full layer {l}: 128 steps against the oracle, worst rel {worst:.2e}")
    finally:
        for buf in (zeros_q, dq, dk, dv, dout):
            buf.free()
        kv.close()
        rope.close()


# ------------------------------------------------------------------ entry-point equivalences

def test_attend_causal_equals_prefill(hip):
    """prefill == append + attend_causal (prepareBatchedAttention then computeBatchedAttention)."""
    hq, hkv, d, n, theta = 12, 4, 128, 300, 1e6
    q = normal(12, "ac/q", (n, hq * d))
    k = normal(12, "ac/k", (n, hkv * d))
    v = normal(12, "ac/v", (n, hkv * d))
    rope = hip.rotary_table(d, theta, 1.0, max_positions=n)
    a = hip.kv_cache(1, n, hkv, d, d, half_precision=True)
    b = hip.kv_cache(1, n, hkv, d, d, half_precision=True)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        want = a.prefill(layer, 0, q, k, v)
        q_rot = b.append(layer, np.arange(n), q, k, v)
        got = b.attend_causal(layer, 0, q_rot)
        np.testing.assert_array_equal(got, want)
    finally:
        a.close()
        b.close()
        rope.close()


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("neox", [False, True])
def test_split_plans_and_fusion_agree(hip, monkeypatch, neox, d):
    """Split-K invariance and fusion equivalence on a ragged multi-session decode batch: many
    splits (one tile per wave, up to 32 splits) or one split per row, with RoPE + append + split
    reduction fused into the decode kernel or run as separate kernels (JMA_UNFUSED=1), change only
    the summation order; the appended cache rows are bit-identical. At head dim 256 the plans of
    one tile per wave run the single-tile-buffer kernel instance, the others the two-buffer one."""
    hq, hkv, theta, B = 8, 2, 1e4, 5
    lens = [40, 700, 1333, 2048, 97]
    outs, rows = [], []
    for env in ({"JMA_DECODE_TILES_PER_WAVE": "1", "JMA_DECODE_TARGET_BLOCKS": "4096"},
                {"JMA_DECODE_TILES_PER_WAVE": "64", "JMA_DECODE_TARGET_BLOCKS": "1"},
                {"JMA_DECODE_TILES_PER_WAVE": "1", "JMA_DECODE_TARGET_BLOCKS": "4096",
                 "JMA_UNFUSED": "1"}):
        for key in ("JMA_DECODE_TILES_PER_WAVE", "JMA_DECODE_TARGET_BLOCKS", "JMA_UNFUSED"):
            monkeypatch.delenv(key, raising=False)
        for key, value in env.items():
            monkeypatch.setenv(key, value)
        lib = A.HipAttentionLibrary(0)
        try:
            rope = lib.rotary_table(d, theta, 1.0, max_positions=2051)
            kv = lib.kv_cache(1, 2051, hkv, d, d, half_precision=True, sequences=B)
            layer = A.AttentionLayer(0, hq, neox=neox, rope=rope)
            for s, L in enumerate(lens):
                kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32),
                          normal(13, f"fs/k{s}", (L, hkv * d)), normal(13, f"fs/v{s}", (L, hkv * d)),
                          sequences=np.full(L, s))
            for step in range(3):
                p = [L + step for L in lens]
                outs.append(kv.decode(layer, p, normal(13, f"fs/q{step}", (B, hq * d)),
                                      normal(13, f"fs/kn{step}", (B, hkv * d)),
                                      normal(13, f"fs/vn{step}", (B, hkv * d)),
                                      sequences=np.arange(B)))
            rows.append([kv.read(0, L, L + 3, sequence=s) for s, L in enumerate(lens)])
            kv.close()
            rope.close()
        finally:
            lib.close()
    for variant in (1, 2):
        for step in range(3):
            np.testing.assert_allclose(outs[3 * variant + step], outs[step], rtol=2e-6, atol=2e-7)
        for s in range(B):
            np.testing.assert_array_equal(rows[variant][s][0], rows[0][s][0])
            np.testing.assert_array_equal(rows[variant][s][1], rows[0][s][1])


@pytest.mark.parametrize("half,d", [(True, 256), (True, 128), (False, 128)])
def test_wide_split_decode_matches_oracle(hip, half, d):
    """Few long rows (MQA, one KV head, contexts up to 16384): the 32-split cap of the fused
    reduction would leave most CUs idle, so the plan cuts the rows into up to 1024 splits and
    reduce_kernel combines them in a second launch. Ragged rows (one long, one short, one at a
    tile boundary) with the new token appended by the decode kernel, against the oracle's GQA
    over the read-back cache."""
    hq, hkv, theta = 4, 1, 1e6
    scale = A.default_scale(d)
    lens = [16383 if half else 8191, 300, 4096]
    B = len(lens)
    rope = hip.rotary_table(d, theta, 1.0, max_positions=max(lens) + 1)
    kv = hip.kv_cache(1, max(lens) + 1, hkv, d, d, half_precision=half, sequences=B)
    close = assert_f16_close if half else assert_f32_close
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        for s_, L in enumerate(lens):
            kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32),
                      normal(15, f"wide/k{s_}", (L, hkv * d)), normal(15, f"wide/v{s_}", (L, hkv * d)),
                      sequences=np.full(L, s_))
        qn = normal(15, "wide/qn", (B, hq * d))
        kn = normal(15, "wide/kn", (B, hkv * d))
        vn = normal(15, "wide/vn", (B, hkv * d))
        got = kv.decode(layer, lens, qn, kn, vn, sequences=np.arange(B)).reshape(B, -1)
        for s_, L in enumerate(lens):
            keys, values = kv.read(0, 0, L + 1, sequence=s_)
            q_rot = rope_rows(qn[s_:s_ + 1], [L], hq, d, d, theta, True, check_against_oracle=False)
            want = oracle.gqa_rows(q_rot[0], keys, values, hq, hkv, d, d, scale)
            err = close(got[s_], want, f"wide split d {d} session {s_} (L={L})", head_dim=d)
            _say(f"wide split half={half} d={d} L={L} err {err:.2e}")
    finally:
        kv.close()
        rope.close()


REDUCE_SHAPE_CASES = {
    # name: (query heads, row length, minimum tiles per split, workgroup target); one f16 row of
    # head dim 128 on one KV head, planned wide so that reduce_kernel combines its splits
    "64 splits: one-wave workgroups": (4, 8191, "4", None),
    "128 splits: four-wave workgroups": (4, 8191, "2", None),
    "256 splits: four-wave workgroups": (4, 8191, "1", None),
    "512 splits: sixteen-wave workgroups": (4, 16383, "1", None),
    "64 query heads, 64 splits: 64-output workgroups": (64, 8191, "4", "4096"),
}


@pytest.mark.parametrize("case", list(REDUCE_SHAPE_CASES))
def test_reduce_workgroup_shapes_match_oracle(monkeypatch, case):
    """reduce_kernel's workgroup shapes, each chosen by the split count and the output count of a
    wide plan: one wave for up to 64 splits, four for up to 256 and sixteen beyond (16 outputs per
    workgroup), or 64 outputs per workgroup when there are enough of them. The split size is
    forced through JMA_DECODE_MIN_SPLIT_TILES; the result is checked against the oracle's GQA over
    the read-back cache, and a repeated call must give the same bits."""
    d, hkv, theta = 128, 1, 1e6
    scale = A.default_scale(d)
    hq, L, tiles, target = REDUCE_SHAPE_CASES[case]
    monkeypatch.setenv("JMA_DECODE_MIN_SPLIT_TILES", tiles)
    if target:
        monkeypatch.setenv("JMA_DECODE_TARGET_BLOCKS", target)
    lib = A.HipAttentionLibrary(0)
    try:
        rope = lib.rotary_table(d, theta, 1.0, max_positions=L + 1)
        kv = lib.kv_cache(1, L + 1, hkv, d, d, half_precision=True)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        tag = f"rshape/{case}"
        kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32),
                  normal(19, f"{tag}/k", (L, hkv * d)), normal(19, f"{tag}/v", (L, hkv * d)))
        qn = normal(19, f"{tag}/qn", (1, hq * d))
        kn = normal(19, f"{tag}/kn", (1, hkv * d))
        vn = normal(19, f"{tag}/vn", (1, hkv * d))
        got = kv.decode(layer, [L], qn, kn, vn).reshape(1, -1)
        again = kv.decode(layer, [L], qn, kn, vn).reshape(1, -1)
        np.testing.assert_array_equal(again, got)  # deterministic, the same row rewritten
        keys, values = kv.read(0, 0, L + 1)
        q_rot = rope_rows(qn, [L], hq, d, d, theta, True, check_against_oracle=False)
        want = oracle.gqa_rows(q_rot[0], keys, values, hq, hkv, d, d, scale)
        err = assert_f16_close(got[0], want, f"reduce shape {case}", head_dim=d)
        _say(f"reduce shape {case} err {err:.2e}")
        kv.close()
        rope.close()
    finally:
        lib.close()


D512_SLICED_CASES = {
    # name: (query heads, row lengths, workgroup target); the plan each gets (tests/plan_check.cpp
    # prints them) follows the name
    "one row @4096: wide, 4 slices": (8, [4096], None),
    "one row @16000: wide, unsliced": (8, [16000], None),
    "three ragged rows, two head groups, target 8192: wide, 4 slices": (20, [9000, 5000, 7000], "8192"),
    "three ragged rows, two head groups: fused, unsliced": (20, [9000, 5000, 7000], None),
}


@pytest.mark.parametrize("half", [True, False])
@pytest.mark.parametrize("case", list(D512_SLICED_CASES))
def test_wide_sliced_d512_decode_matches_oracle(monkeypatch, half, case):
    """Head dim 512 plans with and without column slices: four workgroups per (head group,
    split) in short plans, each forming all of q.K and its share of the V columns, none in long
    ones (where four would exceed the workgroup target). Wide plans write the slices' columns
    into one part_acc item that reduce_kernel combines; fused plans reduce each slice through the
    split exchange.
    One row (8 Q / 1 KV heads: the uniform, single-group instance) and three ragged rows of
    20 Q / 1 KV heads (two head groups, unequal split counts, row starts in virtual items: the
    listed-rows instance); the new token appended by the decode kernel; against the oracle over
    the read-back cache."""
    d, hkv, theta = 512, 1, 1e6
    scale = A.default_scale(d)
    hq, lens, target = D512_SLICED_CASES[case]
    if target:
        monkeypatch.setenv("JMA_DECODE_TARGET_BLOCKS", target)
    B = len(lens)
    lib = A.HipAttentionLibrary(0)
    close = assert_f16_close if half else assert_f32_close
    try:
        rope = lib.rotary_table(d, theta, 1.0, max_positions=max(lens) + 1)
        kv = lib.kv_cache(1, max(lens) + 1, hkv, d, d, half_precision=half, sequences=B)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        tag = f"wsl/{int(half)}/{case}"
        for s_, L in enumerate(lens):
            kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32),
                      normal(18, f"{tag}/k{s_}", (L, hkv * d)), normal(18, f"{tag}/v{s_}", (L, hkv * d)),
                      sequences=np.full(L, s_))
        qn = normal(18, f"{tag}/qn", (B, hq * d))
        kn = normal(18, f"{tag}/kn", (B, hkv * d))
        vn = normal(18, f"{tag}/vn", (B, hkv * d))
        got = kv.decode(layer, lens, qn, kn, vn, sequences=np.arange(B)).reshape(B, -1)
        again = kv.decode(layer, lens, qn, kn, vn, sequences=np.arange(B)).reshape(B, -1)
        np.testing.assert_array_equal(again, got)  # deterministic, the same row rewritten
        for s_, L in enumerate(lens):
            keys, values = kv.read(0, 0, L + 1, sequence=s_)
            q_rot = rope_rows(qn[s_:s_ + 1], [L], hq, d, d, theta, True, check_against_oracle=False)
            want = oracle.gqa_rows(q_rot[0], keys, values, hq, hkv, d, d, scale)
            err = close(got[s_], want, f"sliced wide d 512 {case} session {s_} (L={L})", head_dim=d)
            _say(f"sliced wide d512 half={half} {case} L={L} err {err:.2e}")
        kv.close()
        rope.close()
    finally:
        lib.close()


def test_wide_split_on_a_ring_layer_matches_oracle(hip):
    """A wide plan on a RING layer (LayeredKvCache retention, capacity 16384, window 12000) at a
    position past the first wrap (20000): the 375 visible tiles are cut into wide splits whose
    slots wrap inside the ring; against the oracle's GQA over the window read back from the
    ring, and the stored row bit-exact."""
    hq, hkv, d, theta, cap, w, p = 4, 1, 128, 1e6, 16384, 12000, 20000
    scale = A.default_scale(d)
    rope = hip.rotary_table(d, theta, 1.0, max_positions=p + 1)
    kv = hip.kv_cache(1, p + 1, hkv, d, d, half_precision=True, ring_capacity=[cap])
    try:
        layer = A.AttentionLayer(0, hq, sliding_window=w, neox=True, rope=rope)
        chunk = cap - w
        for start in range(0, p, chunk):
            stop = min(p, start + chunk)
            kv.append(layer, np.arange(start, stop), np.zeros((stop - start, hq * d), np.float32),
                      normal(17, f"wring/k{start}", (stop - start, hkv * d)),
                      normal(17, f"wring/v{start}", (stop - start, hkv * d)))
        qn = normal(17, "wring/qn", (1, hq * d))
        kn = normal(17, "wring/kn", (1, hkv * d))
        vn = normal(17, "wring/vn", (1, hkv * d))
        got = kv.decode(layer, [p], qn, kn, vn).reshape(-1)
        first = p - w + 1
        keys, values = kv.read(0, first, p + 1)
        k_new = oracle.f16_round(rope_rows(kn, [p], hkv, d, d, theta, True, check_against_oracle=False))
        np.testing.assert_array_equal(keys.reshape(w, -1)[-1], k_new[0])
        q_rot = rope_rows(qn, [p], hq, d, d, theta, True, check_against_oracle=False)
        want = oracle.gqa_rows(q_rot[0], keys, values, hq, hkv, d, d, scale)
        err = assert_f16_close(got, want, "wide split on a ring layer", head_dim=d)
        _say(f"wide split ring err {err:.2e}")
    finally:
        kv.close()
        rope.close()


def test_graph_replays_match_eager_decode(hip):
    """Per-token HIP graphs of decode_device (as the benchmark replays them): every replay, with
    eager work and synchronizations in between, reproduces the eager outputs exactly."""
    from models_amd import hip_runtime as rt
    hq, hkv, d, prior, steps, layers = 16, 4, 64, 300, 4, 2
    n = prior + steps
    rope = hip.rotary_table(d, 5e5, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True)
    qd, kd = hq * d, hkv * d
    dq = rt.DeviceArray.from_host(normal(14, "g/q", (layers, n, qd)))
    dk = rt.DeviceArray.from_host(normal(14, "g/k", (layers, n, kd)))
    dv = rt.DeviceArray.from_host(normal(14, "g/v", (layers, n, kd)))
    dout = rt.DeviceArray(layers * n * qd)
    stream = hip.stream()
    try:
        lp = [A.AttentionLayer(l, hq, rope=rope) for l in range(layers)]
        for l in range(layers):
            kv.append_device(lp[l], np.zeros(prior, np.uint32), np.arange(prior),
                             dq.at(l * n * qd), prior * qd, dk.at(l * n * kd), prior * kd,
                             dv.at(l * n * kd), prior * kd)

        def token(s):
            p = prior + s
            for l in range(layers):
                kv.decode_device(lp[l], [0], [p], dq.at((l * n + p) * qd), qd,
                                 dk.at((l * n + p) * kd), kd, dv.at((l * n + p) * kd), kd,
                                 dout.at((l * n + p) * qd), qd)

        dout.zero()
        for s in range(steps):
            token(s)
        hip.synchronize()
        eager = dout.download().reshape(layers, n, qd)[:, prior:]
        assert np.all(np.isfinite(eager)) and np.any(eager)
        kv.discard_from(prior)
        graphs = [rt.Graph(stream, lambda s=s: token(s)) for s in range(steps)]
        kv.discard_from(prior)
        try:
            for replay in range(3):
                dout.zero()
                for s in range(steps):
                    graphs[s].launch()
                hip.synchronize()
                got = dout.download().reshape(layers, n, qd)[:, prior:]
                np.testing.assert_array_equal(got, eager, err_msg=f"replay {replay}")
                kv.discard_from(prior)
                # eager work between replays
                kv.attend(lp[0], [prior - 1], normal(14, "g/x", (qd,)))
        finally:
            for g in graphs:
                g.destroy()
    finally:
        for b in (dq, dk, dv, dout):
            b.free()
        kv.close()
        rope.close()


def test_scratch_growth_and_graph_capture(hip):
    """Scratch memory and graph capture. (1) In a fresh context, the first wide-plan decode
    (one long MQA row: partials for up to 1024 splits) issued while the context stream is being
    captured is refused with NOT_CAPTURABLE, enqueues nothing and records no position; the same
    call then runs eagerly, and a graph captured after it replays the eager result exactly.
    (2) A graph captured with the scratch of a short-context plan still replays its own eager
    result after a longer-context call has grown that scratch (the outgrown buffer stays alive)."""
    import ctypes
    from models_amd import hip_runtime as rt
    lib = A.HipAttentionLibrary(0)
    bufs, graphs = [], []
    try:
        stream = lib.stream()
        h = rt.hip()
        # (1) wide plan: 1 KV head, 8191 cached positions
        hq, hkv, d, L = 4, 1, 128, 8191
        rope = lib.rotary_table(d, 1e6, 1.0, max_positions=L + 1)
        kv = lib.kv_cache(1, L + 1, hkv, d, d, half_precision=True)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        kv.append(layer, np.arange(L), np.zeros((L, hq * d), np.float32),
                  normal(31, "cap/k", (L, hkv * d)), normal(31, "cap/v", (L, hkv * d)))
        dq = rt.DeviceArray.from_host(normal(31, "cap/q", (hq * d,)))
        dk = rt.DeviceArray.from_host(normal(31, "cap/kn", (hkv * d,)))
        dv = rt.DeviceArray.from_host(normal(31, "cap/vn", (hkv * d,)))
        dout = rt.DeviceArray(hq * d)
        bufs += [dq, dk, dv, dout]

        def call():
            kv.decode_device(layer, [0], [L], dq.ptr, hq * d, dk.ptr, hkv * d, dv.ptr, hkv * d,
                             dout.ptr, hq * d)

        rt.check(h.hipStreamBeginCapture(stream, rt.Graph.RELAXED), "hipStreamBeginCapture")
        try:
            with pytest.raises(A.AttentionStatusError) as e:
                call()
        finally:
            g = ctypes.c_void_p()
            rt.check(h.hipStreamEndCapture(stream, ctypes.byref(g)), "hipStreamEndCapture")
            h.hipGraphDestroy(g)
        assert e.value.status == A.NOT_CAPTURABLE, e.value
        assert not kv.contains(0, L)
        dout.zero()
        call()
        lib.synchronize()
        eager = dout.download()
        assert np.all(np.isfinite(eager)) and np.any(eager)
        kv.discard_from(L)
        graphs.append(rt.Graph(stream, call))
        kv.discard_from(L)
        for replay in range(3):
            dout.zero()
            graphs[-1].launch()
            lib.synchronize()
            np.testing.assert_array_equal(dout.download(), eager, err_msg=f"wide replay {replay}")
        kv.close()
        rope.close()

        # (2) fused split exchange: 8 KV heads, a short row then a long one in another session
        hq, hkv, d = 8, 8, 128
        lens = [1000, 8000]
        rope = lib.rotary_table(d, 1e6, 1.0, max_positions=max(lens) + 1)
        kv = lib.kv_cache(1, max(lens) + 1, hkv, d, d, half_precision=True, sequences=2)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        for s, n in enumerate(lens):
            kv.append(layer, np.arange(n), np.zeros((n, hq * d), np.float32),
                      normal(32, f"grow/k{s}", (n, hkv * d)), normal(32, f"grow/v{s}", (n, hkv * d)),
                      sequences=np.full(n, s))
        ins = [[rt.DeviceArray.from_host(normal(32, f"grow/{t}{s}", (hq * d if t == "q" else hkv * d,)))
                for t in "qkv"] for s in range(2)]
        outs = [rt.DeviceArray(hq * d) for _ in range(2)]
        bufs += [b for row in ins for b in row] + outs

        def call_s(s):
            q, k, v = ins[s]
            kv.decode_device(layer, [s], [lens[s]], q.ptr, hq * d, k.ptr, hkv * d, v.ptr, hkv * d,
                             outs[s].ptr, hq * d)

        call_s(0)
        lib.synchronize()
        eager0 = outs[0].download()
        kv.discard_from(lens[0], sequence=0)
        graphs.append(rt.Graph(stream, lambda: call_s(0)))
        kv.discard_from(lens[0], sequence=0)
        call_s(1)  # a wider plan: the exchange scratch grows here
        lib.synchronize()
        assert np.all(np.isfinite(outs[1].download()))
        for replay in range(3):
            outs[0].zero()
            graphs[-1].launch()
            lib.synchronize()
            np.testing.assert_array_equal(outs[0].download(), eager0, err_msg=f"replay {replay}")
        kv.close()
        rope.close()
    finally:
        for g in graphs:
            g.destroy()
        for b in bufs:
            b.free()
        lib.close()

"""The allocation-free decode entry point (jmodels_attn_decode_device_noalloc) against
jmodels_attn_decode_device, through the C ABI: the same launches on the GPU's fixed scratch, so
outputs and appended cache rows must be bit-identical, on consecutive calls whose second is
smaller, on the fused split exchange, the wide plan with the separate reduction and the
separate-kernel path; a plan larger than the fixed scratch is refused before anything runs."""

import numpy as np
import pytest

from gpu_support import assert_f16_close, normal, rope_rows
from models_amd import attention as A
from models_amd import hip_runtime as rt
from oracle import oracle

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _two_caches(lib, layer_of, hkv, d, lens, cap, seed, ring=None):
    caches = []
    for _ in range(2):
        kv = lib.kv_cache(1, cap, hkv, d, d, half_precision=True, sequences=len(lens),
                          ring_capacity=ring)
        layer = layer_of()
        for s, n in enumerate(lens):
            kv.append(layer, np.arange(n), np.zeros((n, layer.num_heads * d), np.float32),
                      normal(seed, f"na/k{s}", (n, hkv * d)), normal(seed, f"na/v{s}", (n, hkv * d)),
                      sequences=np.full(n, s))
        caches.append(kv)
    return caches


def _decode_both(lib, caches, layer, hq, hkv, d, sessions, positions, seed, tag):
    """decode_device on caches[0], decode_device_noalloc on caches[1], same device inputs."""
    B = len(sessions)
    q = normal(seed, f"na/q{tag}", (B, hq * d))
    k = normal(seed, f"na/kn{tag}", (B, hkv * d))
    v = normal(seed, f"na/vn{tag}", (B, hkv * d))
    dq, dk, dv = (rt.DeviceArray.from_host(x) for x in (q, k, v))
    outs = [rt.DeviceArray(B * hq * d) for _ in range(2)]
    try:
        args = (dq.ptr, B * hq * d, dk.ptr, B * hkv * d, dv.ptr, B * hkv * d)
        caches[0].decode_device(layer, sessions, positions, *args, outs[0].ptr, B * hq * d)
        caches[1].decode_device_noalloc(layer, sessions, positions, *args, outs[1].ptr, B * hq * d)
        lib.synchronize()
        got = [o.download().reshape(B, -1) for o in outs]
    finally:
        for b in (dq, dk, dv, *outs):
            b.free()
    np.testing.assert_array_equal(got[1], got[0], err_msg=f"call {tag}")
    for s, p in zip(sessions, positions):
        a = caches[0].read(layer.layer, p, p + 1, sequence=s)
        b = caches[1].read(layer.layer, p, p + 1, sequence=s)
        np.testing.assert_array_equal(b[0], a[0])
        np.testing.assert_array_equal(b[1], a[1])
    return got[1], q


def test_noalloc_decode_matches_decode_device():
    lib = A.HipAttentionLibrary(0)
    try:
        # Fused split exchange: ragged sessions, 16 Q / 4 KV heads, d 128; two calls in a row,
        # the second with fewer sessions and shorter rows.
        hq, hkv, d, theta = 16, 4, 128, 1e6
        lens = [3000, 700, 1500, 4095]
        cap = max(lens) + 2
        rope = lib.rotary_table(d, theta, 1.0, max_positions=cap)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        caches = _two_caches(lib, lambda: layer, hkv, d, lens, cap, 41)
        try:
            got, q = _decode_both(lib, caches, layer, hq, hkv, d, [0, 1, 2, 3], lens, 41, "a")
            q_rot = rope_rows(q, lens, hq, d, d, theta, True)
            for s, L in enumerate(lens):
                keys, values = caches[1].read(0, 0, L + 1, sequence=s)
                want = oracle.gqa_rows(q_rot[s], keys, values, hq, hkv, d, d, A.default_scale(d))
                assert_f16_close(got[s], want, f"noalloc session {s}", head_dim=d)
            _decode_both(lib, caches, layer, hq, hkv, d, [1, 2], [lens[1] + 1, lens[2] + 1], 41, "b")
            _say("fused split exchange: identical on two calls")
        finally:
            for kv in caches:
                kv.close()
            rope.close()

        # Wide plan (one KV head, a long row): partials combined by the separate reduction.
        hq, hkv, d = 4, 1, 256
        lens = [12000]
        cap = lens[0] + 2
        rope = lib.rotary_table(d, theta, 1.0, max_positions=cap)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        caches = _two_caches(lib, lambda: layer, hkv, d, lens, cap, 42)
        try:
            _decode_both(lib, caches, layer, hq, hkv, d, [0], lens, 42, "w1")
            _decode_both(lib, caches, layer, hq, hkv, d, [0], [lens[0] + 1], 42, "w2")
            _say("wide plan: identical on two calls")
        finally:
            for kv in caches:
                kv.close()
            rope.close()

        # Separate-kernel path (10 rotary pairs: not a multiple of 8), rotated queries in the
        # fixed scratch.
        hq, hkv, d = 8, 2, 64
        lens = [900, 2000]
        cap = max(lens) + 2
        rope = lib.rotary_table(20, theta, 1.0, max_positions=cap)
        layer = A.AttentionLayer(0, hq, neox=False, rope=rope)
        caches = _two_caches(lib, lambda: layer, hkv, d, lens, cap, 43)
        try:
            _decode_both(lib, caches, layer, hq, hkv, d, [0, 1], lens, 43, "u1")
            _decode_both(lib, caches, layer, hq, hkv, d, [0], [lens[0] + 1], 43, "u2")
            _say("separate kernels: identical on two calls")
        finally:
            for kv in caches:
                kv.close()
            rope.close()
    finally:
        lib.close()


def test_noalloc_refuses_plans_beyond_the_fixed_scratch(monkeypatch):
    """128 sessions x 8 KV heads x 5 splits (a 100000-workgroup target keeps splits at 4 tiles) of
    4 query heads x 256 elements need tens of MB of split partials, beyond the fixed scratch:
    refused, nothing enqueued or recorded; decode_device itself grows its scratch and runs the
    same call."""
    monkeypatch.setenv("JMA_DECODE_TARGET_BLOCKS", "100000")
    lib = A.HipAttentionLibrary(0)
    try:
        hq, hkv, d, B, n = 32, 8, 256, 128, 544
        rope = lib.rotary_table(d, 1e4, 1.0, max_positions=n + 1)
        kv = lib.kv_cache(1, n + 1, hkv, d, d, half_precision=True, sequences=B)
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        zq = rt.DeviceArray(n * hq * d)
        zq.zero()
        dk = rt.DeviceArray.from_host(normal(44, "big/k", (n, hkv * d)))
        dv = rt.DeviceArray.from_host(normal(44, "big/v", (n, hkv * d)))
        dq = rt.DeviceArray.from_host(normal(44, "big/q", (B, hq * d)))
        dkn = rt.DeviceArray.from_host(normal(44, "big/kn", (B, hkv * d)))
        dvn = rt.DeviceArray.from_host(normal(44, "big/vn", (B, hkv * d)))
        dout = rt.DeviceArray(B * hq * d)
        try:
            for s in range(B):
                kv.append_device(layer, np.full(n, s, np.uint32), np.arange(n), zq.ptr, n * hq * d,
                                 dk.ptr, n * hkv * d, dv.ptr, n * hkv * d)
            lib.synchronize()
            args = ([*range(B)], [n] * B, dq.ptr, B * hq * d, dkn.ptr, B * hkv * d, dvn.ptr,
                    B * hkv * d, dout.ptr, B * hq * d)
            with pytest.raises(A.AttentionStatusError) as e:
                kv.decode_device_noalloc(layer, *args)
            assert e.value.status == A.BUFFER_TOO_SMALL, e.value
            assert not kv.contains(0, n, sequence=0)
            kv.decode_device(layer, *args)
            lib.synchronize()
            assert kv.contains(0, n, sequence=B - 1)
            assert np.all(np.isfinite(dout.download()))
        finally:
            for b in (zq, dk, dv, dq, dkn, dvn, dout):
                b.free()
            kv.close()
            rope.close()
    finally:
        lib.close()


def test_noalloc_refusal_enqueues_nothing_on_any_path(monkeypatch):
    """The fixed-scratch check covers every launch of a call before the first one is enqueued:
    (a) on the separate-kernel path (10 rotary pairs, not a multiple of 8), whose append would
    otherwise run before the attention launch is planned; (b) on the fused path with 256
    sessions, two launches of 128 rows, where only the second launch (long rows) exceeds the
    fixed scratch. Either call is refused with BUFFER_TOO_SMALL and no new row is appended or
    marked; decode_device then runs the same call."""
    monkeypatch.setenv("JMA_DECODE_TARGET_BLOCKS", "100000")
    lib = A.HipAttentionLibrary(0)
    hq, hkv, d, n = 32, 8, 256, 544
    try:
        for case, pairs, B in (("separate kernels", 10, 128), ("second launch", d // 2, 256)):
            rope = lib.rotary_table(2 * pairs, 1e4, 1.0, max_positions=n + 1)
            kv = lib.kv_cache(1, n + 1, hkv, d, d, half_precision=True, sequences=B)
            layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
            # case (b): sessions 0..127 hold 10 rows (one tile, no split), 128..255 hold n - 1
            lens = [n - 1] * B if B == 128 else [10] * 128 + [n - 1] * 128
            zq = rt.DeviceArray(n * hq * d)
            zq.zero()
            dk = rt.DeviceArray.from_host(normal(45, "ref/k", (n, hkv * d)))
            dv = rt.DeviceArray.from_host(normal(45, "ref/v", (n, hkv * d)))
            dq = rt.DeviceArray.from_host(normal(45, "ref/q", (B, hq * d)))
            dkn = rt.DeviceArray.from_host(normal(45, "ref/kn", (B, hkv * d)))
            dvn = rt.DeviceArray.from_host(normal(45, "ref/vn", (B, hkv * d)))
            dout = rt.DeviceArray(B * hq * d)
            try:
                for s, L in enumerate(lens):
                    kv.append_device(layer, np.full(L, s, np.uint32), np.arange(L), zq.ptr,
                                     L * hq * d, dk.ptr, L * hkv * d, dv.ptr, L * hkv * d)
                lib.synchronize()
                args = ([*range(B)], lens, dq.ptr, B * hq * d, dkn.ptr, B * hkv * d, dvn.ptr,
                        B * hkv * d, dout.ptr, B * hq * d)
                with pytest.raises(A.AttentionStatusError) as e:
                    kv.decode_device_noalloc(layer, *args)
                assert e.value.status == A.BUFFER_TOO_SMALL, (case, e.value)
                lib.synchronize()
                for s in (0, B // 2, B - 1):
                    assert not kv.contains(0, lens[s], sequence=s), (case, s)
                kv.decode_device(layer, *args)
                lib.synchronize()
                assert all(kv.contains(0, lens[s], sequence=s) for s in (0, B // 2, B - 1))
                assert np.all(np.isfinite(dout.download()))
                _say(f"{case}: refused before anything ran")
            finally:
                for b in (zq, dk, dv, dq, dkn, dvn, dout):
                    b.free()
                kv.close()
                rope.close()
    finally:
        lib.close()

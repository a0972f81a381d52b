"""GPU parity of the per-layer (LayeredKvCache) device cache: layers with their own KV-head counts,
head lengths and retention in one cache, as Gemma4KvCache builds them
(backend-java gemma4/Gemma4KvCache.java:39-47; cache/LayeredKvCache.java:41-64, 124-156).

Bars: stored rows, retention (contains) and range errors are exact; attention outputs are within
max-abs 1e-3 with f32 KV and normwise relative 2e-2 per (row, head) with f16 KV."""

import ctypes
import sys

import numpy as np
import pytest

from gpu_support import assert_f16_close, assert_f32_close, normal
from models_amd import attention as A
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


# ------------------------------------------------------------------ LayeredKvCacheTest replay

def _device_spec(key_dim, value_dim, ring):
    """A device layer for one of the reference's LayerSpecs. Small widths become one 16-wide head
    (the device's smallest head length), zero padded. Gemma-4 widths keep their head split:
    sliding layers 256-long heads, full layers 512-long heads
    (backend-java gemma4/Gemma4ConfigTest.java:114-117)."""
    if key_dim >= 256:
        length = 256 if ring else 512
        return A.LayerSpec(key_dim // length, length, length, ring)
    return A.LayerSpec(1, 16, 16, ring)


def _pad16(vec):
    out = np.zeros(16, np.float32)
    out[:len(vec)] = vec
    return out


def test_layered_kv_cache_known_answers_on_device(hip, known_answers):
    """Replays backend-java's LayeredKvCacheTest cases (cache/LayeredKvCacheTest.java:28-147, in
    tests/golden) on the device cache built by jmodels_attn_kv_create_layered, with every width
    padded to one 16-wide head. Ring capacities 4, 5, 6 and 8 are not multiples of the device's
    32-row tile: retention follows the logical capacity while the storage is rounded up.

    Checked exactly: contains, oldest/newest retained position (the extremes of contains), the
    rows a view reads (values, in position order), the rows a buffer holds, view and store errors
    (IllegalStateException for overwritten positions -> UNAVAILABLE, IllegalArgumentException for
    ranges wider than the ring, positions past maxSeqLen and layers out of range -> OUT_OF_RANGE,
    short vectors -> BUFFER_TOO_SMALL), and the Gemma-4 cases' maximumBytes: the device holds
    exactly the reference's float storage (without its per-slot int positions, kept on the host).
    Not observable on the device and not checked: the reference's lazily grown host arrays
    (allocatedCapacity, allocatedBytes) and offsets into them (keyOffset, valueOffset)."""
    for case in known_answers["layered_kv_cache"]:
        _say(f"layered case {case['name']}")
        max_seq, ref_specs = case["ctor"]
        specs = [_device_spec(kd, vd, r) for kd, vd, r in ref_specs]
        kv = hip.layered_kv_cache(specs, max_seq, half_precision=False)
        stored = {}
        try:
            def run(ops):
                for op in ops:
                    if op[0] == "store":
                        _, l, p, k, v = op
                        kv.store(l, p, _pad16(k), _pad16(v))
                        stored[(l, p)] = (np.float32(k), np.float32(v))
                    elif op[0] == "clear":
                        kv.clear()
                        stored.clear()
                    elif op[0] == "discard":
                        kv.discard_from(op[1])
                        for key in [key for key in stored if key[1] >= op[1]]:
                            del stored[key]
                    else:
                        raise AssertionError(op)

            def retained(l):
                return [p for p in range(max_seq) if kv.contains(l, p)]

            def check_rows(l, frm, to):
                keys, values = kv.read(l, frm, to)
                keys, values = keys.reshape(to - frm, 16), values.reshape(to - frm, 16)
                kd, vd = ref_specs[l][0], ref_specs[l][1]
                for i, p in enumerate(range(frm, to)):
                    k, v = stored[(l, p)]
                    np.testing.assert_array_equal(keys[i, :kd], k)
                    np.testing.assert_array_equal(values[i, :vd], v)
                    assert not keys[i, kd:].any() and not values[i, vd:].any()

            def buffer_rows(l, values):
                width = ref_specs[l][1 if values else 0]
                return [tuple(kv.read(l, p, p + 1)[1 if values else 0][:width])
                        for p in retained(l)]

            def check(exps):
                for e in exps:
                    kind = e[0]
                    if kind == "contains":
                        assert kv.contains(e[1], e[2]) == e[3], e
                    elif kind in ("oldest", "newest"):
                        held = retained(e[1])
                        got = (held[0] if kind == "oldest" else held[-1]) if held else None
                        assert got == e[2], (e, got)
                    elif kind in ("view", "viewCount"):
                        check_rows(e[1], e[2], e[3])
                        if kind == "viewCount":
                            assert e[3] - e[2] == e[4], e
                    elif kind == "viewError":
                        with pytest.raises(A.AttentionStatusError) as info:
                            kv.read(e[1], e[2], e[3])
                        want = A.UNAVAILABLE if e[4] == "ISE" else A.OUT_OF_RANGE
                        assert info.value.status == want, (e, info.value.status)
                    elif kind == "storeError":
                        _, l, p, k, v, _err = e
                        kd = ref_specs[l][0] if l < len(ref_specs) else len(k)
                        vd = ref_specs[l][1] if l < len(ref_specs) else len(v)
                        kp, vp = _pad16(k), _pad16(v)
                        # the reference's own vector lengths: a short one is too small
                        kn = 16 if len(k) >= kd else len(k)
                        vn = 16 if len(v) >= vd else len(v)
                        st = hip.lib.jmodels_attn_kv_store(hip.ctx, kv.handle, 0, l, p,
                                                           A._ptr(kp), kn, A._ptr(vp), vn)
                        want = (A.BUFFER_TOO_SMALL if (kn < 16 or vn < 16)
                                and l < len(ref_specs) and p < max_seq else A.OUT_OF_RANGE)
                        assert st == want, (e, st)
                    elif kind in ("keyBuffer", "valueBuffer"):
                        values = kind == "valueBuffer"
                        width = ref_specs[e[1]][1 if values else 0]
                        want = np.float32(e[2]).reshape(-1, width)
                        assert sorted(buffer_rows(e[1], values)) == sorted(map(tuple, want)), e
                    elif kind in ("keyBufferContains", "valueBufferContains"):
                        rows = buffer_rows(e[1], kind == "valueBufferContains")
                        assert tuple(np.float32(e[2])) in rows, e
                    elif kind == "maximumBytes":
                        slots = sum(min(sp.ring_capacity, max_seq) if sp.ring_capacity
                                    else max_seq for sp in specs)
                        assert kv.device_bytes() == e[1] - 4 * slots, (e, kv.device_bytes())
                    elif kind == "physicalCapacity":
                        # the device stores ring rows at min(ring, maxSeqLen), linearly when the
                        # ring is at least as long as the context; every layer of these cases is
                        # a multiple of 32 rows, so the bytes below pin it
                        sp = specs[e[1]]
                        cap = min(sp.ring_capacity, max_seq) if sp.ring_capacity else max_seq
                        assert cap == e[2], (e, cap)
                    elif kind in ("allocatedCapacity", "allocatedCapacityAtLeast", "keyOffset",
                                  "valueOffset", "allocatedBytes"):
                        pass  # the reference's host array layout, see the docstring
                    else:
                        raise AssertionError(e)
                if any(e[0] == "physicalCapacity" for e in exps):
                    want = sum((min(s.ring_capacity, max_seq) if s.ring_capacity else max_seq)
                               * (s.key_dim + s.value_dim) * 4 for s in specs)
                    assert kv.device_bytes() == want, (kv.device_bytes(), want)

            check(case.get("expect_before", []))
            run(case["ops"])
            check(case["expect"])
            for ops, exps in (("then_ops", "then_expect"), ("final_ops", "final_expect")):
                if ops in case:
                    run(case[ops])
                    check(case[exps])
        finally:
            kv.close()


def test_layered_cache_rejects_bad_specs(hip):
    """Each layer's shape is validated on its own: a zero head count, a head length that is not a
    multiple of 16, or a null spec array fail before anything is allocated."""
    for bad in (A.LayerSpec(0, 64, 64), A.LayerSpec(2, 40, 64), A.LayerSpec(2, 64, 8)):
        with pytest.raises(A.AttentionStatusError) as info:
            hip.layered_kv_cache([A.LayerSpec(2, 64, 64), bad], 128)
        assert info.value.status == A.INVALID_SHAPE, bad
    out = ctypes.c_void_p()
    st = hip.lib.jmodels_attn_kv_create_layered(hip.ctx, 1, 2, 128, None, A.KV_F16, ctypes.byref(out))
    assert st == A.NULL_POINTER
    # a layer's own kv-head count decides which query-head counts it accepts, and its own widths
    # what a store needs
    kv = hip.layered_kv_cache([A.LayerSpec(4, 64, 64), A.LayerSpec(2, 64, 64)], 64)
    try:
        q, k, v = np.zeros(6 * 64), np.zeros(2 * 64), np.zeros(2 * 64)
        assert kv.decode(A.AttentionLayer(1, 6), [0], q, k, v).shape == (6 * 64,)
        with pytest.raises(ValueError):
            kv.decode(A.AttentionLayer(0, 6), [0], q, np.zeros(4 * 64), np.zeros(4 * 64))
        short = np.zeros(4 * 64, np.float32)
        st = hip.lib.jmodels_attn_kv_store(hip.ctx, kv.handle, 0, 0, 1, A._ptr(short), 2 * 64,
                                           A._ptr(short), 4 * 64)
        assert st == A.BUFFER_TOO_SMALL  # layer 1's key width is too small for layer 0
        st = hip.lib.jmodels_attn_kv_store(hip.ctx, kv.handle, 0, 1, 1, A._ptr(short), 2 * 64,
                                           A._ptr(short), 2 * 64)
        assert st == A.OK
        assert kv.contains(1, 1) and not kv.contains(0, 1)
    finally:
        kv.close()


# ------------------------------------------------------------------ Gemma-4 shaped attention

@pytest.mark.parametrize("half", [True, False])
def test_gemma4_layered_cache_attention(hip, half):
    """A Gemma-4-shaped cache (Gemma4KvCache.java:39-47; Gemma4ForwardPass.executeLayer,
    gemma4/Gemma4ForwardPass.java:955-1006): a sliding layer of 4 KV heads x 256 with window 256
    and a RING of window + prefill chunk = 356 slots (not a multiple of 32), and a full layer of
    2 KV heads x 512, LINEAR. 8 query heads, q/k RMS-normalised with weights, v heads
    RMS-normalised without one, NeoX RoPE, scale 1.0. Two sessions: session 0 prefills 600 rows
    in chunks of 100, session 1 prefills 250 rows in chunks of 50; then 3 decode steps run both
    sessions in one batched call. Every prefill chunk and decode output is checked against the
    oracle fed the host-normalised q, k, v; the retained K/V rows are the oracle's bit for bit
    and ring retention follows the logical capacity."""
    hq, eps, window, chunk = 8, 1e-6, 256, 100
    layers = [dict(hkv=4, d=256, ring=window + chunk, window=window, theta=1e4),
              dict(hkv=2, d=512, ring=0, window=0, theta=1e6)]
    priors, chunks, steps = [600, 250], [100, 50], 3
    max_seq = 640
    close = assert_f16_close if half else assert_f32_close
    specs = [A.LayerSpec(c["hkv"], c["d"], c["d"], c["ring"]) for c in layers]
    kv = hip.layered_kv_cache(specs, max_seq, half_precision=half, sequences=2)
    ropes, norms = [], []
    try:
        for l, c in enumerate(layers):
            hkv, d, theta, w = c["hkv"], c["d"], c["theta"], c["window"]
            wq = normal(21, f"g4l/wq{l}", (d,)) * 0.2 + 1.0
            wk = normal(21, f"g4l/wk{l}", (d,)) * 0.2 + 1.0
            ropes.append(hip.rotary_table(d, theta, 1.0, max_positions=max_seq))
            norms.append(hip.qk_norm(d, wq, wk, eps, value_rms=True))
            layer = A.AttentionLayer(l, hq, sliding_window=w, neox=True, scale=1.0,
                                     rope=ropes[-1], qk_norm=norms[-1])
            data, refs = [], []
            for s in range(2):
                n = priors[s] + steps
                q = normal(21, f"g4l/q{l}s{s}", (n, hq * d))
                k = normal(21, f"g4l/k{l}s{s}", (n, hkv * d))
                v = normal(21, f"g4l/v{l}s{s}", (n, hkv * d))
                qn = np.stack([oracle.qk_norm_heads(r, hq, d, wq, eps) for r in q])
                kn = np.stack([oracle.qk_norm_heads(r, hkv, d, wk, eps) for r in k])
                vn = np.stack([oracle.value_rms_heads(r, hkv, d, eps) for r in v])
                data.append((q, k, v, qn, kn, vn))
                ref = OracleKv(1, max_seq, hkv * d, hkv * d, half_precision=half)
                refs.append(ref)
                worst = 0.0
                for start in range(0, priors[s], chunks[s]):
                    stop = min(priors[s], start + chunks[s])
                    got = kv.prefill(layer, start, q[start:stop], k[start:stop], v[start:stop],
                                     sequence=s)
                    want, _, _ = ref.prefill_layer(0, start, qn[start:stop], kn[start:stop],
                                                   vn[start:stop], hq, hkv, d, d, theta, 1.0,
                                                   True, 1.0, window=w)
                    worst = max(worst, close(got, want, f"layer {l} session {s} prefill @{start}",
                                             head_dim=d))
                _say(f"Gemma-4 layered half={half} layer {l} (d {d}, {hkv} kv heads) session {s} "
                     f"prefill worst {worst:.2e}")
            for t in range(steps):
                pos = [priors[0] + t, priors[1] + t]
                q = np.concatenate([data[s][0][pos[s]] for s in range(2)])
                k = np.concatenate([data[s][1][pos[s]] for s in range(2)])
                v = np.concatenate([data[s][2][pos[s]] for s in range(2)])
                got = kv.decode(layer, pos, q, k, v, sequences=[0, 1]).reshape(2, hq * d)
                for s in range(2):
                    qn, kn, vn = data[s][3:]
                    want, _, _ = refs[s].decode_layer(0, pos[s], qn[pos[s]], kn[pos[s]],
                                                      vn[pos[s]], hq, hkv, d, d, theta, 1.0, True,
                                                      1.0, window=w)
                    e = close(got[s], want, f"layer {l} session {s} decode step {t}", head_dim=d)
                _say(f"Gemma-4 layered half={half} layer {l} decode step {t} error {e:.2e}")
            for s in range(2):
                n = priors[s] + steps
                lo = max(0, n - c["ring"]) if c["ring"] else 0
                np.testing.assert_array_equal(kv.key_slice(l, lo, n, sequence=s),
                                              refs[s].key_slice(0, lo, n))
                np.testing.assert_array_equal(kv.value_slice(l, lo, n, sequence=s),
                                              refs[s].value_slice(0, lo, n))
                if c["ring"] and lo > 0:
                    assert not kv.contains(l, lo - 1, sequence=s) and kv.contains(l, lo, sequence=s)
                    with pytest.raises(A.AttentionStatusError) as info:
                        kv.read(l, lo - 1, n, sequence=s)
                    assert info.value.status == A.OUT_OF_RANGE  # wider than the ring
    finally:
        kv.close()
        for x in norms + ropes:
            x.close()


@pytest.mark.parametrize("half", [True, False])
def test_gemma4_layered_cache_attention_every_unit_split(monkeypatch, half):
    """The Gemma-4-shaped case above with every prefill row block, stripe and stripe pair of two
    or more kv tiles split into two workgroups (JMA_PREFILL_SPLIT_TILES=2), including the sliding
    layer's ring (the halves' tiles wrap around its 356 slots)."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    try:
        test_gemma4_layered_cache_attention(lib, half)
    finally:
        lib.close()

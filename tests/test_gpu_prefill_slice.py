"""GPU parity of the sliced prefill kernels: prefill_slice_kernel (f32 caches at head dims
32-512) and prefill_pair_kernel (f16 caches at head dim 512: two stripes per workgroup, odd stripe
counts leaving the last pair half empty), against the oracle's prefill (computeBatchedAttention,
backend-java llama/LlamaForwardPass.java:1515-1541) on identical seeded inputs.

Bars: attention outputs within max-abs 1e-3 with f32 KV and normwise relative 2e-2 per (row, head)
with f16 KV; the stored K/V rows bit-exact. The cases cover split stripes and stripe pairs (two
workgroups per stripe over halves of its kv tiles, merged), chunked prefill (a chunk start > 0
attends to cached rows), sliding windows, GQA groups that leave padding columns in a stripe
(group 3: 10 rows x 3 heads of 32 columns), ragged tails, non-finite cache contents at positions a
row does not see, a NaN query (status NON_FINITE), and C1's shape (Qwen3-0.6B, 512 rows, f32)."""

import sys

import numpy as np
import pytest

from gpu_support import assert_f16_close, assert_f32_close, normal, rope_rows
from models_amd import attention as A
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


def _chunked_case(hip, half, d, hq, hkv, n1, n2, window, theta, seed, neox=True):
    """Two prefill chunks (0..n1-1, then n1..n1+n2-1) on the device and in the oracle."""
    scale = A.default_scale(d)
    n = n1 + n2
    cap = (n + 31) // 32 * 32 + 32
    tag = f"psl/{int(half)}/{d}/{seed}"
    q = normal(seed, tag + "q", (n, hq * d))
    k = normal(seed, tag + "k", (n, hkv * d))
    v = normal(seed, tag + "v", (n, hkv * d))
    ref = OracleKv(1, cap, hkv * d, hkv * d, half_precision=half)
    r1, _, _ = ref.prefill_layer(0, 0, q[:n1], k[:n1], v[:n1], hq, hkv, d, d, theta, 1.0, neox,
                                 scale, window=window)
    r2, _, _ = ref.prefill_layer(0, n1, q[n1:], k[n1:], v[n1:], hq, hkv, d, d, theta, 1.0, neox,
                                 scale, window=window)
    close = assert_f16_close if half else assert_f32_close
    rope = hip.rotary_table(d, theta, 1.0, max_positions=cap)
    kv = hip.kv_cache(1, cap, hkv, d, d, half_precision=half)
    try:
        layer = A.AttentionLayer(0, hq, sliding_window=window, neox=neox, rope=rope)
        g1 = kv.prefill(layer, 0, q[:n1], k[:n1], v[:n1])
        g2 = kv.prefill(layer, n1, q[n1:], k[n1:], v[n1:])
        e1 = close(g1, r1, f"half={half} d {d} window {window} chunk 1", head_dim=d)
        e2 = close(g2, r2, f"half={half} d {d} window {window} chunk 2", head_dim=d)
        np.testing.assert_array_equal(kv.key_slice(0, 0, n), ref.key_slice(0, 0, n))
        np.testing.assert_array_equal(kv.value_slice(0, 0, n), ref.value_slice(0, 0, n))
        # the same rows again through attend_causal, with q rotated by the oracle's RoPE (the
        # device's is bit-exact to it): the kernel is deterministic
        q_rot = rope_rows(q[n1:], range(n1, n), hq, d, d, theta, neox)
        np.testing.assert_array_equal(kv.attend_causal(layer, n1, q_rot), g2)
    finally:
        kv.close()
        rope.close()
    return max(e1, e2)


@pytest.mark.parametrize("d", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("window", [0, 100])
def test_f32_prefill_matches_oracle(hip, d, window):
    """f32 caches at every head dim the kernel takes (1, 2, 4, 4 and 8 waves of 32- or 64-dim
    slices), group 3 (padding columns in each stripe), chunk start 70, ragged stripe tails."""
    n2 = 229 if d < 512 else 131
    err = _chunked_case(hip, False, d, 12, 4, 70, n2, window, 1e4, 31)
    _say(f"f32 d {d} window {window} max abs err {err:.2e}")


@pytest.mark.parametrize("hq,hkv", [(8, 1), (16, 2), (8, 8)])
@pytest.mark.parametrize("window", [0, 200])
def test_f16_d512_prefill_matches_oracle(hip, hq, hkv, window):
    """f16 caches at head dim 512 (Gemma 4 full layers): 8 or 16 query heads on 1 or 2 kv heads
    (8 rows x 4 heads or 4 rows x 8 heads per stripe) and group 1 (32 rows per stripe); the
    first chunk's 130 rows make an odd stripe count (33, or 5 at group 1)."""
    err = _chunked_case(hip, True, 512, hq, hkv, 130, 350, window, 1e6, 32)
    _say(f"f16 d 512 {hq}/{hkv} window {window} normwise rel err {err:.2e}")


@pytest.mark.parametrize("split", ["2", "0"])
@pytest.mark.parametrize("window", [0, 200])
def test_f16_d512_prefill_split_pairs_match_oracle(monkeypatch, split, window):
    """Stripe pairs cut in two halves of their kv tiles (JMA_PREFILL_SPLIT_TILES=2 splits every
    pair of two or more tiles; 0 splits none): each half a workgroup, the later one merging the
    two states. Both plans against the oracle; a repeated call gives the same bits whichever half
    merges (attend_causal again inside the case)."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", split)
    lib = A.HipAttentionLibrary(0)
    try:
        err = _chunked_case(lib, True, 512, 8, 1, 130, 350, window, 1e6, 35)
        err2 = _chunked_case(lib, True, 512, 16, 2, 70, 200, window, 1e6, 36)
    finally:
        lib.close()
    _say(f"f16 d 512 split tiles {split} window {window} normwise rel err {max(err, err2):.2e}")


@pytest.mark.parametrize("d", [32, 128, 512])
@pytest.mark.parametrize("window", [0, 100])
def test_f32_prefill_split_stripes_match_oracle(monkeypatch, d, window):
    """f32 stripes cut in two halves of their kv tiles (JMA_PREFILL_SPLIT_TILES=2: every stripe of
    two or more tiles), the later half merging the two states: 1, 4 and 8 waves per workgroup
    against the oracle, and the same bits on a repeated call."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    try:
        n2 = 229 if d < 512 else 131
        err = _chunked_case(lib, False, d, 12, 4, 70, n2, window, 1e4, 37)
    finally:
        lib.close()
    _say(f"f32 d {d} split stripes window {window} max abs err {err:.2e}")


@pytest.mark.parametrize("half,d", [(False, 64), (False, 256), (True, 512)])
@pytest.mark.parametrize("which", ["k", "v"])
def test_split_prefill_ignores_rows_it_does_not_see(monkeypatch, half, d, which):
    """The unseen-row case above with every stripe (f32) or stripe pair (f16) split, windowed: the
    infinite rows sit in tiles of both halves."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    try:
        test_slice_prefill_ignores_rows_it_does_not_see(lib, half, d, which, 20)
    finally:
        lib.close()


@pytest.mark.parametrize("which", ["k", "v"])
@pytest.mark.parametrize("window", [0, 20])
def test_f16_d512_split_pairs_ignore_rows_they_do_not_see(monkeypatch, which, window):
    """The unseen-row case above with every stripe pair split: the infinite row sits in the
    second half's tile, whose state goes non-finite in the fast pass and is recomputed in the
    robust pass before the merge."""
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    try:
        test_slice_prefill_ignores_rows_it_does_not_see(lib, True, 512, which, window)
    finally:
        lib.close()


@pytest.mark.parametrize("half,d,hq,hkv", [(True, 512, 8, 1), (False, 128, 16, 8)])
def test_split_prefill_graph_replays_match_eager(monkeypatch, half, d, hq, hkv):
    """Split stripes (f32) and stripe pairs (f16 at 512) from a captured graph: attend_causal on
    device buffers, captured once its scratch exists, replayed three times with an eager call of
    another split shape (same ticket and state buffers) between replays; every replay gives the
    eager call's bits, so the merging halves leave every ticket at zero for the next launch."""
    import importlib
    rt = importlib.import_module("models_amd.hip_runtime")
    monkeypatch.setenv("JMA_PREFILL_SPLIT_TILES", "2")
    lib = A.HipAttentionLibrary(0)
    theta, n, n2 = 1e6, 300, 180
    tag = f"psl-graph/{int(half)}/{d}"
    rope = lib.rotary_table(d, theta, 1.0, max_positions=n + 1)
    kv = lib.kv_cache(1, n + 32, hkv, d, d, half_precision=half)
    bufs, graph = [], None
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        q = normal(38, tag + "q", (n, hq * d))
        kv.append(layer, list(range(n)), q, normal(38, tag + "k", (n, hkv * d)),
                  normal(38, tag + "v", (n, hkv * d)))
        q_rot = rope_rows(q, range(n), hq, d, d, theta, True, check_against_oracle=False)
        dq = rt.DeviceArray.from_host(np.ascontiguousarray(q_rot, np.float32))
        dout = rt.DeviceArray(n * hq * d)
        dout2 = rt.DeviceArray(n2 * hq * d)
        bufs += [dq, dout, dout2]

        def call():
            kv.attend_causal_device(layer, 0, 0, n, dq.ptr, n * hq * d, dout.ptr, n * hq * d)

        def other():  # rows 0 .. n2-1: another split plan on the same scratch
            kv.attend_causal_device(layer, 0, 0, n2, dq.ptr, n2 * hq * d, dout2.ptr, n2 * hq * d)

        call()
        lib.synchronize()
        eager = dout.download()
        assert np.all(np.isfinite(eager))
        graph = rt.Graph(lib.stream(), call)
        for replay in range(3):
            dout.zero()
            graph.launch()
            lib.synchronize()
            np.testing.assert_array_equal(dout.download(), eager, err_msg=f"replay {replay}")
            other()
            lib.synchronize()
    finally:
        if graph is not None:
            graph.destroy()
        for b in bufs:
            b.free()
        kv.close()
        rope.close()
        lib.close()


def test_c1_qwen3_prefill_f32(hip):
    """C1's shape: 16 Q heads, 8 KV heads, d 128, NeoX theta 1e6, f32 KV, the 512-row prompt as
    one chunk, every row against the oracle."""
    err = _chunked_case(hip, False, 128, 16, 8, 256, 256, 0, 1e6, 1)
    _say(f"C1-shaped f32 prefill max abs err {err:.2e}")


@pytest.mark.parametrize("half,d", [(False, 64), (False, 256), (True, 512)])
@pytest.mark.parametrize("which", ["k", "v"])
@pytest.mark.parametrize("window", [0, 20])
def test_slice_prefill_ignores_rows_it_does_not_see(hip, half, d, which, window):
    """Positions a row does not see never reach its result, whatever the cache holds there: 48
    rows are appended with key (or value) row 45 (and, windowed, row 3) infinite, positions 40..
    are discarded (the slots keep their contents) and rows 40..43 are prefilled again; their
    causal (and window) ranges exclude the infinite rows, which share kv tiles with rows they do
    see. The reference's results are finite."""
    hq, hkv, theta, cap = 8, 2, 1e4, 128
    scale = A.default_scale(d)
    tag = f"psl-nf/{int(half)}/{d}/{which}/{window}"
    q = normal(33, tag + "q", (48, hq * d))
    k = normal(33, tag + "k", (48, hkv * d))
    v = normal(33, tag + "v", (48, hkv * d))
    bad = (k if which == "k" else v).copy()
    bad[45] = np.inf if not half else 1e6
    if window:
        bad[3] = -np.inf if not half else -1e6
    k_bad, v_bad = (bad, v) if which == "k" else (k, bad)
    q2 = normal(33, tag + "q2", (4, hq * d))
    k2 = normal(33, tag + "k2", (4, hkv * d))
    v2 = normal(33, tag + "v2", (4, hkv * d))
    ref = OracleKv(1, cap, hkv * d, hkv * d, half_precision=half)
    ref.prefill_layer(0, 0, q[:40], k[:40], v[:40], hq, hkv, d, d, theta, 1.0, True, scale,
                      window=window)
    want, _, _ = ref.prefill_layer(0, 40, q2, k2, v2, hq, hkv, d, d, theta, 1.0, True, scale,
                                   window=window)
    close = assert_f16_close if half else assert_f32_close
    rope = hip.rotary_table(d, theta, 1.0, max_positions=cap)
    kv = hip.kv_cache(1, cap, hkv, d, d, half_precision=half)
    try:
        layer = A.AttentionLayer(0, hq, sliding_window=window, neox=True, rope=rope)
        kv.append(layer, list(range(48)), q, k_bad, v_bad)
        stored = kv.key_slice(0, 45, 46) if which == "k" else kv.value_slice(0, 45, 46)
        assert not np.all(np.isfinite(stored))
        kv.discard_from(40)
        got = kv.prefill(layer, 40, q2, k2, v2)
        close(got, want, f"half={half} d {d} {which} window {window}", head_dim=d)
    finally:
        kv.close()
        rope.close()


@pytest.mark.parametrize("half,d", [(False, 128), (True, 512)])
def test_slice_prefill_nan_query_is_non_finite(hip, half, d):
    """A NaN query element makes its row's scores NaN: the call reports NON_FINITE (softmax
    rejects non-finite scores, ops/TensorOps.java:1247-1279) and the context stays usable."""
    hq, hkv, n, theta = 4, 1, 40, 1e4
    q = normal(34, f"psl-nan/{d}q", (n, hq * d))
    k = normal(34, f"psl-nan/{d}k", (n, hkv * d))
    v = normal(34, f"psl-nan/{d}v", (n, hkv * d))
    rope = hip.rotary_table(d, theta, 1.0, max_positions=64)
    kv = hip.kv_cache(1, 64, hkv, d, d, half_precision=half)
    try:
        layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
        bad = q.copy()
        bad[17, 3] = np.nan
        with pytest.raises(A.AttentionStatusError) as info:
            kv.prefill(layer, 0, bad, k, v)
        assert info.value.status == A.NON_FINITE
        kv.clear()
        out = kv.prefill(layer, 0, q, k, v)
        assert np.all(np.isfinite(out))
    finally:
        kv.close()
        rope.close()

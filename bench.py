"""Benchmark of the GQA decode / prefill attention path on one MI355X.

Headline workload ("C2"): Llama-3.2-1B-shaped decode, batch 1, 32 Q heads,
8 KV heads, head_dim 64, f16 KV cache at context 4096, RoPE theta 5e5 (interleaved pairs), 16
layers with independent seeded N(0,1) K/V per layer, 128 consecutive decode steps appending to the
cache. One bench step = one decode token through all 16 layers: per layer one fused launch (RoPE of q
and the new K, append, split-K attention over the HBM-resident cache, cross-split reduction).
Inputs are resident in HBM before timing; each token's 16 launches are replayed from a HIP graph
captured once per position.

Printed: one JSON line with
  value      decode attention HBM GB/s: algorithmic KV bytes (2 * L * Hkv * d * 2 B per
             layer-step, L = visible positions) / wall time of the timed steps
  roofline   the decode kernel (the only kernel of the timed region): algorithmic bytes per launch
             over its average duration from HIP events bracketing the timed replays on the
             context stream, against 8 TB/s
  cpu_baseline  the CPU oracle (C restatement of backend-java's loop) on a bounded sample,
             1 core, in the same unit (backend-java's decode attention is single-threaded); its
             all_cores field runs the same loop on batches of independent layer-steps over
             (layer-step, kv head) units on up to 16 threads (the GPU box's CPU share)
and, as extra fields, us/token, the same tokens with the Infinity Cache scrubbed before each
(cold_cache), the C1 f32 decode step (16/8 heads, d 128, 513 positions) us and GB/s, the C3
prefill (S 2048, 24/8 heads, d 128) TFLOP/s, the C4 ragged decode (64 sessions up to 16384
positions, new token appended, one launch) GB/s, the C5 long-context decode (26 layers, 32k
context, sliding-window rings) GB/s and us/token, and a vectorised CPU baseline beside the
sequential one.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
F16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix
F32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense f32 matrix
# HBM bytes per decode launch on C2 measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE
# (bench.py --no-cpu --no-prefill --no-c1 --no-c4 --no-c5 --no-proj --no-prefill-others
# --no-decode-others --steps 8 --warmup 2), each scaled by what the counter reads for a 64 MiB
# device copy (FETCH x2.0, WRITE x1.0): 4364.5 KiB x 2.0 + 207.1 KiB. The counter passes are kept
# with the decode profile summary under profiles/; counters cannot be read from inside this
# process.
DECODE_TRAFFIC_BYTES = round((4364.5 * 2.0 + 207.1) * 1024)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def c2_config():
    return dict(hq=32, hkv=8, d=64, prior=4096, steps=128, layers=16, theta=5e5)


def decode_bytes(position: int, hkv: int, d: int) -> int:
    """Algorithmic HBM bytes of one layer's decode attention at `position`: K and V rows of the
    visible positions [0, position], f16."""
    return 2 * (position + 1) * hkv * d * 2


def run_c2(hip, A, rt, synth, steps: int, warmup: int):
    cfg = c2_config()
    hq, hkv, d, prior, layers, theta = cfg["hq"], cfg["hkv"], cfg["d"], cfg["prior"], cfg["layers"], cfg["theta"]
    total_steps = max(cfg["steps"], steps, warmup)
    n = prior + total_steps
    qd, kd = hq * d, hkv * d
    rope = hip.rotary_table(d, theta, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True)
    stream = hip.stream()
    zeros_q = rt.DeviceArray(prior * qd)
    zeros_q.zero()
    dq = rt.DeviceArray(layers * total_steps * qd)
    dk = rt.DeviceArray(layers * n * kd)
    dv = rt.DeviceArray(layers * n * kd)
    dout = rt.DeviceArray(layers * total_steps * qd)
    t0 = time.time()
    dq.upload(synth.normal(2, "bench/c2/q", (layers, total_steps, qd)))
    for l in range(layers):
        dk.upload(synth.normal(2, f"bench/c2/k{l}", (n, kd)), l * n * kd)
        dv.upload(synth.normal(2, f"bench/c2/v{l}", (n, kd)), l * n * kd)
    log(f"C2 inputs generated and resident in HBM ({time.time() - t0:.1f}s)")
    lp = [A.AttentionLayer(l, hq, neox=False, rope=rope) for l in range(layers)]
    zero_seq = np.zeros(prior, np.uint32)
    for l in range(layers):
        kv.append_device(lp[l], zero_seq, np.arange(prior), zeros_q.ptr, prior * qd,
                         dk.at(l * n * kd), prior * kd, dv.at(l * n * kd), prior * kd)
    hip.synchronize()

    def token(s):
        p = prior + s
        for l in range(layers):
            kv.decode_device(lp[l], [0], [p], dq.at((l * total_steps + s) * qd), qd,
                             dk.at((l * n + p) * kd), kd, dv.at((l * n + p) * kd), kd,
                             dout.at((l * total_steps + s) * qd), qd)

    # Eager pass over every position the graphs will replay (it allocates every scratch buffer
    # they need), timed for reference: host enqueue included.
    t = time.perf_counter()
    for s in range(total_steps):
        token(s)
    hip.synchronize()
    eager_us_per_token = (time.perf_counter() - t) / total_steps * 1e6
    eager_out = dout.download()
    kv.discard_from(prior)

    graphs = [rt.Graph(stream, lambda s=s: token(s)) for s in range(total_steps)]
    kv.discard_from(prior)  # capture recorded the appends in the host bookkeeping only
    for s in range(warmup):
        graphs[s].launch()
    hip.synchronize()
    kv.discard_from(prior)

    rt.device_synchronize()
    # HIP events on the context stream bracket the timed replays: every kernel in them is the
    # fused decode kernel (one per layer-step), so their span over the launch count is the
    # kernel's average duration back to back (launch gaps included).
    ev0, ev1 = rt.Event(), rt.Event()
    t = time.perf_counter()
    ev0.record(stream)
    for s in range(steps):
        graphs[s].launch()
    ev1.record(stream)
    rt.device_synchronize()
    elapsed = time.perf_counter() - t
    timed_kernel_ms = ev0.elapsed_ms(ev1) / (steps * layers)
    hip.synchronize()
    replay_out = dout.download()
    eager_out = eager_out.reshape(layers, total_steps, qd)[:, :steps]
    replay_out = replay_out.reshape(layers, total_steps, qd)[:, :steps]
    if not np.array_equal(eager_out, replay_out):
        raise RuntimeError("graph replay differs from the eager decode")
    algo_bytes = sum(decode_bytes(prior + s, hkv, d) for s in range(steps)) * layers

    # Cold cache: the 16 layers' caches (138 MB) fit the 256 MB Infinity Cache and the replays
    # above re-read them every token. Here a 512 MiB device-to-device copy on the same stream
    # before every token evicts them; events bracket only each token's graph.
    cold_tokens = min(steps, 32)
    scrub = rt.DeviceArray(2 * (256 << 20) // 4)
    scrub.zero()
    cold_events = [(rt.Event(), rt.Event()) for _ in range(cold_tokens)]
    for s in range(cold_tokens):
        rt.check(rt.hip().hipMemcpyAsync(scrub.ptr, scrub.at((256 << 20) // 4), 256 << 20, rt.D2D,
                                         stream), "hipMemcpyAsync scrub")
        cold_events[s][0].record(stream)
        graphs[s].launch()
        cold_events[s][1].record(stream)
    rt.device_synchronize()
    cold_ms = sum(a.elapsed_ms(b) for a, b in cold_events)
    cold_bytes = sum(decode_bytes(prior + s, hkv, d) for s in range(cold_tokens)) * layers
    scrub.free()
    # Graph replays do not pass through the host-side populated map; one eager pass restores it.
    kv.discard_from(prior)
    for s in range(steps):
        token(s)
    hip.synchronize()

    # For reference: the kernel in isolation (HIP events around each attention launch at the last
    # decoded position; each pair adds the events' own overhead).
    p_last = prior + steps - 1
    q_last = [dq.at((l * total_steps + steps - 1) * qd) for l in range(layers)]
    for l in range(layers):  # warm
        kv.attend_device(lp[l], [0], [p_last], q_last[l], qd, dout.at(l * total_steps * qd), qd)
    hip.synchronize()
    reps = 8
    events = [(rt.Event(), rt.Event()) for _ in range(reps * layers)]
    i = 0
    for r in range(reps):
        for l in range(layers):
            e0, e1 = events[i]
            e0.record(stream)
            kv.attend_device(lp[l], [0], [p_last], q_last[l], qd, dout.at(l * total_steps * qd), qd)
            e1.record(stream)
            i += 1
    hip.synchronize()
    durations = [e0.elapsed_ms(e1) for e0, e1 in events]
    kernel_ms = float(np.mean(durations))
    kernel_bytes = decode_bytes(p_last, hkv, d)

    # CPU baseline material: layer 0's cache after the run, rotated q of the last step.
    keys, values = kv.read(0, 0, p_last + 1)
    q_host = dq.download(qd, (0 * total_steps + steps - 1) * qd)

    for g in graphs:
        g.destroy()
    for buf in (zeros_q, dq, dk, dv, dout):
        buf.free()
    kv.close()
    rope.close()
    return dict(
        elapsed=elapsed, algo_bytes=algo_bytes, eager_us_per_token=eager_us_per_token,
        timed_kernel_ms=timed_kernel_ms, launches=steps * layers,
        kernel_ms=kernel_ms, kernel_ms_min=float(np.min(durations)), kernel_bytes=kernel_bytes,
        cold_ms=cold_ms, cold_tokens=cold_tokens, cold_bytes=cold_bytes,
        cpu_material=(keys, values, q_host, p_last, hq, hkv, d, theta))


def run_c2_cold(hip, A, rt, synth, steps: int = 64):
    """Profiling aid: the C2 tokens with a 512 MiB device copy on the stream before every token
    (evicting the 256 MB Infinity Cache), in the eager pass and the graph replays alike, so every
    decode dispatch of the run reads its layer from HBM and a profiler's kernel average over the
    run is the cold-cache figure. Returns us per token by events around the tokens only."""
    cfg = c2_config()
    hq, hkv, d, prior, layers, theta = cfg["hq"], cfg["hkv"], cfg["d"], cfg["prior"], cfg["layers"], cfg["theta"]
    n = prior + steps
    qd, kd = hq * d, hkv * d
    rope = hip.rotary_table(d, theta, 1.0, max_positions=n)
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True)
    stream = hip.stream()
    zeros_q = rt.DeviceArray(prior * qd)
    zeros_q.zero()
    dq = rt.DeviceArray.from_host(synth.normal(2, "bench/c2/q", (layers, steps, qd)))
    dk, dv = rt.DeviceArray(layers * n * kd), rt.DeviceArray(layers * n * kd)
    for l in range(layers):
        dk.upload(synth.normal(2, f"bench/c2/k{l}", (n, kd)), l * n * kd)
        dv.upload(synth.normal(2, f"bench/c2/v{l}", (n, kd)), l * n * kd)
    dout = rt.DeviceArray(layers * steps * qd)
    lp = [A.AttentionLayer(l, hq, neox=False, rope=rope) for l in range(layers)]
    for l in range(layers):
        kv.append_device(lp[l], np.zeros(prior, np.uint32), np.arange(prior), zeros_q.ptr,
                         prior * qd, dk.at(l * n * kd), prior * kd, dv.at(l * n * kd), prior * kd)
    scrub = rt.DeviceArray(2 * (256 << 20) // 4)
    scrub.zero()
    hip.synchronize()

    def evict():
        rt.check(rt.hip().hipMemcpyAsync(scrub.ptr, scrub.at((256 << 20) // 4), 256 << 20, rt.D2D,
                                         stream), "hipMemcpyAsync scrub")

    def token(s):
        p = prior + s
        for l in range(layers):
            kv.decode_device(lp[l], [0], [p], dq.at((l * steps + s) * qd), qd,
                             dk.at((l * n + p) * kd), kd, dv.at((l * n + p) * kd), kd,
                             dout.at((l * steps + s) * qd), qd)

    for s in range(steps):
        evict()
        token(s)
    hip.synchronize()
    kv.discard_from(prior)
    graphs = [rt.Graph(stream, lambda s=s: token(s)) for s in range(steps)]
    kv.discard_from(prior)
    events = [(rt.Event(), rt.Event()) for _ in range(steps)]
    for s in range(steps):
        evict()
        events[s][0].record(stream)
        graphs[s].launch()
        events[s][1].record(stream)
    rt.device_synchronize()
    ms = sum(a.elapsed_ms(b) for a, b in events)
    nbytes = sum(decode_bytes(prior + s, hkv, d) for s in range(steps)) * layers
    for g in graphs:
        g.destroy()
    for buf in (zeros_q, dq, dk, dv, dout, scrub):
        buf.free()
    kv.close()
    rope.close()
    return dict(us_per_token=ms / steps * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9,
                kernel_us=ms / (steps * layers) * 1e3)


def run_c3(hip, A, rt, synth, reps: int = 10):
    """C3 causal prefill: S 2048, 24 Q heads, 8 KV heads, d 128, f16, theta 5e5 interleaved."""
    return run_prefill(hip, A, rt, synth, True, 24, 8, 128, 2048, 5e5, False, "bench/c3", reps)


# Causal prefills beside C3 (no BASELINE config of their own): f32 caches run the d-sliced kernel
# on the f32 matrix ops, f16 caches at head dim 512 (Gemma 4 full layers) the same kernel on the
# f16 ones. Fields: name, half, Q heads, KV heads, head dim, rows, RoPE theta, NeoX.
PREFILL_OTHERS = [
    ("c1_shape_f32", False, 16, 8, 128, 512, 1e6, True),
    ("c3_shape_f32", False, 24, 8, 128, 2048, 5e5, False),
    ("gemma4_full_layer_f16_d512", True, 8, 1, 512, 2048, 1e6, True),
]


def run_prefill(hip, A, rt, synth, half, hq, hkv, d, S, theta, neox, tag, reps: int = 10):
    """Causal prefill of S rows (attention over the cached, rotated rows: the kernel alone, the
    append done beforehand); HIP events around `reps` back-to-back launches."""
    rope = hip.rotary_table(d, theta, 1.0, max_positions=S)
    kv = hip.kv_cache(1, S, hkv, d, d, half_precision=half)
    stream = hip.stream()
    dq = rt.DeviceArray.from_host(synth.normal(3, tag + "/q", (S, hq * d)))
    dk = rt.DeviceArray.from_host(synth.normal(3, tag + "/k", (S, hkv * d)))
    dv = rt.DeviceArray.from_host(synth.normal(3, tag + "/v", (S, hkv * d)))
    dqr = rt.DeviceArray(S * hq * d)
    dout = rt.DeviceArray(S * hq * d)
    layer = A.AttentionLayer(0, hq, neox=neox, rope=rope)
    kv.append_device(layer, np.zeros(S, np.uint32), np.arange(S), dq.ptr, dq.count, dk.ptr,
                     dk.count, dv.ptr, dv.count, dqr.ptr, dqr.count)
    kv.attend_causal_device(layer, 0, 0, S, dqr.ptr, dqr.count, dout.ptr, dout.count)
    hip.synchronize()
    # HIP events bracket `reps` back-to-back launches on the context stream.
    e0, e1 = rt.Event(), rt.Event()
    e0.record(stream)
    for _ in range(reps):
        kv.attend_causal_device(layer, 0, 0, S, dqr.ptr, dqr.count, dout.ptr, dout.count)
    e1.record(stream)
    hip.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    flops = 2 * hq * d * S * (S + 1)
    for buf in (dq, dk, dv, dqr, dout):
        buf.free()
    kv.close()
    rope.close()
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12)


def run_prefill_others(hip, A, rt, synth):
    out = {}
    for name, half, hq, hkv, d, S, theta, neox in PREFILL_OTHERS:
        r = run_prefill(hip, A, rt, synth, half, hq, hkv, d, S, theta, neox, "bench/" + name,
                        reps=5)
        peak = F16_MFMA_PEAK_TFLOPS if half else F32_MFMA_PEAK_TFLOPS
        out[name] = {"workload": f"causal prefill S {S}, {hq} Q / {hkv} KV heads, d {d}, "
                                f"{'f16' if half else 'f32'} KV",
                     "us": round(r["ms"] * 1e3, 2), "tflops": round(r["tflops"], 2),
                     "frac_of_mfma_peak": round(r["tflops"] / peak, 4),
                     "mfma_peak_tflops": peak, "flops": r["flops"]}
    return out


def run_c4(hip, A, rt, synth, reps: int = 10):
    """C4 ragged decode at full size: 64 sessions, KV lengths L drawn uniformly from
    [256, 16384], 12 Q / 2 KV heads, d 128, NeoX theta 1e6, f16 KV. The cache holds each session's
    L prior rows; a timed launch is one new token per session (`decode_device`: RoPE, append of
    the new K/V row at position L, split-K attention over L + 1 positions and the cross-split
    reduction, one fused launch), repeated at the same positions with inputs resident."""
    hq, hkv, d, B, theta = 12, 2, 128, 64, 1e6
    lens = [int(x) for x in synth.uniform_int(4, "bench/c4/len", B, 256, 16384)]
    maxlen = max(lens) + 1
    qd, kd = hq * d, hkv * d
    rope = hip.rotary_table(d, theta, 1.0, max_positions=maxlen)
    kv = hip.kv_cache(1, maxlen, hkv, d, d, half_precision=True, sequences=B)
    layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
    zq = rt.DeviceArray(maxlen * qd)
    zq.zero()
    dk, dv = rt.DeviceArray(maxlen * kd), rt.DeviceArray(maxlen * kd)
    t0 = time.time()
    for s, L in enumerate(lens):
        dk.upload(synth.normal(4, f"bench/c4/k{s}", (L, kd)))
        dv.upload(synth.normal(4, f"bench/c4/v{s}", (L, kd)))
        kv.append_device(layer, np.full(L, s, np.uint32), np.arange(L), zq.ptr, L * qd,
                         dk.ptr, L * kd, dv.ptr, L * kd)
    hip.synchronize()
    log(f"C4 cache filled ({sum(lens)} rows, {time.time() - t0:.1f}s)")
    dq = rt.DeviceArray(B * qd)
    dq.upload(synth.normal(4, "bench/c4/q", (B, qd)))
    dkn = rt.DeviceArray.from_host(synth.normal(4, "bench/c4/kn", (B, kd)))
    dvn = rt.DeviceArray.from_host(synth.normal(4, "bench/c4/vn", (B, kd)))
    dout = rt.DeviceArray(B * qd)
    seqs, pos = np.arange(B), np.array(lens)

    def step():
        kv.decode_device(layer, seqs, pos, dq.ptr, B * qd, dkn.ptr, B * kd, dvn.ptr, B * kd,
                         dout.ptr, B * qd)

    for _ in range(2):
        step()
    hip.synchronize()
    stream = hip.stream()
    e0, e1 = rt.Event(), rt.Event()
    e0.record(stream)
    for _ in range(reps):
        step()
    e1.record(stream)
    hip.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    nbytes = 2 * sum(L + 1 for L in lens) * hkv * d * 2
    for buf in (zq, dk, dv, dq, dkn, dvn, dout):
        buf.free()
    kv.close()
    rope.close()
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, rows=sum(lens) + B)


def run_c5_layer(hip, A, rt, synth, sliding: bool, per_graph: int = 32, reps: int = 5):
    """One C5 layer on its own (profiling aid): a sliding-window layer (window 512 on a RING of
    576 slots, theta 1e4) or a global layer (32704 positions, theta 1e6) of the C5 shape (4 Q / 1
    KV heads, d 256, NeoX, f16 KV)."""
    return run_decode_layer(hip, A, rt, synth, 4, 1, 256, 32704, 512 if sliding else 0,
                            per_graph, reps)


# Decode layer-steps beside C1-C5 (no BASELINE config of their own): Gemma 4 full layers (head
# dim 512, 8 Q / 1 KV heads, f16 KV) at a C5-length and a C2-length context. Fields: name, Q
# heads, KV heads, head dim, prior positions.
DECODE_OTHERS = [
    ("gemma4_full_layer_d512_32k", 8, 1, 512, 32704),
    ("gemma4_full_layer_d512_4k", 8, 1, 512, 4096),
]


def run_decode_others(hip, A, rt, synth):
    out = {}
    for name, hq, hkv, d, prior in DECODE_OTHERS:
        r = run_decode_layer(hip, A, rt, synth, hq, hkv, d, prior, 0)
        out[name] = {"workload": f"decode layer-step at position {prior}, {hq} Q / {hkv} KV heads, "
                                 f"d {d}, f16 KV (RoPE, append, attention, reduction)",
                     "us": round(r["us"], 3), "gbs": round(r["gbs"], 1), "bytes": r["bytes"],
                     "frac_of_hbm_peak": round(r["gbs"] / HBM_PEAK_GBS, 4)}
    return out


def run_decode_layer(hip, A, rt, synth, hq, hkv, d, prior, w, per_graph: int = 32, reps: int = 5):
    """One decode layer on its own: filled with its prior positions (the last w of them on a
    RING of w + 64 slots for a sliding-window layer, theta 1e4; all of them, theta 1e6, when w is
    0), the decode step at position `prior` (RoPE, append, attention and the cross-split
    reduction) is replayed from a graph of `per_graph` launches, and HIP events around the
    replays give the per-layer-step time. The step rewrites the same row each time, so every
    launch sees the same cache."""
    sliding = w > 0
    window, ring, theta = (w, w + 64, 1e4) if sliding else (0, 0, 1e6)
    rope = hip.rotary_table(d, theta, 1.0, max_positions=prior + 8)
    kv = hip.kv_cache(1, prior + 8, hkv, d, d, half_precision=True,
                      ring_capacity=[ring] if ring else None)
    layer = A.AttentionLayer(0, hq, sliding_window=window, neox=True, rope=rope)
    first = prior - w if sliding else 0
    rows, qd, kd = prior - first, hq * d, hkv * d
    zq = rt.DeviceArray(rows * qd)
    zq.zero()
    dk = rt.DeviceArray.from_host(synth.normal(5, "bench/c5l/k", (rows, kd)))
    dv = rt.DeviceArray.from_host(synth.normal(5, "bench/c5l/v", (rows, kd)))
    kv.append_device(layer, np.zeros(rows, np.uint32), np.arange(first, prior), zq.ptr, rows * qd,
                     dk.ptr, rows * kd, dv.ptr, rows * kd)
    dq = rt.DeviceArray.from_host(synth.normal(5, "bench/c5l/q", (qd,)))
    dkn = rt.DeviceArray.from_host(synth.normal(5, "bench/c5l/kn", (kd,)))
    dvn = rt.DeviceArray.from_host(synth.normal(5, "bench/c5l/vn", (kd,)))
    dout = rt.DeviceArray(qd)
    stream = hip.stream()

    def one():
        kv.decode_device(layer, [0], [prior], dq.ptr, qd, dkn.ptr, kd, dvn.ptr, kd, dout.ptr, qd)

    one()
    hip.synchronize()
    graph = rt.Graph(stream, lambda: [one() for _ in range(per_graph)])
    for _ in range(2):
        graph.launch()
    rt.device_synchronize()
    e0, e1 = rt.Event(), rt.Event()
    best = float("inf")
    for _ in range(reps):
        e0.record(stream)
        graph.launch()
        e1.record(stream)
        rt.device_synchronize()
        best = min(best, e0.elapsed_ms(e1) / per_graph)
    graph.destroy()
    for buf in (zq, dk, dv, dq, dkn, dvn, dout):
        buf.free()
    kv.close()
    rope.close()
    nbytes = 2 * (min(prior + 1, w) if sliding else prior + 1) * hkv * d * 2
    return dict(us=best * 1e3, bytes=nbytes, gbs=nbytes / (best * 1e-3) / 1e9)


def run_c1(hip, A, rt, synth, reps: int = 20, per_graph: int = 32):
    """C1 Qwen3-0.6B-shaped decode step: 16 Q / 8 KV heads, d 128, NeoX theta 1e6,
    f32 KV, 512 cached positions, the new token at position 512 (RoPE, append, split-K attention
    over 513 positions, one fused launch). The step is repeated at position 512 from a graph of
    `per_graph` launches (the host's per-call overhead would otherwise dominate a ~5 us kernel);
    HIP events around the replays give the per-step time."""
    hq, hkv, d, prior, theta = 16, 8, 128, 512, 1e6
    qd, kd = hq * d, hkv * d
    rope = hip.rotary_table(d, theta, 1.0, max_positions=prior + 1)
    kv = hip.kv_cache(1, prior + 1, hkv, d, d, half_precision=False)
    layer = A.AttentionLayer(0, hq, neox=True, rope=rope)
    zq = rt.DeviceArray(prior * qd)
    zq.zero()
    dk = rt.DeviceArray.from_host(synth.normal(1, "bench/c1/k", (prior, kd)))
    dv = rt.DeviceArray.from_host(synth.normal(1, "bench/c1/v", (prior, kd)))
    kv.append_device(layer, np.zeros(prior, np.uint32), np.arange(prior), zq.ptr, prior * qd,
                     dk.ptr, prior * kd, dv.ptr, prior * kd)
    dq = rt.DeviceArray.from_host(synth.normal(1, "bench/c1/q", (qd,)))
    dkn = rt.DeviceArray.from_host(synth.normal(1, "bench/c1/kn", (kd,)))
    dvn = rt.DeviceArray.from_host(synth.normal(1, "bench/c1/vn", (kd,)))
    dout = rt.DeviceArray(qd)
    stream = hip.stream()

    def steps():
        for _ in range(per_graph):
            kv.decode_device(layer, [0], [prior], dq.ptr, qd, dkn.ptr, kd, dvn.ptr, kd, dout.ptr, qd)

    steps()  # eager pass: every scratch buffer the graph needs exists
    hip.synchronize()
    graph = rt.Graph(stream, steps)
    graph.launch()
    hip.synchronize()
    e0, e1 = rt.Event(), rt.Event()
    e0.record(stream)
    for _ in range(reps):
        graph.launch()
    e1.record(stream)
    hip.synchronize()
    ms = e0.elapsed_ms(e1) / (reps * per_graph)
    nbytes = 2 * (prior + 1) * hkv * d * 4
    graph.destroy()
    for buf in (zq, dk, dv, dq, dkn, dvn, dout):
        buf.free()
    kv.close()
    rope.close()
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9)


def run_c5(hip, A, rt, synth, steps: int = 64, warmup: int = 4):
    """C5 Gemma-3-1B-shaped long-context decode at full size: 4 Q / 1 KV heads (MQA),
    d 256, NeoX RoPE (theta 1e6 on the global layers 5, 11, 17, 23, 1e4 on the sliding ones), f16
    KV, 26 layers in the 5 sliding (window 512) : 1 global pattern, 32704 prior positions, 64
    decode steps. The sliding layers keep LayeredKvCache RING retention of window + 64 slots and
    are filled with the last 512 prior positions (all their window reads); the global layers hold
    all 32704. A step is one token through the 26 layers (one fused decode launch each), replayed
    from per-token HIP graphs with inputs resident in HBM, as for C2."""
    hq, hkv, d, prior, layers, w = 4, 1, 256, 32704, 26, 512
    n = prior + steps
    qd, kd = hq * d, hkv * d
    sliding = [A.uses_sliding_window(l, 6, w) for l in range(layers)]
    rope_swa = hip.rotary_table(d, 1e4, 1.0, max_positions=n)
    rope_glb = hip.rotary_table(d, 1e6, 1.0, max_positions=n)
    ring_cap = w + steps
    kv = hip.kv_cache(layers, n, hkv, d, d, half_precision=True,
                      ring_capacity=[ring_cap if sl else 0 for sl in sliding])
    lp = [A.AttentionLayer(l, hq, sliding_window=w if sliding[l] else 0, neox=True,
                           rope=rope_swa if sliding[l] else rope_glb) for l in range(layers)]
    zq = rt.DeviceArray(prior * qd)
    zq.zero()
    dk, dv = rt.DeviceArray(n * kd), rt.DeviceArray(n * kd)
    t0 = time.time()
    for l in range(layers):
        first = prior - w if sliding[l] else 0
        rows = prior - first
        dk.upload(synth.normal(5, f"bench/c5/k{l}", (rows, kd)))
        dv.upload(synth.normal(5, f"bench/c5/v{l}", (rows, kd)))
        kv.append_device(lp[l], np.zeros(rows, np.uint32), np.arange(first, prior), zq.ptr,
                         rows * qd, dk.ptr, rows * kd, dv.ptr, rows * kd)
    hip.synchronize()
    log(f"C5 cache filled ({time.time() - t0:.1f}s)")
    zq.free()
    # Per layer and step: q, the new k and v rows.
    dq = rt.DeviceArray(layers * steps * qd)
    dkn, dvn = rt.DeviceArray(layers * steps * kd), rt.DeviceArray(layers * steps * kd)
    dq.upload(synth.normal(5, "bench/c5/q", (layers, steps, qd)))
    dkn.upload(synth.normal(5, "bench/c5/kn", (layers, steps, kd)))
    dvn.upload(synth.normal(5, "bench/c5/vn", (layers, steps, kd)))
    dout = rt.DeviceArray(layers * steps * qd)
    stream = hip.stream()

    def token(st):
        p = prior + st
        for l in range(layers):
            i = l * steps + st
            kv.decode_device(lp[l], [0], [p], dq.at(i * qd), qd, dkn.at(i * kd), kd,
                             dvn.at(i * kd), kd, dout.at(i * qd), qd)

    for st in range(steps):  # eager pass: allocates every scratch buffer the graphs need
        token(st)
    hip.synchronize()
    eager_out = dout.download()
    kv.discard_from(prior)
    graphs = [rt.Graph(stream, lambda st=st: token(st)) for st in range(steps)]
    kv.discard_from(prior)
    for st in range(warmup):
        graphs[st].launch()
    hip.synchronize()
    rt.device_synchronize()
    ev0, ev1 = rt.Event(), rt.Event()
    t = time.perf_counter()
    ev0.record(stream)
    for st in range(steps):
        graphs[st].launch()
    ev1.record(stream)
    rt.device_synchronize()
    elapsed = time.perf_counter() - t
    gpu_ms = ev0.elapsed_ms(ev1)
    if not np.array_equal(dout.download(), eager_out):
        raise RuntimeError("C5 graph replay differs from the eager decode")
    nbytes = 0
    for st in range(steps):
        p = prior + st
        for l in range(layers):
            nbytes += 2 * (min(p + 1, w) if sliding[l] else p + 1) * hkv * d * 2
    for g in graphs:
        g.destroy()
    for buf in (dk, dv, dq, dkn, dvn, dout):
        buf.free()
    kv.close()
    rope_swa.close()
    rope_glb.close()
    return dict(elapsed=elapsed, gpu_ms=gpu_ms, bytes=nbytes, steps=steps,
                us_per_token=elapsed / steps * 1e6, gbs=nbytes / elapsed / 1e9)


def _gguf_weights(synth, fmt: int, rows: int, cols: int, key: str) -> np.ndarray:
    """Synthetic GGUF blocks: uniform bytes with f16 N(0, 0.02) scales where the format keeps
    them (Q4_0 / Q8_0 / Q5_0 bytes 0-1, Q4_K / Q5_K bytes 0-3, Q6_K bytes 208-209)."""
    nbytes, elems = {0: (18, 32), 1: (34, 32), 2: (144, 256), 3: (210, 256), 4: (176, 256),
                     5: (22, 32)}[fmt]
    blocks = cols // elems
    raw = synth.uniform_int(9, key, rows * blocks * nbytes, 0, 255).astype(np.uint8)
    raw = raw.reshape(rows, blocks, nbytes)
    scales = (synth.normal(9, key + "/s", (rows, blocks, 2)) * 0.02).astype(np.float16)
    scales = scales.view(np.uint8).reshape(rows, blocks, 4)
    if fmt in (2, 4):
        raw[:, :, 0:4] = scales
    elif fmt == 3:
        raw[:, :, 208:210] = scales[..., :2]
    else:
        raw[:, :, 0:2] = scales[..., :2]
    return raw.reshape(-1)


def run_proj(hip, A, rt, synth, reps: int = 20, per_graph: int = 32):
    """The projections around one C2 layer at decode (batch 1): Llama-3.2-1B's Q (2048 rows), K
    and V (512 rows each) over 2048 inputs as one grouped launch writing q|k|v for the decode,
    and the output projection (2048 x 2048) with the residual added in place; Q4_0, Q8_0, Q5_0,
    Q4_K, Q5_K and Q6_K weights; then C3's grouped Q/K/V projection at its 2048-row prompt. Each
    launch is repeated `per_graph` times in a graph; HIP events around the replays
    give us per launch; GB/s counts the weight bytes (the activations are 8 KB)."""
    cols, rows = 2048, [2048, 512, 512]
    stream = hip.stream()
    result = {}
    for name, fmt in (("q4_0", A.WEIGHTS_Q4_0), ("q8_0", A.WEIGHTS_Q8_0), ("q5_0", A.WEIGHTS_Q5_0),
                      ("q4_k", A.WEIGHTS_Q4_K), ("q5_k", A.WEIGHTS_Q5_K), ("q6_k", A.WEIGHTS_Q6_K)):
        ws = [_gguf_weights(synth, fmt, r, cols, f"bench/proj/{name}/{i}") for i, r in enumerate(rows)]
        wo = _gguf_weights(synth, fmt, cols, cols, f"bench/proj/{name}/wo")
        dws = [rt.DeviceArray.from_host(w) for w in ws]
        dwo = rt.DeviceArray.from_host(wo)
        dx = rt.DeviceArray.from_host(synth.normal(9, "bench/proj/x", (cols,)))
        dqkv = rt.DeviceArray(sum(rows))
        dres = rt.DeviceArray.from_host(synth.normal(9, "bench/proj/res", (cols,)))

        def qkv():
            for _ in range(per_graph):
                hip.quantized_grouped_matmul_device([fmt] * 3, [d.ptr for d in dws],
                                                    [w.size for w in ws], rows, dx.ptr, cols,
                                                    dqkv.ptr, sum(rows), 1, cols)

        def out_proj():
            for _ in range(per_graph):
                hip.quantized_matmul_device(fmt, dwo.ptr, wo.size, dqkv.ptr, cols, dres.ptr, cols,
                                            1, cols, cols, dres.ptr, A.ADDEND_RESIDUAL)

        for label, fn, nbytes in (("qkv", qkv, sum(w.size for w in ws)), ("wo_residual", out_proj, wo.size)):
            graph = rt.Graph(stream, fn)
            graph.launch()
            hip.synchronize()
            e0, e1 = rt.Event(), rt.Event()
            e0.record(stream)
            for _ in range(reps):
                graph.launch()
            e1.record(stream)
            hip.synchronize()
            ms = e0.elapsed_ms(e1) / (reps * per_graph)
            graph.destroy()
            result[f"{label}_{name}"] = dict(us=round(ms * 1e3, 3), weight_bytes=int(nbytes),
                                              gbs=round(nbytes / (ms * 1e-3) / 1e9, 1))
        for d in dws + [dwo, dx, dqkv, dres]:
            d.free()
    # Prefill-sized: C3's Llama-3.2-3B Q (3072 rows), K and V (1024 each) over 3072 inputs for
    # the 2048-row prompt, one grouped call (one launch per format; q4_k_m: Q and K in Q4_K, V in
    # Q6_K, as Q4_K_M files store them), events around 3 replays.
    cols, rows, batch = 3072, [3072, 1024, 1024], 2048
    dx = rt.DeviceArray.from_host(synth.normal(9, "bench/proj/xp", (batch, cols)))
    dqkv = rt.DeviceArray(batch * sum(rows))
    q4k, q6k = A.WEIGHTS_Q4_K, A.WEIGHTS_Q6_K
    for name, fmts in (("q4_0", [A.WEIGHTS_Q4_0] * 3), ("q8_0", [A.WEIGHTS_Q8_0] * 3),
                       ("q4_k", [q4k] * 3), ("q4_k_m", [q4k, q4k, q6k]), ("q6_k", [q6k] * 3)):
        ws = [_gguf_weights(synth, f, r, cols, f"bench/projp/{name}/{i}")
              for i, (f, r) in enumerate(zip(fmts, rows))]
        dws = [rt.DeviceArray.from_host(w) for w in ws]

        def qkv_prefill():
            hip.quantized_grouped_matmul_device(fmts, [d.ptr for d in dws], [w.size for w in ws],
                                                rows, dx.ptr, batch * cols, dqkv.ptr, dqkv.count,
                                                batch, cols)

        qkv_prefill()  # eager first: sizes the activation scratch outside the capture
        hip.synchronize()
        graph = rt.Graph(stream, qkv_prefill)
        graph.launch()
        hip.synchronize()
        e0, e1 = rt.Event(), rt.Event()
        e0.record(stream)
        for _ in range(3):
            graph.launch()
        e1.record(stream)
        hip.synchronize()
        ms = e0.elapsed_ms(e1) / 3
        graph.destroy()
        macs = batch * sum(rows) * cols
        result[f"qkv_prefill2048_{name}"] = dict(
            us=round(ms * 1e3, 1), weight_bytes=int(sum(w.size for w in ws)),
            tops=round(2 * macs / (ms * 1e-3) / 1e12, 2))
        for d in dws:
            d.free()
    dx.free()
    dqkv.free()
    return result


def cpu_baseline_c2(material, budget_s: float):
    """backend-java's decode attention restated in C (oracle/), one thread, on repeated C2
    layer-steps at the last decoded position until about budget_s seconds of CPU work ran."""
    from oracle import oracle
    keys, values, q_raw, p, hq, hkv, d, theta = material
    c, s = oracle.rotary_factors(d, theta, 1.0, p)
    q_rot = np.concatenate([oracle.rope_apply(q_raw[h * d:(h + 1) * d], c, s, False)
                            for h in range(hq)])
    scale = float(np.float32(1.0 / math.sqrt(d)))
    keys = keys.reshape(p + 1, hkv * d)
    values = values.reshape(p + 1, hkv * d)
    runs = 0
    t = time.perf_counter()
    while True:
        oracle.gqa_rows(q_rot, keys, values, hq, hkv, d, d, scale)
        runs += 1
        if time.perf_counter() - t >= budget_s and runs >= 3:
            break
    per = (time.perf_counter() - t) / runs
    return dict(seconds_per_layer_step=per, runs=runs, bytes=decode_bytes(p, hkv, d),
                q_rot=q_rot, keys=keys, values=values, scale=scale)


def cpu_baseline_c2_batched(cpu, material, budget_s: float, threads: int, lanes8: bool):
    """The same layer-step on `threads` threads: batches of 16 independent layer-steps (the 16
    layers of one token), split over (layer-step, kv head) units, until about budget_s seconds.
    lanes8: the vectorised variant (dot products in eight partial sums, as a Vector API loop over
    256-bit vectors computes them) instead of the sequential restatement."""
    from oracle import oracle
    _, _, _, p, hq, hkv, d, _ = material
    batch = 16
    qs, ks, vs = [cpu["q_rot"]] * batch, [cpu["keys"]] * batch, [cpu["values"]] * batch
    runs = 0
    t = time.perf_counter()
    while True:
        oracle.gqa_rows_batch(qs, ks, vs, hq, hkv, d, d, cpu["scale"], threads=threads,
                              lanes8=lanes8)
        runs += 1
        if time.perf_counter() - t >= budget_s and runs >= 2:
            break
    per = (time.perf_counter() - t) / (runs * batch)
    return dict(seconds_per_layer_step=per, runs=runs * batch)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the C3 prefill figure")
    ap.add_argument("--no-c1", action="store_true", help="skip the C1 f32 decode-step figure")
    ap.add_argument("--no-c4", action="store_true", help="skip the C4 ragged decode figure")
    ap.add_argument("--no-c5", action="store_true", help="skip the C5 long-context decode figure")
    ap.add_argument("--no-proj", action="store_true",
                    help="skip the Q4_0 / Q8_0 projection figures")
    ap.add_argument("--proj-only", action="store_true",
                    help="profiling aid: run only the projection measurements, print their figures")
    ap.add_argument("--c5-only", action="store_true",
                    help="profiling aid: run only the C5 long-context decode measurement")
    ap.add_argument("--c5-layers", action="store_true",
                    help="profiling aid: one C5 sliding-window layer and one C5 global layer, each "
                         "replayed on its own from graphs, print their per-layer-step figures")
    ap.add_argument("--c4-only", action="store_true",
                    help="profiling aid: run only the C4 ragged decode measurement, print its figures")
    ap.add_argument("--c2-cold-only", action="store_true",
                    help="profiling aid: only the C2 tokens with the Infinity Cache scrubbed before "
                         "each, in the eager pass and the replays alike")
    ap.add_argument("--c1-only", action="store_true",
                    help="profiling aid: run only the C1 f32 decode-step measurement")
    ap.add_argument("--prefill-only", action="store_true",
                    help="profiling aid: run only the C3 prefill measurement, print its figures")
    ap.add_argument("--prefill-others-only", action="store_true",
                    help="profiling aid: run only the f32 and head-dim-512 prefill measurements")
    ap.add_argument("--no-prefill-others", action="store_true",
                    help="skip the f32 and head-dim-512 prefill figures")
    ap.add_argument("--decode-others-only", action="store_true",
                    help="profiling aid: run only the head-dim-512 decode layer measurements")
    ap.add_argument("--no-decode-others", action="store_true",
                    help="skip the head-dim-512 decode layer figures")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="profiling aid: one device-to-device copy of MIB MiB (the runtime's copy "
                         "kernel), to calibrate the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        return 2
    if args.steps < 1 or args.steps > 128 or args.warmup < 0 or args.warmup > 128:
        print("--steps must be in [1, 128] and --warmup in [0, 128]", file=sys.stderr)
        return 2

    from models_amd import attention as A
    from models_amd import hip_runtime as rt
    from models_amd import synth

    hip = A.HipAttentionLibrary(0)
    log("context created on device 0")
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src, dst = rt.DeviceArray(n), rt.DeviceArray(n)
        src.zero()
        rt.check(rt.hip().hipMemcpy(dst.ptr, src.ptr, src.nbytes, rt.D2D), "hipMemcpy D2D")
        rt.device_synchronize()
        print(json.dumps({"copy_calibration_bytes": src.nbytes}), flush=True)
        return 0
    if args.c2_cold_only:
        cold = run_c2_cold(hip, A, rt, synth)
        print(json.dumps({"c2_cold_us_per_token": round(cold["us_per_token"], 2),
                          "gbs": round(cold["gbs"], 1),
                          "kernel_us_by_events": round(cold["kernel_us"], 3)}), flush=True)
        return 0
    if args.c1_only:
        c1 = run_c1(hip, A, rt, synth)
        print(json.dumps({"c1_us": round(c1["ms"] * 1e3, 3), "gbs": round(c1["gbs"], 1),
                          "bytes": c1["bytes"]}), flush=True)
        return 0
    if args.prefill_only:
        c3 = run_c3(hip, A, rt, synth)
        print(json.dumps({"prefill_us": round(c3["ms"] * 1e3, 2), "tflops": round(c3["tflops"], 2),
                          "flops": c3["flops"]}), flush=True)
        return 0
    if args.decode_others_only:
        print(json.dumps({"decode_others": run_decode_others(hip, A, rt, synth)}), flush=True)
        return 0
    if args.prefill_others_only:
        print(json.dumps({"prefill_others": run_prefill_others(hip, A, rt, synth)}), flush=True)
        return 0
    if args.proj_only:
        print(json.dumps(run_proj(hip, A, rt, synth)), flush=True)
        return 0
    if args.c5_only:
        c5 = run_c5(hip, A, rt, synth)
        print(json.dumps({"c5_us_per_token": round(c5["us_per_token"], 2), "gbs": round(c5["gbs"], 1),
                          "bytes_per_token": c5["bytes"] // c5["steps"]}), flush=True)
        return 0
    if args.c5_layers:
        out = {}
        for name, sl in (("sliding", True), ("global", False)):
            r = run_c5_layer(hip, A, rt, synth, sl)
            out[name] = {"us": round(r["us"], 3), "gbs": round(r["gbs"], 1), "bytes": r["bytes"]}
        print(json.dumps({"c5_layers": out}), flush=True)
        return 0
    if args.c4_only:
        c4 = run_c4(hip, A, rt, synth)
        print(json.dumps({"c4_us": round(c4["ms"] * 1e3, 2), "gbs": round(c4["gbs"], 1),
                          "bytes": c4["bytes"]}), flush=True)
        return 0
    c2 = run_c2(hip, A, rt, synth, args.steps, args.warmup)
    log(f"C2: {args.steps} steps in {c2['elapsed'] * 1e3:.2f} ms; decode kernel "
        f"{c2['timed_kernel_ms'] * 1e3:.2f} us per launch in the timed replays, "
        f"{c2['kernel_ms'] * 1e3:.2f} us isolated")
    c1 = None
    if not args.no_c1:
        c1 = run_c1(hip, A, rt, synth)
        log(f"C1 f32 decode step: {c1['ms'] * 1e3:.2f} us, {c1['gbs']:.0f} GB/s")
    c3 = None
    if not args.no_prefill:
        c3 = run_c3(hip, A, rt, synth)
        log(f"C3 prefill: {c3['ms'] * 1e3:.1f} us, {c3['tflops']:.1f} TFLOP/s")
    others = None
    if not args.no_prefill_others:
        others = run_prefill_others(hip, A, rt, synth)
        log("other prefills: " + ", ".join(f"{k} {v['us']:.1f} us {v['tflops']:.1f} TFLOP/s"
                                           for k, v in others.items()))
    dothers = None
    if not args.no_decode_others:
        dothers = run_decode_others(hip, A, rt, synth)
        log("other decode layers: " + ", ".join(f"{k} {v['us']:.2f} us {v['gbs']:.0f} GB/s"
                                                for k, v in dothers.items()))
    c4 = None
    if not args.no_c4:
        c4 = run_c4(hip, A, rt, synth)
        log(f"C4 ragged decode: {c4['ms'] * 1e3:.1f} us, {c4['gbs']:.0f} GB/s")
    c5 = None
    if not args.no_c5:
        c5 = run_c5(hip, A, rt, synth)
        log(f"C5 long-context decode: {c5['us_per_token']:.1f} us/token, {c5['gbs']:.0f} GB/s")
    proj = None
    if not args.no_proj:
        proj = run_proj(hip, A, rt, synth)
        log("projections (us, then GB/s of weights at decode or integer TOPS at prefill size): " +
            ", ".join(f"{k} {v['us']:.2f} " + (f"{v['gbs']:.0f}" if "gbs" in v else f"{v['tops']:.1f}")
                      for k, v in proj.items()))
    hip.close()

    value = c2["algo_bytes"] / c2["elapsed"] / 1e9
    # Algorithmic bytes of an average launch of the timed region over its event-timed duration.
    achieved = c2["algo_bytes"] / c2["launches"] / (c2["timed_kernel_ms"] * 1e-3) / 1e9
    result = {
        "metric": "decode attn HBM GB/s + us/token @4k ctx; prefill attn TFLOP/s @2k",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["elapsed"] / args.steps * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) Q/K/V, counter-based SplitMix64 + Box-Muller)",
        "config": {
            "workload": "C2 Llama-3.2-1B-shaped decode: 32 Q heads, 8 KV heads, head_dim 64, "
                        "f16 KV, context 4096, 16 layers, RoPE theta 5e5; the eager pass and the "
                        "graph captures cover the configured 128 consecutive decode steps, the "
                        f"timed region replays the first {args.steps} of them",
            "batch": 1, "layers": 16, "context": 4096, "kv_dtype": "f16",
            "accumulate": "f32", "step": "one token through 16 layers (append + attention)",
            "timed_steps": args.steps,
            "timed_positions": [4096, 4096 + args.steps - 1],
            "configured_steps": 128,
        },
        "us_per_token": round(c2["elapsed"] / args.steps * 1e6, 3),
        "us_per_token_eager_python": round(c2["eager_us_per_token"], 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": DECODE_TRAFFIC_BYTES,
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "kernel": "decode_kernel<f16,64,64> (RoPE + append + split-K + fused cross-split reduce)",
            "kernel_us": round(c2["timed_kernel_ms"] * 1e3, 3),
            "kernel_us_source": "HIP events over the timed graph replays / launches",
            "bytes_per_launch": round(c2["algo_bytes"] / c2["launches"]),
            "kernel_us_isolated": round(c2["kernel_ms"] * 1e3, 3),
            "kernel_us_isolated_min": round(c2["kernel_ms_min"] * 1e3, 3),
            "bytes_per_isolated_launch": c2["kernel_bytes"],
        },
    }
    result["cold_cache"] = {
        "what": "C2 tokens with the Infinity Cache scrubbed before each (a 512 MiB device copy "
                "on the stream), HIP events around each token's 16 launches only",
        "us_per_token": round(c2["cold_ms"] / c2["cold_tokens"] * 1e3, 3),
        "gbs": round(c2["cold_bytes"] / (c2["cold_ms"] * 1e-3) / 1e9, 2),
        "frac_of_hbm_peak": round(c2["cold_bytes"] / (c2["cold_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tokens": c2["cold_tokens"],
    }
    if c1 is not None:
        result["c1_decode_step"] = {
            "workload": "C1 Qwen3-0.6B-shaped decode step: 16 Q / 8 KV heads, d 128, f32 KV, "
                        "512 cached positions, new token at position 512 (RoPE, append, "
                        "attention: one launch), replayed from graphs",
            "us": round(c1["ms"] * 1e3, 3),
            "gbs": round(c1["gbs"], 1),
            "frac_of_hbm_peak": round(c1["gbs"] / HBM_PEAK_GBS, 4),
            "bytes": c1["bytes"],
        }
    if c3 is not None:
        result["prefill"] = {
            "workload": "C3 Llama-3.2-3B causal prefill S 2048, 24 Q / 8 KV heads, d 128, f16",
            "tflops": round(c3["tflops"], 2),
            "us": round(c3["ms"] * 1e3, 2),
            "frac_of_f16_mfma_peak": round(c3["tflops"] / F16_MFMA_PEAK_TFLOPS, 4),
            "flops": c3["flops"],
        }
    if others is not None:
        result["prefill_others"] = others
    if dothers is not None:
        result["decode_others"] = dothers
    if c4 is not None:
        result["ragged_decode"] = {
            "workload": "C4 Qwen2.5-1.5B-shaped ragged decode: 64 sessions, KV lengths "
                        "U[256, 16384], 12 Q / 2 KV heads, d 128, f16 KV, one new token per "
                        "session (RoPE, append and attention in one launch)",
            "gbs": round(c4["gbs"], 1),
            "us": round(c4["ms"] * 1e3, 2),
            "frac_of_hbm_peak": round(c4["gbs"] / HBM_PEAK_GBS, 4),
            "bytes": c4["bytes"],
            "kv_rows": c4["rows"],
        }
    if c5 is not None:
        result["long_context_decode"] = {
            "workload": "C5 Gemma-3-1B-shaped decode: 4 Q / 1 KV heads, d 256, f16 KV, 26 layers "
                        "(5 sliding window 512 rings : 1 global), context 32704..32767, 64 steps",
            "gbs": round(c5["gbs"], 1),
            "us_per_token": round(c5["us_per_token"], 2),
            "frac_of_hbm_peak": round(c5["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_token": c5["bytes"] // c5["steps"],
        }
    if proj is not None:
        result["projections"] = {
            "workload": "Llama-3.2-1B layer at decode (batch 1): grouped Q/K/V projection (2048 -> "
                        "2048 + 512 + 512) and output projection 2048 x 2048 plus residual, GGUF "
                        "Q4_0 / Q8_0 / Q5_0 / Q4_K / Q5_K / Q6_K weights, activations quantized "
                        "(Q8_0 or Q8_K) in the launch (us, GB/s of weights); qkv_prefill2048_*: "
                        "C3's grouped Q/K/V (3072 -> 3072 + 1024 + 1024) over its 2048-row prompt, "
                        "activations quantized once, then the register-tiled product (us, integer "
                        "TOPS); q4_k_m: Q and K in Q4_K, V in Q6_K",
            **proj,
        }
    if not args.no_cpu:
        cpu = cpu_baseline_c2(c2["cpu_material"], args.cpu_seconds)
        cpu_gbs = cpu["bytes"] / cpu["seconds_per_layer_step"] / 1e9
        result["cpu_baseline"] = {
            "value": round(cpu_gbs, 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"{cpu['runs']} C2 layer-steps at position {c2['cpu_material'][3]} "
                      f"(backend-java groupedQueryAttention restated in C, oracle/), same "
                      f"algorithmic byte count as the GPU figure",
            "us_per_token": round(cpu["seconds_per_layer_step"] * 16 * 1e6, 1),
        }
        # The GPU box grants one GPU's job 16 CPUs whatever nproc shows; the affinity mask is
        # what this process may use.
        available = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        threads = max(1, min(16, available))
        sample = (f"C2 layer-steps at position {c2['cpu_material'][3]} in batches of 16, "
                  f"(layer-step, kv head) units")
        allc = cpu_baseline_c2_batched(cpu, c2["cpu_material"], args.cpu_seconds / 3, threads, False)
        result["cpu_baseline"]["all_cores"] = {
            "value": round(cpu["bytes"] / allc["seconds_per_layer_step"] / 1e9, 4),
            "cores": threads,
            "available_cpus": available,
            "sample": f"{allc['runs']} {sample} over {threads} threads",
            "us_per_token": round(allc["seconds_per_layer_step"] * 16 * 1e6, 1),
        }
        vec1 = cpu_baseline_c2_batched(cpu, c2["cpu_material"], args.cpu_seconds / 3, 1, True)
        vecn = cpu_baseline_c2_batched(cpu, c2["cpu_material"], args.cpu_seconds / 3, threads, True)
        result["cpu_baseline"]["vectorized"] = {
            "what": "the same loop with dot products in eight partial sums (AVX2 code, the shape "
                    "of a Vector API reduction over 256-bit vectors); timing only, the parity "
                    "oracle is the sequential restatement",
            "value": round(cpu["bytes"] / vec1["seconds_per_layer_step"] / 1e9, 4),
            "cores": 1,
            "us_per_token": round(vec1["seconds_per_layer_step"] * 16 * 1e6, 1),
            "all_cores": {
                "value": round(cpu["bytes"] / vecn["seconds_per_layer_step"] / 1e9, 4),
                "cores": threads,
                "us_per_token": round(vecn["seconds_per_layer_step"] * 16 * 1e6, 1),
            },
            "sample": f"{vec1['runs']} (1 thread) and {vecn['runs']} ({threads} threads) {sample}",
        }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

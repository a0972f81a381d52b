"""Pins the oracle's GGUF block-quantized projection (Q8_0 activation quantization and the Q4_0 /
Q8_0 matmul that backend-native's tests define, NativeKernelLibraryTest.java:909-1023) against
independent statements of the same definitions: numpy's IEEE float32 and float16 arithmetic and
round-half-even, GGML's published block layouts dequantized with numpy, float64 sums, and
hand-computed one-block cases. A swapped nibble, a missing -8 offset, a scale taken from the wrong
block or activation row, or a dropped f16 rounding of the activation scale fails one of them."""

import numpy as np
import pytest

from models_amd import synth


def _quantize_numpy(x, cols):
    """Q8_0 activations from numpy's float32 ops: inverse = 127 / absmax, q = rint(x * inverse),
    scale = float16(absmax / 127)."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    absmax = np.nanmax(np.abs(x), axis=1).astype(np.float32)
    absmax = np.where(np.isnan(absmax), np.float32(0), absmax)
    with np.errstate(divide="ignore", invalid="ignore"):
        inverse = np.where(absmax == 0, np.float32(0), np.float32(127) / absmax).astype(np.float32)
        scaled = (x * inverse[:, None]).astype(np.float32)
    q = np.where(np.isnan(scaled), 0, np.rint(scaled)).astype(np.int8)
    scales = (absmax / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32)
    return q.reshape(-1), scales


def _dequantize_numpy(fmt, weights, rows, cols):
    """GGML Q4_0 / Q8_0 blocks -> (per-block f32 scales [rows, blocks], int values [rows, cols])."""
    blocks = cols // 32
    nbytes = 18 if fmt == 0 else 34
    w = np.frombuffer(bytes(weights), np.uint8)[:rows * blocks * nbytes].reshape(rows, blocks, nbytes)
    scales = w[:, :, :2].copy().view(np.float16).astype(np.float32).reshape(rows, blocks)
    if fmt == 0:
        nib = w[:, :, 2:].astype(np.int32)
        vals = np.concatenate([(nib & 0xF) - 8, (nib >> 4) - 8], axis=2)  # elements 0-15, 16-31
    else:
        vals = w[:, :, 2:].view(np.int8).astype(np.int32)
    return scales, vals.reshape(rows, cols)


def _float64_matmul(fmt, weights, x, batch, rows, cols):
    """float64 sum over blocks of (f32 weight scale * f32 activation scale) * integer block dot."""
    wscale, wvals = _dequantize_numpy(fmt, weights, rows, cols)
    q, ascale = _quantize_numpy(x, cols)
    q = q.reshape(batch, cols // 32, 32).astype(np.int64)
    ascale = ascale.reshape(batch, cols // 32)
    wv = wvals.reshape(rows, cols // 32, 32).astype(np.int64)
    dots = np.einsum("rkj,bkj->brk", wv, q)                           # exact integers
    prod = (wscale[None, :, :] * ascale[:, None, :]).astype(np.float32)  # one f32 rounding
    terms = prod.astype(np.float64) * dots
    return terms.sum(axis=2), np.abs(terms).sum(axis=2)


def _random_weights(fmt, rows, cols, key):
    blocks = cols // 32
    nbytes = 18 if fmt == 0 else 34
    raw = synth.uniform_int(7, key, rows * blocks * nbytes, 0, 255).astype(np.uint8)
    raw = raw.reshape(rows, blocks, nbytes)
    scales = (synth.normal(7, key + "/s", (rows, blocks)) * 0.02).astype(np.float16)
    raw[:, :, :2] = scales.view(np.uint8).reshape(rows, blocks, 2)
    return raw.reshape(-1).tobytes()


def test_q8_0_quantize_matches_numpy_ieee(oracle):
    x = synth.normal(7, "q8/x", (64 * 32,)) * 3.0
    x[:32] = 0.0                                   # all-zero block: scale 0, q 0
    x[32:64] = np.arange(32) - 15.5                # absmax 16.5
    x[64:96] = np.float32(127.0) * (np.arange(32) % 2 * 2 - 1)  # absmax 127: inverse exactly 1
    x[96:128] = np.linspace(-126.5, 126.5, 32)     # with absmax 127 below: ties at .5
    x[127] = 127.0
    q, s = oracle.q8_0_quantize(x, 2, 32 * 32)
    q_ref, s_ref = _quantize_numpy(x, 32 * 32)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.all(q[:32] == 0) and s[0] == 0
    assert int(np.max(np.abs(q.astype(np.int32)))) <= 127
    # ties round half to even: 126.5 * 1 -> 126, -125.5 -> -126
    blk = q[96:128].astype(np.int32)
    np.testing.assert_array_equal(blk[:31], np.rint(np.linspace(-126.5, 126.5, 32)[:31]))
    # dequantized, every element lies within half a quantization step of x
    qs = q.astype(np.float32).reshape(-1, 32)
    err = np.abs(qs * (np.float32(127) / np.maximum(np.abs(x).reshape(-1, 32).max(1), 1e-30))[:, None] ** -1
                 - x.reshape(-1, 32))
    step = np.abs(x).reshape(-1, 32).max(1) / 127
    assert np.all(err <= step[:, None] * 0.5 * (1 + 1e-5) + 1e-30)


def test_q8_0_quantize_skips_nan(oracle):
    x = np.linspace(-2.0, 2.0, 32).astype(np.float32)
    x[5] = np.nan
    q, s = oracle.q8_0_quantize(x, 1, 32)
    q_ref, s_ref = _quantize_numpy(x, 32)
    assert q[5] == 0
    np.testing.assert_array_equal(q, q_ref)
    assert s[0] == s_ref[0] == np.float32(np.float16(np.float32(2.0) / np.float32(127)))


def test_q4_0_one_block_by_hand(oracle):
    # scale 1.0; every byte 0x98: low nibble 8 (element i -> 0), high nibble 9 (element i+16 -> 1)
    w = bytes([0x00, 0x3C]) + bytes([0x98] * 16)
    x = np.concatenate([np.full(16, 100.0), np.arange(16) + 1.0]).astype(np.float32)
    x[0] = 127.0  # absmax 127: q == x, activation scale f16(1.0) = 1
    out = oracle.quantized_matmul(0, w, x, 1, 1, 32)
    assert out[0, 0] == np.float32(np.sum(np.arange(16) + 1.0))  # 136: only the high half counts
    # the -8 offset: bytes 0x00 -> every element -8
    w0 = bytes([0x00, 0x3C]) + bytes(16)
    assert oracle.quantized_matmul(0, w0, x, 1, 1, 32)[0, 0] == np.float32(-8 * np.sum(x))
    # a weight scale of 0.5 and an activation absmax of 254 (activation scale 2): product 1.0
    x2 = x * 2
    w2 = bytes([0x00, 0x38]) + bytes([0x98] * 16)
    assert oracle.quantized_matmul(0, w2, x2, 1, 1, 32)[0, 0] == np.float32(136.0)


def test_q8_0_one_block_by_hand(oracle):
    vals = (np.arange(32) - 16).astype(np.int8)
    w = bytes([0x00, 0x3C]) + vals.tobytes()
    x = np.zeros(32, np.float32)
    x[3], x[30] = 127.0, -1.0  # q = x exactly
    out = oracle.quantized_matmul(1, w, x, 1, 1, 32)
    assert out[0, 0] == np.float32(127 * (3 - 16) + (-1) * (30 - 16))


@pytest.mark.parametrize("fmt", [0, 1])
def test_quantized_matmul_matches_float64_dequantized(oracle, fmt):
    batch, rows, cols = 3, 40, 512
    w = _random_weights(fmt, rows, cols, f"qm/w{fmt}")
    x = synth.normal(7, f"qm/x{fmt}", (batch, cols))
    out = oracle.quantized_matmul(fmt, w, x, batch, rows, cols)
    ref, mag = _float64_matmul(fmt, w, x, batch, rows, cols)
    # the oracle's per-block fma chain rounds once per block: |err| <= blocks * 2^-24 * sum|term|
    bound = (cols // 32) * 2.0 ** -24 * mag + 1e-30
    assert np.all(np.abs(out.astype(np.float64) - ref) <= bound)


def test_quantized_matmul_rows_and_batches_are_independent(oracle):
    fmt, batch, rows, cols = 0, 4, 7, 256
    w = _random_weights(fmt, rows, cols, "qm/ind")
    x = synth.normal(7, "qm/ind/x", (batch, cols))
    full = oracle.quantized_matmul(fmt, w, x, batch, rows, cols)
    row_bytes = cols // 32 * 18
    for b in range(batch):
        for r in (0, 3, 6):
            one = oracle.quantized_matmul(fmt, w[r * row_bytes:(r + 1) * row_bytes], x[b], 1, 1, cols)
            assert one[0, 0] == full[b, r]


def test_reference_fixtures_against_float64(oracle, known_answers):
    for case in known_answers["quantized_matmul"]:
        w = bytes.fromhex(case["weights_hex"])
        b, r, c = case["batch"], case["rows"], case["cols"]
        x = np.float32(case["input"])
        out = oracle.quantized_matmul(case["format"], w, x, b, r, c)
        ref, mag = _float64_matmul(case["format"], w, x, b, r, c)
        assert np.all(np.abs(out - ref) <= (c // 32) * 2.0 ** -24 * mag + 1e-30), case["name"]


def test_quantized_matmul_rejects_bad_shapes(oracle):
    with pytest.raises(oracle.OracleError):
        oracle.quantized_matmul(0, bytes(18), np.zeros(31, np.float32), 1, 1, 31)
    with pytest.raises(oracle.OracleError):
        oracle.quantized_matmul(7, bytes(18), np.zeros(32, np.float32), 1, 1, 32)

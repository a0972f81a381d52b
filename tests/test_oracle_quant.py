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


_NBYTES = {0: 18, 1: 34, 5: 22}


def _dequantize_numpy(fmt, weights, rows, cols):
    """GGML Q4_0 / Q8_0 / Q5_0 blocks -> (per-block f32 scales [rows, blocks], int values
    [rows, cols])."""
    blocks = cols // 32
    nbytes = _NBYTES[fmt]
    w = np.frombuffer(bytes(weights), np.uint8)[:rows * blocks * nbytes].reshape(rows, blocks, nbytes)
    scales = w[:, :, :2].copy().view(np.float16).astype(np.float32).reshape(rows, blocks)
    if fmt == 0:
        nib = w[:, :, 2:].astype(np.int32)
        vals = np.concatenate([(nib & 0xF) - 8, (nib >> 4) - 8], axis=2)  # elements 0-15, 16-31
    elif fmt == 5:
        high = w[:, :, 2:6].copy().view("<u4").astype(np.int64)[..., 0]  # bit j: element j's 5th bit
        bits = (high[..., None] >> np.arange(32)) & 1
        nib = w[:, :, 6:].astype(np.int32)
        vals = np.concatenate([nib & 0xF, nib >> 4], axis=2) + 16 * bits - 16
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
    nbytes = _NBYTES[fmt]
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


def test_q5_0_one_block_by_hand(oracle):
    # scale 1.0; every nibble 0: elements whose fifth bit is set are 16 - 16 = 0, the others -16
    x = np.zeros(32, np.float32)
    x[0], x[5], x[16], x[31] = 127.0, 2.0, 3.0, -4.0  # absmax 127: q == x
    high = (1 << 5) | (1 << 16)                       # elements 5 and 16 read 0
    w = bytes([0x00, 0x3C]) + high.to_bytes(4, "little") + bytes(16)
    out = oracle.quantized_matmul(5, w, x, 1, 1, 32)
    assert out[0, 0] == np.float32(-16 * (127.0 - 4.0))
    # nibble 0xF in the low half of byte 3 (element 3) and the high half (element 19), fifth
    # bits set on both: 31 - 16 = 15 each; every other element -16
    x2 = np.zeros(32, np.float32)
    x2[3], x2[19], x2[0] = 2.0, 3.0, 127.0
    packed = bytearray(16)
    packed[3] = 0xFF
    w2 = bytes([0x00, 0x3C]) + ((1 << 3) | (1 << 19)).to_bytes(4, "little") + bytes(packed)
    out2 = oracle.quantized_matmul(5, w2, x2, 1, 1, 32)
    assert out2[0, 0] == np.float32(15 * 2.0 + 15 * 3.0 - 16 * 127.0)


def test_q5_0_fixture_blocks_dequantize_to_their_logical_values(known_answers):
    """fillQ5_0Weights records each lane's 5-bit low and high values; numpy's GGML Q5_0
    dequantization recovers them (before the -16 offset)."""
    for case in (c for c in known_answers["quantized_matmul"] if c["format"] == 5):
        w, rows, cols = bytes.fromhex(case["weights_hex"]), case["rows"], case["cols"]
        _, vals = _dequantize_numpy(5, w, rows, cols)
        np.testing.assert_array_equal(vals.reshape(-1, 32) + 16, np.array(case["logical"]["quants"]))


@pytest.mark.parametrize("fmt", [0, 1, 5])
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
        if case["format"] not in (0, 1, 5):
            continue  # the K-quant cases: test_kquant_matmul_matches_float64
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


# ------------------------------------------------------------------ K-quants (Q8_K activations)

def _q8_k_numpy(x, cols):
    """Q8_K from numpy's float32 ops: the block's largest-magnitude element (first on ties, NaN
    skipped) sets inverse = -127 / max; q = min(rint(inverse * x), 127); 16-element sums;
    scale = 1 / inverse."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    q = np.zeros(x.shape, np.int32)
    scales = np.zeros(x.shape[0], np.float32)
    for i, v in enumerate(x):
        a = np.where(np.isnan(v), np.float32(-1), np.abs(v))
        k = int(np.argmax(a))  # first index of the largest magnitude
        if a[k] <= 0:
            continue
        inverse = np.float32(-127) / v[k]
        with np.errstate(invalid="ignore"):
            scaled = (inverse * v).astype(np.float32)
        q[i] = np.minimum(np.where(np.isnan(scaled), 0, np.rint(scaled)), 127)
        scales[i] = np.float32(1) / inverse
    sums = q.reshape(-1, 16).sum(axis=1)
    return q.reshape(-1).astype(np.int8), scales, sums.astype(np.int16)


def _dequant_q4_k(w, rows, cols):
    """GGML Q4_K (144-byte blocks of 256): d, dmin, 6-bit scales and mins of 8 groups packed in 12
    bytes, group g's 32 nibbles in bytes 32(g/2) .. +31 (low nibble for even g)."""
    b = np.frombuffer(bytes(w), np.uint8).reshape(rows, cols // 256, 144)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
    dmin = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
    sc = b[:, :, 4:16].astype(np.int32)
    scales = np.zeros((rows, cols // 256, 8), np.int32)
    mins = np.zeros_like(scales)
    scales[..., :4] = sc[..., 0:4] & 63
    mins[..., :4] = sc[..., 4:8] & 63
    scales[..., 4:] = (sc[..., 8:12] & 15) | ((sc[..., 0:4] >> 6) << 4)
    mins[..., 4:] = (sc[..., 8:12] >> 4) | ((sc[..., 4:8] >> 6) << 4)
    qs = b[:, :, 16:144].astype(np.int32).reshape(rows, cols // 256, 4, 32)
    quants = np.stack([qs & 15, qs >> 4], axis=3).reshape(rows, cols // 256, 8, 32)
    return d, dmin, scales, mins, quants


def _dequant_q5_k(w, rows, cols):
    """GGML Q5_K (176-byte blocks of 256): Q4_K's d, dmin and 6-bit scales and mins, qh[32] at
    byte 16 (bit g of qh[i] is the fifth bit of element i of group g), the nibbles at byte 48."""
    b = np.frombuffer(bytes(w), np.uint8).reshape(rows, cols // 256, 176)
    q4 = np.concatenate([b[:, :, :16], b[:, :, 48:]], axis=2).reshape(-1).tobytes()
    d, dmin, scales, mins, nib = _dequant_q4_k(q4, rows, cols)
    qh = b[:, :, 16:48].astype(np.int32)
    fifth = (qh[:, :, None, :] >> np.arange(8)[None, None, :, None]) & 1
    return d, dmin, scales, mins, nib + 16 * fifth


def _dequant_q6_k(w, rows, cols):
    """GGML Q6_K (210-byte blocks of 256): element 128h + 32t + i of half h takes the low nibble
    of ql[64h + i (+32 for t odd)] (high nibble for t >= 2) and bits 2t..2t+1 of qh[32h + i] as
    its top two bits, minus 32; int8 scale per 16 elements; f16 d at byte 208."""
    b = np.frombuffer(bytes(w), np.uint8).reshape(rows, cols // 256, 210).astype(np.int32)
    q = np.zeros((rows, cols // 256, 256), np.int32)
    for h in range(2):
        ql = b[..., 64 * h:64 * h + 64]
        qh = b[..., 128 + 32 * h:128 + 32 * h + 32]
        for t in range(4):
            low = (ql[..., 32 * (t & 1):32 * (t & 1) + 32] >> (4 * (t >> 1))) & 15
            q[..., 128 * h + 32 * t:128 * h + 32 * t + 32] = (low | (((qh >> (2 * t)) & 3) << 4)) - 32
    scales = b[..., 192:208].astype(np.int8).astype(np.int32)
    d = np.frombuffer(bytes(w), np.uint8).reshape(rows, cols // 256, 210)[..., 208:210].copy()
    d = d.view(np.float16).astype(np.float32)[..., 0]
    return d, scales, q


def _float64_kquant(fmt, w, x, batch, rows, cols):
    q, ascale, asum = _q8_k_numpy(x, cols)
    nb = cols // 256
    q = q.reshape(batch, nb, 256).astype(np.int64)
    ascale = ascale.reshape(batch, nb)
    if fmt in (2, 4):
        d, dmin, scales, mins, quants = (_dequant_q4_k if fmt == 2 else _dequant_q5_k)(w, rows, cols)
        dots = np.einsum("rkgj,bkgj->brkg", quants.astype(np.int64), q.reshape(batch, nb, 8, 32))
        qsum = (dots * scales[None]).sum(axis=3)
        gsum = asum.reshape(batch, nb, 8, 2).sum(axis=3).astype(np.int64)
        msum = (mins[None] * gsum[:, None]).sum(axis=3)
        dd = (d[None] * ascale[:, None]).astype(np.float32).astype(np.float64)
        dm = (dmin[None] * ascale[:, None]).astype(np.float32).astype(np.float64)
        terms = np.stack([dd * qsum, -dm * msum], axis=-1)
    else:
        d, scales, quants = _dequant_q6_k(w, rows, cols)
        per16 = scales.repeat(16, axis=2)  # scale of each element
        prods = np.einsum("rke,bke->brk", (quants * per16).astype(np.int64), q)
        dd = (d[None] * ascale[:, None]).astype(np.float32).astype(np.float64)
        terms = (dd * prods)[..., None]
    return terms.sum(axis=(2, 3)), np.abs(terms).sum(axis=(2, 3)), terms.shape[2] * terms.shape[3] + 8


def test_q8_k_quantize_matches_numpy(oracle):
    x = synth.normal(7, "q8k/x", (6 * 256,)) * 2.0
    x[:256] = 0.0                              # zero block
    x[256:512] *= 0.1
    x[256 + 10] = 5.0                          # ties of magnitude: the first one sets the sign
    x[256 + 20] = -5.0
    x[512 + 3] = np.nan                        # NaN skipped by the maximum
    x[768:1024] = np.linspace(-127, 127, 256)  # max 127 at the end: inverse -1
    q, s, sums = oracle.q8_k_quantize(x, 1, 6 * 256)
    q_ref, s_ref, sums_ref = _q8_k_numpy(x, 6 * 256)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(sums, sums_ref)
    assert s[0] == 0 and not q[:256].any()
    assert s[1] < 0  # first of +5 / -5 is +5: inverse -127 / 5, scale -5 / 127
    assert int(q[256 + 10]) == -127 and int(q[256 + 20]) == 127


@pytest.mark.parametrize("fmt", [2, 3, 4])
def test_kquant_fixture_blocks_dequantize_to_their_logical_values(known_answers, fmt):
    """The reference test's block builders record what each element means; numpy's GGML
    dequantization recovers exactly that, which pins the layouts the float64 check below uses."""
    case = next(c for c in known_answers["quantized_matmul"] if c["format"] == fmt)
    w, rows, cols = bytes.fromhex(case["weights_hex"]), case["rows"], case["cols"]
    lg = case["logical"]
    if fmt in (2, 4):
        d, dmin, scales, mins, quants = (_dequant_q4_k if fmt == 2 else _dequant_q5_k)(w, rows, cols)
        assert (scales == np.array(lg["scales"])).all() and (mins == np.array(lg["mins"])).all()
        np.testing.assert_array_equal(quants.reshape(-1, 256), np.array(lg["quants"]))
        np.testing.assert_array_equal(d[:, 0], (np.arange(rows) + 1) * 0.03125)
    else:
        d, scales, quants = _dequant_q6_k(w, rows, cols)
        np.testing.assert_array_equal(quants.reshape(-1, 256), np.array(lg["quants"]))
        np.testing.assert_array_equal(scales.reshape(-1, 16), np.array(lg["scales"]))


@pytest.mark.parametrize("fmt", [2, 3, 4])
def test_kquant_matmul_matches_float64(oracle, known_answers, fmt):
    cases = [c for c in known_answers["quantized_matmul"] if c["format"] == fmt]
    rnd = _random_kquant(fmt, 9, 1024, f"kq/{fmt}")
    for w, x, b, r, c in [(bytes.fromhex(k["weights_hex"]), np.float32(k["input"]), k["batch"],
                           k["rows"], k["cols"]) for k in cases] + [
            (rnd, synth.normal(7, f"kq/x{fmt}", (2, 1024)), 2, 9, 1024)]:
        out = oracle.quantized_matmul(fmt, w, x, b, r, c)
        ref, mag, n = _float64_kquant(fmt, w, x, b, r, c)
        assert np.all(np.abs(out.astype(np.float64) - ref) <= n * 2.0 ** -24 * mag + 1e-30), fmt


def _random_kquant(fmt, rows, cols, key):
    nbytes = {2: 144, 3: 210, 4: 176}[fmt]
    raw = synth.uniform_int(7, key, rows * cols // 256 * nbytes, 0, 255).astype(np.uint8)
    raw = raw.reshape(rows, cols // 256, nbytes)
    d = (synth.normal(7, key + "/d", (rows, cols // 256, 2)) * 0.01).astype(np.float16).view(np.uint8)
    if fmt in (2, 4):
        raw[:, :, 0:4] = d.reshape(rows, cols // 256, 4)
    else:
        raw[:, :, 208:210] = d.reshape(rows, cols // 256, 4)[..., :2]
    return raw.reshape(-1).tobytes()


def test_q5_k_without_fifth_bits_is_q4_k_and_each_fifth_bit_adds_16(oracle):
    """A Q5_K block with qh cleared is the Q4_K block of the same d, dmin, scales, mins and
    nibbles (the same outputs bit for bit); setting every fifth bit of group g adds
    16 * scale_g * (sum of that group's Q8_K activations) to the block's integer sum, which the
    float64 reference of the dequantized blocks prices exactly."""
    rows, cols = 6, 512
    w5 = np.frombuffer(_random_kquant(4, rows, cols, "q5k/eq"), np.uint8).reshape(rows, 2, 176).copy()
    w5[:, :, 16:48] = 0
    w4 = np.concatenate([w5[:, :, :16], w5[:, :, 48:]], axis=2)
    x = synth.normal(7, "q5k/eq/x", (2, cols))
    a = oracle.quantized_matmul(4, w5.reshape(-1).tobytes(), x, 2, rows, cols)
    b = oracle.quantized_matmul(2, w4.reshape(-1).tobytes(), x, 2, rows, cols)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    w5[:, 1, 16:48] = 0x24  # fifth bits of groups 2 and 5 in the second block
    out = oracle.quantized_matmul(4, w5.reshape(-1).tobytes(), x, 2, rows, cols)
    ref, mag, n = _float64_kquant(4, w5.reshape(-1).tobytes(), x, 2, rows, cols)
    assert np.all(np.abs(out.astype(np.float64) - ref) <= n * 2.0 ** -24 * mag + 1e-30)
    assert not np.array_equal(out, a)

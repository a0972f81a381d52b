"""Pins the CPU oracle against the known answers of the reference's own unit tests
(tests/golden/reference_known_answers.json, transcribed from backend-java's tests)."""

import math

import numpy as np
import pytest

from oracle.oracle import ILLEGAL_ARGUMENT, ILLEGAL_STATE, KvCache, LayeredKvCache, OracleError

ERR = {"IAE": ILLEGAL_ARGUMENT, "ISE": ILLEGAL_STATE}


def _num(x):
    return {"inf": math.inf, "-inf": -math.inf, "nan": math.nan}.get(x, x) if isinstance(x, str) \
        else x


def _run_kv_ops(cache, ops):
    for op in ops:
        if op[0] == "store":
            cache.store(op[1], op[2], op[3], op[4])
        elif op[0] == "reserve":
            cache.reserve_sequence_capacity(op[1])
        elif op[0] == "clear":
            cache.clear()
        elif op[0] == "discard":
            cache.discard_from(op[1])
        else:
            raise AssertionError(op)


def _check_kv(cache, expectations):
    for e in expectations:
        kind = e[0]
        if kind in ("key", "value"):
            got = getattr(cache, kind)(e[1], e[2])
            if e[3] is None:
                assert got is None, e
            else:
                np.testing.assert_array_equal(got, np.float32(e[3]), err_msg=str(e))
        elif kind in ("keyNotNull", "valueNotNull"):
            assert getattr(cache, kind[:-7])(e[1], e[2]) is not None, e
        elif kind == "keyOffset":
            assert cache.key_offset(e[1], e[2]) == e[3], e
        elif kind == "valueOffset":
            assert cache.value_offset(e[1], e[2]) == e[3], e
        elif kind == "keyBuffer":
            np.testing.assert_array_equal(cache.key_buffer(), np.float32(e[1]))
        elif kind == "valueBuffer":
            np.testing.assert_array_equal(cache.value_buffer(), np.float32(e[1]))
        elif kind == "keyBufferLength":
            assert cache.key_buffer().size == e[1]
        elif kind == "valueBufferLength":
            assert cache.value_buffer().size == e[1]
        elif kind == "capacity":
            assert cache.allocated_sequence_capacity() == e[1]
        elif kind in ("keySlice", "valueSlice"):
            fn = cache.key_slice if kind == "keySlice" else cache.value_slice
            if isinstance(e[4], str):
                with pytest.raises(OracleError) as info:
                    fn(e[1], e[2], e[3])
                assert info.value.status == ERR[e[4]], e
            else:
                np.testing.assert_array_equal(fn(e[1], e[2], e[3]), np.float32(e[4]))
        elif kind == "storeError":
            with pytest.raises(OracleError) as info:
                cache.store(e[1], e[2], np.zeros(cache.key_dim), np.zeros(cache.value_dim))
            assert info.value.status == ERR[e[3]], e
        elif kind == "reserveError":
            with pytest.raises(OracleError) as info:
                cache.reserve_sequence_capacity(e[1])
            assert info.value.status == ERR[e[2]], e
        else:
            raise AssertionError(e)


def test_kv_cache_known_answers(oracle, known_answers):
    for case in known_answers["kv_cache"]:
        cache = KvCache(*case["ctor"], half_precision=case.get("half_precision", False))
        _run_kv_ops(cache, case["ops"])
        _check_kv(cache, case["expect"])
        if "then_ops" in case:
            _run_kv_ops(cache, case["then_ops"])
            _check_kv(cache, case["then_expect"])


def _run_lkv_ops(cache, ops):
    for op in ops:
        if op[0] == "store":
            cache.store(op[1], op[2], op[3], op[4])
        elif op[0] == "clear":
            cache.clear()
        elif op[0] == "discard":
            cache.discard_from(op[1])
        else:
            raise AssertionError(op)


def _contains_sequence(buf, seq):
    seq = np.float32(seq)
    n = len(seq)
    return any(np.array_equal(buf[i:i + n], seq) for i in range(len(buf) - n + 1))


def _check_lkv(cache, expectations):
    for e in expectations:
        kind = e[0]
        if kind == "allocatedCapacity":
            assert cache.allocated_sequence_capacity(e[1]) == e[2], e
        elif kind == "allocatedCapacityAtLeast":
            assert cache.allocated_sequence_capacity(e[1]) >= e[2], e
        elif kind == "physicalCapacity":
            assert cache.physical_sequence_capacity(e[1]) == e[2], e
        elif kind == "contains":
            assert cache.contains(e[1], e[2]) == e[3], e
        elif kind == "keyOffset":
            assert cache.key_offset(e[1], e[2]) == e[3], e
        elif kind == "valueOffset":
            dv = cache.specs[e[1]][1]
            assert cache.key_offset(e[1], e[2]) // cache.specs[e[1]][0] * dv == e[3], e
        elif kind == "keyBufferContains":
            assert _contains_sequence(cache.key_buffer(e[1]), e[2]), e
        elif kind == "valueBufferContains":
            assert _contains_sequence(cache.value_buffer(e[1]), e[2]), e
        elif kind == "keyBuffer":
            np.testing.assert_array_equal(cache.key_buffer(e[1]), np.float32(e[2]))
        elif kind == "valueBuffer":
            np.testing.assert_array_equal(cache.value_buffer(e[1]), np.float32(e[2]))
        elif kind == "oldest":
            assert cache.oldest_retained_position(e[1]) == e[2], e
        elif kind == "newest":
            assert cache.newest_retained_position(e[1]) == e[2], e
        elif kind == "view":
            assert [list(s) for s in cache.attention_view(e[1], e[2], e[3])] == e[4], e
        elif kind == "viewCount":
            spans = cache.attention_view(e[1], e[2], e[3])
            assert sum(s[1] for s in spans) == e[4], e
        elif kind == "viewError":
            with pytest.raises(OracleError) as info:
                cache.attention_view(e[1], e[2], e[3])
            assert info.value.status == ERR[e[4]], e
        elif kind == "storeError":
            with pytest.raises(OracleError) as info:
                cache.store(e[1], e[2], e[3], e[4])
            assert info.value.status == ERR[e[5]], e
        elif kind == "allocatedBytes":
            assert cache.allocated_bytes() == e[1], e
        elif kind == "maximumBytes":
            assert cache.maximum_bytes() == e[1], e
        else:
            raise AssertionError(e)


def test_layered_kv_cache_known_answers(oracle, known_answers):
    for case in known_answers["layered_kv_cache"]:
        cache = LayeredKvCache(case["ctor"][0], case["ctor"][1])
        _check_lkv(cache, case.get("expect_before", []))
        _run_lkv_ops(cache, case["ops"])
        _check_lkv(cache, case["expect"])
        if "then_ops" in case:
            _run_lkv_ops(cache, case["then_ops"])
            _check_lkv(cache, case["then_expect"])
        if "final_ops" in case:
            _run_lkv_ops(cache, case["final_ops"])
            _check_lkv(cache, case["final_expect"])


def test_rope_known_answers(oracle, known_answers):
    for case in known_answers["rope"]:
        x = np.float32(case["input"])
        if case.get("direct"):
            out = oracle.rope_direct(x, case["position"], case["head_dim"], case["theta"],
                                     case["frequency_scale"], case["neox"])
        else:
            c, s = oracle.rotary_factors(case["rotary_dim"], case["theta"],
                                         case["frequency_scale"], case["position"],
                                         factors=case.get("factors"))
            out = oracle.rope_apply(x, c, s, case["neox"])
        for idx, value, tol in case.get("expect_close", []):
            assert abs(float(out[idx]) - value) <= tol, (case["name"], idx, out[idx], value)
        for idx, value in case.get("expect_exact", []):
            assert out[idx] == np.float32(value), (case["name"], idx)
        if case.get("neox_equals_standard"):
            other = oracle.rope_direct(x, case["position"], case["head_dim"], case["theta"],
                                       case["frequency_scale"], not case["neox"])
            np.testing.assert_array_equal(other, out)


def test_softmax_known_answers(oracle, known_answers):
    for case in known_answers["softmax"]:
        x = np.array([_num(v) for v in case["input"]], dtype=np.float32)
        if "expect_error" in case:
            with pytest.raises(OracleError) as info:
                oracle.softmax(x)
            assert info.value.status == ERR[case["expect_error"]], case["name"]
            continue
        out = oracle.softmax(x)
        for idx, value, tol in case.get("expect_close", []):
            assert abs(float(out[idx]) - value) <= tol, case["name"]
        if "expect_sum" in case:
            assert abs(float(out.sum(dtype=np.float32)) - case["expect_sum"][0]) <= \
                case["expect_sum"][1], case["name"]
        if case.get("expect_positive_finite"):
            assert np.all(np.isfinite(out)) and np.all(out > 0), case["name"]
        if "expect_pair_sum" in case:
            i, j, value, tol = case["expect_pair_sum"]
            assert abs(float(out[i] + out[j]) - value) <= tol, case["name"]


def test_attention_start_known_answers(oracle, known_answers):
    for case in known_answers["attention_start"]:
        assert oracle.attention_start(case["position"], case["window"]) == case["expect"], case


def test_sliding_layer_pattern(known_answers):
    from models_amd.attention import uses_sliding_window
    case = known_answers["sliding_layers"]
    got = [uses_sliding_window(l, case["pattern"], 512) for l in range(case["layers"])]
    assert got == case["sliding"]


def test_rms_norm_known_answers(oracle, known_answers):
    # TensorOpsTest.RmsNorm (ops/TensorOpsTest.java:42-67).
    for case in known_answers["rms_norm"]:
        out = oracle.rms_norm(case["x"], case["weight"], case["eps"])
        for i, want, tol in case["expect_close"]:
            assert abs(float(out[i]) - want) <= tol, (case["name"], i, out[i], want)


def test_value_norm_known_answers(oracle, known_answers):
    # Gemma4MathTest.normalizesAnUnweightedHeadInPlaceWithoutTouchingAdjacentValues
    # (gemma4/Gemma4MathTest.java:28-38).
    for case in known_answers["value_norm"]:
        out = oracle.value_rms_norm(case["values"], case["eps"], case["offset"], case["length"])
        for i, want in case["expect_equal"]:
            assert float(out[i]) == want, (case["name"], i)
        for i, want, tol in case["expect_close"]:
            assert abs(float(out[i]) - want) <= tol, (case["name"], i, out[i], want)

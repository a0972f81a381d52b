"""Writes ``reference_known_answers.json``: the known-answer cases of the reference's own unit
tests for the attention/KV-cache path, transcribed as data (inputs, operations, expected outputs).

Every case names the test file:line it comes from, relative to
``backend-java/src/test/java/com/integrallis/models/backend/purejava/``. Nothing here imports or
runs the reference; the values are the literals its assertions hold. Run it to regenerate the
fixture (it is deterministic):

    python tests/golden/make_fixtures.py
"""

import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def kv_cases():
    # Ops: ["store", layer, pos, key, value] | ["reserve", n] | ["clear"] | ["discard", pos]
    # Expectations: key/value (None = null), keyOffset/valueOffset, keyBuffer/valueBuffer,
    # capacity, slices, and errors ("IAE" IllegalArgumentException / "ISE" IllegalStateException).
    return [
        {
            "name": "storeAndRetrieveSinglePosition", "src": "cache/KvCacheTest.java:42-51",
            "ctor": [2, 10, 4, 4],
            "ops": [["store", 0, 0, [1, 2, 3, 4], [5, 6, 7, 8]]],
            "expect": [["key", 0, 0, [1, 2, 3, 4]], ["value", 0, 0, [5, 6, 7, 8]]],
        },
        {
            "name": "sequentialPositions", "src": "cache/KvCacheTest.java:53-62",
            "ctor": [1, 10, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]], ["store", 0, 1, [3, 4], [30, 40]],
                    ["store", 0, 2, [5, 6], [50, 60]]],
            "expect": [["key", 0, 1, [3, 4]], ["value", 0, 2, [50, 60]]],
        },
        {
            "name": "storesVectorsFromBatchOffsets", "src": "cache/KvCacheTest.java:64-74",
            "ctor": [1, 10, 2, 3],
            # store(0, 1, {99,1,2,98}, 1, {97,96,10,20,30,95}, 2): the offset windows are [1,2]
            # and [10,20,30]
            "ops": [["store", 0, 1, [1, 2], [10, 20, 30]]],
            "expect": [["key", 0, 1, [1, 2]], ["value", 0, 1, [10, 20, 30]]],
        },
        {
            "name": "storesVectorsInContiguousFlatBuffers", "src": "cache/KvCacheTest.java:76-93",
            "ctor": [2, 3, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]], ["store", 0, 1, [3, 4], [30, 40]],
                    ["store", 1, 0, [5, 6], [50, 60]]],
            "expect": [["keyOffset", 0, 0, 0], ["keyOffset", 0, 1, 2], ["keyOffset", 1, 0, 6],
                       ["valueOffset", 0, 0, 0], ["valueOffset", 0, 1, 2],
                       ["valueOffset", 1, 0, 6],
                       ["keyBuffer", [1, 2, 3, 4, 0, 0, 5, 6, 0, 0, 0, 0]],
                       ["valueBuffer", [10, 20, 30, 40, 0, 0, 50, 60, 0, 0, 0, 0]]],
        },
        {
            "name": "sliceCorrectRange", "src": "cache/KvCacheTest.java:113-125",
            "ctor": [1, 10, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]], ["store", 0, 1, [3, 4], [30, 40]],
                    ["store", 0, 2, [5, 6], [50, 60]]],
            "expect": [["keySlice", 0, 0, 3, [1, 2, 3, 4, 5, 6]],
                       ["valueSlice", 0, 1, 3, [30, 40, 50, 60]]],
        },
        {
            "name": "keySliceRejectsAnUnpopulatedPosition", "src": "cache/KvCacheTest.java:127-137",
            "ctor": [1, 10, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]], ["store", 0, 2, [5, 6], [50, 60]]],
            "expect": [["keySlice", 0, 0, 3, "ISE"]],
        },
        {
            "name": "valueSliceRejectsAPositionWithoutAllocatedStorage",
            "src": "cache/KvCacheTest.java:139-148",
            "ctor": [1, 40, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]]],
            "expect": [["valueSlice", 0, 16, 17, "ISE"]],
        },
        {
            "name": "layersAreIndependent", "src": "cache/KvCacheTest.java:154-162",
            "ctor": [2, 10, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [10, 20]], ["store", 1, 0, [3, 4], [30, 40]]],
            "expect": [["key", 0, 0, [1, 2]], ["key", 1, 0, [3, 4]]],
        },
        {
            "name": "clearResetsAllEntries", "src": "cache/KvCacheTest.java:168-181",
            "ctor": [1, 10, 2, 2],
            "ops": [["store", 0, 0, [1, 2], [3, 4]], ["clear"]],
            "expect": [["key", 0, 0, None], ["value", 0, 0, None]],
            "then_ops": [["store", 0, 0, [5, 6], [7, 8]]],
            "then_expect": [["key", 0, 0, [5, 6]], ["value", 0, 0, [7, 8]]],
        },
        {
            "name": "discardFromPreservesAcceptedPrefixAndClearsSpeculativeTail",
            "src": "cache/KvCacheTest.java:183-207",
            "ctor": [2, 10, 2, 2],
            "ops": [["store", l, p, [l * 10 + p, l * 10 + p + 0.25],
                     [l * 10 + p + 0.5, l * 10 + p + 0.75]] for l in range(2) for p in range(4)]
            + [["discard", 2]],
            "expect": [["keyNotNull", 0, 1], ["valueNotNull", 1, 1], ["key", 0, 2, None],
                       ["value", 1, 3, None]],
        },
        {
            "name": "largeLogicalContextStartsWithSmallPhysicalCapacity",
            "src": "cache/KvCacheTest.java:209-216",
            "ctor": [2, 10000, 4, 4],
            "ops": [],
            "expect": [["capacity", 16], ["keyBufferLength", 2 * 16 * 4],
                       ["valueBufferLength", 2 * 16 * 4]],
        },
        {
            "name": "growthPreservesEntriesAndLayerIsolation", "src": "cache/KvCacheTest.java:218-232",
            "ctor": [2, 40, 2, 3],
            "ops": [["store", 0, 0, [1, 2], [10, 20, 30]], ["store", 1, 0, [3, 4], [40, 50, 60]],
                    ["store", 0, 20, [5, 6], [70, 80, 90]]],
            "expect": [["capacity", 32], ["key", 0, 0, [1, 2]], ["value", 1, 0, [40, 50, 60]],
                       ["key", 0, 20, [5, 6]], ["keyOffset", 1, 0, 64],
                       ["valueOffset", 1, 0, 96]],
        },
        {
            "name": "reservationGrowsStorageBeforeDisjointBatchWrites",
            "src": "cache/KvCacheTest.java:234-244",
            "ctor": [2, 40, 2, 3],
            "ops": [["reserve", 24], ["store", 0, 23, [1, 2], [3, 4, 5]]],
            "expect": [["capacity", 32], ["key", 0, 23, [1, 2]]],
        },
        {
            "name": "positionBeyondMaxThrows", "src": "cache/KvCacheTest.java:249-263",
            "ctor": [1, 5, 2, 2],
            "ops": [],
            "expect": [["storeError", 0, 5, "IAE"], ["reserveError", 6, "IAE"]],
        },
        {
            "name": "layerOutOfRangeThrows", "src": "cache/KvCacheTest.java:266-279",
            "ctor": [2, 10, 2, 2],
            "ops": [],
            "expect": [["storeError", -1, 0, "IAE"], ["storeError", 2, 0, "IAE"]],
        },
        {
            "name": "keepsExactlyRepresentableValuesUnchanged",
            "src": "cache/KvCacheTest.java:293-301",
            "ctor": [1, 2, 2, 2],
            "half_precision": True,
            "ops": [["store", 0, 0, [0.5, -2.25], [0.5, -2.25]]],
            "expect": [["keySlice", 0, 0, 1, [0.5, -2.25]], ["valueSlice", 0, 0, 1, [0.5, -2.25]]],
        },
    ]


def layered_cases():
    # ctor: [maxSeqLen, [[keyDim, valueDim, ringCapacity(0 = linear)], ...]]
    def seq(size, start):
        return [start + i for i in range(size)]

    return [
        {
            "name": "linearLayerGrowsLazilyAndPreservesAbsoluteHistory",
            "src": "cache/LayeredKvCacheTest.java:28-46",
            "ctor": [64, [[2, 1, 0]]],
            "expect_before": [["allocatedCapacity", 0, 0]],
            "ops": [["store", 0, 0, [1, 2], [3]], ["store", 0, 20, [4, 5], [6]]],
            "expect": [["allocatedCapacityAtLeast", 0, 21], ["contains", 0, 0, True],
                       ["contains", 0, 20, True], ["keyOffset", 0, 20, 40],
                       ["valueOffset", 0, 20, 20], ["keyBufferContains", 0, [1, 2]],
                       ["keyBufferContains", 0, [4, 5]], ["oldest", 0, 0], ["newest", 0, 20]],
        },
        {
            "name": "ringLayerRejectsOverwrittenPositionsAndSplitsAViewAtWraparound",
            "src": "cache/LayeredKvCacheTest.java:48-77",
            "ctor": [16, [[2, 1, 4]]],
            "ops": [["store", 0, p, [p * 10.0, p * 10.0 + 1], [p * 100.0]] for p in range(6)],
            "expect": [["contains", 0, 0, False], ["contains", 0, 1, False], ["oldest", 0, 2],
                       ["newest", 0, 5],
                       ["view", 0, 2, 6, [[2, 2, 4, 2], [4, 2, 0, 0]]],
                       ["keyBuffer", 0, [40, 41, 50, 51, 20, 21, 30, 31]],
                       ["valueBuffer", 0, [400, 500, 200, 300]],
                       ["viewError", 0, 1, 5, "ISE"]],
        },
        {
            "name": "ringCapacityCanRetainAWindowWhileAnEntirePrefillChunkIsWritten",
            "src": "cache/LayeredKvCacheTest.java:79-93",
            "ctor": [32, [[1, 1, 5]]],
            "ops": [["store", 0, p, [p], [-p]] for p in range(2, 7)],
            "expect": [["viewCount", 0, 2, 5, 3], ["viewCount", 0, 4, 7, 3],
                       ["contains", 0, 2, True], ["contains", 0, 6, True]],
        },
        {
            "name": "mixedLayerShapesUseIndependentLinearAndRingStorage",
            "src": "cache/LayeredKvCacheTest.java:95-112",
            "ctor": [32, [[4, 2, 8], [2, 3, 0]]],
            "ops": [["store", 0, 3, seq(4, 10), seq(2, 20)], ["store", 1, 3, seq(2, 30), seq(3, 40)]],
            "expect": [["keyBufferContains", 0, [10, 11, 12, 13]],
                       ["valueBufferContains", 1, [40, 41, 42]],
                       ["allocatedBytes", (8 * (4 + 2) * 4 + 8 * 4) + (16 * (2 + 3) * 4 + 16 * 4)]],
        },
        {
            "name": "discardFromPreservesTheAcceptedPrefixAcrossLinearAndRingLayers",
            "src": "cache/LayeredKvCacheTest.java:114-139",
            "ctor": [32, [[1, 1, 6], [1, 1, 0]]],
            "ops": [op for p in range(8)
                    for op in (["store", 0, p, [p], [p]], ["store", 1, p, [p], [p]])]
            + [["discard", 6]],
            "expect": [["contains", 0, 5, True], ["contains", 0, 6, False],
                       ["contains", 0, 7, False], ["contains", 1, 5, True],
                       ["contains", 1, 6, False], ["contains", 1, 7, False]],
            "then_ops": [["store", 0, 6, [60], [61]], ["store", 1, 6, [60], [61]]],
            "then_expect": [["viewCount", 0, 2, 7, 5], ["viewCount", 1, 0, 7, 7]],
            "final_ops": [["clear"]],
            "final_expect": [["oldest", 0, None], ["oldest", 1, None]],
        },
        {
            "name": "validatesCoordinatesVectorRangesAndAttentionRanges",
            "src": "cache/LayeredKvCacheTest.java:141-158",
            "ctor": [8, [[2, 1, 4]]],
            "ops": [],
            "expect": [["storeError", 0, 0, [1], [2], "IAE"], ["storeError", 1, 0, [1, 2], [3], "IAE"],
                       ["storeError", 0, 8, [1, 2], [3], "IAE"], ["viewError", 0, 0, 5, "IAE"]],
        },
        {
            "name": "gemma4MapsSlidingAndFullAttentionLayers",
            "src": "gemma4/Gemma4KvCacheTest.java:28-45 (Gemma4KvCache.create, gemma4/Gemma4KvCache.java:27-50)",
            # 30 layers; full layers (layer+1) % 6 == 0 hold 2 KV heads of 512, sliding layers
            # 8 KV heads of 256 in a ring of window 1024 + prefill chunk 128.
            "ctor": [8192, [[1024, 1024, 0] if (l + 1) % 6 == 0 else [2048, 2048, 1152]
                            for l in range(30)]],
            "ops": [],
            "expect": [["physicalCapacity", 0, 1152], ["physicalCapacity", 5, 8192],
                       ["allocatedBytes", 0], ["maximumBytes", 807682560]],
        },
        {
            "name": "gemma4CapsSlidingStorageWhenTheRuntimeContextIsShorter",
            "src": "gemma4/Gemma4KvCacheTest.java:48-53",
            "ctor": [512, [[1024, 1024, 0] if (l + 1) % 6 == 0 else [2048, 2048, 1152]
                           for l in range(30)]],
            "ops": [],
            "expect": [["physicalCapacity", 0, 512], ["physicalCapacity", 5, 512]],
        },
    ]


def rope_cases():
    return [
        {
            "name": "ggufFrequencyFactorsPreserveGemma4ProportionalRopeLayout",
            "src": "ops/RotaryTableTest.java:80-91",
            "rotary_dim": 8, "theta": 1000000.0, "frequency_scale": 1.0,
            "factors": [1.0, 1.0e30, 1.0e30, 1.0e30], "position": 2, "neox": True,
            "input": [1, 2, 3, 4, 5, 6, 7, 8],
            "expect_close": [[0, -4.9626341, 1e-6], [4, -1.1714368, 1e-6]],
            "expect_exact": [[1, 2], [2, 3], [3, 4], [5, 6], [6, 7], [7, 8]],
        },
        {
            "name": "neoxLayoutRotatesPairsSeparatedByHalfAHead",
            "src": "ops/TensorOpsTest.java:1527-1541",
            "direct": True, "head_dim": 4, "theta": 10000.0, "frequency_scale": 1.0,
            "position": 1, "neox": True, "input": [1.0, 2.0, 3.0, 4.0],
            # pair 0 angle 1.0, pair 1 angle 0.01
            "expect_close": [
                [0, 1.0 * math.cos(1.0) - 3.0 * math.sin(1.0), 1e-6],
                [2, 1.0 * math.sin(1.0) + 3.0 * math.cos(1.0), 1e-6],
                [1, 2.0 * math.cos(0.01) - 4.0 * math.sin(0.01), 1e-6],
                [3, 2.0 * math.sin(0.01) + 4.0 * math.cos(0.01), 1e-6]],
        },
        {
            "name": "appliesFrequencyScaleToNormalAndNeoxRope",
            "src": "ops/TensorOpsTest.java:1543-1556",
            "direct": True, "head_dim": 2, "theta": 10000.0, "frequency_scale": 0.25,
            "position": 2, "neox": False, "input": [1.0, 2.0],
            "expect_close": [[0, math.cos(0.5) - 2.0 * math.sin(0.5), 1e-6],
                             [1, math.sin(0.5) + 2.0 * math.cos(0.5), 1e-6]],
            "neox_equals_standard": True,
        },
    ]


def softmax_cases():
    inf = "inf"
    return [
        {"name": "uniformInputProducesUniform", "src": "ops/TensorOpsTest.java:1371-1378",
         "input": [1, 1, 1, 1], "expect_close": [[i, 0.25, 1e-5] for i in range(4)]},
        {"name": "sumsToOne", "src": "ops/TensorOpsTest.java:1381-1387",
         "input": [1, 2, 3], "expect_sum": [1.0, 1e-5]},
        {"name": "numericallyStableWithLargeValues", "src": "ops/TensorOpsTest.java:1390-1401",
         "input": [1000, 1001, 1002], "expect_sum": [1.0, 1e-5], "expect_positive_finite": True},
        {"name": "preservesNegativeInfinityAsAZeroProbabilityMask",
         "src": "ops/TensorOpsTest.java:1415-1422",
         "input": [1.0, "-inf", 2.0], "expect_close": [[1, 0.0, 0.0]],
         "expect_pair_sum": [0, 2, 1.0, 1e-5]},
        {"name": "rejectsEmptyAndNegativeSizes", "src": "ops/TensorOpsTest.java:1425-1434",
         "input": [], "expect_error": "IAE"},
        {"name": "rejectsAnAllMaskedRow", "src": "ops/TensorOpsTest.java:1437-1443",
         "input": ["-inf", "-inf"], "expect_error": "IAE"},
        {"name": "rejectsNaN", "src": "ops/TensorOpsTest.java:1446-1453",
         "input": [1.0, "nan"], "expect_error": "IAE"},
        {"name": "rejectsPositiveInfinity", "src": "ops/TensorOpsTest.java:1446-1453",
         "input": [1.0, inf], "expect_error": "IAE"},
    ]


def rms_norm_cases():
    # TensorOpsTest.RmsNorm (:42-67): out = x * (1 / rms) * w, rms = sqrt(mean(x^2) + eps).
    return [
        {"name": "identityWeightNormalizesCorrectly", "src": "ops/TensorOpsTest.java:42-54",
         "x": [3.0, 4.0], "weight": [1.0, 1.0], "eps": 1e-5,
         "expect_close": [[0, 3.0 / math.sqrt(12.5), 1e-4], [1, 4.0 / math.sqrt(12.5), 1e-4]]},
        {"name": "weightScalesOutput", "src": "ops/TensorOpsTest.java:56-67",
         "x": [1.0, 1.0], "weight": [2.0, 3.0], "eps": 1e-5,
         "expect_close": [[0, 2.0, 1e-4], [1, 3.0, 1e-4]]},
    ]


def value_norm_cases():
    # Gemma4MathTest (gemma4/Gemma4MathTest.java:28-38): normalizeWithoutWeight over values[1..2]
    # of {99, 3, 4, 98} with eps 1e-6; the neighbours stay untouched.
    return [
        {"name": "normalizesAnUnweightedHeadInPlaceWithoutTouchingAdjacentValues",
         "src": "gemma4/Gemma4MathTest.java:28-38",
         "values": [99.0, 3.0, 4.0, 98.0], "offset": 1, "length": 2, "eps": 1e-6,
         "expect_equal": [[0, 99.0], [3, 98.0]],
         "expect_close": [[1, 0.8485281, 1e-6], [2, 1.1313708, 1e-6]]},
    ]


def window_cases():
    # EncoderAttentionWindowTest CausalWindow (GEMMA3, window 512, pattern 6): layer 0 slides,
    # layer 5 is global (:37-40, 128-145); LlamaConfig.usesSlidingWindow (:157-162).
    return [
        {"src": "llama/EncoderAttentionWindowTest.java:133-136", "position": 700, "window": 512,
         "expect": 700 - 512 + 1},
        {"src": "llama/LlamaConfig.java:184-195 (global layer)", "position": 700, "window": 0,
         "expect": 0},
        {"src": "llama/LlamaConfig.java:194 (clamps at 0)", "position": 10, "window": 512,
         "expect": 0},
        {"src": "llama/LlamaConfig.java:194 (first full window)", "position": 511,
         "window": 512, "expect": 0},
        {"src": "llama/LlamaConfig.java:194 (window starts sliding)", "position": 512,
         "window": 512, "expect": 1},
    ]


def sliding_layers():
    # usesSlidingWindow(layer) = layer % pattern < pattern - 1 (LlamaConfig.java:157-162) and
    # EncoderAttentionWindowTest :110-118 for 24 layers, pattern 6.
    return {"src": "llama/EncoderAttentionWindowTest.java:110-118", "layers": 24, "pattern": 6,
            "sliding": [l % 6 != 5 for l in range(24)]}


def _f16_bits(x):
    import numpy as np
    return int(np.array([x], np.float32).astype(np.float16).view(np.uint16)[0])


def quantized_matmul_cases():
    # backend-native/src/test/java/com/integrallis/models/backend/nativekernel/
    # NativeKernelLibraryTest.java: the synthetic activations and weights its quantized-matmul
    # tests build (inputs :660-668, fillWeights :670-684, fillQ8_0Weights :686-702), written out
    # as data. The relation each test asserts between the native kernel and the test's own
    # reference (:909-1023) is kept with the case: "exact" (containsExactly) or an absolute
    # tolerance (BLOCK_QUANT_REDUCTION_TOLERANCE 2e-5, :35).
    def activations(batch, cols):
        return [((col * 17 + b * 11) % 29 - 14) * 0.125 for b in range(batch) for col in range(cols)]

    def q4_0_weights(rows, cols):
        out = bytearray()
        for row in range(rows):
            for block in range(cols // 32):
                out += _f16_bits((row + block + 1) * 0.125).to_bytes(2, "little")
                for lane in range(16):
                    low = (row * 3 + block * 5 + lane) & 0xF
                    high = (row * 7 + block * 2 + lane * 3) & 0xF
                    out.append(low | high << 4)
        return out.hex()

    def q8_0_weights(rows, cols):
        out = bytearray()
        for row in range(rows):
            for block in range(cols // 32):
                out += _f16_bits((row + block + 1) * 0.03125).to_bytes(2, "little")
                for lane in range(32):
                    out.append(((row * 37 + block * 19 + lane * 11) & 0xFF) - 128 & 0xFF)
        return out.hex()

    cases = []
    for name, src, batch, rows in (
            ("computesQ4_0BatchedMatrixMultiplication", ":67-84", 2, 3),
            ("reusableGgufKernelComputesAcrossWorkspaceGrowth[1x2]", ":101-126", 1, 2),
            ("reusableGgufKernelComputesAcrossWorkspaceGrowth[3x128]", ":101-126", 3, 128)):
        cases.append({"name": name, "src": "NativeKernelLibraryTest.java" + src, "format": 0,
                      "batch": batch, "rows": rows, "cols": 64, "relation": "exact",
                      "input": activations(batch, 64), "weights_hex": q4_0_weights(rows, 64)})
    # K-quant blocks (q4KBlock :740-764, q6KBlock :830-858, q6Quant :860-862), each with the
    # logical values its builder encodes (what a correct dequantization must recover), under the
    # reference's K-quant relation (K_QUANT_REDUCTION_TOLERANCE 2e-3, :36).
    q4_scales = [5, 12, 30, 60, 7, 15, 31, 63]
    q4_mins = [3, 8, 20, 45, 1, 10, 25, 50]

    def q4_k(rows, cols):
        out, quants = bytearray(), []
        for row in range(rows):
            for block in range(cols // 256):
                b = bytearray(144)
                b[0:2] = _f16_bits((row + 1) * 0.03125).to_bytes(2, "little")
                b[2:4] = _f16_bits((block + 1) * 0.015625).to_bytes(2, "little")
                for g in range(4):
                    b[4 + g] = q4_scales[g]
                    b[8 + g] = q4_mins[g]
                for g in range(4, 8):
                    b[8 + g] = (q4_scales[g] & 0x0F) | ((q4_mins[g] & 0x0F) << 4)
                    b[g] |= (q4_scales[g] >> 4) << 6
                    b[4 + g] |= (q4_mins[g] >> 4) << 6
                qv = []
                for g in range(8):
                    off, shift = 16 + (g >> 1) * 32, (g & 1) * 4
                    for i in range(32):
                        quant = (row * 13 + block * 7 + g * 5 + i * 3) & 0x0F
                        b[off + i] |= quant << shift
                        qv.append(quant)
                quants.append(qv)
                out += b
        return out.hex(), quants

    def q6_k(rows, cols):
        out, quants, scales = bytearray(), [], []
        for row in range(rows):
            for block in range(cols // 256):
                b = bytearray(210)
                sc = [(row * 5 + block * 3 + i * 7) % 17 - 8 for i in range(16)]
                for i in range(16):
                    b[192 + i] = sc[i] & 0xFF
                b[208:210] = _f16_bits((row + block + 1) * 0.015625).to_bytes(2, "little")
                qv = [(row * 19 + block * 11 + i * 7) % 64 - 32 for i in range(256)]
                for sb in range(2):
                    pb, lb, hb = sb * 128, sb * 64, 128 + sb * 32
                    for i in range(32):
                        q1, q2, q3, q4 = (qv[pb + i + 32 * t] + 32 for t in range(4))
                        b[lb + i] = (q1 & 0x0F) | ((q3 & 0x0F) << 4)
                        b[lb + 32 + i] = (q2 & 0x0F) | ((q4 & 0x0F) << 4)
                        b[hb + i] = (((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) | (((q3 >> 4) & 3) << 4)
                                     | (((q4 >> 4) & 3) << 6))
                quants.append(qv)
                scales.append(sc)
                out += b
        return out.hex(), quants, scales

    def q5_0_weights(rows, cols):
        # fillQ5_0Weights (:701-722): per lane a 5-bit low and high value, nibbles at byte 6 +
        # lane, fifth bits as bits lane and lane + 16 of the little-endian word at byte 2.
        out, quants = bytearray(), []
        for row in range(rows):
            for block in range(cols // 32):
                b = bytearray(22)
                b[0:2] = _f16_bits((row + block + 1) * 0.0625).to_bytes(2, "little")
                high_bits, lows, highs = 0, [], []
                for lane in range(16):
                    low = (row * 17 + block * 11 + lane * 5) & 0x1F
                    high = (row * 13 + block * 7 + lane * 9) & 0x1F
                    b[6 + lane] = (low & 0x0F) | ((high & 0x0F) << 4)
                    high_bits |= ((low >> 4) & 1) << lane
                    high_bits |= ((high >> 4) & 1) << (lane + 16)
                    lows.append(low)
                    highs.append(high)
                b[2:6] = high_bits.to_bytes(4, "little")
                quants.append(lows + highs)  # elements 0-15, then 16-31 (before the -16 offset)
                out += b
        return out.hex(), quants

    def q5_k(rows, cols):
        # q5KBlock (:799-828): q4KBlock's scales and mins, 5-bit quants whose fifth bit of group
        # g sits in bit g of byte 16 + index.
        out, quants = bytearray(), []
        for row in range(rows):
            for block in range(cols // 256):
                b = bytearray(176)
                b[0:2] = _f16_bits((row + 1) * 0.03125).to_bytes(2, "little")
                b[2:4] = _f16_bits((block + 1) * 0.015625).to_bytes(2, "little")
                for g in range(4):
                    b[4 + g] = q4_scales[g]
                    b[8 + g] = q4_mins[g]
                for g in range(4, 8):
                    b[8 + g] = (q4_scales[g] & 0x0F) | ((q4_mins[g] & 0x0F) << 4)
                    b[g] |= (q4_scales[g] >> 4) << 6
                    b[4 + g] |= (q4_mins[g] >> 4) << 6
                qv = []
                for g in range(8):
                    off, shift = 48 + (g >> 1) * 32, (g & 1) * 4
                    for i in range(32):
                        quant = (row * 17 + block * 11 + g * 7 + i * 5) & 0x1F
                        b[off + i] |= (quant & 0x0F) << shift
                        if quant & 0x10:
                            b[16 + i] |= 1 << g
                        qv.append(quant)
                quants.append(qv)
                out += b
        return out.hex(), quants

    hx, quants = q5_0_weights(5, 64)
    cases.append({"name": "reusableGgufKernelComputesQ5_0BatchedMatrixMultiplicationWithinReductionTolerance",
                  "src": "NativeKernelLibraryTest.java:199-220", "format": 5, "batch": 3, "rows": 5,
                  "cols": 64, "relation": 2e-5, "input": activations(3, 64), "weights_hex": hx,
                  "logical": {"quants": quants}})
    hx, quants = q5_0_weights(5, 256)
    cases.append({"name": "reusableGgufKernelComputesQ5_0SingleTokenProjectionWithinQuantizedTolerance",
                  "src": "NativeKernelLibraryTest.java:222-244", "format": 5, "batch": 1, "rows": 5,
                  "cols": 256, "relation": 1e-3, "input": activations(1, 256), "weights_hex": hx,
                  "logical": {"quants": quants}})
    hx, quants = q5_k(5, 512)
    cases.append({"name": "reusableGgufKernelMatchesVectorSemanticsForKQuantizedBatchedMultiplication[Q5_K]",
                  "src": "NativeKernelLibraryTest.java:246-271", "format": 4, "batch": 3, "rows": 5,
                  "cols": 512, "relation": 2e-3, "input": activations(3, 512), "weights_hex": hx,
                  "logical": {"scales": q4_scales, "mins": q4_mins, "quants": quants}})
    hx, quants = q4_k(5, 512)
    cases.append({"name": "reusableGgufKernelMatchesVectorSemanticsForKQuantizedBatchedMultiplication[Q4_K]",
                  "src": "NativeKernelLibraryTest.java:246-271", "format": 2, "batch": 3, "rows": 5,
                  "cols": 512, "relation": 2e-3, "input": activations(3, 512), "weights_hex": hx,
                  "logical": {"scales": q4_scales, "mins": q4_mins, "quants": quants}})
    hx, quants, scales = q6_k(5, 512)
    cases.append({"name": "reusableGgufKernelMatchesVectorSemanticsForKQuantizedBatchedMultiplication[Q6_K]",
                  "src": "NativeKernelLibraryTest.java:246-271", "format": 3, "batch": 3, "rows": 5,
                  "cols": 512, "relation": 2e-3, "input": activations(3, 512), "weights_hex": hx,
                  "logical": {"quants": quants, "scales": scales}})
    cases.append({"name": "reusableGgufKernelComputesQ8_0BatchedMatrixMultiplicationWithinReductionTolerance",
                  "src": "NativeKernelLibraryTest.java:176-196", "format": 1, "batch": 3, "rows": 5,
                  "cols": 64, "relation": 2e-5, "input": activations(3, 64),
                  "weights_hex": q8_0_weights(5, 64)})
    return cases


def main():
    data = {
        "about": "Known answers transcribed from backend-java unit tests (see each 'src').",
        "kv_cache": kv_cases(),
        "layered_kv_cache": layered_cases(),
        "rope": rope_cases(),
        "softmax": softmax_cases(),
        "rms_norm": rms_norm_cases(),
        "value_norm": value_norm_cases(),
        "attention_start": window_cases(),
        "sliding_layers": sliding_layers(),
        "quantized_matmul": quantized_matmul_cases(),
    }
    path = os.path.join(HERE, "reference_known_answers.json")
    with open(path, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")
    print(path)


if __name__ == "__main__":
    main()

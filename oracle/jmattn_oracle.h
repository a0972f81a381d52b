/*
 * CPU oracle for the grouped-query attention + KV-cache path of integrallis/models backend-java.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's Java algorithm, used
 * by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. The product
 * (models_amd/, libjmodels_attn.so) never links, loads or calls it.
 *
 * Reference paths are relative to
 *   backend-java/src/main/java/com/integrallis/models/backend/purejava/
 * Every function names the file:line it follows.
 *
 * Floating-point model: Java float arithmetic is IEEE binary32 with round-to-nearest and no
 * fused multiply-add; the library is built with -ffp-contract=off so C matches that. Java's
 * (float)Math.exp/cos/sin/pow(double) are restated as (float)exp/cos/sin/pow(double).
 *
 * Parity status per function (what pins it) is listed in the header of oracle.py.
 */
#ifndef JMATTN_ORACLE_H
#define JMATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by oracle functions (mirrors the reference's exception kinds). */
#define JMO_OK 0
#define JMO_ILLEGAL_ARGUMENT 1 /* IllegalArgumentException */
#define JMO_ILLEGAL_STATE 2    /* IllegalStateException */

/* ---------------------------------------------------------------- half precision */

/* Float.floatToFloat16: IEEE binary16 with round-to-nearest-even (KvCache.java:94-100). */
uint16_t jmo_float_to_f16(float x);
/* Float.float16ToFloat. */
float jmo_f16_to_float(uint16_t h);
/* float16ToFloat(floatToFloat16(x)) element-wise: the "half-precision KV" store rounding. */
void jmo_f16_round_array(const float* in, float* out, size_t n);

/* ---------------------------------------------------------------- RoPE */

/* RotaryTable ctor frequencies: freq[p] = (float)(1/pow(theta, (2p)/rotaryDim))
 * (ops/RotaryTable.java:69-72). Returns JMO_ILLEGAL_ARGUMENT on odd/zero dims or bad theta. */
int jmo_rotary_frequencies(int rotary_dim, float theta, float* freq_out);

/* RotaryTable.fillFactors for one position (ops/RotaryTable.java:177-186).
 * factors may be NULL (no GGUF frequency divisors). */
int jmo_rotary_factors(int rotary_dim, float theta, float frequency_scale, const float* factors,
                       int position, float* cos_out, float* sin_out);

/* TensorOps.rope(vector, offset, cosine, sine, factorOffset, pairCount) and ropeNeox(...)
 * (ops/TensorOps.java:1336-1346, 1373-1390; rotatePair/rotateSplitPair :1474-1486). */
void jmo_rope_apply(float* vec, const float* cos_f, const float* sin_f, int pairs, int neox);

/* TensorOps.rope/ropeNeox with inline per-pair factors (ops/TensorOps.java:1296-1319, 1356-1371). */
void jmo_rope_direct(float* vec, int position, int head_dim, float theta, float frequency_scale,
                     int neox);

/* ---------------------------------------------------------------- softmax / norm */

/* TensorOps.softmax (ops/TensorOps.java:1247-1279). Returns JMO_ILLEGAL_ARGUMENT for size<=0,
 * NaN, +inf or no finite input (x is left partially untouched in that case, like the Java). */
int jmo_softmax(float* x, int size);

/* TensorOps.rmsNorm (ops/TensorOps.java:50-58); out may alias x. */
void jmo_rms_norm(float* out, const float* x, const float* weight, int size, float eps);
/* normalizeHead over `heads` consecutive heads of x, in place. */
void jmo_qk_norm_heads(float* x, int heads, int head_dim, const float* weight, float eps);

/* VectorUtil.dotProduct restated as a sequential float sum (vectors-core is not vendored, so its
 * lane order is unpinned; see oracle.py). */
float jmo_dot(const float* a, const float* b, int n);
/* Gemma4Math.normalizeWithoutWeight (gemma4/Gemma4Math.java:38-55); ILLEGAL_ARGUMENT for
 * length <= 0 or eps not finite and > 0. out may equal in. */
int jmo_value_rms_norm(float* out, const float* in, int length, float eps);

/* ---------------------------------------------------------------- KvCache (linear, growing) */

typedef struct jmo_kv jmo_kv;

/* KvCache ctor (cache/KvCache.java:35-48); half_precision mirrors
 * -Dmodels.purejava.halfPrecisionKvCache (KvCache.java:84-85). Returns NULL on bad arguments. */
jmo_kv* jmo_kv_create(int num_layers, int max_seq_len, int key_dim, int value_dim,
                      int half_precision);
void jmo_kv_destroy(jmo_kv* kv);
/* KvCache.store(layer, position, key, keyOffset, value, valueOffset) (KvCache.java:58-73). */
int jmo_kv_store(jmo_kv* kv, int layer, int position, const float* key, const float* value);
/* keyOffset / valueOffset (KvCache.java:142-153); -1 when the Java would throw. */
int64_t jmo_kv_key_offset(const jmo_kv* kv, int layer, int position);
int64_t jmo_kv_value_offset(const jmo_kv* kv, int layer, int position);
/* keySlice/valueSlice (KvCache.java:105-115, 208-230): copies rows [from,to) into out. */
int jmo_kv_key_slice(const jmo_kv* kv, int layer, int from, int to, float* out);
int jmo_kv_value_slice(const jmo_kv* kv, int layer, int from, int to, float* out);
/* key(layer,pos)/value: 1 = copied, 0 = null (unpopulated), <0 = argument error. */
int jmo_kv_key(const jmo_kv* kv, int layer, int position, float* out);
int jmo_kv_value(const jmo_kv* kv, int layer, int position, float* out);
void jmo_kv_clear(jmo_kv* kv);                                 /* KvCache.java:156-158 */
int jmo_kv_discard_from(jmo_kv* kv, int position);             /* KvCache.java:161-173 */
int jmo_kv_reserve(jmo_kv* kv, int required_capacity);         /* KvCache.java:197-206 */
int jmo_kv_allocated_capacity(const jmo_kv* kv);               /* KvCache.java:176-178 */
const float* jmo_kv_key_buffer(const jmo_kv* kv);              /* KvCache.java:130-132 */
const float* jmo_kv_value_buffer(const jmo_kv* kv);            /* KvCache.java:137-139 */
int64_t jmo_kv_buffer_length(const jmo_kv* kv, int values);    /* keys.length / values.length */

/* ---------------------------------------------------------------- LayeredKvCache (linear/ring) */

typedef struct jmo_lkv jmo_lkv;
/* LayeredKvCache ctor (cache/LayeredKvCache.java:137-150). ring_capacity[l] == 0 → LINEAR. */
jmo_lkv* jmo_lkv_create(int max_seq_len, int num_layers, const int* key_dims,
                        const int* value_dims, const int* ring_capacity);
void jmo_lkv_destroy(jmo_lkv* kv);
int jmo_lkv_store(jmo_lkv* kv, int layer, int position, const float* key, const float* value);
int jmo_lkv_contains(const jmo_lkv* kv, int layer, int position);            /* :172-175 */
/* attentionView (:178-209): span_out holds up to 2 x (firstPosition, count, keyOff, valueOff). */
int jmo_lkv_attention_view(const jmo_lkv* kv, int layer, int from, int to, int* span_count,
                           int* span_out);
int jmo_lkv_discard_from(jmo_lkv* kv, int position);                          /* :212-223 */
void jmo_lkv_clear(jmo_lkv* kv);                                              /* :226-230 */
int jmo_lkv_oldest(const jmo_lkv* kv, int layer);  /* -1 = empty (:233-235, 310-319) */
int jmo_lkv_newest(const jmo_lkv* kv, int layer);
int jmo_lkv_allocated_capacity(const jmo_lkv* kv, int layer);
int jmo_lkv_physical_capacity(const jmo_lkv* kv, int layer);
int64_t jmo_lkv_allocated_bytes(const jmo_lkv* kv);                           /* :285-291 */
int64_t jmo_lkv_maximum_bytes(const jmo_lkv* kv);                             /* :294-300 */
int64_t jmo_lkv_key_offset(const jmo_lkv* kv, int layer, int position);
const float* jmo_lkv_key_buffer(const jmo_lkv* kv, int layer);
const float* jmo_lkv_value_buffer(const jmo_lkv* kv, int layer);
int64_t jmo_lkv_buffer_length(const jmo_lkv* kv, int layer, int values);

/* ---------------------------------------------------------------- attention */

/* LlamaConfig.attentionStartPosition for a causal layer (llama/LlamaConfig.java:184-195):
 * window 0 = global layer → 0; else max(0, position - window + 1). */
int jmo_attention_start(int position, int window);

/* LlamaForwardPass.groupedQueryAttention (llama/LlamaForwardPass.java:1543-1593) with
 * computeAttentionScores (:1595-1631) and accumulateAttentionValues (:1633-1670) over a
 * KvCache. scores must hold max_seq_len floats. */
int jmo_gqa(const jmo_kv* kv, int layer, int position, int window, const float* q, int num_heads,
            int num_kv_heads, int key_length, int value_length, float scale, float* out,
            float* scores);

/* The same arithmetic over caller-supplied contiguous rows: keys[r*key_row_stride + kvh*dk]
 * holds position first+r. Used for ragged sequences and for the CPU baseline timing. */
int jmo_gqa_rows(const float* q, const float* keys, const float* values, int rows,
                 int key_row_stride, int value_row_stride, int num_heads, int num_kv_heads,
                 int key_length, int value_length, float scale, float* out, float* scores);

/* Gemma4ForwardPass.computeAttention (gemma4/Gemma4ForwardPass.java:1186-1230): the same GQA math
 * over a 1-2 span LayeredKvCache view, with an explicit scale (Gemma 4 uses 1.0). */
int jmo_gqa_layered(const jmo_lkv* kv, int layer, int position, int window, const float* q,
                    int num_heads, int num_kv_heads, int head_dim, float scale, float* out,
                    float* scores);

/* One decode token through one layer exactly as LlamaForwardPass.forwardSequenceInternal runs it
 * (llama/LlamaForwardPass.java:1069-1128): RoPE on every Q and K head (RotaryTable.prepare +
 * apply, :1070-1083), KvCache.store (:1086), GQA (:1090-1128). q/k are rotated in place.
 * rope_theta <= 0 → the layer applies no RoPE (LlamaConfig.usesRope false). */
int jmo_decode_layer(jmo_kv* kv, int layer, int position, int window, float* q, float* k,
                     const float* v, int num_heads, int num_kv_heads, int key_length,
                     int value_length, float rope_theta, float rope_scale, int neox, float scale,
                     float* out, float* scores);

/* Causal prefill of n rows at start..start+n-1 (prepareBatchedAttention + computeBatchedAttention,
 * llama/LlamaForwardPass.java:1479-1541): RoPE + store for every row, then per-row GQA. */
int jmo_prefill_layer(jmo_kv* kv, int layer, int start, int n, int window, float* q, float* k,
                      const float* v, int num_heads, int num_kv_heads, int key_length,
                      int value_length, float rope_theta, float rope_scale, int neox, float scale,
                      float* out, float* scores);

/* Multi-threaded variant of jmo_gqa_rows over independent (sequence, head) units, used only for
 * the all-cores CPU baseline figure. Identical arithmetic per unit. */
int jmo_gqa_rows_batch(int count, const float* const* q, const float* const* keys,
                       const float* const* values, const int* rows, int key_row_stride,
                       int value_row_stride, int num_heads, int num_kv_heads, int key_length,
                       int value_length, float scale, float* const* out, int threads);
/* jmo_gqa_rows_batch with dot products in eight partial sums (a vectorised loop, timing only:
 * the bench's vectorised CPU baseline; parity is pinned on the sequential variant). */
int jmo_gqa_rows_batch8(int count, const float* const* q, const float* const* keys,
                       const float* const* values, const int* rows, int key_row_stride,
                       int value_row_stride, int num_heads, int num_kv_heads, int key_length,
                       int value_length, float scale, float* const* out, int threads);

/* ---------------------------------------------------------------- GGUF block-quantized projection
 *
 * The Q/K/V and output projections around attention (llama/LlamaForwardPass.java:1043-1067,
 * 1131-1138) multiply a GGUF block-quantized weight matrix [rows][cols] by f32 activations. For
 * Q4_0 and Q8_0 weights both backend-native (backend-native/src/main/rust/model-kernels/src/
 * lib.rs, the batched matmul exports at RS:540-700) and vectors-core quantize each 32-element
 * activation block to Q8_0 and take integer dot products per block. Restated here from the
 * reference implementation in backend-native's tests, which the native Q4_0 kernel must match
 * exactly (backend-native/src/test/java/com/integrallis/models/backend/nativekernel/
 * NativeKernelLibraryTest.java:67-84 with :909-1023). */
#define JMO_FMT_Q4_0 0 /* 18-byte blocks: f16 scale, 16 bytes of nibbles (RS:87) */
#define JMO_FMT_Q8_0 1 /* 34-byte blocks: f16 scale, 32 int8 (RS:89) */
#define JMO_FMT_Q4_K 2 /* 144-byte blocks of 256: d, dmin, 12 bytes of 6-bit scales/mins, nibbles (RS:90) */
#define JMO_FMT_Q6_K 3 /* 210-byte blocks of 256: ql[128], qh[64], int8 scales[16], d (RS:92) */
#define JMO_FMT_Q5_K 4 /* 176-byte blocks of 256: d, dmin, 12 bytes of scales/mins, qh[32], nibbles (RS:91) */
#define JMO_FMT_Q5_0 5 /* 22-byte blocks: f16 scale, 32 high bits, 16 bytes of nibbles (RS:88) */

/* quantizeInputs (NativeKernelLibraryTest.java:998-1017; RS quantize_q8_0_batch_scalar): per
 * 32-element block, absmax (a NaN element is skipped, as Rust's f32::max does), inverse scale
 * 127 / absmax (0 for an all-zero block), scale = f16-rounded absmax / 127, element =
 * ggmlNearestInt(x * inverse) (:1019-1022). q [batch*cols], scales [batch*cols/32]. */
void jmo_q8_0_quantize(const float* x, int batch, int cols, int8_t* q, float* scales);

/* quantize_q8_k_batch (RS:3906-3952), the activations of the K-quant formats: per 256-element
 * block, the element of largest magnitude (the first on ties; NaN skipped) sets
 * inverse = -127 / max; element = min(nearest(inverse * x), 127); sums of 16 consecutive
 * elements; scale = 1 / inverse; an all-zero block has scale 0, elements 0, sums 0.
 * q [batch*cols], scales [batch*cols/256], sums [batch*cols/16]. */
void jmo_q8_k_quantize(const float* x, int batch, int cols, int8_t* q, float* scales,
                       int16_t* sums);

/* referenceQ4_0F32BatchedMatmul / referenceQ8_0F32BatchedMatmul (NativeKernelLibraryTest.java:
 * 909-936, 938-965): out[b*rows + r] = sum over blocks in order of
 * fma(weightScale * activationScale, integerDot, sum). Q4_K and Q6_K with Q8_K activations as
 * backend-native's scalar row kernels compute them (dot_q4_k_q8_k_row_scalar, RS:3410-3459:
 * per block sum = fma(d, sum_g scale_g * dot_g, sum) then fma(-dmin, sum_g min_g * sums_g, sum),
 * d and dmin the weight's f16 factors times the activation scale; dot_q6_k_q8_k_row_scalar,
 * RS:3519-3577: eight integer lane sums per block (lane = element index within its 32-run mod 8),
 * eight fma chains over the blocks, the lanes added in order at the end). JMO_ILLEGAL_ARGUMENT for
 * an unknown format or cols not a multiple of the block size (32, or 256 for K-quants). */
int jmo_quantized_matmul(int format, const uint8_t* weights, const float* input, int batch,
                         int rows, int cols, float* out);

#ifdef __cplusplus
}
#endif
#endif

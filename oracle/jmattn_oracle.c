/*
 * CPU oracle: plain-C restatement of backend-java's GQA + KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY (checker for tests/, smoke() and the bench cpu_baseline leg). The
 * product library never links or calls this file. Paths below are relative to
 *   backend-java/src/main/java/com/integrallis/models/backend/purejava/
 * Build with -ffp-contract=off so float expressions round like Java's binary32 arithmetic.
 */
#include "jmattn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ================================================================ half precision */

uint16_t jmo_float_to_f16(float x) {
  /* IEEE 754 binary32 -> binary16, round to nearest, ties to even; overflow -> infinity.
   * Behaviour of Float.floatToFloat16 as used by KvCache.storeHalfPrecision (KvCache.java:94-100). */
  uint32_t bits;
  memcpy(&bits, &x, sizeof bits);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  uint32_t mag = bits & 0x7fffffffu;
  if (mag > 0x7f800000u) { /* NaN: keep it quiet and keep the top payload bits */
    return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x03ffu));
  }
  if (mag >= 0x477ff000u) { /* >= 65520 = 65504 + half an ulp: rounds past the largest finite */
    return (uint16_t)(sign | 0x7c00u);
  }
  int exponent = (int)(mag >> 23) - 127;
  if (exponent < -25) { /* below half the smallest subnormal (2^-24): rounds to zero */
    return sign;
  }
  uint32_t significand = (mag & 0x7fffffu) | 0x800000u; /* 24 bits, value = s * 2^(e-23) */
  uint32_t shift;
  uint32_t result;
  if (exponent >= -14) { /* normal binary16 */
    shift = 13;
    result = ((uint32_t)(exponent + 15) << 10) | ((significand >> shift) & 0x3ffu);
  } else { /* subnormal binary16: unit 2^-24 */
    shift = (uint32_t)(-exponent - 1);
    result = significand >> shift;
  }
  uint32_t remainder = significand & ((1u << shift) - 1u);
  uint32_t halfway = 1u << (shift - 1u);
  if (remainder > halfway || (remainder == halfway && (result & 1u))) {
    result += 1u; /* a carry out of the significand bumps the exponent, as it should */
  }
  return (uint16_t)(sign | result);
}

float jmo_f16_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exponent = (h >> 10) & 0x1fu;
  uint32_t mantissa = h & 0x3ffu;
  uint32_t bits;
  if (exponent == 0x1fu) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else if (exponent != 0) {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  } else if (mantissa == 0) {
    bits = sign;
  } else { /* subnormal: normalise */
    int e = -1;
    do {
      mantissa <<= 1;
      e++;
    } while ((mantissa & 0x400u) == 0);
    bits = sign | ((uint32_t)(112 - e) << 23) | ((mantissa & 0x3ffu) << 13);
  }
  float out;
  memcpy(&out, &bits, sizeof out);
  return out;
}

void jmo_f16_round_array(const float* in, float* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = jmo_f16_to_float(jmo_float_to_f16(in[i]));
}

/* ================================================================ RoPE */

static int finite_positive(float v) { return v > 0.0f && isfinite(v); }

int jmo_rotary_frequencies(int rotary_dim, float theta, float* freq_out) {
  /* RotaryTable ctor (ops/RotaryTable.java:48-75). */
  if (rotary_dim <= 0 || (rotary_dim & 1) != 0 || !finite_positive(theta)) {
    return JMO_ILLEGAL_ARGUMENT;
  }
  int pairs = rotary_dim / 2;
  for (int pair = 0; pair < pairs; pair++) {
    freq_out[pair] = (float)(1.0 / pow((double)theta, (double)(pair * 2) / rotary_dim));
  }
  return JMO_OK;
}

int jmo_rotary_factors(int rotary_dim, float theta, float frequency_scale, const float* factors,
                       int position, float* cos_out, float* sin_out) {
  /* RotaryTable.fillFactors (ops/RotaryTable.java:177-186). */
  if (position < 0 || !finite_positive(frequency_scale)) return JMO_ILLEGAL_ARGUMENT;
  int pairs = rotary_dim / 2;
  float* freq = (float*)malloc(sizeof(float) * (size_t)(pairs > 0 ? pairs : 1));
  int status = jmo_rotary_frequencies(rotary_dim, theta, freq);
  if (status == JMO_OK) {
    float scaled_position = (float)position * frequency_scale;
    for (int pair = 0; pair < pairs; pair++) {
      float divisor = factors == NULL ? 1.0f : factors[pair];
      float angle = scaled_position * freq[pair] / divisor;
      cos_out[pair] = (float)cos((double)angle);
      sin_out[pair] = (float)sin((double)angle);
    }
  }
  free(freq);
  return status;
}

void jmo_rope_apply(float* vec, const float* cos_f, const float* sin_f, int pairs, int neox) {
  /* TensorOps.rope / ropeNeox over precomputed factors (ops/TensorOps.java:1336-1346,
   * 1373-1390); each pair is rotated as x0*c - x1*s, x0*s + x1*c (:1474-1486). */
  for (int pair = 0; pair < pairs; pair++) {
    int first = neox ? pair : 2 * pair;
    int second = neox ? pair + pairs : 2 * pair + 1;
    float x0 = vec[first];
    float x1 = vec[second];
    vec[first] = x0 * cos_f[pair] - x1 * sin_f[pair];
    vec[second] = x0 * sin_f[pair] + x1 * cos_f[pair];
  }
}

void jmo_rope_direct(float* vec, int position, int head_dim, float theta, float frequency_scale,
                     int neox) {
  /* TensorOps.rope(vector, offset, position, headDim, theta, scale) (ops/TensorOps.java:1296-1319)
   * and ropeNeox (:1356-1371): factors computed inline per pair. */
  float scaled_position = (float)position * frequency_scale;
  int pairs = head_dim / 2;
  for (int pair = 0; pair < pairs; pair++) {
    float freq = (float)(1.0 / pow((double)theta, (double)(2 * pair) / head_dim));
    float angle = scaled_position * freq;
    float c = (float)cos((double)angle);
    float s = (float)sin((double)angle);
    int first = neox ? pair : 2 * pair;
    int second = neox ? pair + pairs : 2 * pair + 1;
    float x0 = vec[first];
    float x1 = vec[second];
    vec[first] = x0 * c - x1 * s;
    vec[second] = x0 * s + x1 * c;
  }
}

/* ================================================================ softmax / norm / dot */

int jmo_softmax(float* x, int size) {
  /* TensorOps.softmax (ops/TensorOps.java:1247-1279): float max with NaN/+inf rejection,
   * (float)Math.exp(x - max) in double, sequential float sum, multiply by 1/sum. */
  if (size <= 0) return JMO_ILLEGAL_ARGUMENT;
  float max = -INFINITY;
  for (int i = 0; i < size; i++) {
    float value = x[i];
    if (isnan(value)) return JMO_ILLEGAL_ARGUMENT;
    if (value == INFINITY) return JMO_ILLEGAL_ARGUMENT;
    if (value > max) max = value;
  }
  if (!isfinite(max)) return JMO_ILLEGAL_ARGUMENT;
  float sum = 0.0f;
  for (int i = 0; i < size; i++) {
    x[i] = (float)exp((double)(x[i] - max));
    sum += x[i];
  }
  float inv_sum = 1.0f / sum;
  for (int i = 0; i < size; i++) x[i] *= inv_sum;
  return JMO_OK;
}

int jmo_value_rms_norm(float* out, const float* in, int length, float eps) {
  /* Gemma4Math.normalizeWithoutWeight (gemma4/Gemma4Math.java:38-55): sumSquares as a float dot
   * product (sequential here; vectors-core's lane order is unpinned), inverse =
   * (float)(1.0 / Math.sqrt(sumSquares / length + eps)) with the mean and the epsilon added in
   * float and the square root and reciprocal in double, then out = in * inverse. */
  if (length <= 0 || !(eps > 0.0f) || !isfinite(eps)) return JMO_ILLEGAL_ARGUMENT;
  float sum_sq = jmo_dot(in, in, length);
  float inverse = (float)(1.0 / sqrt((double)(sum_sq / (float)length + eps)));
  for (int i = 0; i < length; i++) out[i] = in[i] * inverse;
  return JMO_OK;
}

float jmo_dot(const float* a, const float* b, int n) {
  float sum = 0.0f;
  for (int i = 0; i < n; i++) sum += a[i] * b[i];
  return sum;
}

void jmo_rms_norm(float* out, const float* x, const float* weight, int size, float eps) {
  /* TensorOps.rmsNorm (ops/TensorOps.java:50-58). */
  float sum_sq = jmo_dot(x, x, size);
  float rms = (float)sqrt((double)(sum_sq / (float)size + eps));
  float scale = 1.0f / rms;
  for (int i = 0; i < size; i++) out[i] = x[i] * scale * weight[i];
}

void jmo_qk_norm_heads(float* x, int heads, int head_dim, const float* weight, float eps) {
  /* normalizeHead per head, in place (llama/LlamaForwardPass.java:1070-1083, 1672-1676): the
   * reference calls rmsNorm(vector, offset, vector, offset, ...), which reads each element before
   * writing it. */
  for (int h = 0; h < heads; h++) jmo_rms_norm(x + (int64_t)h * head_dim, x + (int64_t)h * head_dim,
                                                weight, head_dim, eps);
}

/* ================================================================ KvCache */

struct jmo_kv {
  int num_layers, max_seq_len, key_dim, value_dim, half_precision;
  int capacity; /* allocatedSequenceCapacity */
  float* keys;
  float* values;
  unsigned char* populated;
};

static int checked_product(int64_t a, int64_t b, int64_t* out) {
  int64_t p = a * b;
  if (p > 2147483647LL) return 0;
  *out = p;
  return 1;
}

jmo_kv* jmo_kv_create(int num_layers, int max_seq_len, int key_dim, int value_dim,
                      int half_precision) {
  /* KvCache ctor (cache/KvCache.java:35-48): capacity min(maxSeqLen, 16). */
  if (num_layers <= 0 || max_seq_len <= 0 || key_dim <= 0 || value_dim <= 0) return NULL;
  jmo_kv* kv = (jmo_kv*)calloc(1, sizeof(jmo_kv));
  kv->num_layers = num_layers;
  kv->max_seq_len = max_seq_len;
  kv->key_dim = key_dim;
  kv->value_dim = value_dim;
  kv->half_precision = half_precision;
  kv->capacity = max_seq_len < 16 ? max_seq_len : 16;
  int64_t slots, kn, vn;
  if (!checked_product(num_layers, kv->capacity, &slots) || !checked_product(slots, key_dim, &kn) ||
      !checked_product(slots, value_dim, &vn)) {
    free(kv);
    return NULL;
  }
  kv->keys = (float*)calloc((size_t)kn, sizeof(float));
  kv->values = (float*)calloc((size_t)vn, sizeof(float));
  kv->populated = (unsigned char*)calloc((size_t)slots, 1);
  return kv;
}

void jmo_kv_destroy(jmo_kv* kv) {
  if (!kv) return;
  free(kv->keys);
  free(kv->values);
  free(kv->populated);
  free(kv);
}

static int kv_check_bounds(const jmo_kv* kv, int layer, int position) {
  /* KvCache.checkBounds (KvCache.java:237-244). */
  return layer >= 0 && layer < kv->num_layers && position >= 0 && position < kv->max_seq_len;
}

static int64_t kv_slot(const jmo_kv* kv, int layer, int position) {
  return (int64_t)layer * kv->capacity + position; /* KvCache.slotIndex (:280-282) */
}

static int kv_ensure_capacity(jmo_kv* kv, int required) {
  /* KvCache.ensureCapacity (KvCache.java:284-322): double up to maxSeqLen and move each layer's
   * rows to layer * newCapacity. */
  if (required <= kv->capacity) return JMO_OK;
  int new_capacity = kv->capacity;
  while (new_capacity < required) {
    int64_t doubled = (int64_t)new_capacity * 2;
    new_capacity = doubled < kv->max_seq_len ? (int)doubled : kv->max_seq_len;
  }
  int64_t slots, kn, vn;
  if (!checked_product(kv->num_layers, new_capacity, &slots) ||
      !checked_product(slots, kv->key_dim, &kn) || !checked_product(slots, kv->value_dim, &vn)) {
    return JMO_ILLEGAL_ARGUMENT;
  }
  float* keys = (float*)calloc((size_t)kn, sizeof(float));
  float* values = (float*)calloc((size_t)vn, sizeof(float));
  unsigned char* populated = (unsigned char*)calloc((size_t)slots, 1);
  for (int layer = 0; layer < kv->num_layers; layer++) {
    memcpy(keys + (int64_t)layer * new_capacity * kv->key_dim,
           kv->keys + (int64_t)layer * kv->capacity * kv->key_dim,
           sizeof(float) * (size_t)kv->capacity * kv->key_dim);
    memcpy(values + (int64_t)layer * new_capacity * kv->value_dim,
           kv->values + (int64_t)layer * kv->capacity * kv->value_dim,
           sizeof(float) * (size_t)kv->capacity * kv->value_dim);
    memcpy(populated + (int64_t)layer * new_capacity,
           kv->populated + (int64_t)layer * kv->capacity, (size_t)kv->capacity);
  }
  free(kv->keys);
  free(kv->values);
  free(kv->populated);
  kv->keys = keys;
  kv->values = values;
  kv->populated = populated;
  kv->capacity = new_capacity;
  return JMO_OK;
}

int jmo_kv_store(jmo_kv* kv, int layer, int position, const float* key, const float* value) {
  /* KvCache.store (KvCache.java:58-73). */
  if (!kv_check_bounds(kv, layer, position)) return JMO_ILLEGAL_ARGUMENT;
  int status = kv_ensure_capacity(kv, position + 1);
  if (status != JMO_OK) return status;
  int64_t slot = kv_slot(kv, layer, position);
  float* kd = kv->keys + slot * kv->key_dim;
  float* vd = kv->values + slot * kv->value_dim;
  if (kv->half_precision) {
    jmo_f16_round_array(key, kd, (size_t)kv->key_dim);
    jmo_f16_round_array(value, vd, (size_t)kv->value_dim);
  } else {
    memcpy(kd, key, sizeof(float) * (size_t)kv->key_dim);
    memcpy(vd, value, sizeof(float) * (size_t)kv->value_dim);
  }
  kv->populated[slot] = 1;
  return JMO_OK;
}

int64_t jmo_kv_key_offset(const jmo_kv* kv, int layer, int position) {
  /* keyOffset: bounds then allocation check (KvCache.java:142-146, 324-328). */
  if (!kv_check_bounds(kv, layer, position) || position >= kv->capacity) return -1;
  return kv_slot(kv, layer, position) * kv->key_dim;
}

int64_t jmo_kv_value_offset(const jmo_kv* kv, int layer, int position) {
  if (!kv_check_bounds(kv, layer, position) || position >= kv->capacity) return -1;
  return kv_slot(kv, layer, position) * kv->value_dim;
}

static int kv_slice(const jmo_kv* kv, const float* store, int dim, int layer, int from, int to,
                    float* out) {
  /* KvCache.slice (KvCache.java:208-230). */
  if (layer < 0 || layer >= kv->num_layers) return JMO_ILLEGAL_ARGUMENT;
  if (from < 0 || to > kv->max_seq_len || from > to) return JMO_ILLEGAL_ARGUMENT;
  for (int p = 0; p < to - from; p++) {
    int position = from + p;
    if (position >= kv->capacity) return JMO_ILLEGAL_STATE;
    int64_t slot = kv_slot(kv, layer, position);
    if (!kv->populated[slot]) return JMO_ILLEGAL_STATE;
    memcpy(out + (int64_t)p * dim, store + slot * dim, sizeof(float) * (size_t)dim);
  }
  return JMO_OK;
}

int jmo_kv_key_slice(const jmo_kv* kv, int layer, int from, int to, float* out) {
  return kv_slice(kv, kv->keys, kv->key_dim, layer, from, to, out);
}

int jmo_kv_value_slice(const jmo_kv* kv, int layer, int from, int to, float* out) {
  return kv_slice(kv, kv->values, kv->value_dim, layer, from, to, out);
}

static int kv_vector(const jmo_kv* kv, const float* store, int dim, int layer, int position,
                     float* out) {
  /* key/value -> vectorOrNull (KvCache.java:118-127, 246-256). */
  if (!kv_check_bounds(kv, layer, position)) return -JMO_ILLEGAL_ARGUMENT;
  if (position >= kv->capacity) return 0;
  int64_t slot = kv_slot(kv, layer, position);
  if (!kv->populated[slot]) return 0;
  memcpy(out, store + slot * dim, sizeof(float) * (size_t)dim);
  return 1;
}

int jmo_kv_key(const jmo_kv* kv, int layer, int position, float* out) {
  return kv_vector(kv, kv->keys, kv->key_dim, layer, position, out);
}

int jmo_kv_value(const jmo_kv* kv, int layer, int position, float* out) {
  return kv_vector(kv, kv->values, kv->value_dim, layer, position, out);
}

void jmo_kv_clear(jmo_kv* kv) {
  memset(kv->populated, 0, (size_t)kv->num_layers * kv->capacity);
}

int jmo_kv_discard_from(jmo_kv* kv, int position) {
  /* KvCache.discardFrom (KvCache.java:161-173). */
  if (position < 0 || position > kv->max_seq_len) return JMO_ILLEGAL_ARGUMENT;
  if (position >= kv->capacity) return JMO_OK;
  for (int layer = 0; layer < kv->num_layers; layer++) {
    int64_t from = (int64_t)layer * kv->capacity + position;
    int64_t to = (int64_t)(layer + 1) * kv->capacity;
    memset(kv->populated + from, 0, (size_t)(to - from));
  }
  return JMO_OK;
}

int jmo_kv_reserve(jmo_kv* kv, int required_capacity) {
  /* KvCache.reserveSequenceCapacity (KvCache.java:197-206). */
  if (required_capacity < 0 || required_capacity > kv->max_seq_len) return JMO_ILLEGAL_ARGUMENT;
  return kv_ensure_capacity(kv, required_capacity);
}

int jmo_kv_allocated_capacity(const jmo_kv* kv) { return kv->capacity; }
const float* jmo_kv_key_buffer(const jmo_kv* kv) { return kv->keys; }
const float* jmo_kv_value_buffer(const jmo_kv* kv) { return kv->values; }

int64_t jmo_kv_buffer_length(const jmo_kv* kv, int values) {
  return (int64_t)kv->num_layers * kv->capacity * (values ? kv->value_dim : kv->key_dim);
}

/* ================================================================ LayeredKvCache */

typedef struct {
  int key_dim, value_dim, ring; /* ring capacity, 0 = LINEAR */
  int physical_limit, allocated;
  float* keys;
  float* values;
  int* positions;
} jmo_layer_state;

struct jmo_lkv {
  int max_seq_len, num_layers;
  jmo_layer_state* layers;
};

jmo_lkv* jmo_lkv_create(int max_seq_len, int num_layers, const int* key_dims,
                        const int* value_dims, const int* ring_capacity) {
  /* LayeredKvCache ctor + LayerState (cache/LayeredKvCache.java:126-150); physicalLimit is
   * min(ringCapacity, maxSeqLen) for RING layers, maxSeqLen for LINEAR ones. */
  if (max_seq_len <= 0 || num_layers <= 0) return NULL;
  for (int l = 0; l < num_layers; l++) {
    if (key_dims[l] <= 0 || value_dims[l] <= 0 || ring_capacity[l] < 0) return NULL;
  }
  jmo_lkv* kv = (jmo_lkv*)calloc(1, sizeof(jmo_lkv));
  kv->max_seq_len = max_seq_len;
  kv->num_layers = num_layers;
  kv->layers = (jmo_layer_state*)calloc((size_t)num_layers, sizeof(jmo_layer_state));
  for (int l = 0; l < num_layers; l++) {
    jmo_layer_state* s = &kv->layers[l];
    s->key_dim = key_dims[l];
    s->value_dim = value_dims[l];
    s->ring = ring_capacity[l];
    s->physical_limit =
        s->ring > 0 ? (s->ring < max_seq_len ? s->ring : max_seq_len) : max_seq_len;
  }
  return kv;
}

void jmo_lkv_destroy(jmo_lkv* kv) {
  if (!kv) return;
  for (int l = 0; l < kv->num_layers; l++) {
    free(kv->layers[l].keys);
    free(kv->layers[l].values);
    free(kv->layers[l].positions);
  }
  free(kv->layers);
  free(kv);
}

static int lkv_slot(const jmo_layer_state* s, int position) {
  return s->ring > 0 ? position % s->physical_limit : position; /* :354-356 */
}

static void lkv_reallocate(jmo_layer_state* s, int capacity) {
  /* allocate + grow (:380-396): old contents are copied to the front of the new arrays. */
  float* keys = (float*)calloc((size_t)capacity * s->key_dim, sizeof(float));
  float* values = (float*)calloc((size_t)capacity * s->value_dim, sizeof(float));
  int* positions = (int*)malloc(sizeof(int) * (size_t)capacity);
  for (int i = 0; i < capacity; i++) positions[i] = -1;
  if (s->allocated > 0) {
    memcpy(keys, s->keys, sizeof(float) * (size_t)s->allocated * s->key_dim);
    memcpy(values, s->values, sizeof(float) * (size_t)s->allocated * s->value_dim);
    memcpy(positions, s->positions, sizeof(int) * (size_t)s->allocated);
  }
  free(s->keys);
  free(s->values);
  free(s->positions);
  s->keys = keys;
  s->values = values;
  s->positions = positions;
  s->allocated = capacity;
}

static void lkv_ensure_capacity(const jmo_lkv* kv, jmo_layer_state* s, int required) {
  /* LayeredKvCache.ensureCapacity (:358-378). */
  if (s->ring > 0) {
    if (s->allocated == 0) lkv_reallocate(s, s->physical_limit);
    return;
  }
  if (required <= s->allocated) return;
  int capacity = s->allocated;
  if (capacity == 0) capacity = kv->max_seq_len < 16 ? kv->max_seq_len : 16;
  while (capacity < required) {
    int doubled = capacity <= kv->max_seq_len / 2 ? capacity * 2 : kv->max_seq_len;
    capacity = doubled < kv->max_seq_len ? doubled : kv->max_seq_len;
  }
  lkv_reallocate(s, capacity);
}

int jmo_lkv_store(jmo_lkv* kv, int layer, int position, const float* key, const float* value) {
  /* LayeredKvCache.store (:158-169). */
  if (layer < 0 || layer >= kv->num_layers) return JMO_ILLEGAL_ARGUMENT;
  if (position < 0 || position >= kv->max_seq_len) return JMO_ILLEGAL_ARGUMENT;
  jmo_layer_state* s = &kv->layers[layer];
  lkv_ensure_capacity(kv, s, position + 1);
  int slot = lkv_slot(s, position);
  memcpy(s->keys + (int64_t)slot * s->key_dim, key, sizeof(float) * (size_t)s->key_dim);
  memcpy(s->values + (int64_t)slot * s->value_dim, value, sizeof(float) * (size_t)s->value_dim);
  s->positions[slot] = position;
  return JMO_OK;
}

int jmo_lkv_contains(const jmo_lkv* kv, int layer, int position) {
  if (layer < 0 || layer >= kv->num_layers) return -JMO_ILLEGAL_ARGUMENT;
  if (position < 0 || position >= kv->max_seq_len) return -JMO_ILLEGAL_ARGUMENT;
  const jmo_layer_state* s = &kv->layers[layer];
  return s->allocated != 0 && s->positions[lkv_slot(s, position)] == position;
}

int jmo_lkv_attention_view(const jmo_lkv* kv, int layer, int from, int to, int* span_count,
                           int* span_out) {
  /* LayeredKvCache.attentionView (:178-209). */
  if (layer < 0 || layer >= kv->num_layers) return JMO_ILLEGAL_ARGUMENT;
  const jmo_layer_state* s = &kv->layers[layer];
  if (from < 0 || to > kv->max_seq_len || from >= to) return JMO_ILLEGAL_ARGUMENT;
  int count = to - from;
  if (s->ring > 0 && count > s->physical_limit) return JMO_ILLEGAL_ARGUMENT;
  for (int p = from; p < to; p++) {
    if (s->allocated == 0 || s->positions[lkv_slot(s, p)] != p) return JMO_ILLEGAL_STATE;
  }
  int first_slot = lkv_slot(s, from);
  if (s->ring == 0) {
    *span_count = 1;
    span_out[0] = from;
    span_out[1] = count;
    span_out[2] = first_slot * s->key_dim;
    span_out[3] = first_slot * s->value_dim;
    return JMO_OK;
  }
  int first_count = count < s->allocated - first_slot ? count : s->allocated - first_slot;
  span_out[0] = from;
  span_out[1] = first_count;
  span_out[2] = first_slot * s->key_dim;
  span_out[3] = first_slot * s->value_dim;
  int second = count - first_count;
  *span_count = second == 0 ? 1 : 2;
  if (second) {
    span_out[4] = from + first_count;
    span_out[5] = second;
    span_out[6] = 0;
    span_out[7] = 0;
  }
  return JMO_OK;
}

int jmo_lkv_discard_from(jmo_lkv* kv, int position) {
  if (position < 0 || position > kv->max_seq_len) return JMO_ILLEGAL_ARGUMENT;
  for (int l = 0; l < kv->num_layers; l++) {
    jmo_layer_state* s = &kv->layers[l];
    for (int i = 0; i < s->allocated; i++) {
      if (s->positions[i] >= position) s->positions[i] = -1;
    }
  }
  return JMO_OK;
}

void jmo_lkv_clear(jmo_lkv* kv) {
  for (int l = 0; l < kv->num_layers; l++) {
    jmo_layer_state* s = &kv->layers[l];
    for (int i = 0; i < s->allocated; i++) s->positions[i] = -1;
  }
}

static int lkv_retained(const jmo_lkv* kv, int layer, int oldest) {
  /* retainedPosition (:310-319). */
  const jmo_layer_state* s = &kv->layers[layer];
  int result = oldest ? 2147483647 : -1;
  for (int i = 0; i < s->allocated; i++) {
    int p = s->positions[i];
    if (p >= 0) result = oldest ? (p < result ? p : result) : (p > result ? p : result);
  }
  return (result == 2147483647 || result < 0) ? -1 : result;
}

int jmo_lkv_oldest(const jmo_lkv* kv, int layer) { return lkv_retained(kv, layer, 1); }
int jmo_lkv_newest(const jmo_lkv* kv, int layer) { return lkv_retained(kv, layer, 0); }
int jmo_lkv_allocated_capacity(const jmo_lkv* kv, int layer) { return kv->layers[layer].allocated; }
int jmo_lkv_physical_capacity(const jmo_lkv* kv, int layer) {
  return kv->layers[layer].physical_limit;
}

static int64_t lkv_storage_bytes(const jmo_layer_state* s, int capacity) {
  /* storageBytes (:420-426): floats for keys+values plus one int position per slot. */
  return (int64_t)capacity * (s->key_dim + s->value_dim) * 4 + (int64_t)capacity * 4;
}

int64_t jmo_lkv_allocated_bytes(const jmo_lkv* kv) {
  int64_t bytes = 0;
  for (int l = 0; l < kv->num_layers; l++) {
    bytes += lkv_storage_bytes(&kv->layers[l], kv->layers[l].allocated);
  }
  return bytes;
}

int64_t jmo_lkv_maximum_bytes(const jmo_lkv* kv) {
  int64_t bytes = 0;
  for (int l = 0; l < kv->num_layers; l++) {
    bytes += lkv_storage_bytes(&kv->layers[l], kv->layers[l].physical_limit);
  }
  return bytes;
}

int64_t jmo_lkv_key_offset(const jmo_lkv* kv, int layer, int position) {
  int c = jmo_lkv_contains(kv, layer, position);
  if (c <= 0) return -1;
  const jmo_layer_state* s = &kv->layers[layer];
  return (int64_t)lkv_slot(s, position) * s->key_dim;
}

const float* jmo_lkv_key_buffer(const jmo_lkv* kv, int layer) { return kv->layers[layer].keys; }
const float* jmo_lkv_value_buffer(const jmo_lkv* kv, int layer) {
  return kv->layers[layer].values;
}

int64_t jmo_lkv_buffer_length(const jmo_lkv* kv, int layer, int values) {
  const jmo_layer_state* s = &kv->layers[layer];
  return (int64_t)s->allocated * (values ? s->value_dim : s->key_dim);
}

/* ================================================================ attention */

int jmo_attention_start(int position, int window) {
  /* LlamaConfig.attentionStartPosition, causal branch (llama/LlamaConfig.java:184-195). */
  if (window <= 0) return 0;
  int first = position - window + 1;
  return first > 0 ? first : 0;
}

static int gqa_core(const float* q, const float* keys, const float* values, int rows,
                    int key_row_stride, int value_row_stride, int num_heads, int num_kv_heads,
                    int key_length, int value_length, float scale, float* out, float* scores) {
  /* groupedQueryAttention (llama/LlamaForwardPass.java:1543-1593): zero the output, then per
   * head: scores = dot(q_h, K_row) * scale (:1625-1630), softmax over the visible rows
   * (TensorOps.softmax), out_h += p * V_row in ascending position order (:1660-1669). */
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || rows <= 0) return JMO_ILLEGAL_ARGUMENT;
  int group = num_heads / num_kv_heads;
  memset(out, 0, sizeof(float) * (size_t)num_heads * value_length);
  for (int head = 0; head < num_heads; head++) {
    int kv_head = head / group;
    const float* qh = q + (int64_t)head * key_length;
    for (int r = 0; r < rows; r++) {
      const float* krow = keys + (int64_t)r * key_row_stride + (int64_t)kv_head * key_length;
      scores[r] = jmo_dot(qh, krow, key_length) * scale;
    }
    int status = jmo_softmax(scores, rows);
    if (status != JMO_OK) return status;
    float* oh = out + (int64_t)head * value_length;
    for (int r = 0; r < rows; r++) {
      const float* vrow = values + (int64_t)r * value_row_stride + (int64_t)kv_head * value_length;
      float p = scores[r];
      for (int i = 0; i < value_length; i++) oh[i] += p * vrow[i];
    }
  }
  return JMO_OK;
}

int jmo_gqa_rows(const float* q, const float* keys, const float* values, int rows,
                 int key_row_stride, int value_row_stride, int num_heads, int num_kv_heads,
                 int key_length, int value_length, float scale, float* out, float* scores) {
  return gqa_core(q, keys, values, rows, key_row_stride, value_row_stride, num_heads, num_kv_heads,
                  key_length, value_length, scale, out, scores);
}

int jmo_gqa(const jmo_kv* kv, int layer, int position, int window, const float* q, int num_heads,
            int num_kv_heads, int key_length, int value_length, float scale, float* out,
            float* scores) {
  /* Rows are addressed from keyOffset(layer, firstPosition) + (pos - first) * keyDim, exactly as
   * computeAttentionScores does (:1608-1630); values by valueOffset per position (:1660-1668). */
  if (kv->key_dim != num_kv_heads * key_length || kv->value_dim != num_kv_heads * value_length) {
    return JMO_ILLEGAL_ARGUMENT;
  }
  int first = jmo_attention_start(position, window);
  int64_t koff = jmo_kv_key_offset(kv, layer, first);
  int64_t voff = jmo_kv_value_offset(kv, layer, first);
  if (koff < 0 || voff < 0 || position >= kv->capacity) return JMO_ILLEGAL_STATE;
  return gqa_core(q, kv->keys + koff, kv->values + voff, position - first + 1, kv->key_dim,
                  kv->value_dim, num_heads, num_kv_heads, key_length, value_length, scale, out,
                  scores + first);
}

int jmo_gqa_layered(const jmo_lkv* kv, int layer, int position, int window, const float* q,
                    int num_heads, int num_kv_heads, int head_dim, float scale, float* out,
                    float* scores) {
  /* Gemma4ForwardPass.computeAttention (gemma4/Gemma4ForwardPass.java:1186-1230). */
  int first = jmo_attention_start(position, window);
  int spans = 0;
  int span[8];
  int status = jmo_lkv_attention_view(kv, layer, first, position + 1, &spans, span);
  if (status != JMO_OK) return status;
  const jmo_layer_state* s = &kv->layers[layer];
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return JMO_ILLEGAL_ARGUMENT;
  int group = num_heads / num_kv_heads;
  memset(out, 0, sizeof(float) * (size_t)num_heads * head_dim);
  for (int head = 0; head < num_heads; head++) {
    int kv_head = head / group;
    int count = 0;
    for (int sp = 0; sp < spans; sp++) {
      for (int row = 0; row < span[4 * sp + 1]; row++) {
        const float* krow = s->keys + span[4 * sp + 2] + (int64_t)row * s->key_dim +
                            (int64_t)kv_head * head_dim;
        scores[count++] = jmo_dot(q + (int64_t)head * head_dim, krow, head_dim) * scale;
      }
    }
    status = jmo_softmax(scores, count);
    if (status != JMO_OK) return status;
    int idx = 0;
    float* oh = out + (int64_t)head * head_dim;
    for (int sp = 0; sp < spans; sp++) {
      for (int row = 0; row < span[4 * sp + 1]; row++) {
        const float* vrow = s->values + span[4 * sp + 3] + (int64_t)row * s->value_dim +
                            (int64_t)kv_head * head_dim;
        float p = scores[idx++];
        for (int i = 0; i < head_dim; i++) oh[i] += p * vrow[i];
      }
    }
  }
  return JMO_OK;
}

static int rope_heads(float* x, int heads, int key_length, const float* cos_f, const float* sin_f,
                      int neox) {
  for (int h = 0; h < heads; h++) {
    jmo_rope_apply(x + (int64_t)h * key_length, cos_f, sin_f, key_length / 2, neox);
  }
  return JMO_OK;
}

int jmo_decode_layer(jmo_kv* kv, int layer, int position, int window, float* q, float* k,
                     const float* v, int num_heads, int num_kv_heads, int key_length,
                     int value_length, float rope_theta, float rope_scale, int neox, float scale,
                     float* out, float* scores) {
  /* forwardSequenceInternal per-layer attention block (llama/LlamaForwardPass.java:1069-1128). */
  if (position < 0 || position >= kv->max_seq_len) return JMO_ILLEGAL_ARGUMENT;
  if (rope_theta > 0.0f) {
    int pairs = key_length / 2;
    float* cos_f = (float*)malloc(sizeof(float) * (size_t)pairs);
    float* sin_f = (float*)malloc(sizeof(float) * (size_t)pairs);
    int status =
        jmo_rotary_factors(key_length, rope_theta, rope_scale, NULL, position, cos_f, sin_f);
    if (status == JMO_OK) {
      rope_heads(q, num_heads, key_length, cos_f, sin_f, neox);
      rope_heads(k, num_kv_heads, key_length, cos_f, sin_f, neox);
    }
    free(cos_f);
    free(sin_f);
    if (status != JMO_OK) return status;
  }
  int status = jmo_kv_store(kv, layer, position, k, v);
  if (status != JMO_OK) return status;
  return jmo_gqa(kv, layer, position, window, q, num_heads, num_kv_heads, key_length,
                 value_length, scale, out, scores);
}

int jmo_prefill_layer(jmo_kv* kv, int layer, int start, int n, int window, float* q, float* k,
                      const float* v, int num_heads, int num_kv_heads, int key_length,
                      int value_length, float rope_theta, float rope_scale, int neox, float scale,
                      float* out, float* scores) {
  /* prepareBatchedAttention (:1479-1513) stores every row first; computeBatchedAttention
   * (:1515-1541) then attends row b at position start + b, so causality is the loop bound. */
  int query_dim = num_heads * key_length;
  int key_dim = num_kv_heads * key_length;
  int value_dim = num_kv_heads * value_length;
  int pairs = key_length / 2;
  float* cos_f = (float*)malloc(sizeof(float) * (size_t)(pairs > 0 ? pairs : 1));
  float* sin_f = (float*)malloc(sizeof(float) * (size_t)(pairs > 0 ? pairs : 1));
  int status = JMO_OK;
  for (int b = 0; b < n && status == JMO_OK; b++) {
    if (rope_theta > 0.0f) {
      status =
          jmo_rotary_factors(key_length, rope_theta, rope_scale, NULL, start + b, cos_f, sin_f);
      if (status != JMO_OK) break;
      rope_heads(q + (int64_t)b * query_dim, num_heads, key_length, cos_f, sin_f, neox);
      rope_heads(k + (int64_t)b * key_dim, num_kv_heads, key_length, cos_f, sin_f, neox);
    }
    status = jmo_kv_store(kv, layer, start + b, k + (int64_t)b * key_dim,
                          v + (int64_t)b * value_dim);
  }
  free(cos_f);
  free(sin_f);
  for (int b = 0; b < n && status == JMO_OK; b++) {
    status = jmo_gqa(kv, layer, start + b, window, q + (int64_t)b * query_dim, num_heads,
                     num_kv_heads, key_length, value_length, scale,
                     out + (int64_t)b * num_heads * value_length, scores);
  }
  return status;
}

/* ---------------------------------------------------------------- 8-lane timing variant */

/* A dot product in eight partial sums (lane j accumulates elements i with i % 8 == j, then the
 * lanes are added pairwise: (0+4, 1+5, 2+6, 3+7), then (0+2, 1+3), then (0+1)), followed by the
 * scalar tail: the shape of a Vector API reduction over 256-bit float vectors, which the compiler
 * turns into AVX2 code. Used only to time a vectorised CPU baseline; parity is pinned on the
 * sequential jmo_dot. */
static float dot8(const float* a, const float* b, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int i = 0;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; j++) acc[j] += a[i + j] * b[i + j];
  for (int j = 0; j < 4; j++) acc[j] += acc[j + 4];
  acc[0] += acc[2];
  acc[1] += acc[3];
  float sum = acc[0] + acc[1];
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

static int gqa_core8(const float* q, const float* keys, const float* values, int rows,
                     int key_row_stride, int value_row_stride, int num_heads, int num_kv_heads,
                     int key_length, int value_length, float scale, float* out, float* scores) {
  /* gqa_core with dot8 for the scores; the weighted V sum is element-wise (no reduction), so
   * the compiler vectorises it as written. */
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || rows <= 0) return JMO_ILLEGAL_ARGUMENT;
  int group = num_heads / num_kv_heads;
  memset(out, 0, sizeof(float) * (size_t)num_heads * value_length);
  for (int head = 0; head < num_heads; head++) {
    int kv_head = head / group;
    const float* qh = q + (int64_t)head * key_length;
    for (int r = 0; r < rows; r++) {
      const float* krow = keys + (int64_t)r * key_row_stride + (int64_t)kv_head * key_length;
      scores[r] = dot8(qh, krow, key_length) * scale;
    }
    int status = jmo_softmax(scores, rows);
    if (status != JMO_OK) return status;
    float* oh = out + (int64_t)head * value_length;
    for (int r = 0; r < rows; r++) {
      const float* vrow = values + (int64_t)r * value_row_stride + (int64_t)kv_head * value_length;
      float p = scores[r];
      for (int i = 0; i < value_length; i++) oh[i] += p * vrow[i];
    }
  }
  return JMO_OK;
}

/* ---------------------------------------------------------------- threaded baseline */

typedef struct {
  int begin, end;
  int count;
  const float* const* q;
  const float* const* keys;
  const float* const* values;
  const int* rows;
  int key_row_stride, value_row_stride, num_heads, num_kv_heads, key_length, value_length;
  float scale;
  float* const* out;
  int lanes8;
  int status;
} jmo_batch_job;

static void* batch_worker(void* arg) {
  /* Work unit = (sequence, kv head): the heads of one GQA group run gqa_core on a view. */
  jmo_batch_job* job = (jmo_batch_job*)arg;
  int group = job->num_heads / job->num_kv_heads;
  int max_rows = 1;
  for (int s = 0; s < job->count; s++) max_rows = job->rows[s] > max_rows ? job->rows[s] : max_rows;
  float* scores = (float*)malloc(sizeof(float) * (size_t)max_rows);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)group * job->value_length);
  for (int unit = job->begin; unit < job->end && job->status == JMO_OK; unit++) {
    int s = unit / job->num_kv_heads;
    int kvh = unit % job->num_kv_heads;
    /* one kv head, its `group` query heads: a 1-kv-head GQA over offset views */
    int status = (job->lanes8 ? gqa_core8 : gqa_core)(job->q[s] + (int64_t)kvh * group * job->key_length,
                          job->keys[s] + (int64_t)kvh * job->key_length,
                          job->values[s] + (int64_t)kvh * job->value_length, job->rows[s],
                          job->key_row_stride, job->value_row_stride, group, 1, job->key_length,
                          job->value_length, job->scale, tmp, scores);
    if (status != JMO_OK) job->status = status;
    memcpy(job->out[s] + (int64_t)kvh * group * job->value_length, tmp,
           sizeof(float) * (size_t)group * job->value_length);
  }
  free(scores);
  free(tmp);
  return NULL;
}

static int gqa_rows_batch(int count, const float* const* q, const float* const* keys,
                          const float* const* values, const int* rows, int key_row_stride,
                          int value_row_stride, int num_heads, int num_kv_heads, int key_length,
                          int value_length, float scale, float* const* out, int threads,
                          int lanes8) {
  if (count <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return JMO_ILLEGAL_ARGUMENT;
  if (threads < 1) threads = 1;
  int units = count * num_kv_heads;
  if (threads > units) threads = units;
  pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  jmo_batch_job* jobs = (jmo_batch_job*)calloc((size_t)threads, sizeof(jmo_batch_job));
  for (int t = 0; t < threads; t++) {
    jmo_batch_job* j = &jobs[t];
    j->begin = (int)((int64_t)units * t / threads);
    j->end = (int)((int64_t)units * (t + 1) / threads);
    j->count = count;
    j->q = q;
    j->keys = keys;
    j->values = values;
    j->rows = rows;
    j->key_row_stride = key_row_stride;
    j->value_row_stride = value_row_stride;
    j->num_heads = num_heads;
    j->num_kv_heads = num_kv_heads;
    j->key_length = key_length;
    j->value_length = value_length;
    j->scale = scale;
    j->out = out;
    j->lanes8 = lanes8;
    j->status = JMO_OK;
    if (threads == 1) {
      batch_worker(j);
    } else {
      pthread_create(&tids[t], NULL, batch_worker, j);
    }
  }
  int status = JMO_OK;
  for (int t = 0; t < threads; t++) {
    if (threads > 1) pthread_join(tids[t], NULL);
    if (jobs[t].status != JMO_OK) status = jobs[t].status;
  }
  free(tids);
  free(jobs);
  return status;
}

int jmo_gqa_rows_batch(int count, const float* const* q, const float* const* keys,
                       const float* const* values, const int* rows, int key_row_stride,
                       int value_row_stride, int num_heads, int num_kv_heads, int key_length,
                       int value_length, float scale, float* const* out, int threads) {
  return gqa_rows_batch(count, q, keys, values, rows, key_row_stride, value_row_stride, num_heads,
                        num_kv_heads, key_length, value_length, scale, out, threads, 0);
}

int jmo_gqa_rows_batch8(int count, const float* const* q, const float* const* keys,
                        const float* const* values, const int* rows, int key_row_stride,
                        int value_row_stride, int num_heads, int num_kv_heads, int key_length,
                        int value_length, float scale, float* const* out, int threads) {
  return gqa_rows_batch(count, q, keys, values, rows, key_row_stride, value_row_stride, num_heads,
                        num_kv_heads, key_length, value_length, scale, out, threads, 1);
}

/* ================================================================ GGUF block-quantized projection */

/* ggmlNearestInt (NativeKernelLibraryTest.java:1019-1022; RS:4072-4075): adding 1.5 * 2^23 puts
 * the value's integer part in the low mantissa bits, rounded to nearest even. */
static int ggml_nearest_int(float value) {
  const float shifted = value + 12582912.0f;
  uint32_t bits;
  memcpy(&bits, &shifted, 4);
  return (int)(bits & 0x007fffffu) - 0x00400000;
}

void jmo_q8_0_quantize(const float* x, int batch, int cols, int8_t* q, float* scales) {
  const int blocks = cols / 32;
  for (int b = 0; b < batch; b++) {
    for (int blk = 0; blk < blocks; blk++) {
      const float* v = x + (size_t)b * cols + (size_t)blk * 32;
      float absmax = 0.0f;
      for (int i = 0; i < 32; i++) {
        const float a = fabsf(v[i]);
        if (a > absmax) absmax = a; /* a NaN compares false and is skipped */
      }
      const float inverse = absmax == 0.0f ? 0.0f : 127.0f / absmax;
      scales[(size_t)b * blocks + blk] = jmo_f16_to_float(jmo_float_to_f16(absmax / 127.0f));
      for (int i = 0; i < 32; i++) {
        const float scaled = v[i] * inverse;
        q[(size_t)b * cols + (size_t)blk * 32 + i] = (int8_t)ggml_nearest_int(scaled);
      }
    }
  }
}

void jmo_q8_k_quantize(const float* x, int batch, int cols, int8_t* q, float* scales,
                       int16_t* sums) {
  const int blocks = cols / 256;
  for (int b = 0; b < batch; b++) {
    for (int blk = 0; blk < blocks; blk++) {
      const size_t off = (size_t)b * cols + (size_t)blk * 256;
      const float* v = x + off;
      float max = 0.0f, absmax = 0.0f;
      for (int i = 0; i < 256; i++) {
        const float a = fabsf(v[i]);
        if (a > absmax) { /* strict: the first of equal magnitudes wins; NaN compares false */
          absmax = a;
          max = v[i];
        }
      }
      int16_t* s16 = sums + (size_t)b * (cols / 16) + (size_t)blk * 16;
      if (absmax == 0.0f) {
        memset(q + off, 0, 256);
        memset(s16, 0, 16 * sizeof(int16_t));
        scales[(size_t)b * blocks + blk] = 0.0f;
        continue;
      }
      const float inverse = -127.0f / max;
      int block_sum = 0;
      for (int i = 0; i < 256; i++) {
        const float scaled = inverse * v[i];
        int quant = ggml_nearest_int(scaled);
        if (quant > 127) quant = 127;
        q[off + i] = (int8_t)quant;
        block_sum += (int8_t)quant;
        if ((i + 1) % 16 == 0) {
          s16[i / 16] = (int16_t)block_sum;
          block_sum = 0;
        }
      }
      scales[(size_t)b * blocks + blk] = 1.0f / inverse;
    }
  }
}

/* qk_scale / qk_min (RS:3861-3878): 6-bit scale and min of 32-element group g of a Q4_K block. */
static int qk_scale(const uint8_t* sc, int g) {
  if (g < 4) return sc[g] & 0x3f;
  return (sc[g + 4] & 0x0f) | ((sc[g - 4] >> 6) << 4);
}
static int qk_min(const uint8_t* sc, int g) {
  if (g < 4) return sc[g + 4] & 0x3f;
  return (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
}

static float kquant_row(int format, const uint8_t* w_row, const int8_t* aq, const float* ascale,
                        const int16_t* asum, int blocks) {
  if (format == JMO_FMT_Q4_K) {
    float sum = 0.0f;
    for (int blk = 0; blk < blocks; blk++) {
      const uint8_t* w = w_row + (size_t)blk * 144;
      const float d = jmo_f16_to_float((uint16_t)(w[0] | (w[1] << 8))) * ascale[blk];
      const float dmin = jmo_f16_to_float((uint16_t)(w[2] | (w[3] << 8))) * ascale[blk];
      const uint8_t* sc = w + 4;
      const uint8_t* qs = w + 16;
      const int8_t* a = aq + (size_t)blk * 256;
      const int16_t* s16 = asum + (size_t)blk * 16;
      int qsum = 0, msum = 0;
      for (int g = 0; g < 8; g++) {
        const uint8_t* packed = qs + (g >> 1) * 32;
        const int shift = (g & 1) * 4;
        int dot = 0;
        for (int i = 0; i < 32; i++) dot += ((packed[i] >> shift) & 0x0f) * a[g * 32 + i];
        qsum += qk_scale(sc, g) * dot;
        msum += qk_min(sc, g) * (s16[2 * g] + s16[2 * g + 1]);
      }
      sum = fmaf(d, (float)qsum, sum);
      sum = fmaf(-dmin, (float)msum, sum);
    }
    return sum;
  }
  if (format == JMO_FMT_Q5_K) {
    /* dot_q5_k_q8_k_row_scalar (RS:3461-3518): Q4_K's arithmetic, each quant taking bit g of
     * qh[index] as its fifth bit (value 16). */
    float sum = 0.0f;
    for (int blk = 0; blk < blocks; blk++) {
      const uint8_t* w = w_row + (size_t)blk * 176;
      const float d = jmo_f16_to_float((uint16_t)(w[0] | (w[1] << 8))) * ascale[blk];
      const float dmin = jmo_f16_to_float((uint16_t)(w[2] | (w[3] << 8))) * ascale[blk];
      const uint8_t* sc = w + 4;
      const uint8_t* qh = w + 16;
      const uint8_t* qs = w + 48;
      const int8_t* a = aq + (size_t)blk * 256;
      const int16_t* s16 = asum + (size_t)blk * 16;
      int qsum = 0, msum = 0;
      for (int g = 0; g < 8; g++) {
        const uint8_t* packed = qs + (g >> 1) * 32;
        const int shift = (g & 1) * 4;
        int dot = 0;
        for (int i = 0; i < 32; i++) {
          const int quant = ((packed[i] >> shift) & 0x0f) | ((qh[i] >> g) & 1 ? 16 : 0);
          dot += quant * a[g * 32 + i];
        }
        qsum += qk_scale(sc, g) * dot;
        msum += qk_min(sc, g) * (s16[2 * g] + s16[2 * g + 1]);
      }
      sum = fmaf(d, (float)qsum, sum);
      sum = fmaf(-dmin, (float)msum, sum);
    }
    return sum;
  }
  /* Q6_K */
  float lane_sums[8] = {0};
  for (int blk = 0; blk < blocks; blk++) {
    const uint8_t* w = w_row + (size_t)blk * 210;
    const float d = jmo_f16_to_float((uint16_t)(w[208] | (w[209] << 8))) * ascale[blk];
    const uint8_t* ql = w;
    const uint8_t* qh = w + 128;
    const int8_t* sc = (const int8_t*)(w + 192);
    const int8_t* a = aq + (size_t)blk * 256;
    int isum[8] = {0};
    for (int sb = 0; sb < 2; sb++) {
      for (int i = 0; i < 32; i++) {
        const int si = i / 16;
        const int l1 = ql[sb * 64 + i], l2 = ql[sb * 64 + 32 + i], hi = qh[sb * 32 + i];
        const int q1 = ((l1 & 0x0f) | ((hi & 3) << 4)) - 32;
        const int q2 = ((l2 & 0x0f) | (((hi >> 2) & 3) << 4)) - 32;
        const int q3 = ((l1 >> 4) | (((hi >> 4) & 3) << 4)) - 32;
        const int q4 = ((l2 >> 4) | (((hi >> 6) & 3) << 4)) - 32;
        const int8_t* aa = a + sb * 128;
        int* acc = &isum[i & 7];
        *acc += sc[sb * 8 + si] * q1 * aa[i];
        *acc += sc[sb * 8 + si + 2] * q2 * aa[i + 32];
        *acc += sc[sb * 8 + si + 4] * q3 * aa[i + 64];
        *acc += sc[sb * 8 + si + 6] * q4 * aa[i + 96];
      }
    }
    for (int l = 0; l < 8; l++) lane_sums[l] = fmaf(d, (float)isum[l], lane_sums[l]);
  }
  float sum = 0.0f;
  for (int l = 0; l < 8; l++) sum += lane_sums[l];
  return sum;
}

static int kquant_matmul(int format, const uint8_t* weights, const float* input, int batch,
                         int rows, int cols, float* out) {
  const int blocks = cols / 256;
  const int block_bytes = format == JMO_FMT_Q4_K ? 144 : format == JMO_FMT_Q5_K ? 176 : 210;
  int8_t* q = (int8_t*)malloc((size_t)batch * cols);
  float* scales = (float*)malloc((size_t)batch * blocks * sizeof(float));
  int16_t* sums = (int16_t*)malloc((size_t)batch * (cols / 16) * sizeof(int16_t));
  if (!q || !scales || !sums) {
    free(q);
    free(scales);
    free(sums);
    return JMO_ILLEGAL_STATE;
  }
  jmo_q8_k_quantize(input, batch, cols, q, scales, sums);
  for (int b = 0; b < batch; b++)
    for (int r = 0; r < rows; r++)
      out[(size_t)b * rows + r] =
          kquant_row(format, weights + (size_t)r * blocks * block_bytes, q + (size_t)b * cols,
                     scales + (size_t)b * blocks, sums + (size_t)b * (cols / 16), blocks);
  free(q);
  free(scales);
  free(sums);
  return JMO_OK;
}

int jmo_quantized_matmul(int format, const uint8_t* weights, const float* input, int batch,
                         int rows, int cols, float* out) {
  if (rows <= 0 || batch <= 0 || cols <= 0) return JMO_ILLEGAL_ARGUMENT;
  if (format == JMO_FMT_Q4_K || format == JMO_FMT_Q5_K || format == JMO_FMT_Q6_K) {
    if (cols % 256 != 0) return JMO_ILLEGAL_ARGUMENT;
    return kquant_matmul(format, weights, input, batch, rows, cols, out);
  }
  if ((format != JMO_FMT_Q4_0 && format != JMO_FMT_Q8_0 && format != JMO_FMT_Q5_0) ||
      cols % 32 != 0)
    return JMO_ILLEGAL_ARGUMENT;
  const int blocks = cols / 32;
  const int block_bytes = format == JMO_FMT_Q4_0 ? 18 : format == JMO_FMT_Q5_0 ? 22 : 34;
  int8_t* q = (int8_t*)malloc((size_t)batch * cols);
  float* scales = (float*)malloc((size_t)batch * blocks * sizeof(float));
  if (!q || !scales) {
    free(q);
    free(scales);
    return JMO_ILLEGAL_STATE;
  }
  jmo_q8_0_quantize(input, batch, cols, q, scales);
  for (int b = 0; b < batch; b++) {
    for (int r = 0; r < rows; r++) {
      float sum = 0.0f;
      for (int blk = 0; blk < blocks; blk++) {
        const uint8_t* w = weights + ((size_t)r * blocks + blk) * block_bytes;
        const float weight_scale = jmo_f16_to_float((uint16_t)(w[0] | (w[1] << 8)));
        const int8_t* a = q + (size_t)b * cols + (size_t)blk * 32;
        int dot = 0;
        if (format == JMO_FMT_Q4_0) {
          /* byte i holds element i in its low nibble and element i + 16 in its high one, each
           * offset by 8 (:921-926) */
          for (int i = 0; i < 16; i++) {
            const int packed = w[2 + i];
            dot += ((packed & 0xf) - 8) * a[i];
            dot += ((packed >> 4) - 8) * a[i + 16];
          }
        } else if (format == JMO_FMT_Q5_0) {
          /* referenceQ5_0F32BatchedMatmul (NativeKernelLibraryTest.java:966-993; RS:3204-3252):
           * byte i holds the low nibbles of elements i and i + 16, bits i and i + 16 of the
           * little-endian word at byte 2 their fifth bits, each element offset by 16 */
          const uint32_t high = (uint32_t)w[2] | ((uint32_t)w[3] << 8) | ((uint32_t)w[4] << 16) |
                                ((uint32_t)w[5] << 24);
          for (int i = 0; i < 16; i++) {
            const int packed = w[6 + i];
            const int lo = ((packed & 0xf) | (int)(((high >> i) & 1u) << 4)) - 16;
            const int hi = ((packed >> 4) | (int)(((high >> (i + 16)) & 1u) << 4)) - 16;
            dot += lo * a[i];
            dot += hi * a[i + 16];
          }
        } else {
          for (int i = 0; i < 32; i++) dot += (int8_t)w[2 + i] * a[i];
        }
        const float scale = weight_scale * scales[(size_t)b * blocks + blk];
        sum = fmaf(scale, (float)dot, sum); /* Math.fma (:929-930) */
      }
      out[(size_t)b * rows + r] = sum;
    }
  }
  free(q);
  free(scales);
  return JMO_OK;
}

/*
 * tlm_oracle.c -- CPU restatement of three-llm's per-token decoder path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared
 * against; it is imported by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, and by nothing else.  The product library never
 * links, loads or calls it.
 *
 * Semantics follow the reference's CPU runner, which is JavaScript: every
 * scalar is an IEEE double, every stored array is a Float32Array.  So each
 * function below accumulates in double and rounds to float exactly where the
 * reference stores into a Float32Array.  Build with -ffp-contract=off: the
 * reference rounds every product and sum separately, an FMA would not.
 *
 * Reference files are cited relative to packages/three-llm/src/.
 *
 * Parity pins (tests/test_oracle.py):
 *   orc_f16_to_f32, orc_bf16_to_f32  exhaustive 65536 patterns vs IEEE (numpy),
 *                                    known answers of engine.test.ts:599-610.
 *   orc_f32_to_f16                   exhaustive round trip + numpy RNE on 1M values.
 *   orc_linear / orc_linear_t        closed forms engine.test.ts:491-505, HF fixture.
 *   orc_rmsnorm, orc_silu, softmax   closed forms engine.test.ts:507-548.
 *   orc_rope_parameters, orc_apply_rope  HF fixture inv_freq / rotated Q,K (5 cases).
 *   orc_attention                    HF fixture logits; brute force on tiny shapes,
 *                                    pos=0 -> V row, softmax shift invariance.
 *   orc_forward_token                HF fixture logits + final hidden, fp32 and
 *                                    fp16-storage variants (19 positions x 5 cases).
 *   orc_argmax                       tie/first-max KATs of tsl.browser.test.ts:82-103.
 *   orc_topk_candidates              KATs of tsl.browser.test.ts:82-120 (chunked
 *                                    candidates, softcap); brute force (sort by
 *                                    score desc, id asc) with ties, -inf and NaN;
 *                                    the result does not depend on the chunk size.
 *   orc_q4_quantize, orc_q4_dequant  build-defined format (no reference counterpart):
 *                                    exhaustive codes x scale set, round-trip bound.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

/* ---------------------------------------------------------------- dtypes -- */

/* float16ToFloat32, load/tensors.ts:29-45.  The reference builds the value in
 * double from sign, exponent and fraction; every fp16 is exact in fp32. */
float orc_f16_to_f32(uint16_t value) {
  int sign = (value >> 15) & 1;
  int exponent = (value >> 10) & 0x1f;
  int fraction = value & 0x3ff;
  double r;
  if (exponent == 0) {
    if (fraction == 0) return sign ? -0.0f : 0.0f;
    r = (sign ? -1.0 : 1.0) * pow(2.0, -14) * (fraction / 1024.0);
  } else if (exponent == 31) {
    return fraction ? NAN : (sign ? -INFINITY : INFINITY);
  } else {
    r = (sign ? -1.0 : 1.0) * pow(2.0, exponent - 15) * (1.0 + fraction / 1024.0);
  }
  return (float)r;
}

/* bfloat16ToFloat32, load/tensors.ts:65-68: the 16 bits become the high half. */
float orc_bf16_to_f32(uint16_t value) {
  uint32_t bits = (uint32_t)value << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* fp32 -> fp16, round to nearest even (IEEE 754 binary16).  The reference has
 * no such function; it is the rounding the fp16 storage fixture uses
 * (torch .half(), scripts/reference/generate.py) and the device KV cache. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u | ((absx >> 13) & 0x3ffu) : 0u));
  if (absx >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7c00u);
  if (absx < 0x38800000u) { /* below the fp16 normal range: subnormal or zero */
    if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to zero */
    uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    int e = (int)(absx >> 23); /* 102..112 */
    int shift = 126 - e;       /* so that the result is mant >> shift in units of 2^-24 */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (absx >> 23) - 112u; /* rebias 127 -> 15 */
  uint32_t mant = absx & 0x7fffffu;
  uint32_t q = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------- math -- */

/* linear, runtime/math.ts:6-25.  Weight layout [in][out] exactly as the
 * reference: y[o] = b[o] + sum_i x[i] * W[i*out + o], i ascending, double sum. */
void orc_linear(const float* x, const float* w, const float* bias, int in, int out, float* y) {
  for (int o = 0; o < out; o++) {
    double sum = bias ? (double)bias[o] : 0.0;
    for (int i = 0; i < in; i++) sum += (double)x[i] * (double)w[(size_t)i * out + o];
    y[o] = (float)sum;
  }
}

/* The same reduction with the weight stored [out][in] (Hugging Face
 * orientation, the transpose the reference builds at DecoderWeights.ts:224-235).
 * The order of the additions is unchanged, so results are bit-identical to
 * orc_linear on the transposed matrix.  Rows are independent, so threads split
 * rows without changing any sum. */
void orc_linear_t(const float* x, const float* wt, const float* bias, int in, int out, float* y) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && (long)in * out > (1L << 18))
  for (int o = 0; o < out; o++) {
    const float* row = wt + (size_t)o * in;
    double sum = bias ? (double)bias[o] : 0.0;
    for (int i = 0; i < in; i++) sum += (double)x[i] * (double)row[i];
    y[o] = (float)sum;
  }
}

/* rmsNorm, runtime/math.ts:78-97.  weight may be NULL (scale 1); offset selects
 * the `1 + weight` (Gemma) variant. */
void orc_rmsnorm(const float* x, const float* w, int n, double eps, int offset, float* y) {
  double sum_squares = 0.0;
  for (int i = 0; i < n; i++) sum_squares += (double)x[i] * (double)x[i];
  double inv_rms = 1.0 / sqrt(sum_squares / n + eps);
  for (int i = 0; i < n; i++) {
    double scale = w == NULL ? 1.0 : offset ? 1.0 + (double)w[i] : (double)w[i];
    y[i] = (float)((double)x[i] * inv_rms * scale);
  }
}

/* softmax, runtime/math.ts:60-76.  The running sum adds the unrounded double
 * exponentials; the division uses the stored (rounded) value. */
void orc_softmax(const float* v, int n, float* out) {
  double max_value = -INFINITY;
  for (int i = 0; i < n; i++) max_value = fmax(max_value, (double)v[i]);
  double sum = 0.0;
  for (int i = 0; i < n; i++) {
    double value = exp((double)v[i] - max_value);
    out[i] = (float)value;
    sum += value;
  }
  for (int i = 0; i < n; i++) out[i] = (float)((double)out[i] / sum);
}

/* silu, runtime/math.ts:99-101 (evaluated in double). */
double orc_silu(double x) { return x / (1.0 + exp(-x)); }

/* ropeParameters, runtime/rope.ts:4-52.
 * kind: 0 default, 1 linear, 2 yarn, 3 llama3.  For yarn, attn_factor < 0
 * means "not given" (the reference's `?? 1 + 0.1 ln factor`).  Returns 0, or
 * -1 for the inputs the reference rejects with an Error. */
int orc_rope_parameters(int dim, double theta, int kind, double factor, double orig_ctx, double beta_fast,
                        double beta_slow, double attn_factor, double low_freq, double high_freq, float* inv_freq,
                        double* attention_factor_out) {
  if (dim < 0 || dim % 2 != 0) return -1;
  if (!isfinite(theta) || theta <= 1) return -1;
  if (kind != 0 && (!isfinite(factor) || factor < 1)) return -1;
  double attention_factor = 1.0;
  double low = 0, high = 0;
  if (kind == 2) {
    if (!(isfinite(orig_ctx) && isfinite(beta_fast) && isfinite(beta_slow))) return -1;
    if (!(orig_ctx > 0 && beta_fast > 0 && beta_slow > 0 && beta_fast >= beta_slow)) return -1;
    attention_factor = attn_factor >= 0 ? attn_factor : 1 + 0.1 * log(factor);
    if (!isfinite(attention_factor) || attention_factor <= 0) return -1;
#define CORRECTION(r) ((dim * log(orig_ctx / ((r) * 2 * M_PI))) / (2 * log(theta)))
    low = fmax(0, floor(CORRECTION(beta_fast)));
    high = fmin(dim - 1, ceil(CORRECTION(beta_slow)));
#undef CORRECTION
    if (low == high) high += 0.001;
  }
  if (kind == 3) {
    if (!(isfinite(orig_ctx) && isfinite(low_freq) && isfinite(high_freq))) return -1;
    if (!(orig_ctx > 0 && low_freq > 0 && high_freq > low_freq)) return -1;
  }
  for (int i = 0; i < dim / 2; i++) {
    double frequency = 1.0 / pow(theta, (2.0 * i) / dim);
    if (kind == 1) frequency /= factor;
    if (kind == 2) {
      double ramp = fmin(1, fmax(0, (i - low) / (high - low)));
      frequency *= 1 - ramp + ramp / factor;
    }
    if (kind == 3) {
      double wavelength = (2 * M_PI) / frequency;
      if (wavelength > orig_ctx / low_freq)
        frequency /= factor;
      else if (wavelength >= orig_ctx / high_freq) {
        double smooth = (orig_ctx / wavelength - low_freq) / (high_freq - low_freq);
        frequency *= (1 - smooth) / factor + smooth;
      }
    }
    inv_freq[i] = (float)frequency;
  }
  *attention_factor_out = attention_factor;
  return 0;
}

/* applyRoPE, runtime/math.ts:118-152 (rotate-half over [0, rotary_dim)).
 * inv_freq holds the ropeParameters table, pair_count the reference's
 * ropePairCount (default rotary_dim / 2). */
void orc_apply_rope(float* v, int head_offset, int rotary_dim, int position, const float* inv_freq, int pair_count,
                    double attention_factor) {
  if (rotary_dim <= 0) return;
  int half = rotary_dim / 2;
  float rotated[1024];
  for (int i = 0; i < rotary_dim; i++) {
    double x = v[head_offset + i];
    int freq_index = i < half ? i : i - half;
    if (freq_index >= pair_count) {
      rotated[i] = (float)x;
      continue;
    }
    double partner = i < half ? -(double)v[head_offset + i + half] : (double)v[head_offset + i - half];
    double angle = (double)position * (double)inv_freq[freq_index];
    rotated[i] = (float)((x * cos(angle) + partner * sin(angle)) * attention_factor);
  }
  for (int i = 0; i < rotary_dim; i++) v[head_offset + i] = rotated[i];
}

static float round_f16(float f) { return orc_f16_to_f32(orc_f32_to_f16(f)); }

typedef struct {
  int heads, kv_heads, head_dim, rotary_dim, sliding_window, kv_f16;
  const float* inv_freq;
  int pair_count;
  double attention_factor;
  double attn_scale;
} orc_attn_opts;

/* causalAttention, runtime/math.ts:179-276, for the Llama/Qwen2 recipe: no
 * q/k-norm, no v-norm, no output gate.  qkv is [q | k | v] (fp32, not
 * modified).  The caches are [max_tokens][kv_heads*head_dim].  kv_f16 = 1
 * stores K and V rounded to fp16, the precision of the device cache; 0 keeps
 * the reference's fp32 cache. */
static void attention_impl(const float* qkv, const orc_attn_opts* o, int position, float* key_cache,
                           float* value_cache, float* output) {
  int D = o->head_dim;
  int q_size = o->heads * D;
  int kv_size = o->kv_heads * D;
  float* query = (float*)malloc(sizeof(float) * q_size);
  float* key = (float*)malloc(sizeof(float) * kv_size);
  memcpy(query, qkv, sizeof(float) * q_size);
  memcpy(key, qkv + q_size, sizeof(float) * kv_size);
  int first = o->sliding_window > 0 ? (position - o->sliding_window + 1 > 0 ? position - o->sliding_window + 1 : 0) : 0;
  for (int h = 0; h < o->heads; h++)
    orc_apply_rope(query, h * D, o->rotary_dim, position, o->inv_freq, o->pair_count, o->attention_factor);
  for (int h = 0; h < o->kv_heads; h++)
    orc_apply_rope(key, h * D, o->rotary_dim, position, o->inv_freq, o->pair_count, o->attention_factor);
  const float* value = qkv + q_size + kv_size;
  for (int d = 0; d < kv_size; d++) {
    key_cache[(size_t)position * kv_size + d] = o->kv_f16 ? round_f16(key[d]) : key[d];
    value_cache[(size_t)position * kv_size + d] = o->kv_f16 ? round_f16(value[d]) : value[d];
  }
  int count = position - first + 1;
  float* scores = (float*)malloc(sizeof(float) * count);
  float* weights = (float*)malloc(sizeof(float) * count);
  for (int h = 0; h < o->heads; h++) {
    int q_off = h * D;
    int kv_head = (h * o->kv_heads) / o->heads;
    int kv_off = kv_head * D;
    for (int t = first; t <= position; t++) {
      double dot = 0.0;
      for (int i = 0; i < D; i++) dot += (double)query[q_off + i] * (double)key_cache[(size_t)t * kv_size + kv_off + i];
      scores[t - first] = (float)(dot * o->attn_scale);
    }
    orc_softmax(scores, count, weights);
    for (int i = 0; i < D; i++) {
      double sum = 0.0;
      for (int t = first; t <= position; t++)
        sum += (double)weights[t - first] * (double)value_cache[(size_t)t * kv_size + kv_off + i];
      output[q_off + i] = (float)sum;
    }
  }
  free(scores);
  free(weights);
  free(query);
  free(key);
}

/* One causalAttention call (tests drive it directly).  attn_scale <= 0 selects
 * the reference default 1/sqrt(head_dim) (math.ts:190). */
void orc_attention(const float* qkv, int heads, int kv_heads, int head_dim, int rotary_dim, const float* inv_freq,
                   int pair_count, double attention_factor, double attn_scale, int sliding_window, int kv_f16,
                   int position, float* key_cache, float* value_cache, float* output) {
  orc_attn_opts o = {heads, kv_heads, head_dim, rotary_dim, sliding_window, kv_f16, inv_freq,
                     pair_count, attention_factor, attn_scale > 0 ? attn_scale : 1.0 / sqrt((double)head_dim)};
  attention_impl(qkv, &o, position, key_cache, value_cache, output);
}

/* Greedy branch of sampleTopK, runtime/math.ts:581-593: first maximum wins. */
int orc_argmax(const float* logits, int n) {
  int best = 0;
  float best_value = logits[0];
  for (int i = 1; i < n; i++)
    if (logits[i] > best_value) {
      best = i;
      best_value = logits[i];
    }
  return best;
}

/* TSLLogitSampler candidate levels, TSLLogits.ts:245-330.  Per chunk of
 * `chunk` logits and rank r < k: the best (score, id) not already taken in
 * this chunk, starting from (id 0, LOWEST_FLOAT) and taking strictly higher
 * scores or equal scores with a lower id (:248-266).  Then per rank r: the
 * best chunk candidate of rank <= r not already taken globally (:268-300).
 * Scores pass through cap * tanh(x / cap) first when softcap > 0 (:185-191),
 * in float as the shader does. */
void orc_topk_candidates(const float* logits, int n, int chunk, int k, double softcap, int* tokens,
                         float* scores) {
  const float lowest = -3.4028234663852886e38f;
  const int nchunks = (n + chunk - 1) / chunk;
  int* ct = (int*)malloc(sizeof(int) * (size_t)nchunks * k);
  float* cs = (float*)malloc(sizeof(float) * (size_t)nchunks * k);
  for (int c = 0; c < nchunks; c++) {
    const int off = c * chunk, size = n - off < chunk ? n - off : chunk;
    for (int r = 0; r < k; r++) {
      int best = 0;
      float best_score = lowest;
      for (int i = 0; i < size; i++) {
        const int id = off + i;
        float score = logits[id];
        if (softcap > 0) score = (float)softcap * tanhf(score / (float)softcap);
        int selected = 0;
        for (int p = 0; p < r; p++)
          if (ct[c * k + p] == id) selected = 1;
        if (!selected && (score > best_score || (score == best_score && id < best))) {
          best = id;
          best_score = score;
        }
      }
      ct[c * k + r] = best;
      cs[c * k + r] = best_score;
    }
  }
  for (int r = 0; r < k; r++) {
    int best = 0;
    float best_score = lowest;
    for (int c = 0; c < nchunks; c++)
      for (int q = 0; q <= r; q++) {
        const int id = ct[c * k + q];
        const float score = cs[c * k + q];
        int selected = 0;
        for (int p = 0; p < r; p++)
          if (tokens[p] == id) selected = 1;
        if (!selected && (score > best_score || (score == best_score && id < best))) {
          best = id;
          best_score = score;
        }
      }
    tokens[r] = best;
    scores[r] = best_score;
  }
  free(ct);
  free(cs);
}

/* ------------------------------------------------------------------- q4 ---
 * Build-defined 4-bit format (the reference has no quantized format; it would
 * consume these weights only after dequantizing them to fp32):
 *   W is [N][K] (row = output feature), K a multiple of 32.  For each row n and
 *   group g of 32 consecutive k: s = fp16(fp32(max|w| / 7)), clamped to the
 *   largest finite fp16; q = clamp(rint(w / f32(s)), -8, 7) (ties to even),
 *   q = 0 when s == 0; stored as the nibble q + 8, two per byte, even k in the
 *   low nibble: byte (n, k/2) = (q[k] + 8) | (q[k+1] + 8) << 4.
 *   Scales are [N][K/32] fp16 bits.  Dequant: w' = f32(s) * (nibble - 8),
 *   exact in fp32. */
void orc_q4_quantize(const float* w, int N, int K, uint8_t* packed, uint16_t* scales) {
  int G = K / 32;
  for (int n = 0; n < N; n++) {
    for (int g = 0; g < G; g++) {
      const float* src = w + (size_t)n * K + g * 32;
      float maxabs = 0.0f;
      for (int j = 0; j < 32; j++) maxabs = fmaxf(maxabs, fabsf(src[j]));
      float s32 = maxabs / 7.0f;
      uint16_t s16 = orc_f32_to_f16(s32);
      if ((s16 & 0x7c00u) == 0x7c00u) s16 = (uint16_t)((s16 & 0x8000u) | 0x7bffu);
      float s = orc_f16_to_f32(s16);
      scales[(size_t)n * G + g] = s16;
      for (int j = 0; j < 32; j += 2) {
        int q[2];
        for (int u = 0; u < 2; u++) {
          float r = s == 0.0f ? 0.0f : rintf(src[j + u] / s);
          if (r < -8.0f) r = -8.0f;
          if (r > 7.0f) r = 7.0f;
          q[u] = (int)r;
        }
        packed[(size_t)n * (K / 2) + (g * 32 + j) / 2] = (uint8_t)((q[0] + 8) | ((q[1] + 8) << 4));
      }
    }
  }
}

void orc_q4_dequant(const uint8_t* packed, const uint16_t* scales, int N, int K, float* out) {
  int G = K / 32;
  /* rows are independent: threads split them without changing any value */
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && (long)N * K > (1L << 20))
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) {
      uint8_t b = packed[(size_t)n * (K / 2) + k / 2];
      int nib = (k & 1) ? (b >> 4) : (b & 15);
      out[(size_t)n * K + k] = orc_f16_to_f32(scales[(size_t)n * G + k / 32]) * (float)(nib - 8);
    }
}

/* ------------------------------------------------------------ the model --- */

enum {
  ORC_EMBED = 0,
  ORC_LM_HEAD = 1,
  ORC_FINAL_NORM = 2,
  ORC_ATTN_NORM = 3,
  ORC_FFN_NORM = 4,
  ORC_WQKV = 5,
  ORC_BQKV = 6,
  ORC_WO = 7,
  ORC_WGATE = 8,
  ORC_WUP = 9,
  ORC_WDOWN = 10,
};

typedef struct {
  int hidden, inter, layers, heads, kv_heads, head_dim, vocab, max_tokens;
  double eps;
  orc_attn_opts attn;
  float* inv_freq;
  const float* embed;
  const float* lm_head;
  const float* final_norm;
  const float** attn_norm;
  const float** ffn_norm;
  const float** wqkv;
  const float** bqkv;
  const float** wo;
  const float** wgate;
  const float** wup;
  const float** wdown;
  float* kcache;
  float* vcache;
  int* windows; /* per layer (block.slidingWindow); NULL: attn.sliding_window */
} orc_model;

/* Weights are borrowed (not copied): the caller keeps the arrays alive.  All
 * matrices are fp32 in Hugging Face orientation [out][in]. */
orc_model* orc_model_new(int hidden, int inter, int layers, int heads, int kv_heads, int head_dim, int vocab,
                         int max_tokens, double eps, int rotary_dim, const float* inv_freq, int pair_count,
                         double attention_factor, int sliding_window, int kv_f16) {
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->hidden = hidden;
  m->inter = inter;
  m->layers = layers;
  m->heads = heads;
  m->kv_heads = kv_heads;
  m->head_dim = head_dim;
  m->vocab = vocab;
  m->max_tokens = max_tokens;
  m->eps = eps;
  m->inv_freq = (float*)malloc(sizeof(float) * (rotary_dim / 2 + 1));
  memcpy(m->inv_freq, inv_freq, sizeof(float) * (rotary_dim / 2));
  orc_attn_opts a = {heads,    kv_heads, head_dim,         rotary_dim, sliding_window, kv_f16, m->inv_freq,
                     pair_count, attention_factor, 1.0 / sqrt((double)head_dim)};
  m->attn = a;
#define ALLOC_LAYERS(f) m->f = (const float**)calloc(layers, sizeof(float*))
  ALLOC_LAYERS(attn_norm);
  ALLOC_LAYERS(ffn_norm);
  ALLOC_LAYERS(wqkv);
  ALLOC_LAYERS(bqkv);
  ALLOC_LAYERS(wo);
  ALLOC_LAYERS(wgate);
  ALLOC_LAYERS(wup);
  ALLOC_LAYERS(wdown);
#undef ALLOC_LAYERS
  size_t cache = (size_t)layers * max_tokens * kv_heads * head_dim;
  m->kcache = (float*)calloc(cache, sizeof(float));
  m->vcache = (float*)calloc(cache, sizeof(float));
  return m;
}

void orc_model_set(orc_model* m, int tensor, int layer, const float* data) {
  switch (tensor) {
    case ORC_EMBED: m->embed = data; break;
    case ORC_LM_HEAD: m->lm_head = data; break;
    case ORC_FINAL_NORM: m->final_norm = data; break;
    case ORC_ATTN_NORM: m->attn_norm[layer] = data; break;
    case ORC_FFN_NORM: m->ffn_norm[layer] = data; break;
    case ORC_WQKV: m->wqkv[layer] = data; break;
    case ORC_BQKV: m->bqkv[layer] = data; break;
    case ORC_WO: m->wo[layer] = data; break;
    case ORC_WGATE: m->wgate[layer] = data; break;
    case ORC_WUP: m->wup[layer] = data; break;
    case ORC_WDOWN: m->wdown[layer] = data; break;
  }
}

/* recipe.attnScale (<= 0: 1/sqrt(head_dim)) and the blocks' slidingWindow,
 * as DecoderCPURunner.attention passes them (decoder/DecoderCPURunner.ts:
 * 140-160; per-layer windows from DecoderWeights.ts:307-311).  windows may be
 * NULL (every layer keeps the model's window); it is copied. */
void orc_model_set_attention(orc_model* m, double attn_scale, const int* windows) {
  m->attn.attn_scale = attn_scale > 0 ? attn_scale : 1.0 / sqrt((double)m->head_dim);
  free(m->windows);
  m->windows = NULL;
  if (windows) {
    m->windows = (int*)malloc(sizeof(int) * m->layers);
    memcpy(m->windows, windows, sizeof(int) * m->layers);
  }
}

void orc_model_free(orc_model* m) {
  free(m->windows);
  free(m->attn_norm);
  free(m->ffn_norm);
  free(m->wqkv);
  free(m->bqkv);
  free(m->wo);
  free(m->wgate);
  free(m->wup);
  free(m->wdown);
  free(m->kcache);
  free(m->vcache);
  free(m->inv_freq);
  free(m);
}

/* resetCache, decoder/DecoderCPURunner.ts:163-171. */
void orc_model_reset(orc_model* m) {
  size_t cache = (size_t)m->layers * m->max_tokens * m->kv_heads * m->head_dim;
  memset(m->kcache, 0, cache * sizeof(float));
  memset(m->vcache, 0, cache * sizeof(float));
}

/* Read back the cache rows [0, count) of one layer ([count][kv_heads*D]). */
void orc_model_read_cache(const orc_model* m, int layer, int count, float* k, float* v) {
  size_t kv = (size_t)m->kv_heads * m->head_dim;
  memcpy(k, m->kcache + (size_t)layer * m->max_tokens * kv, sizeof(float) * kv * count);
  memcpy(v, m->vcache + (size_t)layer * m->max_tokens * kv, sizeof(float) * kv * count);
}

/* Write cache rows [pos0, pos0 + count) of one layer ([count][kv_heads*D]
 * fp32), e.g. rows a device produced, so that the oracle continues from
 * that cache (positions past the rows it computed itself). */
int orc_model_write_cache(orc_model* m, int layer, int pos0, int count, const float* k, const float* v) {
  if (layer < 0 || layer >= m->layers || pos0 < 0 || count < 0 || pos0 + count > m->max_tokens) return -1;
  size_t kv = (size_t)m->kv_heads * m->head_dim;
  size_t off = ((size_t)layer * m->max_tokens + pos0) * kv;
  memcpy(m->kcache + off, k, sizeof(float) * kv * count);
  memcpy(m->vcache + off, v, sizeof(float) * kv * count);
  return 0;
}

/* forwardToken, decoder/DecoderCPURunner.ts:47-138: the sequential
 * (Llama/Qwen2) branch :102-132, then final norm and logits :135-137.
 * hidden_out (optional) receives the final normed hidden state. */
int orc_forward_token(orc_model* m, int token, int position, float* logits, float* hidden_out) {
  if (token < 0 || token >= m->vocab || position < 0 || position >= m->max_tokens) return -1;
  int H = m->hidden, I = m->inter, D = m->head_dim;
  int q_size = m->heads * D, kv_size = m->kv_heads * D, qkv_n = q_size + 2 * kv_size;
  float* x = (float*)malloc(sizeof(float) * H);
  float* norm = (float*)malloc(sizeof(float) * H);
  float* qkv = (float*)malloc(sizeof(float) * qkv_n);
  float* attn = (float*)malloc(sizeof(float) * q_size);
  float* proj = (float*)malloc(sizeof(float) * H);
  float* gate = (float*)malloc(sizeof(float) * I);
  float* up = (float*)malloc(sizeof(float) * I);
  float* act = (float*)malloc(sizeof(float) * I);
  /* embedding: copyTensorRow with embedScale 1 (DecoderWeights.ts:355-383). */
  memcpy(x, m->embed + (size_t)token * H, sizeof(float) * H);
  for (int l = 0; l < m->layers; l++) {
    size_t cache_off = (size_t)l * m->max_tokens * kv_size;
    orc_rmsnorm(x, m->attn_norm[l], H, m->eps, 0, norm);
    orc_linear_t(norm, m->wqkv[l], m->bqkv[l], H, qkv_n, qkv);
    orc_attn_opts ao = m->attn;
    if (m->windows) ao.sliding_window = m->windows[l];
    attention_impl(qkv, &ao, position, m->kcache + cache_off, m->vcache + cache_off, attn);
    orc_linear_t(attn, m->wo[l], NULL, q_size, H, proj);
    for (int d = 0; d < H; d++) x[d] = (float)((double)x[d] + (double)proj[d]);
    orc_rmsnorm(x, m->ffn_norm[l], H, m->eps, 0, norm);
    orc_linear_t(norm, m->wgate[l], NULL, H, I, gate);
    orc_linear_t(norm, m->wup[l], NULL, H, I, up);
    for (int d = 0; d < I; d++) act[d] = (float)(orc_silu((double)gate[d]) * (double)up[d]);
    orc_linear_t(act, m->wdown[l], NULL, I, H, proj);
    for (int d = 0; d < H; d++) x[d] = (float)((double)x[d] + (double)proj[d]);
  }
  orc_rmsnorm(x, m->final_norm, H, m->eps, 0, norm);
  if (hidden_out) memcpy(hidden_out, norm, sizeof(float) * H);
  if (logits) orc_linear_t(norm, m->lm_head, NULL, H, m->vocab, logits);
  free(x);
  free(norm);
  free(qkv);
  free(attn);
  free(proj);
  free(gate);
  free(up);
  free(act);
  return 0;
}

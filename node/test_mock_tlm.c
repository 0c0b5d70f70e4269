/* A stand-in for libtlm.so with the same C ABI (include/tlm.h), for testing
 * the N-API binding and runner.js on a machine without a GPU.  It is a test
 * double, not a decoder: a "model" computes logits by a fixed formula,
 *   next(token, pos) = (7 token + 3 pos + 1) mod V,
 *   logits[v] = 1 for v = next, else ((37 v + token) mod 101) / 1000,
 * so every greedy step, top-k list and prompt-cache decision is predictable.
 * The reads sleep (TLM_MOCK_READ_MS, default 20 ms) so the addon's thread-pool
 * path is observable, and a model created with max_tokens 13 fails every read
 * with TLM_ERR_HIP and "TLMModel: mock read failure" (set in the reading
 * thread's tlm_last_error).
 *
 *   gcc -shared -fPIC -O2 -I include -o <out>.so node/test_mock_tlm.c -lpthread */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "tlm.h"

static __thread char g_err[256];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

struct tlm_ctx {
  int device;
  int closed;
};

struct tlm_model {
  int vocab, max_tokens;
  int token, pos, has_token;
  int fail_reads;
  tlm_model_counts counts;
};

static void nap(void) {
  const char* e = getenv("TLM_MOCK_READ_MS");
  const long ms = e ? atol(e) : 20;
  struct timespec ts = {ms / 1000, (ms % 1000) * 1000000L};
  nanosleep(&ts, NULL);
}

static int next_token(const tlm_model* m) { return (int)((7L * m->token + 3L * m->pos + 1) % m->vocab); }

static float logit(const tlm_model* m, int v) {
  return v == next_token(m) ? 1.0f : (float)((37L * v + m->token) % 101) / 1000.0f;
}

int tlm_abi_version(void) { return TLM_ABI_VERSION; }
const char* tlm_last_error(void) { return g_err; }

int tlm_open(int device, tlm_ctx** out) {
  if (!out) return fail(TLM_ERR_INVALID, "TLMContext: null output");
  *out = calloc(1, sizeof(tlm_ctx));
  (*out)->device = device;
  return TLM_OK;
}
void tlm_close(tlm_ctx* c) { free(c); }
int tlm_sync(tlm_ctx* c) { return c ? TLM_OK : fail(TLM_ERR_INVALID, "TLMContext: null"); }
int tlm_device_info(tlm_ctx* c, char* name, size_t len, int* cus) {
  (void)c;
  snprintf(name, len, "mock");
  *cus = 1;
  return TLM_OK;
}

int tlm_model_create(tlm_ctx* c, const tlm_model_desc* d, tlm_model** out) {
  if (!c || !d || !out) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  if (d->vocab_size < 2 || d->max_tokens < 1) return fail(TLM_ERR_INVALID, "TLMModel: bad sizes");
  tlm_model* m = calloc(1, sizeof(tlm_model));
  m->vocab = d->vocab_size;
  m->max_tokens = d->max_tokens;
  m->fail_reads = d->max_tokens == 13;
  *out = m;
  return TLM_OK;
}
void tlm_model_destroy(tlm_model* m) { free(m); }
int tlm_model_upload(tlm_model* m, int t, int l, const void* h, size_t b) {
  (void)m, (void)t, (void)l, (void)h, (void)b;
  return TLM_OK;
}
int tlm_model_finalize(tlm_model* m) { return m ? TLM_OK : fail(TLM_ERR_INVALID, "TLMModel: null model"); }
int tlm_model_set_prefill(tlm_model* m, int32_t r, int32_t c) {
  (void)m, (void)r, (void)c;
  return TLM_OK;
}

int tlm_compute_token(tlm_model* m, int32_t token, int32_t pos, int flags) {
  (void)flags;
  if (token < 0 || token >= m->vocab) return fail(TLM_ERR_RANGE, "TLMModel: token %d outside [0, %d)", token, m->vocab);
  if (pos < 0 || pos >= m->max_tokens) return fail(TLM_ERR_RANGE, "TLMModel: position %d out of range", pos);
  m->token = token, m->pos = pos, m->has_token = 1;
  m->counts.graph_launches++;
  m->counts.kernel_launches++;
  return TLM_OK;
}

int tlm_prefill(tlm_model* m, const int32_t* tokens, int32_t start, int32_t end) {
  if (start < 0 || end > m->max_tokens || start > end)
    return fail(TLM_ERR_RANGE, "TLMModel: prefill range [%d, %d) outside [0, %d)", start, end, m->max_tokens);
  nap();
  if (m->fail_reads) return fail(TLM_ERR_HIP, "TLMModel: mock read failure");
  if (end > start) m->token = tokens[end - 1], m->pos = end - 1, m->has_token = 1;
  m->counts.replayed_positions += (uint64_t)(end - start);
  return TLM_OK;
}

static int read_check(tlm_model* m) {
  nap();
  if (m->fail_reads) return fail(TLM_ERR_HIP, "TLMModel: mock read failure");
  if (!m->has_token) return fail(TLM_ERR_STATE, "TLMModel: nothing computed");
  return TLM_OK;
}

int tlm_read_logits(tlm_model* m, float* out, size_t n) {
  int rc = read_check(m);
  if (rc) return rc;
  for (size_t v = 0; v < n && v < (size_t)m->vocab; v++) out[v] = logit(m, (int)v);
  return TLM_OK;
}

int tlm_read_token(tlm_model* m, int32_t* token) {
  int rc = read_check(m);
  if (rc) return rc;
  *token = next_token(m);
  return TLM_OK;
}

int tlm_read_candidates(tlm_model* m, int k, double softcap, int32_t* tokens, float* scores) {
  (void)softcap;
  int rc = read_check(m);
  if (rc) return rc;
  for (int i = 0; i < k; i++) tokens[i] = -1, scores[i] = -INFINITY;
  for (int v = 0; v < m->vocab; v++) {  /* the k best, ties to the lower id */
    const float s = logit(m, v);
    int j = k;
    while (j > 0 && (tokens[j - 1] < 0 || s > scores[j - 1])) j--;
    if (j == k) continue;
    memmove(tokens + j + 1, tokens + j, sizeof(int32_t) * (size_t)(k - 1 - j));
    memmove(scores + j + 1, scores + j, sizeof(float) * (size_t)(k - 1 - j));
    tokens[j] = v, scores[j] = s;
  }
  return TLM_OK;
}

int tlm_decode_greedy(tlm_model* m, int32_t token, int32_t pos, int n, int32_t* out) {
  if ((long)pos + n > m->max_tokens) return fail(TLM_ERR_RANGE, "TLMModel: decode passes max_tokens");
  nap();
  if (m->fail_reads) return fail(TLM_ERR_HIP, "TLMModel: mock read failure");
  m->token = token, m->pos = pos, m->has_token = 1;
  for (int i = 0; i < n; i++) {
    out[i] = next_token(m);
    m->token = out[i], m->pos = pos + i + 1;
  }
  m->counts.graph_launches += (uint64_t)n;
  return TLM_OK;
}

int tlm_reset_cache(tlm_model* m) {
  m->has_token = 0;
  return TLM_OK;
}

int tlm_model_counts_read(tlm_model* m, tlm_model_counts* out) {
  *out = m->counts;
  return TLM_OK;
}

int tlm_quantize_q4(const float* w, int n_out, int k_in, uint8_t* packed, uint16_t* scales) {
  (void)w;
  memset(packed, 0x88, (size_t)n_out * (size_t)k_in / 2);
  memset(scales, 0, sizeof(uint16_t) * (size_t)n_out * (size_t)(k_in / 32));
  return TLM_OK;
}
int tlm_f32_to_f16(const float* in, size_t n, uint16_t* out) {
  (void)in;
  memset(out, 0, 2 * n);
  return TLM_OK;
}
int tlm_synth_normal(uint64_t s, uint64_t st, size_t n, float sd, float* out) {
  (void)s, (void)st, (void)sd;
  memset(out, 0, sizeof(float) * n);
  return TLM_OK;
}
int tlm_synth_tokens(uint64_t s, uint64_t st, size_t n, int32_t vocab, int32_t* out) {
  for (size_t i = 0; i < n; i++) out[i] = (int32_t)((s + st + i) % (uint64_t)vocab);
  return TLM_OK;
}

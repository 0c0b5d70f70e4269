/*
 * tlm.h -- C ABI of the MI355X-native per-token decoder path of three-llm.
 *
 * Every compute entry point runs hand-written HIP kernels for gfx950.  All
 * functions return 0 (TLM_OK) or a negative TLM_ERR_* code; the message of the
 * last failure on the calling thread is tlm_last_error(), formatted like the
 * reference's errors ("Component: message").
 *
 * Reference interfaces replaced (paths relative to packages/three-llm/src/):
 *   ops      tsl/TSLLinear.ts:13-82, tsl/TSLRMSNorm.ts:18-81, tsl/TSLSiLUMul.ts:10-36,
 *            tsl/TSLGatedMLP.ts:17-90, tsl/TSLAttention.ts:19-449,
 *            tsl/TSLLogits.ts:40-69 and :201-274 (chunked logits + greedy sampler)
 *   runner   decoder/DecoderTSLRunner.ts:62-594 (computeToken :487-502,
 *            prefillTokens :504-530, readLogits :532-535, sampleToken :537-539,
 *            resetCache :541-546), driven by runtime/generate.ts:31-49.
 *
 * Device pointers are plain `void*`/`float*` obtained from tlm_alloc (or any
 * HIP allocation on the context's device).  Work is enqueued on the context's
 * stream; tlm_download / tlm_read_* / tlm_sync wait for it.  A context or model
 * must not be used from two threads at once.
 */
#ifndef TLM_H
#define TLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TLM_ABI_VERSION 3

enum {
  TLM_OK = 0,
  TLM_ERR_INVALID = -1, /* bad argument (shape, range, null) */
  TLM_ERR_HIP = -2,     /* HIP runtime error */
  TLM_ERR_OOM = -3,     /* device allocation failed */
  TLM_ERR_STATE = -4,   /* call not valid in the current state */
  TLM_ERR_RANGE = -5    /* token or position out of range */
};

/* Weight storage formats (canonical host layouts):
 *   TLM_FMT_F16: uint16 fp16 bits, [N][K] row-major (row = output feature).
 *   TLM_FMT_Q4 : packed nibbles uint8 [N][K/2] (even k in the low nibble,
 *                value q+8 for q in [-8,7]) plus fp16 scales uint16 [N][K/32];
 *                w = f32(scale[n][k/32]) * q.  K must be a multiple of 32.
 *   TLM_FMT_F32: float [N][K] (embedding tables only). */
enum { TLM_FMT_F16 = 1, TLM_FMT_Q4 = 2, TLM_FMT_F32 = 3 };

typedef struct tlm_ctx tlm_ctx;
typedef struct tlm_linear tlm_linear;
typedef struct tlm_attn tlm_attn;
typedef struct tlm_model tlm_model;

/* ---------------------------------------------------------------- context */
int tlm_abi_version(void);
const char* tlm_last_error(void);
/* Opens device `device` (HIP ordinal) with one stream of default priority. */
int tlm_open(int device, tlm_ctx** out);
void tlm_close(tlm_ctx* ctx);
int tlm_sync(tlm_ctx* ctx);
/* Device name and compute-unit count (for reports). */
int tlm_device_info(tlm_ctx* ctx, char* name, size_t name_len, int* cu_count);
/* Free and total device memory of the context's GPU (hipMemGetInfo; for
 * reports and for checking that an entry point allocates nothing).  No
 * counterpart in the reference (the browser exposes no device memory). */
int tlm_device_memory(tlm_ctx* ctx, size_t* free_bytes, size_t* total_bytes);

/* Device buffers (thin helpers so hosts need no HIP binding of their own). */
int tlm_alloc(tlm_ctx* ctx, size_t bytes, void** dptr);
int tlm_free(tlm_ctx* ctx, void* dptr);
int tlm_upload(tlm_ctx* ctx, void* dst, const void* src, size_t bytes);   /* blocking */
int tlm_download(tlm_ctx* ctx, void* dst, const void* src, size_t bytes); /* waits for the stream */
/* Device-to-device copy enqueued on the context stream (bytes % 16 == 0): a
 * plain streaming kernel of known size.  A utility with no reference
 * counterpart (the reference copies through WebGPU buffers); it also scales
 * hardware byte counters against a known transfer. */
int tlm_copy(tlm_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ------------------------------------------------------------------ linear
 * TSLLinear (tsl/TSLLinear.ts:13-82): y[n] = b[n] + sum_k W[n][k] x[k].
 * The reference takes fp32 W [in][out]; here W is fp16 or q4 in the canonical
 * [out][in] layout above, repacked at creation into the device tile layout. */
int tlm_linear_create(tlm_ctx* ctx, int fmt, int n_out, int k_in, const void* weights, const uint16_t* scales,
                      tlm_linear** out);
void tlm_linear_destroy(tlm_linear* lin);
/* Dequantizes the device copy back to fp32 [N][K] on the host (bit-exact
 * parity check of the device layout: q4 -> f32(s)*q, fp16 -> f32). */
int tlm_linear_dequant(tlm_linear* lin, float* host_out);
/* y = bias + W x.  x: fp32[K] device, bias: fp32[N] device or NULL, y: fp32[N] device. */
int tlm_op_linear(tlm_linear* lin, const float* x, const float* bias, float* y);
/* The same linear over `rows` tokens at once, as one MFMA GEMM (the batched
 * prefill's linear; the reference applies TSLLinear once per replayed token,
 * DecoderTSLRunner.ts:472-480).  x: fp16 bits device [rows][K] (K % 32 == 0),
 * y: fp32 device [rows][N].  W is dequantised to fp16 ((code - 8) * s rounded
 * once), products accumulate in fp32.  Enqueue only. */
int tlm_op_linear_rows(tlm_linear* lin, const uint16_t* x, int32_t rows, const float* bias, float* y);

/* ----------------------------------------------------------- element ops */
/* TSLRMSNorm (tsl/TSLRMSNorm.ts:18-81): y = x * rsqrt(mean(x^2) + eps) * (offset ? 1 + w : w). */
int tlm_op_rmsnorm(tlm_ctx* ctx, const float* x, const float* w, int n, double eps, int offset, float* y);
/* TSLSiLUMul (tsl/TSLSiLUMul.ts:10-36): out = silu(gate) * up. */
int tlm_op_silu_mul(tlm_ctx* ctx, const float* gate, const float* up, int n, float* out);
/* TSLGatedMLP (tsl/TSLGatedMLP.ts:17-90), SwiGLU: y = down(silu(gate x) * (up x)).
 * gate_up holds 2*I rows (gate rows then up rows), down is [H][I]. */
int tlm_op_gated_mlp(tlm_linear* gate_up, tlm_linear* down, const float* x, float* y);

/* --------------------------------------------------------------- attention
 * TSLAttention (tsl/TSLAttention.ts:19-449) for the Llama/Qwen2 recipe:
 * RoPE (rotate-half over rotary_dim, table from ropeParameters), KV append
 * at `position`, causal softmax attention over [max(0,pos-W+1), pos] with
 * grouped KV heads, split over the sequence with an online-softmax combine. */
typedef struct tlm_attn_desc {
  int32_t heads, kv_heads, head_dim, max_tokens;
  int32_t rotary_dim;       /* 0 disables RoPE */
  int32_t sliding_window;   /* 0 = full causal */
  int32_t kv_fmt;           /* TLM_FMT_F16 (default) or TLM_FMT_F32 */
  int32_t reserved;
  const float* inv_freq;    /* host, rotary_dim/2 entries (ropeParameters) */
  double attention_factor;  /* ropeParameters().attentionFactor */
  double attn_scale;        /* <= 0 selects 1/sqrt(head_dim) */
} tlm_attn_desc;

int tlm_attn_create(tlm_ctx* ctx, const tlm_attn_desc* desc, tlm_attn** out);
void tlm_attn_destroy(tlm_attn* attn);
/* qkv: fp32 device [(heads + 2 kv_heads) * head_dim] (packed Q|K|V, pre-RoPE);
 * out: fp32 device [heads * head_dim]. */
int tlm_op_attention(tlm_attn* attn, const float* qkv, int position, float* out);
/* `rows` consecutive positions position0.. at once (the batched prefill's
 * attention; the reference runs TSLAttention once per replayed token): qkv fp32
 * device [rows][(heads + 2 kv_heads) * head_dim], bias included; RoPE, the K/V
 * rows appended to the cache, causal attention of each row over
 * [max(0, pos - W + 1), pos] on MFMA; out: fp16 bits device [rows][heads * head_dim].
 * Needs an fp16 cache and head_dim 64 or 128.  Waits for the stream. */
int tlm_op_attention_rows(tlm_attn* attn, const float* qkv, int32_t rows, int32_t position0, uint16_t* out);
/* Allocation-free tlm_op_attention_rows.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  The same kernels and results; the rotated
 * fp16 queries are staged in a fixed 4 MiB device array of the library (one
 * per device, held until the process ends) instead of a buffer allocated per
 * call, so rows * heads * head_dim * 2 may not exceed 4 MiB (TLM_ERR_RANGE
 * otherwise).  Enqueue only: no allocation, free or wait.  Every call on one
 * device shares that array, so calls that overlap on one device (other
 * streams or contexts) race. */
int tlm_op_attention_rows_noalloc(tlm_attn* attn, const float* qkv, int32_t rows, int32_t position0, uint16_t* out);
int tlm_attn_reset(tlm_attn* attn);
/* Cache rows [0, count) as fp32 [count][kv_heads*head_dim] (host). */
int tlm_attn_read_cache(tlm_attn* attn, int count, float* k_out, float* v_out);

/* ------------------------------------------------------------------ logits
 * TSLLogits chunk layers + greedy sampler (tsl/TSLLogits.ts:40-69, :201-274):
 * logits = head x; token = argmax, ties to the lower id.  logits may be NULL. */
int tlm_op_logits(tlm_linear* head, const float* x, float* logits, int32_t* token);
int tlm_op_argmax(tlm_ctx* ctx, const float* logits, int n, int32_t* token);
/* TSLLogitSampler candidate levels (tsl/TSLLogits.ts:276-330): the k best
 * (token, score) of logits[0, n) in the greedy order (higher score, ties to
 * the lower id), scores after the softcap cap * tanh(x / cap) when softcap > 0
 * (:185-191).  Entries at or below LOWEST_FLOAT (-inf, NaN included) never
 * take part; missing slots are (0, LOWEST_FLOAT).  1 <= k <= 16; device
 * tokens[k], scores[k].  Enqueue only. */
int tlm_op_topk(tlm_ctx* ctx, const float* logits, int n, int k, double softcap, int32_t* tokens, float* scores);

/* ------------------------------------------------------------------- model */
typedef struct tlm_model_desc {
  int32_t hidden_size, intermediate_size, num_layers, num_heads, num_kv_heads, head_dim, vocab_size;
  int32_t max_tokens;
  int32_t rotary_dim;
  int32_t sliding_window;
  int32_t linear_fmt;  /* TLM_FMT_Q4 or TLM_FMT_F16 for the decoder linears */
  int32_t head_fmt;    /* TLM_FMT_F16 or TLM_FMT_Q4 for an untied LM head */
  int32_t embed_fmt;   /* TLM_FMT_F16 or TLM_FMT_F32 embedding table */
  int32_t kv_fmt;      /* TLM_FMT_F16 or TLM_FMT_F32 cache */
  int32_t qkv_bias;    /* 1: upload TLM_T_BQKV per layer */
  int32_t tied;        /* 1: LM head = embedding table (fp16 embedding only) */
  double rms_eps;
  double attention_factor;
  const float* inv_freq; /* host, rotary_dim/2 entries */
  /* ABI 2.  DecoderCPURunner.attention (decoder/DecoderCPURunner.ts:140-160)
   * passes recipe.attnScale and the block's slidingWindow per layer
   * (DecoderWeights.ts:307-311: sliding_attention layers get the recipe's
   * window, full_attention layers 0 when the config lists layer types). */
  double attn_scale;             /* <= 0 selects 1/sqrt(head_dim) (attnScale undefined) */
  const int32_t* layer_windows;  /* host, num_layers entries (0 = full causal), copied at
                                    create; NULL: every layer uses sliding_window */
} tlm_model_desc;

enum {
  TLM_T_EMBED = 0,      /* [V][H] embed_fmt */
  TLM_T_LM_HEAD = 1,    /* [V][H] head_fmt (untied only) */
  TLM_T_LM_HEAD_SCALES = 2,
  TLM_T_FINAL_NORM = 3, /* fp32 [H] */
  TLM_T_ATTN_NORM = 4,  /* fp32 [H] per layer */
  TLM_T_FFN_NORM = 5,   /* fp32 [H] per layer */
  TLM_T_WQKV = 6,       /* [(Hq+2Hkv)*D][H], rows Q|K|V */
  TLM_T_WQKV_SCALES = 7,
  TLM_T_BQKV = 8,       /* fp32 [(Hq+2Hkv)*D] */
  TLM_T_WO = 9,         /* [H][Hq*D] */
  TLM_T_WO_SCALES = 10,
  TLM_T_WGATE = 11,     /* [I][H] */
  TLM_T_WGATE_SCALES = 12,
  TLM_T_WUP = 13,       /* [I][H] */
  TLM_T_WUP_SCALES = 14,
  TLM_T_WDOWN = 15,     /* [H][I] */
  TLM_T_WDOWN_SCALES = 16
};

/* Flags of tlm_compute_token. */
enum { TLM_LOGITS = 1 };

int tlm_model_create(tlm_ctx* ctx, const tlm_model_desc* desc, tlm_model** out);
void tlm_model_destroy(tlm_model* model);
/* Copies a canonical host tensor to the device (the caller keeps ownership,
 * like uploadAndReleaseStaticWeights in tsl/releaseCPU.ts:79-110). */
int tlm_model_upload(tlm_model* model, int tensor, int layer, const void* host, size_t bytes);
/* Builds the per-token HIP graphs; implicit on the first compute. */
int tlm_model_finalize(tlm_model* model);
/* computeToken (DecoderTSLRunner.ts:487-502): enqueue one token at `position`.
 * With TLM_LOGITS the LM head and the greedy argmax run too. */
int tlm_compute_token(tlm_model* model, int32_t token, int32_t position, int flags);
/* prefillTokens (DecoderTSLRunner.ts:504-530): positions [start, end), no logits. */
int tlm_prefill(tlm_model* model, const int32_t* tokens, int32_t start, int32_t end);
/* Batched prefill control: tlm_prefill runs chunks of up to `chunk` positions
 * with at least `min_rows` positions (default 64, chunk 2048) as row batches
 * (MFMA GEMMs and flash attention per layer, tlm_op_linear_rows /
 * tlm_op_attention_rows) and replays the decode graph per position below
 * that, as the reference always does (DecoderTSLRunner.ts:472-480).
 * min_rows <= 0 turns the batched path off; TLM_ERR_INVALID names why a model
 * cannot use it (fp32 cache, head_dim other than 64/128, sizes not multiples
 * of 32, a q4 scale above 8188).  The row batches keep activations in fp16:
 * when one rounds to inf or is NaN, a device flag trips and tlm_prefill
 * replays that chunk on the fp32 decode graph (it waits for the stream after
 * each batched chunk to read the flag; tlm_model_describe counts such chunks). */
int tlm_model_set_prefill(tlm_model* model, int32_t min_rows, int32_t chunk);
/* readLogits (DecoderTSLRunner.ts:532-535): waits, copies n <= vocab floats. */
int tlm_read_logits(tlm_model* model, float* out, size_t n);
/* sampleToken greedy (TSLLogits.ts:359-361): waits, returns the argmax. */
int tlm_read_token(tlm_model* model, int32_t* token);
/* Greedy decode on the device: computes `token` at `position`, then feeds each
 * argmax back for n steps without host round trips; out[i] = argmax after
 * position+i.  Equals n rounds of computeToken + sampleToken. */
int tlm_decode_greedy(tlm_model* model, int32_t token, int32_t position, int n, int32_t* out);
/* resetCache (DecoderTSLRunner.ts:541-546): every cache row reads back zero
 * afterwards.  Only the rows some call could have written since the last
 * reset are cleared (positions below the highest one a compute, decode,
 * prefill, fill, write or timing call named), so a reset after a short
 * sequence costs little and leaves the weights in the last-level cache. */
int tlm_reset_cache(tlm_model* model);
/* Cache access in the canonical [count][kv_heads][head_dim] order, kv_fmt
 * element type (uint16 fp16 bits or float). */
int tlm_kv_write(tlm_model* model, int layer, int pos0, int count, const void* k, const void* v);
int tlm_kv_read(tlm_model* model, int layer, int pos0, int count, void* k, void* v);
/* Fills positions [0, count) of every layer with N(0,1) values from a
 * counter-based generator on the device (long-context benchmarks). */
int tlm_kv_fill_normal(tlm_model* model, uint64_t seed, int count);
/* readCandidates (TSLLogits.ts:336-349) over the model's last logits
 * (a token computed with TLM_LOGITS): k <= 16 (token, score) pairs to host
 * memory, best first; waits for the stream.  sampleTopKCandidates
 * (runtime/math.ts:527-547) then draws from them on the host. */
int tlm_read_candidates(tlm_model* model, int k, double softcap, int32_t* tokens, float* scores);
/* Final hidden state (after the final norm) of the last token with logits. */
int tlm_read_hidden(tlm_model* model, float* out, size_t n);

/* Timing with HIP events on the model stream.  tlm_time_decode: greedy
 * decode of n tokens after `warmup` untimed ones, from `position`; ms total.
 * tlm_time_kernel: average ms of one launch of kernel `which` (0 = LM head,
 * 1 = attention of layer 0, 2 = fused gate|up/SwiGLU/down MLP of layer 0,
 * 4 = QKV of layer 0, 5 = O of layer 0, 6 = top-8 candidates over the logits)
 * over iters back-to-back launches;
 * afterwards the residual accumulators are cleared (the next token starts
 * from the cache and ctrl state as left). */
int tlm_time_decode(tlm_model* model, int32_t token, int32_t position, int warmup, int n, double* ms);
int tlm_time_kernel(tlm_model* model, int which, int iters, double* avg_ms);
/* tlm_time_head / tlm_time_layers: n greedy decode steps from (token,
 * position), each the layer part (the persistent kernel, or the layer graph in
 * the long-window case) then the LM head, each part bracketed by its own pair
 * of events on the model stream; average ms of the LM head launch, or of the
 * layer part, inside a real step (weights cold in the caches, as in decode).
 * Leaves the cache and ctrl state advanced like tlm_decode_greedy.  No
 * reference counterpart (measurement). */
int tlm_time_head(tlm_model* model, int32_t token, int32_t position, int n, double* avg_ms);
int tlm_time_layers(tlm_model* model, int32_t token, int32_t position, int n, double* avg_ms);
/* tlm_trace_decode: n greedy decode steps from (token, position) through the
 * persistent schedule, launched directly with its timeline on; `out` receives
 * the last step's timeline: for every (block, wave), layer l < L and stage
 * (0 qkv, 1 attention, 2 O, 3 gate|up, 4 down), 4 wall-clock stamps (100 MHz:
 * weights issued, input ready, computed, published; 0 where the wave had no
 * such work); layer slot L, stage 0 holds the kernel's start and end.
 * n_out must be blocks * 16 * (L + 1) * 5 * 4 (see tlm_model_describe for the
 * block count).  TLM_ERR_STATE when the model has no
 * persistent schedule or a position needs the long-window kernels.  Tracing
 * has no counterpart in the reference (the browser has no device clock). */
int tlm_trace_decode(tlm_model* model, int32_t token, int32_t position, int n, uint64_t* out, size_t n_out);
/* Launch layout chosen for the model (for reports): per-stage grid sizes. */
int tlm_model_describe(tlm_model* model, char* out, size_t len);
/* Work the model has handed to its stream since it was created: the
 * counterpart of the reference's submission count
 * (src/test/submission.browser.test.ts:46-57: one submission per decode token,
 * one per prefill chunk).  A captured per-token graph is one graph launch;
 * kernels enqueued directly (the token/position write before a token, the
 * kernels of a batched prefill chunk, the eager schedule with graphs off)
 * count one each. */
typedef struct tlm_model_counts {
  uint64_t graph_launches;
  uint64_t kernel_launches;
  uint64_t prefill_chunks;      /* batched row chunks run (replayed ones excluded) */
  uint64_t replayed_positions;  /* prompt positions run through the decode graph */
  uint64_t recomputed_positions; /* positions recomputed on the per-stage graph after a failed
                                    token of the persistent schedule (a wait ran out, or an
                                    fp16 input overflow of its q4 linears) */
  uint64_t persistent_tokens;    /* token steps run on the persistent schedule (the rest ran
                                    the per-stage graph: long windows, shapes without it) */
} tlm_model_counts;
int tlm_model_counts_read(tlm_model* model, tlm_model_counts* out);

/* ------------------------------------------------------- host-side helpers
 * Synthetic inputs: N(0, std) from SplitMix64 -> Box-Muller, one counter
 * stream per (seed, stream id); identical output for any thread count. */
int tlm_synth_normal(uint64_t seed, uint64_t stream, size_t n, float stddev, float* out);
int tlm_synth_tokens(uint64_t seed, uint64_t stream, size_t n, int32_t vocab, int32_t* out);
/* q4 quantizer of the canonical format (fp16 scale = max|w|/7, ties-to-even codes). */
int tlm_quantize_q4(const float* w, int n_out, int k_in, uint8_t* packed, uint16_t* scales);
int tlm_f32_to_f16(const float* in, size_t n, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif /* TLM_H */

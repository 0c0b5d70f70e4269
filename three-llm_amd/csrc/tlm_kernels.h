// Kernel argument blocks and launchers shared by tlm_kernels.hip and tlm_api.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tlm {

constexpr int kTile = 64;      // output rows per tile: one row per lane of a wave64
constexpr int kMaxChunks = 8;  // most 16-byte chunks a wave keeps in flight per batch
constexpr int kMaxPart = 8;    // partial vectors a consumer folds in with one round trip
constexpr int kAttnWaves = 4;  // decode attention: waves per block, each a quarter of the block's chunk
constexpr int kGqaWaves = 8;   // matrix-core decode attention (long windows): waves per block
constexpr int kGqaTile = 32;   // its positions per wave tile
constexpr int kGqaPro = 3;     // its q|k|v elements per thread: (G + 2) head_dim <= 3 * 64 kGqaWaves
inline bool gqa_attention_fits(int G, int D) {
  return (D == 64 || D == 128) && G >= 1 && G <= 16 && (G + 2) * D <= kGqaPro * 64 * kGqaWaves;
}
constexpr int kLongWindow = 1024; // decode attention: windows above this many positions run the long-window kernels
// Residual stream accumulators: up to kRep replicas of an int64 fixed-point
// vector (value * 2^32).  Producers add into replica (block % nrep) with
// device-scope atomics; integer addition is associative, so the sum is exact
// and the same in every run, whatever nrep.  Readers add the nrep replicas:
// more replicas mean fewer atomics per address in the producer and more reads
// in every reader (a model's count: rep_count).
constexpr int kRep = 4;
constexpr float kFxScale = 4294967296.0f;        // 2^32
constexpr float kFxInv = 2.3283064365386963e-10f;  // 2^-32

enum WeightFmt { WF_F16 = 1, WF_Q4 = 2 };

// GEMV prologues: how the input slice x[k0, k1) is formed in LDS.
enum Prologue {
  PRO_COPY = 0,    // x = in
  PRO_RMS = 1,     // x = rmsnorm(base + sum_j pin[j]) * w
  PRO_SWIGLU = 2,  // x = silu(sum_j pin[j][k]) * (sum_j pin[j][up_off + k])
  PRO_ATTN = 3,    // x = flash-decoding combine of the attention chunk partials
  PRO_RMS2 = 4,    // PRO_RMS for K up to 8 elements per thread (chosen by launch_gemv)
  PRO_RMSF = 5,    // x = rmsnorm(sum of the kRep fixed-point replicas acc_in) * w
  PRO_RMSF2 = 6,   // PRO_RMSF for K up to 8 elements per thread (chosen by launch_gemv)
  PRO_ATTN3 = 7,   // PRO_ATTN folding 32 chunk partials per round trip instead of 16 (long windows)
  PRO_RMSFH = 8,   // PRO_RMSF over 2 replicas (models whose MLP adds into 2)
  PRO_RMSF2H = 9,  // PRO_RMSF2 over 2 replicas
};

// Split of the attention window [first, pos] into chunks; identical on host and device.
struct ChunkPlan {
  int first, n, chunk, nact;
};
__host__ __device__ inline ChunkPlan chunk_plan(int pos, int window, int nsplit, int chmin) {
  ChunkPlan p;
  p.first = window > 0 ? (pos - window + 1 > 0 ? pos - window + 1 : 0) : 0;
  p.n = pos - p.first + 1;
  const int c = (p.n + nsplit - 1) / nsplit;
  p.chunk = c > chmin ? c : chmin;
  p.nact = (p.n + p.chunk - 1) / p.chunk;
  return p;
}

// ctrl block (device int32[8]): per-token state read by every kernel so that one
// captured graph serves every position.  C_SEQ numbers the tokens of the
// persistent schedule (the tag of its published words, never 0); C_ERR
// collects its failures (kPsErr*); C_FXR is set when a residual value of the
// per-stage kernels leaves their fixed-point range (fx_guard).
enum Ctrl { C_TOKEN = 0, C_POS = 1, C_STEP = 2, C_BASE = 3, C_LEN = 4, C_SEQ = 5, C_FXR = 6, C_ERR = 7 };

// Embedding row staging: the kernels that choose the next token (set_ctrl,
// prefill_advance, argmax_merge) also write its embedding row, in fixed point,
// to replica 0 of x0, the residual accumulator layer 0 reads (replicas 1..3
// stay zero).  x0 == null disables the copy.
struct EmbStage {
  const void* emb;  // [V][H] fp16 or fp32
  int f32;
  int H;
  unsigned long long* x0;
};

struct GemvArgs {
  const uint4* w;      // [T][C][64] 16-byte chunks (q4: 32 k, fp16: 8 k)
  const uint16_t* s;   // q4 scales [T][C][64] (fp16 bits)
  int N, T, C, K, cps; // rows, tiles, chunks/row, logical K, chunks per split
  float* out;          // [S][N] partial sums (S = gridDim.y)
  const float* bias;   // added by split 0 (may be null)
  // PRO_COPY
  const float* in;
  // PRO_RMS
  const float* base;   // fp32 [K] residual stream
  const unsigned long long* acc_in;  // PRO_RMSF: [kRep][K] fixed-point residual (PRO_RMSFH: [2][K])
  unsigned long long* zero_ptr;      // optional: the grid zeroes zero_ptr[0, zero_n)
  int zero_n;
  const int* ctrl;
  const float* pin;    // partials to add (RMS) / gate|up partials (SWIGLU)
  int n_pin, pin_stride;
  const float* norm_w;
  float eps;
  float* xout;         // block (0,0) stores base + sum pin here (residual stream)
  int up_off;          // SWIGLU: offset of the up rows in pin
  // PRO_ATTN: chunk partials of the attention kernel
  const float* pacc;   // [Hq][nsplit][D]
  const float* pml;    // [Hq][nsplit][2]
  int att_D, att_nsplit, att_chmin, att_window, att_max_tokens;
  // LM head
  float* xnorm;        // with an RMS prologue: block 0 stores the normalised input here (may be null)
  float* logits;       // full logits (may be null)
  float* arg_val;      // per-block argmax partials
  int* arg_idx;
  int* tokens_out;     // greedy stream (indexed by ctrl[C_STEP]), may be null
  int advance;         // 1: the merge advances ctrl (token <- argmax, pos++, step++)
  int max_steps;
  // LM head: each block also folds its best into *arg_key, an atomic max of
  // greedy_key (zero between launches; may be null)
  unsigned long long* arg_key;
  // with arg_key: the merge in the same launch.  A block counts itself in
  // *arrived (zero between launches) once its max has returned; the block
  // that counts last writes the token and advances position, step and token
  // number in mctrl (the persistent schedule's step; no embedding row is
  // staged), then clears the key and the count.  Null: greedy_pick_kernel.
  unsigned* arrived;
  int* mctrl;
  // PRO_RMSF input of the persistent schedule: acc_in holds kRep partials of
  // published words (fp32 value in bits 0..31), summed as floats
  int ps_words;
};

// Fused gate|up -> SwiGLU -> down of one 32-index slice of the intermediate
// dimension per block.  The gate|up linear is stored in row pairs: tile t holds
// gate rows 32t..32t+31 in lanes 0..31 and the matching up rows in lanes 32..63.
struct MlpArgs {
  GemvArgs g;               // gate|up (K = H) and the PRO_RMS prologue inputs
  const uint4* wd;          // down linear tiles [Td][Cd][64]
  const uint16_t* sd;       // q4 scales of the down linear
  int Td, Cd;               // down tiles (ceil(H / 64)) and chunks per row
  int H;                    // output rows
  unsigned long long* acc;  // [nrep][H] fixed-point accumulator, zero on entry
  int nrep;                 // replicas of acc: 2 or kRep
};

struct AttnArgs {
  const float* src;     // q|k|v partial sums [n_src][src_stride]
  int n_src, src_stride;
  const float* bias;    // [(Hq + 2Hkv) D] or null
  const int* ctrl;      // position at ctrl[C_POS]
  void* kc;             // [Hkv][max_tokens][D] (this layer)
  void* vc;
  const float* rope_cos;  // [max_tokens][rd/2], attention factor folded in
  const float* rope_sin;
  float* out;           // [Hq D] (combine kernel)
  float* pacc;          // [Hq][nsplit][D] unnormalised chunk outputs
  float* pml;           // [Hq][nsplit][2] (max score, sum of exp)
  int Hq, Hkv, D, G, rd, max_tokens, window, nsplit, chmin;
  int lpp;              // lanes per position in the score pass (1, 2 or 4)
  float scale;
  int gqa;              // long windows: the matrix-core kernel (one block per kv head and chunk)
};

// launchers (stream-ordered, graph-capturable: no memset, no host sync)
// launchers return false when no compiled variant matches (nothing is launched)
// waves in {4, 8}; nch in {1, 2, 4, 8}: chunks per wave and load batch
bool launch_gemv(int fmt, int pro, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st);
// fused MLP: kMlpWaves waves, one block per 32 intermediate indices; nch: gate|up
// chunks per wave, ndb: down (tile, chunk) items per wave per batch (1, 2, 4)
bool launch_mlp(int fmt, int nch, int ndb, int blocks, const MlpArgs& a, hipStream_t st);
size_t mlp_smem_bytes(int fmt, int C, int K);
// 16 waves (1024 threads, the most a block holds): four waves per SIMD hide
// the dequant-dot's LDS reads of x, each wave carries half the chunks it
// would in an 8-wave block, and the prologue's residual loads come from the
// first waves only.  Measured against 8 waves: Qwen2.5-0.5B shape 451 -> 439 us per
// decode token, Llama-3.2-1B (4096 positions) 602 -> 576, Llama-3.2-3B
// (16384 positions) 1675 -> 1649.
constexpr int kMlpWaves = 16;
// pro: PRO_COPY (input a.in) or PRO_RMSF (the final norm fused in); nch up to 16
bool launch_lm_head(int fmt, int pro, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st);
// attention chunk partials; with `combine` also the combine kernel writing a.out
bool launch_attention(bool kv_f32, int gmax, const AttnArgs& a, bool combine, bool long_win, hipStream_t st);
// long windows, fp16 cache, head_dim 64 or 128, G <= 16: grid Hkv x nsplit
bool launch_gqa_attention(const AttnArgs& a, hipStream_t st);
size_t gemv_smem_bytes(int fmt, int cps, int waves);
void launch_rmsnorm(const float* x, const float* w, int n, float eps, int offset, float* y, hipStream_t st);
void launch_silu_mul(const float* g, const float* u, int n, float* out, hipStream_t st);
void launch_reduce(const float* part, int n_part, int stride, const float* bias, int n, float* y, hipStream_t st);
void launch_argmax(const float* logits, int n, float* pval, int* pidx, int* token, int blocks, hipStream_t st);
// second pass of the greedy sampler; `ctrl` receives the token at ctrl[C_TOKEN]
// ps: the token came from the persistent schedule; advance its token number (C_SEQ)
void launch_argmax_merge(const float* pval, const int* pidx, int n, int* ctrl, int* tokens_out, int advance,
                         int max_steps, const EmbStage& es, hipStream_t st, int ps = 0);
// The merge of an LM head launch that folded into key (greedy_key order),
// with argmax_merge_kernel's control-word updates; clears key.
void launch_greedy_pick(unsigned long long* key, int* ctrl, int* tokens_out, int advance, int max_steps,
                        const EmbStage& es, hipStream_t st, int ps);
void launch_set_ctrl(int* ctrl, int token, int pos, int step, int base, int len, const EmbStage& es,
                     hipStream_t st);
void launch_prefill_advance(int* ctrl, const int* prompt, const EmbStage& es, hipStream_t st, int ps = 0);
// Stages the embedding row of ctrl[C_TOKEN] (a token chosen by a persistent
// step, which does not stage it, before a step on the per-stage graph).
void launch_stage_ctrl(const int* ctrl, const EmbStage& es, hipStream_t st);
void launch_copy(uint4* dst, const uint4* src, size_t n16, hipStream_t st);
void launch_dequant(int fmt, const uint4* w, const uint16_t* s, int N, int T, int C, int K, float* out,
                    hipStream_t st);
void launch_kv_fill(void* kc, void* vc, bool f32, size_t heads_stride, int Hkv, int max_tokens, int D, int count,
                    uint64_t seed, hipStream_t st);
size_t attn_smem_bytes(int gmax, int D, bool kv_f32, bool long_win);
int attn_lpp(int D, bool kv_f32);
// top-k candidates (k <= kTopkMax) of an fp32 vector in the greedy order; the
// workspace holds two levels of wcap (score, id) pairs each
constexpr int kTopkMax = 16;
bool launch_topk(const float* logits, int n, int k, float softcap, float* wv, int* wi, size_t wcap, float* out_v,
                 int* out_i, hipStream_t st);

// --------------------------------------------- persistent per-token schedule --
// One launch computes every layer of one token on one 1024-thread block per
// CU.  A layer is five stages; every block holds at most kPsRoles (stage, item)
// roles, fixed for the launch, so it issues a role's weights as soon as its
// previous role is published, then waits.  The stages run one after another,
// so a block's later role costs no time.  Linears are split along K over
// several items (more CUs per stage); their consumers add the partial sums:
//   QKV   (item = head x one of kq K-splits: Hq q, Hkv k, Hkv v heads)  RMSNorm
//         of the residual, the head's D rows of q|k|v partial sums, RoPE (linear,
//         so applied per partial), bias in split 0
//   ATT   (item = query head)  sums the q|k|v partials, appends the rounded k
//         and v to the cache, attention over the window split over the 16
//         waves and merged in LDS
//   O     (item = 64-row tile of H x one of ko K-splits)  partial x_mid rows
//         (split 0 adds the residual rows)
//   GU    (item = mw paired 32-index gate|up tiles)  RMSNorm of x_mid, gate|up,
//         SwiGLU
//   DOWN  (item = 64-row tile x one of ks K-splits)  partial rows of the down
//         projection (split 0 adds x_mid): the residual is the sum of the ks
//         partials
// Producers publish 8-byte words (fp32 value, token number ctrl[C_SEQ]) with
// device-scope stores (past the per-XCD L2), or with plain stores into their
// XCD's L2 where every consumer runs on the same XCD (ps_localize); a consumer
// polls its words with device-scope loads until they all carry the current
// token number.  No atomics, no clearing between
// tokens.  Every wait is bounded (kPsTimeoutTicks); a time-out sets ctrl[C_ERR].
// The q4 linears dot fp16 copies of their inputs (two weights per
// v_dot2_f32_f16, fp32 sums); an input past the fp16 range makes the last
// residual NaN, and the last layer's down items then set a bit of
// ctrl[C_ERR] too.
constexpr int kPsWaves = 16;
constexpr int kPsMaxKs = 4;        // K-splits of a linear (partials its consumers add)
constexpr int kPsRoles = 3;        // (stage, item) roles per block
constexpr long long kPsTimeoutTicks = 10000000;  // 100 ms of the 100 MHz wall clock
// ctrl[C_ERR] bits of a persistent-schedule token (the host recomputes it on
// the per-stage graph): a bounded wait ran out; the last residual was not
// finite (an input of a q4 linear overflowed its fp16 copy)
constexpr int kPsErrTimeout = 1, kPsErrRange = 2;
enum PsStage { PS_QKV = 0, PS_ATT = 1, PS_O = 2, PS_GU = 3, PS_DOWN = 4, PS_STAGES = 5 };
// Role code bit: the item publishes through its XCD's L2 (its consumers share
// the XCD); the stage is the code's low byte.
constexpr int kPsLocal = 0x100, kPsStageMask = 0xFF;
struct PsLayer {
  const uint4* wqkv;
  const uint16_t* sqkv;
  const float* bqkv;      // [Nqkv] (zeros without a bias)
  const float* attn_norm;
  const uint4* wo;
  const uint16_t* so;
  const uint4* wgu;       // paired gate|up tiles
  const uint16_t* sgu;
  const float* ffn_norm;
  const uint4* wd;
  const uint16_t* sd;
  void* kc;               // [Hkv][max_tokens][D]
  void* vc;
  int window;             // this layer's sliding window (0: full causal)
};
struct PsArgs {
  const PsLayer* layers;  // [L]
  const int* roles;       // [blocks][kPsRoles][2]: (stage code, item) pairs in stage order; stage -1: none
  const int* xcc;         // [blocks] the XCD each block ran on when the roles were placed (null: no
                          // handoff through an L2; a block on another XCD publishes device-scope)
  int L, H, I, Hq, Hkv, D, G, rd, max_tokens;
  int Nqkv, QS;
  int Cx, Co, Cd;         // chunks per row: H-input linears (qkv, gate|up), O (K = QS), down (K = I)
  int To, Tgu, Tq;        // 64-row tiles: H outputs (O, down), gate|up (paired), qkv
  int mw;                 // gate|up tiles per GU item
  int kq, cq, ko, co, ks, cs;  // K-splits and chunks per split: qkv, O, down
  float eps, scale;
  int* ctrl;
  const void* emb;        // [V][H] fp16 or fp32 (layer 0's residual)
  int emb_f32;
  const float* rope_cos;  // [max_tokens][max(rd / 2, 1)]
  const float* rope_sin;
  // published words (fp32 value, token number), per layer
  unsigned long long* pub_x;    // [L][kPsMaxKs][H] down partials (splits >= ks stay zero)
  unsigned long long* pub_qkv;  // [L][kq][Nqkv] partial q, k (RoPE applied), v
  unsigned long long* pub_o;    // [L][QS] attention output
  unsigned long long* pub_xm;   // [L][ko][H] partial x_mid
  unsigned long long* pub_h;    // [L][Tgu * 32] silu(gate) * up (zero past I)
  // optional timeline: per (block, wave), per layer and stage, kPsEvents
  // wall-clock stamps (100 MHz) taken by the wave's first lane; stage slot
  // PS_STAGES of layer L holds the kernel's start and end
  unsigned long long* trace;
  // bounded waits: give up after timeout ticks of the 100 MHz wall clock
  // (kPsTimeoutTicks); fail_layer >= 0 makes the QKV stage of that layer
  // report a time-out without waiting (the failure path, forced from the host
  // by tests)
  long long timeout;
  int fail_layer;
};
constexpr int kPsEvents = 4;  // weights issued, input ready, computed, published
// Template choice of the persistent kernel for a model (dt == 0: none).
struct PsShape {
  int fmt, kv_f32, dt, nx, no, nd, mw, kq, ko, ks;
  int l2;  // launch the variant whose marked roles publish through their XCD's L2
};
PsShape ps_shape(int fmt, int kv_f32, int H, int I, int D, int Hq, int Hkv, int cus);
size_t ps_smem_bytes(const PsShape& sh, int H, int QS);
// Block roles of a shape: [blocks][kPsRoles][2] (stage, item), stage -1 = none;
// false when the items need more than kPsRoles roles per block.
bool ps_roles(const PsShape& sh, int blocks, int H, int Hq, int Hkv, int Tgu, int* roles);
// The XCD (XCC id) of each block of a `blocks`-block launch; false on a HIP error.
bool ps_xcc_probe(int blocks, int* xcc);
// Moves the roles so that each group of k|v, attention and (when an O split
// covers whole kv heads) O items shares one class of blocks (equal b % 8,
// one XCD by xcc) and marks the items whose consumers all share it
// (kPsLocal); returns how many it marked, 0 (roles unchanged) when the
// blocks' XCDs are not one per class or a group does not fit its class.
int ps_localize(const PsShape& sh, int blocks, int Hq, int Hkv, int To, const int* xcc, int* roles);
// once per model, outside stream capture: allows the kernel smem bytes of LDS
bool ps_prepare(const PsShape& sh, size_t smem);
// a_dev: the arguments in device memory (kernel reads them with scalar loads)
bool launch_ps_token(const PsShape& sh, int blocks, size_t smem, const PsArgs* a_dev, hipStream_t st);

// ------------------------------------------------------------ batched prefill --
// A chunk of M prompt positions per pass: row-major activations, linears as
// MFMA GEMMs C[M][N] = A[M][K] * W^T over the tiled weight layout.
enum GemmEpi {
  GEMM_STORE = 0,   // Cf[m][n] = acc + bias[n] (no split-K)
  GEMM_PART = 1,    // Cf[z][m][n] = split z's sum (the consumer adds the slices)
  GEMM_SWIGLU = 2,  // Ch[m][i] = fp16(silu(gate) * up), paired gate|up weight rows (no split-K)
  GEMM_ROPE = 3,    // q|k|v rows, head_dim 64, full rotary: + bias, RoPE at position p0 + m; q to
                    // Ch (fp16 [M][Hq 64]), k and v to the fp16 caches (K-wave kernel, no split-K)
  GEMM_FOLD = 4,    // residual rows and the next RMSNorm's operand (K-wave kernel, no split-K):
                    // Cf[m][n] += acc (the fp32 residual rows), Ch[m][n] = fp16(x nw[n] 2^ex[m]),
                    // ss[m][t] = sum of x^2 over the 64 columns of tile t
};
struct GemmArgs {
  const uint16_t* A;   // fp16 [M][lda]
  int lda, M, N, K;    // N: physical weight rows (64 per tile)
  const uint4* w;      // [T][C][64] 16-byte chunks
  const uint16_t* s;   // q4 scales [T][C][64]
  int C;               // chunks per row in the weight layout
  const float* bias;   // GEMM_STORE, may be null
  float* Cf;           // fp32 [M][ldc]
  uint16_t* Ch;        // GEMM_SWIGLU: fp16 [M][ldc]
  int ldc;
  int n_out;           // GEMM_SWIGLU: intermediate size I (outputs i < n_out)
  int spc;             // 32-k steps per split (set by launch_gemm)
  // GEMM_ROPE
  const float* rope_cos;  // [max_tokens][32], attention factor folded in
  const float* rope_sin;
  int p0, Hq, Hkv, max_tokens;
  uint16_t* kc;        // fp16 [Hkv][max_tokens][64] (this layer)
  uint16_t* vc;
  int* ovf;            // set to 1 when an fp16 output (h, q, k, v) is not finite; may be null
  const int* ctrl;     // non-null: the first row's position is ctrl[C_POS] instead of p0 (a
                       // captured prefill chunk serves every chunk of its size)
  // GEMM_FOLD: nw the norm weight, ex the rows' exponents, ss the tile sums
  // ([M][ss_ld]).  GEMM_SWIGLU with ss non-null: its operand rows came from a
  // GEMM_FOLD; the products of row m are scaled by
  // rsqrt(sum_t ss[m][t] / n_norm + eps) 2^-ex[m] (the RMSNorm applied after the dot).
  const float* nw;
  const int* ex;
  float* ss;
  int ss_ld, n_norm;
  float eps;
};
// Tile and split-K choice of one GEMM (gemm_shape is the only planner, so the
// host sizes the slice buffers from the same numbers the launch uses).
struct GemmShape {
  int ring;  // 1: the q4 LDS-ring kernel (wn waves over 64 wn columns, 32 mt rows)
  int kw;    // 1 (with ring): four waves split K on one 64-column tile
  int wn;
  int mt, nb, gx, gy, spc, splits;
};
// Rows of the residual stream: X[m] += sum of n_part slices part[s][m]
// (slice stride pstride floats, rows of H), then Y[m] = fp16(rmsnorm(X[m]) w)
// unless Y is null.
struct RowsArgs {
  float* X;
  const float* part;
  int n_part;
  size_t pstride;
  int H;
  const float* w;
  float eps;
  uint16_t* Y;
  int* ovf;             // set to 1 when a normed fp16 value is not finite; may be null
  int* ex;              // with Y: row m's ilogb(rsqrt(mean(x^2) + eps)), the scale exponent of a
                        // later GEMM_FOLD of the same rows; may be null
  // non-null emb: X[m] is first set to the embedding row of token tokens[i + m],
  // i = ctrl[C_POS] - ctrl[C_BASE] (0 without ctrl), fp32 or fp16 table (emb_f32)
  const void* emb;
  int emb_f32;
  const int* tokens;
  const int* ctrl;
};
struct PrefillAttnArgs {
  const uint16_t* q;    // fp16 [M][Hq D], RoPE applied
  const void* kc;       // fp16 [Hkv][max_tokens][D] (this layer)
  const void* vc;
  uint16_t* out;        // fp16 [M][Hq D]
  int M, p0, Hq, Hkv, D, G, max_tokens, window;
  float scale_log2;     // softmax scale * log2(e)
  const int* ctrl;      // non-null: the first row's position is ctrl[C_POS] instead of p0
};
struct RopeKvArgs {
  const float* qkv;     // fp32 [n_part][M][Nqkv] split-K slices (summed here)
  int n_part;
  size_t pstride;       // floats between slices
  const float* bias;    // [Nqkv] or null
  int M, p0, Hq, Hkv, D, rd, max_tokens;
  const float* rope_cos;  // [max_tokens][rd / 2]
  const float* rope_sin;
  uint16_t* q;          // fp16 [M][Hq D]
  void* kc;             // [Hkv][max_tokens][D]
  void* vc;
  int kv_f32;
  int* ovf;             // set to 1 when an fp16 q, k or v is not finite; may be null
  const int* ctrl;      // non-null: the first row's position is ctrl[C_POS] instead of p0
};
GemmShape gemm_shape(int fmt, int epi, int M, int N, int K, int cus);
bool launch_gemm(int fmt, int epi, const GemmShape& sh, const GemmArgs& g, hipStream_t st);
void launch_rms_rows(const RowsArgs& a, int M, hipStream_t st);
void launch_rope_kv(const RopeKvArgs& a, hipStream_t st);
bool launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t st);
void launch_rows_to_f16(const float* x, size_t n, uint16_t* y, hipStream_t st);

}  // namespace tlm

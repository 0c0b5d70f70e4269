// Kernel argument blocks and launchers shared by tlm_kernels.hip and tlm_api.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tlm {

constexpr int kTile = 64;      // output rows per tile: one row per lane of a wave64
constexpr int kMaxChunks = 8;  // most 16-byte chunks a wave keeps in flight per batch
constexpr int kMaxPart = 8;    // partial vectors a consumer folds in with one round trip

enum WeightFmt { WF_F16 = 1, WF_Q4 = 2 };

// GEMV prologues: how the input slice x[k0, k1) is formed in LDS.
enum Prologue {
  PRO_COPY = 0,    // x = in
  PRO_RMS = 1,     // x = rmsnorm(base + sum_j pin[j]) * w
  PRO_SWIGLU = 2,  // x = silu(sum_j pin[j][k]) * (sum_j pin[j][up_off + k])
  PRO_ATTN = 3,    // x = flash-decoding combine of the attention chunk partials
  PRO_RMS2 = 4,    // PRO_RMS for K up to 8 elements per thread (chosen by launch_gemv)
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
// captured graph serves every position.
enum Ctrl { C_TOKEN = 0, C_POS = 1, C_STEP = 2, C_BASE = 3, C_LEN = 4 };

// Embedding row staging: the kernels that choose the next token (set_ctrl,
// prefill_advance, argmax_merge) also copy its embedding row to x0, the
// residual base of layer 0.  x0 == null disables the copy.
struct EmbStage {
  const void* emb;  // [V][H] fp16 or fp32
  int f32;
  int H;
  float* x0;
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
  const float* base;   // fp32 [K] residual stream (layer 0: the staged embedding row)
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
  // LM head epilogue
  float* logits;       // full logits (may be null)
  float* arg_val;      // per-block argmax partials
  int* arg_idx;
  int* tokens_out;     // greedy stream (indexed by ctrl[C_STEP]), may be null
  int advance;         // 1: last block advances ctrl (token <- argmax, pos++, step++)
  int max_steps;
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
};

// launchers (stream-ordered, graph-capturable: no memset, no host sync)
// launchers return false when no compiled variant matches (nothing is launched)
// waves in {4, 8}; nch in {1, 2, 4, 8}: chunks per wave and load batch
bool launch_gemv(int fmt, int pro, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st);
bool launch_lm_head(int fmt, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st);
// attention chunk partials; with `combine` also the combine kernel writing a.out
bool launch_attention(bool kv_f32, int gmax, const AttnArgs& a, bool combine, hipStream_t st);
size_t gemv_smem_bytes(int fmt, int cps, int waves);
void launch_final_norm(const float* base, const float* pin, int n_pin, int pin_stride, const float* w, int n,
                       float eps, float* y, hipStream_t st);
void launch_rmsnorm(const float* x, const float* w, int n, float eps, int offset, float* y, hipStream_t st);
void launch_silu_mul(const float* g, const float* u, int n, float* out, hipStream_t st);
void launch_reduce(const float* part, int n_part, int stride, const float* bias, int n, float* y, hipStream_t st);
void launch_argmax(const float* logits, int n, float* pval, int* pidx, int* token, int blocks, hipStream_t st);
// second pass of the greedy sampler; `ctrl` receives the token at ctrl[C_TOKEN]
void launch_argmax_merge(const float* pval, const int* pidx, int n, int* ctrl, int* tokens_out, int advance,
                         int max_steps, const EmbStage& es, hipStream_t st);
void launch_set_ctrl(int* ctrl, int token, int pos, int step, int base, int len, const EmbStage& es,
                     hipStream_t st);
void launch_prefill_advance(int* ctrl, const int* prompt, const EmbStage& es, hipStream_t st);
void launch_copy(uint4* dst, const uint4* src, size_t n16, hipStream_t st);
void launch_dequant(int fmt, const uint4* w, const uint16_t* s, int N, int T, int C, int K, float* out,
                    hipStream_t st);
void launch_kv_fill(void* kc, void* vc, bool f32, size_t heads_stride, int Hkv, int max_tokens, int D, int count,
                    uint64_t seed, hipStream_t st);
size_t attn_smem_bytes(int gmax, int D, bool kv_f32);
int attn_lpp(int D, bool kv_f32);

}  // namespace tlm

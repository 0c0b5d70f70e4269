// C ABI (include/tlm.h) over the gfx950 kernels of tlm_kernels.hip.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tlm.h"
#include "tlm_kernels.h"

using namespace tlm;

// ----------------------------------------------------------------- errors --

static thread_local std::string g_error;

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                                   \
  do {                                                                                                  \
    hipError_t e_ = (expr);                                                                             \
    if (e_ != hipSuccess)                                                                               \
      return fail(e_ == hipErrorOutOfMemory ? TLM_ERR_OOM : TLM_ERR_HIP, "HIP: %s failed: %s", #expr,   \
                  hipGetErrorString(e_));                                                               \
  } while (0)

#define CHECK_LAUNCH(component)                                                                         \
  do {                                                                                                  \
    hipError_t e_ = hipGetLastError();                                                                  \
    if (e_ != hipSuccess) return fail(TLM_ERR_HIP, "%s: launch failed: %s", component, hipGetErrorString(e_)); \
  } while (0)

// ------------------------------------------------- allocation-free scratch --
// tlm_op_attention_rows_noalloc stages the batched attention's rotated fp16
// queries here instead of in a hipMalloc'd buffer.  Each device that loads the
// library holds its own copy until the process ends.  In host code the name
// `scratch` is only a stand-in for the device array: kernels and copies get
// the device address that hipGetSymbolAddress returns (once per device, at
// tlm_open, with that device current).  Every call on a device shares that
// device's copy, so calls that overlap on one device race.
constexpr size_t kScratchBytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[kScratchDevices] = {};

static int scratch_address(int device, void** out) {  // device current
  if (device < 0 || device >= kScratchDevices)
    return fail(TLM_ERR_INVALID, "TLMContext: device %d beyond the %d the scratch table holds", device,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TLM_ERR_HIP, "TLMContext: scratch address on device %d: %s", device, hipGetErrorString(e));
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return TLM_OK;
}

// ---------------------------------------------------------------- objects --

struct tlm_ctx {
  int device = 0;
  int cus = 256;
  char name[256] = {0};
  hipStream_t stream = nullptr;
  // scratch for op-level argmax
  float* arg_val = nullptr;
  int* arg_idx = nullptr;
  // top-k levels: two levels of kTopkWork (score, id) pairs
  float* topk_v = nullptr;
  int* topk_i = nullptr;
  void* scratch = nullptr;  // this device's copy of `scratch` (device address)
};
constexpr size_t kTopkWork = 32768;

struct GemvPlan {
  int waves = 4, cps = 1, splits = 1, gx = 1;
  int nch = 1;  // chunks per wave per load batch
};

struct tlm_linear {
  tlm_ctx* ctx = nullptr;
  int fmt = TLM_FMT_F16;
  int N = 0, K = 0, T = 0, C = 0;
  uint4* w = nullptr;
  uint16_t* s = nullptr;
  GemvPlan plan;
  float* part = nullptr;  // op-level partials [splits][N]
  // paired layout (fused MLP gate|up, N = 2I): canonical gate row i sits in
  // tile i / 32, lane i % 32; up row I + i in the same tile, lane 32 + i % 32
  int pair_half = 0;  // I when paired, else 0
  uint16_t smax = 0;  // q4: largest scale magnitude uploaded (fp16 bits)
};

// Physical row of canonical row r.
static int phys_row(const tlm_linear* L, int r) {
  if (!L->pair_half) return r;
  const int I = L->pair_half, up = r >= I, i = up ? r - I : r;
  return (i / 32) * kTile + (up ? 32 : 0) + i % 32;
}

struct tlm_attn {
  tlm_ctx* ctx = nullptr;
  tlm_attn_desc d{};
  // chunks per query head: short windows (one wave each) and long windows
  // (up to kAttnWaves waves each, or with `gqa` one kGqaWaves-wave block per
  // kv head and chunk); pacc / pml hold the larger.  chmin*: smallest chunk.
  int G = 1, gmax = 1, nsplit = 1, nsplit_long = 1, chmin = 32, chmin_long = 32, lpp = 1;
  bool gqa = false;
  float scale = 1.f;
  void* kc = nullptr;
  void* vc = nullptr;
  float* rope_cos = nullptr;
  float* rope_sin = nullptr;
  float* pacc = nullptr;
  float* pml = nullptr;
  float* zero_bias = nullptr;  // stands in for an absent QKV bias
  int* ctrl = nullptr;
};

struct Layer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* bqkv = nullptr;
  tlm_linear* qkv = nullptr;
  tlm_linear* o = nullptr;
  tlm_linear* gu = nullptr;
  tlm_linear* down = nullptr;
  void* kc = nullptr;
  void* vc = nullptr;
};

// One logged run of tokens: n positions from pos, the first with `token`;
// device: the later tokens came from the device's argmax (a greedy run),
// else n is 1.  logits: the run computed the LM head.
struct RedoEntry {
  int32_t token, pos, n;
  bool logits, device;
};
constexpr size_t kRedoMax = (size_t)1 << 20;

// Persistent-schedule launches of every model on one device, in the order
// they are enqueued: each needs all of the device's CUs at once, so two of
// them running together (two models on two streams) would each wait for
// blocks the other holds.  While more than one model of the device has the
// schedule, a launch waits for the device's previous one (event `ev`,
// recorded on stream `last`).
struct PsDevice {
  std::mutex mu;
  int models = 0;
  hipEvent_t ev = nullptr;
  hipStream_t last = nullptr;
};
static PsDevice g_ps_dev[kScratchDevices];

constexpr int kPinPrompt = 16;  // first prompt word of tlm_model::host_pin

struct tlm_model {
  tlm_ctx* ctx = nullptr;
  tlm_model_desc d{};
  int Nqkv = 0, QS = 0;
  std::vector<Layer> layers;
  void* emb = nullptr;
  tlm_linear* head = nullptr;
  float* final_norm = nullptr;
  // activations and partials
  int* ctrl = nullptr;
  int* tokens_out = nullptr;
  int* prompt = nullptr;
  float *xa = nullptr, *xf = nullptr, *attn_out = nullptr;
  // residual accumulators (fixed point, nrep of kRep replica slots of H): x0 holds the
  // current token's embedding row (staged by the control kernels), rb[l] the
  // residual after layer l's MLP
  unsigned long long *x0 = nullptr, *rb = nullptr;
  int nrep = kRep;  // replicas the MLP adds into and the residual readers add (rep_count)
  float *pq = nullptr, *po = nullptr;
  int mlp_nch = 1, mlp_ndb = 1;
  float* logits = nullptr;
  float* arg_val = nullptr;
  int* arg_idx = nullptr;
  unsigned long long* arg_key = nullptr;  // the LM head's folded argmax (zero between launches)
  unsigned* arg_arrived = nullptr;        // LM head blocks done, for its in-launch merge (zero between launches)
  float* cand_v = nullptr;  // top-k candidates of the last logits (kTopkMax)
  int* cand_i = nullptr;
  // attention (shared by the layers; they run one after another)
  tlm_attn attn;
  GemvPlan lm_plan;
  // batched prefill: chunks of at least pf_min_rows positions (0: off) run as
  // MFMA GEMMs over pf_chunk rows at a time; row buffers for pf_cap rows are
  // allocated on first use
  int pf_min_rows = 64, pf_chunk = 2048, pf_cap = 0;
  float *pf_x = nullptr, *pf_part = nullptr;  // residual rows, split-K slices
  int* pf_ovf = nullptr;   // device flag: a batched chunk rounded a non-finite fp16 activation
  // pinned host words: [0, 8) the control block read back, [8] the fp16 flag
  // read back, [kPinPrompt, + max_tokens) the prompt ids on their way to the
  // device (asynchronous copies: the host does not wait for a staging copy)
  int* host_pin = nullptr;
  int pf_replayed = 0;     // batched chunks replayed on the decode graph after such a flag
  size_t pf_part_n = 0;
  uint16_t *pf_xn = nullptr, *pf_q = nullptr, *pf_att = nullptr, *pf_h = nullptr;
  int* pf_ex = nullptr;      // per row: the exponent of the attention norm's scale (GEMM_FOLD)
  float* pf_ss = nullptr;    // per row and 64-column tile: sums of squares of the residual (GEMM_FOLD)
  // per attention mode: [0] short windows, [1] long windows (long_window)
  hipGraphExec_t g_logits[2] = {}, g_prefill[2] = {}, g_layers[2] = {};
  hipGraph_t graph_logits[2] = {}, graph_prefill[2] = {}, graph_layers[2] = {};
  // persistent schedule (windows up to kLongWindow positions): one kernel per
  // token for every layer; ps_on when the model's shape has a compiled variant
  PsShape ps{};
  bool ps_on = false;
  bool ps_registered = false;  // counted in g_ps_dev[device].models
  int ps_blocks = 0;
  size_t ps_smem = 0;
  PsLayer* ps_layers = nullptr;  // device [L]
  int* ps_roles = nullptr;       // device [blocks][kPsRoles][2]
  int* ps_xcc = nullptr;         // device [blocks]: each block's XCD when the roles were placed
  int ps_l2_items = 0;           // items that publish through their XCD's L2 (0: none)
  PsArgs* ps_args_dev = nullptr;  // the kernel's arguments (device memory)
  unsigned long long *ps_pub_x = nullptr, *ps_pub_qkv = nullptr, *ps_pub_o = nullptr, *ps_pub_xm = nullptr,
                     *ps_pub_h = nullptr;
  // x0_stale: a persistent step chose the current token without staging its
  // embedding row in x0, which the per-stage graph's first layer reads
  // (stage_x0 does it before that graph's next step)
  bool x0_stale = false;
  // captured prompt chunks: batched chunks by row count, replayed chunks by
  // (schedule, position count); captured on first use
  std::map<int, std::pair<hipGraph_t, hipGraphExec_t>> pf_graphs, replay_graphs;
  // Tokens enqueued since the last clean check of the persistent schedule's
  // flags, in order: a token whose wait ran out or whose last residual was
  // not finite (fp16 input overflow) is recomputed with everything after it
  // on the per-stage graph (ps_recover).  redo_lost: the log outgrew
  // kRedoMax, so such a token can only be reported.
  std::vector<RedoEntry> redo;
  bool redo_lost = false;
  bool ps_suspend = false;   // recomputing: every token on the per-stage graph
  bool ps_range_off = false;  // the persistent schedule is off after an fp16 range overflow
  int host_pos = 0;  // position of the last token enqueued (selects the attention mode)
  int kv_hi = 0;     // cache rows [0, kv_hi) may hold values since the cache was last cleared
  std::vector<int> windows;  // per-layer sliding window (0: full causal)
  tlm_model_counts counts{};  // work handed to the stream (tlm_model_counts_read)
  bool finalized = false;
  bool use_graphs = true;  // TLM_GRAPHS=0 enqueues the same kernels directly (profilers, debugging)
};

// ------------------------------------------------------------ layout/plan --

// Chunks per row: 16-byte units of 32 q4 weights or 8 fp16 weights.
static int chunk_k(int fmt) { return fmt == TLM_FMT_Q4 ? 32 : 8; }

// Chunks a wave loads per batch: its chunk count rounded up to a power of two
// (at most kMaxChunks; more chunks run in several batches).
static void set_nch(GemvPlan& p) {
  const int per_wave = (p.cps + p.waves - 1) / p.waves;
  p.nch = per_wave <= 1 ? 1 : per_wave <= 2 ? 2 : per_wave <= 4 ? 4 : 8;
}

// Split-K plan for one GEMV: enough waves to keep every CU busy on a latency-
// bound batch-1 product, at least one 16-byte chunk per wave, and few partial
// vectors for the consumer to fold in.
static GemvPlan plan_gemv(int T, int C, int cus, int CK, bool single_split) {
  GemvPlan p;
  if (single_split) {
    p.waves = C >= 64 ? 8 : 4;
    p.cps = C;
    p.splits = 1;
    p.gx = T;
    set_nch(p);
    return p;
  }
  const long units = (long)T * C;
  const long target = 8L * cus;
  const int cpw = (int)std::max(1L, (units + target - 1) / target);
  p.waves = C >= 64 ? 8 : 4;
  int cps = std::max(1, std::min(C, p.waves * cpw));
  int S = (C + cps - 1) / cps;
  S = std::min(S, kMaxPart);  // consumers fold at most kMaxPart partials in one round trip
  cps = (C + S - 1) / S;
  const int max_cps = 8192 / CK;  // x slice <= 32 KB of LDS
  if (cps > max_cps) {
    cps = max_cps;
    S = (C + cps - 1) / cps;
  }
  p.cps = cps;
  p.splits = S;
  p.gx = T;
  if (p.waves > cps) p.waves = cps >= 8 ? 8 : 4;
  set_nch(p);
  return p;
}

// A GEMV whose prologue RMS-normalises the whole input row keeps 8 elements
// of it per thread: K <= 512 * waves.
static void rms_waves(tlm_linear* L) {
  while (L->plan.waves < 8 && L->K > 512 * L->plan.waves) L->plan.waves *= 2;
  set_nch(L->plan);
}

// Host repack of canonical rows [r0, r0 + rows) into the device tile layout.
// Tiles shared with rows outside the range are read back first.
static int linear_write_rows(tlm_linear* L, int r0, int rows, const void* data, const uint16_t* scales) {
  if (rows <= 0) return TLM_OK;
  int t0 = r0 / kTile, t1 = (r0 + rows - 1) / kTile + 1;
  if (L->pair_half) t0 = 0, t1 = L->T;
  const size_t tiles = (size_t)(t1 - t0);
  const size_t chunk_elems = (size_t)L->C * kTile;  // chunks per tile
  const bool aligned =
      !L->pair_half && (r0 % kTile == 0) && ((r0 + rows) % kTile == 0 || r0 + rows == L->N);
  hipStream_t st = L->ctx->stream;
  HIP_TRY(hipStreamSynchronize(st));
  if (data) {
    std::vector<uint4> host(tiles * chunk_elems);
    uint4* dst = L->w + (size_t)t0 * chunk_elems;
    if (!aligned) HIP_TRY(hipMemcpy(host.data(), dst, host.size() * sizeof(uint4), hipMemcpyDeviceToHost));
    const int CK = chunk_k(L->fmt);
    const int Kc = L->fmt == TLM_FMT_Q4 ? L->K / 2 : L->K;  // canonical row length in units
    for (int r = r0; r < r0 + rows; r++) {
      const int pr = phys_row(L, r);
      const int t = pr / kTile - t0, lane = pr % kTile;
      for (int c = 0; c < L->C; c++) {
        uint4 v = {0, 0, 0, 0};
        if (L->fmt == TLM_FMT_Q4) {
          const uint8_t* src = (const uint8_t*)data + (size_t)(r - r0) * Kc + (size_t)c * 16;
          memcpy(&v, src, 16);
        } else {
          uint16_t tmp[8] = {0};
          const uint16_t* src = (const uint16_t*)data + (size_t)(r - r0) * Kc;
          for (int j = 0; j < 8; j++) {
            const int k = c * CK + j;
            if (k < L->K) tmp[j] = src[k];
          }
          memcpy(&v, tmp, 16);
        }
        host[((size_t)t * L->C + c) * kTile + lane] = v;
      }
    }
    HIP_TRY(hipMemcpy(dst, host.data(), host.size() * sizeof(uint4), hipMemcpyHostToDevice));
  }
  if (scales && L->fmt == TLM_FMT_Q4) {
    std::vector<uint16_t> host(tiles * chunk_elems);
    uint16_t* dst = L->s + (size_t)t0 * chunk_elems;
    if (!aligned) HIP_TRY(hipMemcpy(host.data(), dst, host.size() * sizeof(uint16_t), hipMemcpyDeviceToHost));
    const int G = L->K / 32;
    for (int r = r0; r < r0 + rows; r++) {
      const int pr = phys_row(L, r);
      const int t = pr / kTile - t0, lane = pr % kTile;
      for (int c = 0; c < L->C; c++) {
        const uint16_t sv = c < G ? scales[(size_t)(r - r0) * G + c] : 0;
        host[((size_t)t * L->C + c) * kTile + lane] = sv;
        L->smax = std::max<uint16_t>(L->smax, sv & 0x7fff);
      }
    }
    HIP_TRY(hipMemcpy(dst, host.data(), host.size() * sizeof(uint16_t), hipMemcpyHostToDevice));
  }
  return TLM_OK;
}

static int linear_alloc(tlm_ctx* ctx, int fmt, int N, int K, bool single_split, tlm_linear** out,
                        bool paired = false) {
  if (fmt != TLM_FMT_F16 && fmt != TLM_FMT_Q4) return fail(TLM_ERR_INVALID, "TLMLinear: unsupported format %d", fmt);
  if (N <= 0 || K <= 0) return fail(TLM_ERR_INVALID, "TLMLinear: invalid shape %dx%d", N, K);
  if (fmt == TLM_FMT_Q4 && K % 32 != 0) return fail(TLM_ERR_INVALID, "TLMLinear: q4 needs K %% 32 == 0 (K=%d)", K);
  tlm_linear* L = new tlm_linear();
  L->ctx = ctx;
  L->fmt = fmt;
  L->N = N;
  L->K = K;
  L->T = (N + kTile - 1) / kTile;
  if (paired) {
    L->pair_half = N / 2;
    L->T = (N / 2 + 31) / 32;
  }
  L->C = (K + chunk_k(fmt) - 1) / chunk_k(fmt);
  L->plan = plan_gemv(L->T, L->C, ctx->cus, chunk_k(fmt), single_split);
  const size_t chunks = (size_t)L->T * L->C * kTile;
  hipError_t e = hipMalloc(&L->w, chunks * 16);
  if (e == hipSuccess && fmt == TLM_FMT_Q4) e = hipMalloc(&L->s, chunks * 2);
  if (e == hipSuccess) e = hipMemset(L->w, 0, chunks * 16);
  if (e == hipSuccess && L->s) e = hipMemset(L->s, 0, chunks * 2);
  if (e != hipSuccess) {
    hipFree(L->w);
    hipFree(L->s);
    delete L;
    return fail(TLM_ERR_OOM, "TLMLinear: device allocation of %zu bytes failed", chunks * 18);
  }
  *out = L;
  return TLM_OK;
}

static void fill_gemv_args(GemvArgs& a, const tlm_linear* L, float* out) {
  memset(&a, 0, sizeof a);
  a.w = L->w;
  a.s = L->s;
  a.N = L->N;
  a.T = L->T;
  a.C = L->C;
  a.K = L->K;
  a.cps = L->plan.cps;
  a.out = out;
}

static int wfmt(int fmt) { return fmt == TLM_FMT_Q4 ? WF_Q4 : WF_F16; }

// One GEMV launch of a linear with its split-K plan.
static bool launch_linear(const tlm_linear* L, int pro, const GemvArgs& a, hipStream_t st) {
  return launch_gemv(wfmt(L->fmt), pro, L->plan.waves, L->plan.nch, dim3(L->plan.gx, L->plan.splits), a, st);
}

// ------------------------------------------------------------------ context --

// The host-side helpers of tlm_host.cpp report through the same message.
int tlm_host_fail(int code, const char* msg) { return fail(code, "%s", msg); }

// Counts the model in (or out of) its device's persistent-schedule launches;
// the device's ordering event is created with the first model (device current).
static int ps_register(tlm_model* m, bool on) {
  if (on == m->ps_registered) return TLM_OK;
  PsDevice& pd = g_ps_dev[m->ctx->device];
  std::lock_guard<std::mutex> lock(pd.mu);
  if (on && !pd.ev) HIP_TRY(hipEventCreateWithFlags(&pd.ev, hipEventDisableTiming));
  pd.models += on ? 1 : -1;
  m->ps_registered = on;
  return TLM_OK;
}

// One persistent-schedule launch (enqueue(): the graph or the kernels) in the
// device's order: while several models of the device have the schedule, it
// waits for the previous launch of any of them and becomes the one the next
// waits for.
template <typename F>
static int ps_ordered(tlm_model* m, F enqueue) {
  PsDevice& pd = g_ps_dev[m->ctx->device];
  hipStream_t st = m->ctx->stream;
  std::lock_guard<std::mutex> lock(pd.mu);
  const bool order = pd.models > 1;
  if (order && pd.last && pd.last != st) HIP_TRY(hipStreamWaitEvent(st, pd.ev, 0));
  const int rc = enqueue();
  if (rc) return rc;
  if (order) {
    HIP_TRY(hipEventRecord(pd.ev, st));
    pd.last = st;
  }
  return TLM_OK;
}

static int model_check(tlm_model* m, const int* ctrl_host = nullptr);
static int read_ctrl(tlm_model* m, int* c);
// Positions up to `end` (exclusive) may now hold cache rows (what
// tlm_reset_cache clears).
static void kv_touch(tlm_model* m, long end) {
  m->kv_hi = (int)std::max<long>(m->kv_hi, std::min<long>(end, m->d.max_tokens));
}
static int kv_clear(tlm_model* m, int pos0, int n);


extern "C" {

int tlm_abi_version(void) { return TLM_ABI_VERSION; }

const char* tlm_last_error(void) { return g_error.c_str(); }


int tlm_open(int device, tlm_ctx** out) {
  if (!out) return fail(TLM_ERR_INVALID, "TLMContext: null output");
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) return fail(TLM_ERR_INVALID, "TLMContext: no device %d (%d present)", device, count);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(TLM_ERR_STATE, "TLMContext: device %d is %s; this library is built for gfx950", device,
                prop.gcnArchName);
  tlm_ctx* c = new tlm_ctx();
  c->device = device;
  c->cus = prop.multiProcessorCount;
  // the marketing name can be empty (a driver without the product table): the
  // architecture and the CU count name the part then
  snprintf(c->name, sizeof c->name, "%s (%s, %d CUs)", prop.name[0] ? prop.name : "AMD Instinct", prop.gcnArchName,
           prop.multiProcessorCount);
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->arg_val, 4096 * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&c->arg_idx, 4096 * sizeof(int));
  if (e == hipSuccess) e = hipMalloc(&c->topk_v, 2 * kTopkWork * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&c->topk_i, 2 * kTopkWork * sizeof(int));
  if (e != hipSuccess) {
    tlm_close(c);
    return fail(TLM_ERR_HIP, "TLMContext: setup failed: %s", hipGetErrorString(e));
  }
  const int rc = scratch_address(device, &c->scratch);
  if (rc) {
    tlm_close(c);
    return rc;
  }
  *out = c;
  return TLM_OK;
}

void tlm_close(tlm_ctx* ctx) {
  if (!ctx) return;
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  hipFree(ctx->arg_val);
  hipFree(ctx->arg_idx);
  hipFree(ctx->topk_v);
  hipFree(ctx->topk_i);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

int tlm_sync(tlm_ctx* ctx) {
  if (!ctx) return fail(TLM_ERR_INVALID, "TLMContext: null context");
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return TLM_OK;
}

int tlm_device_info(tlm_ctx* ctx, char* name, size_t name_len, int* cu_count) {
  if (!ctx) return fail(TLM_ERR_INVALID, "TLMContext: null context");
  if (name && name_len) snprintf(name, name_len, "%s", ctx->name);
  if (cu_count) *cu_count = ctx->cus;
  return TLM_OK;
}

int tlm_device_memory(tlm_ctx* ctx, size_t* free_bytes, size_t* total_bytes) {
  if (!ctx || !free_bytes || !total_bytes) return fail(TLM_ERR_INVALID, "TLMContext: null argument");
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipMemGetInfo(free_bytes, total_bytes));
  return TLM_OK;
}

int tlm_alloc(tlm_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return fail(TLM_ERR_INVALID, "TLMBuffer: null argument");
  HIP_TRY(hipMalloc(dptr, std::max<size_t>(bytes, 4)));
  return TLM_OK;
}

int tlm_free(tlm_ctx* ctx, void* dptr) {
  if (!ctx) return fail(TLM_ERR_INVALID, "TLMBuffer: null context");
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  HIP_TRY(hipFree(dptr));
  return TLM_OK;
}

int tlm_upload(tlm_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(TLM_ERR_INVALID, "TLMBuffer: null argument");
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return TLM_OK;
}

int tlm_download(tlm_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(TLM_ERR_INVALID, "TLMBuffer: null argument");
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return TLM_OK;
}

int tlm_copy(tlm_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(TLM_ERR_INVALID, "TLMBuffer: null argument");
  if (bytes % 16 != 0) return fail(TLM_ERR_INVALID, "TLMBuffer: copy size %zu is not a multiple of 16", bytes);
  if (bytes == 0) return TLM_OK;
  launch_copy(static_cast<uint4*>(dst), static_cast<const uint4*>(src), bytes / 16, ctx->stream);
  CHECK_LAUNCH("TLMBuffer");
  return TLM_OK;
}

// ------------------------------------------------------------------ linear --

int tlm_linear_create(tlm_ctx* ctx, int fmt, int n_out, int k_in, const void* weights, const uint16_t* scales,
                      tlm_linear** out) {
  if (!ctx || !out || !weights || (fmt == TLM_FMT_Q4 && !scales))
    return fail(TLM_ERR_INVALID, "TLMLinear: null argument");
  tlm_linear* L = nullptr;
  int rc = linear_alloc(ctx, fmt, n_out, k_in, false, &L);
  if (rc) return rc;
  rc = linear_write_rows(L, 0, n_out, weights, scales);
  if (rc == TLM_OK && hipMalloc(&L->part, sizeof(float) * (size_t)L->plan.splits * L->N) != hipSuccess)
    rc = fail(TLM_ERR_OOM, "TLMLinear: partials allocation failed");
  if (rc) {
    tlm_linear_destroy(L);
    return rc;
  }
  *out = L;
  return TLM_OK;
}

void tlm_linear_destroy(tlm_linear* L) {
  if (!L) return;
  hipStreamSynchronize(L->ctx->stream);
  hipFree(L->w);
  hipFree(L->s);
  hipFree(L->part);
  delete L;
}

int tlm_linear_dequant(tlm_linear* L, float* host_out) {
  if (!L || !host_out) return fail(TLM_ERR_INVALID, "TLMLinear: null argument");
  float* d = nullptr;
  const size_t bytes = sizeof(float) * (size_t)L->N * L->K;
  HIP_TRY(hipMalloc(&d, bytes));
  launch_dequant(wfmt(L->fmt), L->w, L->s, L->N, L->T, L->C, L->K, d, L->ctx->stream);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(L->ctx->stream);
  if (e == hipSuccess) e = hipMemcpy(host_out, d, bytes, hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) return fail(TLM_ERR_HIP, "TLMLinear: dequant failed: %s", hipGetErrorString(e));
  return TLM_OK;
}

int tlm_op_linear(tlm_linear* L, const float* x, const float* bias, float* y) {
  if (!L || !x || !y) return fail(TLM_ERR_INVALID, "TLMLinear: null argument");
  GemvArgs a;
  const bool direct = L->plan.splits == 1;
  fill_gemv_args(a, L, direct ? y : L->part);
  a.in = x;
  a.bias = direct ? bias : nullptr;
  if (!launch_linear(L, PRO_COPY, a, L->ctx->stream))
    return fail(TLM_ERR_STATE, "TLMLinear: no kernel variant for this shape");
  CHECK_LAUNCH("TLMLinear");
  if (!direct) {
    launch_reduce(L->part, L->plan.splits, L->N, bias, L->N, y, L->ctx->stream);
    CHECK_LAUNCH("TLMLinear");
  }
  return TLM_OK;
}

int tlm_op_linear_rows(tlm_linear* L, const uint16_t* x, int32_t rows, const float* bias, float* y) {
  if (!L || !x || !y || rows <= 0) return fail(TLM_ERR_INVALID, "TLMLinear: invalid argument");
  if (L->pair_half) return fail(TLM_ERR_INVALID, "TLMLinear: paired layout");
  if (L->K % 32) return fail(TLM_ERR_INVALID, "TLMLinear: batched rows need K %% 32 == 0 (K = %d)", L->K);
  GemmArgs g;
  memset(&g, 0, sizeof g);
  g.A = x;
  g.lda = L->K;
  g.M = rows;
  g.N = L->N;
  g.K = L->K;
  g.w = L->w;
  g.s = L->s;
  g.C = L->C;
  g.bias = bias;
  g.Cf = y;
  g.ldc = L->N;
  if (L->fmt == TLM_FMT_Q4 && L->smax > 0x6FFF)
    return fail(TLM_ERR_INVALID, "TLMLinear: q4 scale above 8188 overflows the fp16 GEMM operand");
  const GemmShape sh = gemm_shape(wfmt(L->fmt), GEMM_STORE, rows, L->N, L->K, L->ctx->cus);
  if (!launch_gemm(wfmt(L->fmt), GEMM_STORE, sh, g, L->ctx->stream))
    return fail(TLM_ERR_STATE, "TLMLinear: no batched kernel variant for %d x %d", L->N, L->K);
  CHECK_LAUNCH("TLMLinear");
  return TLM_OK;
}

// -------------------------------------------------------------- element ops --

int tlm_op_rmsnorm(tlm_ctx* ctx, const float* x, const float* w, int n, double eps, int offset, float* y) {
  if (!ctx || !x || !y || n <= 0) return fail(TLM_ERR_INVALID, "TLMRMSNorm: invalid argument");
  launch_rmsnorm(x, w, n, (float)eps, offset, y, ctx->stream);
  CHECK_LAUNCH("TLMRMSNorm");
  return TLM_OK;
}

int tlm_op_silu_mul(tlm_ctx* ctx, const float* gate, const float* up, int n, float* out) {
  if (!ctx || !gate || !up || !out || n <= 0) return fail(TLM_ERR_INVALID, "TLMSiLUMul: invalid argument");
  launch_silu_mul(gate, up, n, out, ctx->stream);
  CHECK_LAUNCH("TLMSiLUMul");
  return TLM_OK;
}

int tlm_op_gated_mlp(tlm_linear* gu, tlm_linear* down, const float* x, float* y) {
  if (!gu || !down || !x || !y) return fail(TLM_ERR_INVALID, "TLMGatedMLP: null argument");
  if (gu->N != 2 * down->K || gu->K != down->N)
    return fail(TLM_ERR_INVALID, "TLMGatedMLP: gate/up %dx%d does not match down %dx%d", gu->N, gu->K, down->N,
                down->K);
  hipStream_t st = gu->ctx->stream;
  GemvArgs a;
  fill_gemv_args(a, gu, gu->part);
  a.in = x;
  if (!launch_linear(gu, PRO_COPY, a, st))
    return fail(TLM_ERR_STATE, "TLMGatedMLP: no kernel variant for this shape");
  CHECK_LAUNCH("TLMGatedMLP");
  GemvArgs b;
  const bool direct = down->plan.splits == 1;
  fill_gemv_args(b, down, direct ? y : down->part);
  b.pin = gu->part;
  b.n_pin = gu->plan.splits;
  b.pin_stride = gu->N;
  b.up_off = down->K;
  if (!launch_linear(down, PRO_SWIGLU, b, st))
    return fail(TLM_ERR_STATE, "TLMGatedMLP: no kernel variant for this shape");
  CHECK_LAUNCH("TLMGatedMLP");
  if (!direct) {
    launch_reduce(down->part, down->plan.splits, down->N, nullptr, down->N, y, st);
    CHECK_LAUNCH("TLMGatedMLP");
  }
  return TLM_OK;
}

// ---------------------------------------------------------------- attention --

// cos/sin of pos * inv_freq[j] in double, times the attention factor, rounded
// to fp32 (the CPU reference evaluates the angle in double, math.ts:144-146).
static void rope_tables(int max_tokens, int rd, const float* inv_freq, double af, std::vector<float>& cs,
                        std::vector<float>& sn) {
  const int half = rd / 2;
  cs.assign((size_t)max_tokens * half, 0.f);
  sn.assign((size_t)max_tokens * half, 0.f);
  for (int p = 0; p < max_tokens; p++)
    for (int j = 0; j < half; j++) {
      const double angle = (double)p * (double)inv_freq[j];
      cs[(size_t)p * half + j] = (float)(cos(angle) * af);
      sn[(size_t)p * half + j] = (float)(sin(angle) * af);
    }
}

static int attn_init(tlm_ctx* ctx, const tlm_attn_desc* d, tlm_attn* A, bool own_cache) {
  if (d->heads <= 0 || d->kv_heads <= 0 || d->heads % d->kv_heads != 0)
    return fail(TLM_ERR_INVALID, "TLMAttention: heads %d must be a multiple of kv heads %d", d->heads, d->kv_heads);
  if (d->head_dim <= 0 || d->head_dim % 2 != 0 || d->head_dim > 128)
    return fail(TLM_ERR_INVALID, "TLMAttention: head_dim %d must be even and <= 128", d->head_dim);
  if (d->rotary_dim < 0 || d->rotary_dim > d->head_dim || d->rotary_dim % 2 != 0)
    return fail(TLM_ERR_INVALID, "TLMAttention: invalid rotary dimension %d", d->rotary_dim);
  if (d->rotary_dim > 0 && !d->inv_freq) return fail(TLM_ERR_INVALID, "TLMAttention: missing inv_freq");
  if (d->max_tokens <= 0) return fail(TLM_ERR_INVALID, "TLMAttention: max_tokens must be positive");
  A->ctx = ctx;
  A->d = *d;
  A->G = d->heads / d->kv_heads;
  if (A->G > 16) return fail(TLM_ERR_INVALID, "TLMAttention: more than 16 query heads per kv head");
  A->gmax = A->G <= 1 ? 1 : A->G <= 2 ? 2 : A->G <= 4 ? 4 : A->G <= 8 ? 8 : 16;
  A->scale = (float)(d->attn_scale > 0 ? d->attn_scale : 1.0 / sqrt((double)d->head_dim));
  A->lpp = attn_lpp(d->head_dim, d->kv_fmt == TLM_FMT_F32);
  if (attn_smem_bytes(A->gmax, d->head_dim, d->kv_fmt == TLM_FMT_F32, true) > 65536)
    return fail(TLM_ERR_INVALID, "TLMAttention: %d heads per kv head x head_dim %d exceed the LDS budget", A->G,
                d->head_dim);
  // per wave: chunks of at least 32 positions, at most 256, about two waves
  // per CU and kv head at the longest window.  Long windows: a block spreads
  // its chunk over up to kAttnWaves waves, so a quarter as many chunks.
  const int by_tile = (d->max_tokens + 255) / 256;
  const int by_cus = std::max(1, 2 * ctx->cus / d->kv_heads);
  const int by_min = (d->max_tokens + 31) / 32;
  A->chmin = 32;
  A->nsplit = std::max(by_tile, std::min(by_min, by_cus));
  A->nsplit_long = (A->nsplit + kAttnWaves - 1) / kAttnWaves;
  A->chmin_long = A->chmin;
  // Long windows with an fp16 cache, head_dim 64 / 128 and (G + 2) head_dim
  // <= 1536: the matrix-core kernel, one block per (kv head, chunk) for all G
  // query heads; about one block per CU, chunks of at least four 32-position
  // tiles (128 against 256 positions: Llama-3.2-1B at 4096, 32 blocks per kv
  // head instead of 17, 1870 -> 1879 tok/s; 64: no better), and at most 32
  // chunks (the O projection's combine folds 32 in one round trip).
  // TLM_GQA=0 keeps the one-head-per-block kernel (comparisons).
  const char* gq = getenv("TLM_GQA");
  A->gqa = d->kv_fmt == TLM_FMT_F16 && gqa_attention_fits(A->G, d->head_dim) && !(gq && gq[0] == '0');
  if (A->gqa) {
    A->nsplit_long = std::max(1, std::min(32, ctx->cus / d->kv_heads));
    A->chmin_long = 4 * kGqaTile;
  }
  const int D = d->head_dim;
  const size_t esz = d->kv_fmt == TLM_FMT_F32 ? 4 : 2;
  std::vector<float> cs, sn;
  const int half = std::max(1, d->rotary_dim / 2);
  if (d->rotary_dim > 0) rope_tables(d->max_tokens, d->rotary_dim, d->inv_freq, d->attention_factor, cs, sn);
  else cs.assign((size_t)d->max_tokens * half, 0.f), sn.assign((size_t)d->max_tokens * half, 0.f);
  HIP_TRY(hipMalloc(&A->rope_cos, cs.size() * sizeof(float)));
  HIP_TRY(hipMalloc(&A->rope_sin, sn.size() * sizeof(float)));
  HIP_TRY(hipMemcpy(A->rope_cos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(A->rope_sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice));
  const size_t nsp = (size_t)std::max(A->nsplit, A->nsplit_long);
  HIP_TRY(hipMalloc(&A->pacc, sizeof(float) * (size_t)d->heads * nsp * D));
  HIP_TRY(hipMalloc(&A->pml, sizeof(float) * (size_t)d->heads * nsp * 2));
  const size_t nqkv = (size_t)(d->heads + 2 * d->kv_heads) * D;
  HIP_TRY(hipMalloc(&A->zero_bias, sizeof(float) * nqkv));
  HIP_TRY(hipMemset(A->zero_bias, 0, sizeof(float) * nqkv));
  if (own_cache) {
    const size_t cache = (size_t)d->kv_heads * d->max_tokens * D * esz;
    HIP_TRY(hipMalloc(&A->kc, cache));
    HIP_TRY(hipMalloc(&A->vc, cache));
    HIP_TRY(hipMemset(A->kc, 0, cache));
    HIP_TRY(hipMemset(A->vc, 0, cache));
    HIP_TRY(hipMalloc(&A->ctrl, sizeof(int) * 8));
    HIP_TRY(hipMemset(A->ctrl, 0, sizeof(int) * 8));
  }
  return TLM_OK;
}

static void attn_free(tlm_attn* A, bool own_cache) {
  hipFree(A->rope_cos);
  hipFree(A->rope_sin);
  hipFree(A->pacc);
  hipFree(A->pml);
  hipFree(A->zero_bias);
  if (own_cache) {
    hipFree(A->kc);
    hipFree(A->vc);
    hipFree(A->ctrl);
  }
}

// Windows above kLongWindow positions run the long-window attention kernels.
static bool long_window(const tlm_attn* A, int pos) {
  const int n = A->d.sliding_window > 0 ? std::min(pos + 1, A->d.sliding_window) : pos + 1;
  return n > kLongWindow;
}

static AttnArgs attn_args(const tlm_attn* A, const float* src, int n_src, int stride, const float* bias,
                          const int* ctrl, void* kc, void* vc, float* out, bool long_win) {
  AttnArgs a;
  memset(&a, 0, sizeof a);
  a.src = src;
  a.n_src = n_src;
  a.src_stride = stride;
  a.bias = bias ? bias : A->zero_bias;
  a.ctrl = ctrl;
  a.kc = kc;
  a.vc = vc;
  a.rope_cos = A->rope_cos;
  a.rope_sin = A->rope_sin;
  a.out = out;
  a.pacc = A->pacc;
  a.pml = A->pml;
  a.Hq = A->d.heads;
  a.Hkv = A->d.kv_heads;
  a.D = A->d.head_dim;
  a.G = A->G;
  a.rd = A->d.rotary_dim;
  a.max_tokens = A->d.max_tokens;
  a.window = A->d.sliding_window;
  a.nsplit = long_win ? A->nsplit_long : A->nsplit;
  a.chmin = long_win ? A->chmin_long : A->chmin;
  a.gqa = long_win && A->gqa ? 1 : 0;
  a.lpp = A->lpp;
  a.scale = A->scale;
  return a;
}

int tlm_attn_create(tlm_ctx* ctx, const tlm_attn_desc* desc, tlm_attn** out) {
  if (!ctx || !desc || !out) return fail(TLM_ERR_INVALID, "TLMAttention: null argument");
  tlm_attn* A = new tlm_attn();
  int rc = attn_init(ctx, desc, A, true);
  if (rc) {
    attn_free(A, true);
    delete A;
    return rc;
  }
  *out = A;
  return TLM_OK;
}

void tlm_attn_destroy(tlm_attn* A) {
  if (!A) return;
  hipStreamSynchronize(A->ctx->stream);
  attn_free(A, true);
  delete A;
}

int tlm_op_attention(tlm_attn* A, const float* qkv, int position, float* out) {
  if (!A || !qkv || !out) return fail(TLM_ERR_INVALID, "TLMAttention: null argument");
  if (position < 0 || position >= A->d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMAttention: position %d outside [0, %d)", position, A->d.max_tokens);
  hipStream_t st = A->ctx->stream;
  launch_set_ctrl(A->ctrl, 0, position, 0, 0, 0, EmbStage{}, st);
  const int total = (A->d.heads + 2 * A->d.kv_heads) * A->d.head_dim;
  const bool lw = long_window(A, position);
  AttnArgs a = attn_args(A, qkv, 1, total, nullptr, A->ctrl, A->kc, A->vc, out, lw);
  if (!launch_attention(A->d.kv_fmt == TLM_FMT_F32, A->gmax, a, true, lw, st))
    return fail(TLM_ERR_STATE, "TLMAttention: no kernel variant for this shape");
  CHECK_LAUNCH("TLMAttention");
  return TLM_OK;
}

// RoPE + cache append of `rows` positions from position0, then their causal
// attention, enqueued on the context's stream; q: fp16 staging of the rotated
// queries, [rows][heads * head_dim].
static int check_attention_rows(const tlm_attn* A, const float* qkv, int32_t rows, int32_t position0,
                                const uint16_t* out) {
  if (!A || !qkv || !out || rows <= 0) return fail(TLM_ERR_INVALID, "TLMAttention: invalid argument");
  const tlm_attn_desc& d = A->d;
  if (position0 < 0 || position0 + rows > d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMAttention: rows [%d, %d) outside [0, %d)", position0, position0 + rows,
                d.max_tokens);
  if (d.kv_fmt == TLM_FMT_F32 || (d.head_dim != 64 && d.head_dim != 128))
    return fail(TLM_ERR_INVALID, "TLMAttention: batched rows need an fp16 cache and head_dim 64 or 128");
  return TLM_OK;
}

static bool enqueue_attention_rows(tlm_attn* A, const float* qkv, int32_t rows, int32_t position0, uint16_t* out,
                                   uint16_t* q) {
  const tlm_attn_desc& d = A->d;
  hipStream_t st = A->ctx->stream;
  RopeKvArgs r;
  memset(&r, 0, sizeof r);
  r.qkv = qkv;
  r.n_part = 1;
  r.pstride = 0;
  r.M = rows;
  r.p0 = position0;
  r.Hq = d.heads;
  r.Hkv = d.kv_heads;
  r.D = d.head_dim;
  r.rd = d.rotary_dim;
  r.max_tokens = d.max_tokens;
  r.rope_cos = A->rope_cos;
  r.rope_sin = A->rope_sin;
  r.q = q;
  r.kc = A->kc;
  r.vc = A->vc;
  launch_rope_kv(r, st);
  PrefillAttnArgs pa;
  memset(&pa, 0, sizeof pa);
  pa.q = q;
  pa.kc = A->kc;
  pa.vc = A->vc;
  pa.out = out;
  pa.M = rows;
  pa.p0 = position0;
  pa.Hq = d.heads;
  pa.Hkv = d.kv_heads;
  pa.D = d.head_dim;
  pa.G = A->G;
  pa.max_tokens = d.max_tokens;
  pa.window = d.sliding_window;
  pa.scale_log2 = A->scale * 1.4426950408889634f;
  return launch_prefill_attention(pa, st);
}

int tlm_op_attention_rows(tlm_attn* A, const float* qkv, int32_t rows, int32_t position0, uint16_t* out) {
  int rc = check_attention_rows(A, qkv, rows, position0, out);
  if (rc) return rc;
  uint16_t* q = nullptr;
  HIP_TRY(hipMalloc(&q, sizeof(uint16_t) * (size_t)rows * A->d.heads * A->d.head_dim));
  const bool launched = enqueue_attention_rows(A, qkv, rows, position0, out, q);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(A->ctx->stream);
  hipFree(q);
  if (e != hipSuccess) return fail(TLM_ERR_HIP, "TLMAttention: batched rows failed: %s", hipGetErrorString(e));
  if (!launched) return fail(TLM_ERR_STATE, "TLMAttention: no batched attention kernel for this shape");
  return TLM_OK;
}

int tlm_op_attention_rows_noalloc(tlm_attn* A, const float* qkv, int32_t rows, int32_t position0, uint16_t* out) {
  int rc = check_attention_rows(A, qkv, rows, position0, out);
  if (rc) return rc;
  const size_t need = sizeof(uint16_t) * (size_t)rows * A->d.heads * A->d.head_dim;
  if (need > kScratchBytes)
    return fail(TLM_ERR_RANGE, "TLMAttention: %d rows need %zu bytes of query staging; the allocation-free "
                "entry point holds %zu (at most %zu rows of this shape)", rows, need, kScratchBytes,
                kScratchBytes / (sizeof(uint16_t) * A->d.heads * A->d.head_dim));
  if (!A->ctx->scratch) return fail(TLM_ERR_STATE, "TLMAttention: the context has no scratch address");
  if (!enqueue_attention_rows(A, qkv, rows, position0, out, static_cast<uint16_t*>(A->ctx->scratch)))
    return fail(TLM_ERR_STATE, "TLMAttention: no batched attention kernel for this shape");
  CHECK_LAUNCH("TLMAttention");
  return TLM_OK;
}

int tlm_attn_reset(tlm_attn* A) {
  if (!A) return fail(TLM_ERR_INVALID, "TLMAttention: null argument");
  const size_t esz = A->d.kv_fmt == TLM_FMT_F32 ? 4 : 2;
  const size_t cache = (size_t)A->d.kv_heads * A->d.max_tokens * A->d.head_dim * esz;
  HIP_TRY(hipMemsetAsync(A->kc, 0, cache, A->ctx->stream));
  HIP_TRY(hipMemsetAsync(A->vc, 0, cache, A->ctx->stream));
  return TLM_OK;
}

static float elem_to_f32(const void* p, size_t i, bool f32) {
  if (f32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu, bits;
  if (e == 0) {
    if (m == 0)
      bits = sign;
    else {
      int sh = 0;
      while (!(m & 0x400u)) {
        m <<= 1;
        sh++;
      }
      bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 31)
    bits = sign | 0x7f800000u | (m << 13);
  else
    bits = sign | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

int tlm_attn_read_cache(tlm_attn* A, int count, float* k_out, float* v_out) {
  if (!A || !k_out || !v_out || count < 0 || count > A->d.max_tokens)
    return fail(TLM_ERR_INVALID, "TLMAttention: invalid read");
  const bool f32 = A->d.kv_fmt == TLM_FMT_F32;
  const size_t esz = f32 ? 4 : 2;
  const int Hkv = A->d.kv_heads, D = A->d.head_dim, M = A->d.max_tokens;
  std::vector<uint8_t> kbuf((size_t)Hkv * M * D * esz), vbuf(kbuf.size());
  HIP_TRY(hipStreamSynchronize(A->ctx->stream));
  HIP_TRY(hipMemcpy(kbuf.data(), A->kc, kbuf.size(), hipMemcpyDeviceToHost));
  HIP_TRY(hipMemcpy(vbuf.data(), A->vc, vbuf.size(), hipMemcpyDeviceToHost));
  for (int t = 0; t < count; t++)
    for (int h = 0; h < Hkv; h++)
      for (int d = 0; d < D; d++) {
        const size_t src = ((size_t)h * M + t) * D + d, dst = ((size_t)t * Hkv + h) * D + d;
        k_out[dst] = elem_to_f32(kbuf.data(), src, f32);
        v_out[dst] = elem_to_f32(vbuf.data(), src, f32);
      }
  return TLM_OK;
}

// ------------------------------------------------------------------- logits --

// LM head grid: every block resident at once (two 8-wave blocks per CU) with
// the same number of 64-row tiles, at most 4096 blocks (the argmax partials).
// One block per tile ran ~4.6 rounds with a ragged last one (47 us at
// 151936 x 896 on 256 CUs); five tiles per block (475 blocks) took 44.5 us.
// Counts that leave some CUs a block more than others were slower (6, 7 and 8
// tiles per block: 48-58 us).
static int lm_head_grid(int T, int cus) {
  const int per = std::max((T + 2 * cus - 1) / (2 * cus), (T + 4095) / 4096);
  return (T + per - 1) / per;
}

int tlm_op_logits(tlm_linear* head, const float* x, float* logits, int32_t* token) {
  if (!head || !x || !token) return fail(TLM_ERR_INVALID, "TLMLogits: null argument");
  tlm_ctx* ctx = head->ctx;
  GemvPlan p = plan_gemv(head->T, head->C, ctx->cus, chunk_k(head->fmt), true);
  p.gx = lm_head_grid(head->T, ctx->cus);
  GemvArgs a;
  fill_gemv_args(a, head, nullptr);
  a.cps = p.cps;
  a.in = x;
  a.logits = logits;
  a.arg_val = ctx->arg_val;
  a.arg_idx = ctx->arg_idx;
  if (gemv_smem_bytes(wfmt(head->fmt), p.cps, p.waves) > 65536)
    return fail(TLM_ERR_INVALID, "TLMLogits: hidden size %d too large for one block", head->K);
  if (!launch_lm_head(wfmt(head->fmt), PRO_COPY, p.waves, p.nch, dim3(p.gx), a, ctx->stream))
    return fail(TLM_ERR_STATE, "TLMLogits: no kernel variant for this shape");
  // the sampled token lands in token[0] (the merge's ctrl[C_TOKEN])
  launch_argmax_merge(ctx->arg_val, ctx->arg_idx, p.gx, token, nullptr, 0, 0, EmbStage{}, ctx->stream);
  CHECK_LAUNCH("TLMLogits");
  return TLM_OK;
}

int tlm_op_argmax(tlm_ctx* ctx, const float* logits, int n, int32_t* token) {
  if (!ctx || !logits || !token || n <= 0) return fail(TLM_ERR_INVALID, "TLMLogits: invalid argmax argument");
  const int blocks = std::max(1, std::min(1024, (n + 1023) / 1024));
  launch_argmax(logits, n, ctx->arg_val, ctx->arg_idx, token, blocks, ctx->stream);
  CHECK_LAUNCH("TLMLogits");
  return TLM_OK;
}

int tlm_op_topk(tlm_ctx* ctx, const float* logits, int n, int k, double softcap, int32_t* tokens, float* scores) {
  if (!ctx || !logits || !tokens || !scores || n <= 0) return fail(TLM_ERR_INVALID, "TLMLogitSampler: invalid argument");
  if (k < 1 || k > kTopkMax)
    return fail(TLM_ERR_INVALID, "TLMLogitSampler: candidate count %d outside [1, %d]", k, kTopkMax);
  if (!launch_topk(logits, n, k, (float)(softcap > 0 ? softcap : 0), ctx->topk_v, ctx->topk_i, kTopkWork, scores,
                   tokens, ctx->stream))
    return fail(TLM_ERR_INVALID, "TLMLogitSampler: %d logits exceed the candidate workspace", n);
  CHECK_LAUNCH("TLMLogitSampler");
  return TLM_OK;
}

// -------------------------------------------------------------------- model --

static int model_alloc(void** p, size_t bytes) {
  if (hipMalloc(p, std::max<size_t>(bytes, 4)) != hipSuccess)
    return fail(TLM_ERR_OOM, "TLMModel: device allocation of %zu bytes failed", bytes);
  if (hipMemset(*p, 0, std::max<size_t>(bytes, 4)) != hipSuccess)
    return fail(TLM_ERR_HIP, "TLMModel: memset failed");
  return TLM_OK;
}

void tlm_model_destroy(tlm_model* m);

// Replicas of the fixed-point residual for a hidden size: the MLP's down
// atomics hit each address (blocks / nrep) times and every residual reader
// (the next QKV GEMV, the LM head) adds nrep vectors.  Measured at long
// windows (us per token): Llama-3.2-1B shape (hidden 2048) 502 with 2 against
// 515 with 4; Llama-3.2-3B (3072) 1363 with 2, 1345 with 4, 1385 with 8.
// TLM_REPLICAS=2 or 4 at model creation overrides it (comparisons).
static int rep_count(int H) {
  const char* e = getenv("TLM_REPLICAS");
  const int v = e ? atoi(e) : 0;
  if (v == 2 || v == kRep) return v;
  return H <= 2048 ? 2 : kRep;
}

static PsArgs ps_args(const tlm_model* m) {
  const tlm_model_desc& d = m->d;
  const Layer& L0 = m->layers[0];
  PsArgs a;
  memset(&a, 0, sizeof a);
  a.layers = m->ps_layers;
  a.roles = m->ps_roles;
  a.L = d.num_layers;
  a.H = d.hidden_size;
  a.I = d.intermediate_size;
  a.Hq = d.num_heads;
  a.Hkv = d.num_kv_heads;
  a.D = d.head_dim;
  a.G = d.num_heads / d.num_kv_heads;
  a.rd = d.rotary_dim;
  a.max_tokens = d.max_tokens;
  a.Nqkv = m->Nqkv;
  a.QS = m->QS;
  a.Cx = L0.qkv->C;
  a.Co = L0.o->C;
  a.Cd = L0.down->C;
  a.To = L0.o->T;
  a.Tgu = L0.gu->T;
  a.Tq = L0.qkv->T;
  a.mw = m->ps.mw;
  a.kq = m->ps.kq;
  a.cq = (a.Cx + a.kq - 1) / a.kq;
  a.ko = m->ps.ko;
  a.co = (a.Co + a.ko - 1) / a.ko;
  a.ks = m->ps.ks;
  a.cs = (a.Cd + a.ks - 1) / a.ks;
  a.eps = (float)d.rms_eps;
  a.scale = m->attn.scale;
  a.ctrl = m->ctrl;
  a.emb = m->emb;
  a.emb_f32 = d.embed_fmt == TLM_FMT_F32 ? 1 : 0;
  a.rope_cos = m->attn.rope_cos;
  a.rope_sin = m->attn.rope_sin;
  a.pub_x = m->ps_pub_x;
  a.pub_qkv = m->ps_pub_qkv;
  a.pub_o = m->ps_pub_o;
  a.pub_xm = m->ps_pub_xm;
  a.pub_h = m->ps_pub_h;
  a.xcc = m->ps_l2_items > 0 ? m->ps_xcc : nullptr;
  // TLM_PS_TIMEOUT_US / TLM_PS_FAIL_LAYER: a shorter bound of every wait and a
  // layer whose QKV stage reports a time-out (tests of the failure path)
  a.timeout = kPsTimeoutTicks;
  a.fail_layer = -1;
  if (const char* e = getenv("TLM_PS_TIMEOUT_US")) a.timeout = std::max(1LL, atoll(e)) * 100;  // 100 MHz clock
  if (const char* e = getenv("TLM_PS_FAIL_LAYER")) a.fail_layer = atoi(e);
  return a;
}

// The persistent schedule of a model whose shape has a compiled variant
// (TLM_PERSISTENT=0 turns it off): the device table of layer pointers, the
// handoff buffers (zeroed: token number 0 never matches) and ctrl[C_SEQ] = 1.
static int ps_setup(tlm_model* m) {
  const tlm_model_desc& d = m->d;
  const char* env = getenv("TLM_PERSISTENT");
  if (env && env[0] == '0') return TLM_OK;
  const int H = d.hidden_size, L = d.num_layers;
  const Layer& L0 = m->layers[0];
  m->ps = ps_shape(wfmt(d.linear_fmt), d.kv_fmt == TLM_FMT_F32 ? 1 : 0, H, d.intermediate_size, d.head_dim,
                   d.num_heads, d.num_kv_heads, m->ctx->cus);
  if (!m->ps.dt) return TLM_OK;
  m->ps_blocks = m->ctx->cus;
  std::vector<int> roles((size_t)2 * kPsRoles * m->ps_blocks);
  if (!ps_roles(m->ps, m->ps_blocks, H, d.num_heads, d.num_kv_heads, L0.gu->T, roles.data())) {
    m->ps = PsShape{};
    return TLM_OK;
  }
  // handoffs through an XCD's L2 where a producer's consumers share its XCD
  // (TLM_PS_L2=0: every handoff device-scope, for comparisons)
  std::vector<int> xcc(m->ps_blocks);
  const char* l2e = getenv("TLM_PS_L2");
  if (!(l2e && l2e[0] == '0') && ps_xcc_probe(m->ps_blocks, xcc.data()))
    m->ps_l2_items = ps_localize(m->ps, m->ps_blocks, d.num_heads, d.num_kv_heads, L0.o->T, xcc.data(), roles.data());
  m->ps.l2 = m->ps_l2_items > 0 ? 1 : 0;
  m->ps_smem = ps_smem_bytes(m->ps, H, m->QS);
  if (!ps_prepare(m->ps, m->ps_smem)) {
    m->ps = PsShape{};
    return TLM_OK;
  }
  std::vector<PsLayer> tab(L);
  for (int l = 0; l < L; l++) {
    const Layer& Ly = m->layers[l];
    PsLayer& t = tab[l];
    t.wqkv = Ly.qkv->w;
    t.sqkv = Ly.qkv->s;
    t.bqkv = Ly.bqkv ? Ly.bqkv : m->attn.zero_bias;
    t.attn_norm = Ly.attn_norm;
    t.wo = Ly.o->w;
    t.so = Ly.o->s;
    t.wgu = Ly.gu->w;
    t.sgu = Ly.gu->s;
    t.ffn_norm = Ly.ffn_norm;
    t.wd = Ly.down->w;
    t.sd = Ly.down->s;
    t.kc = Ly.kc;
    t.vc = Ly.vc;
    t.window = m->windows[l];
  }
  const size_t w8 = sizeof(unsigned long long);
  int rc = model_alloc((void**)&m->ps_layers, sizeof(PsLayer) * L);
  if (!rc) rc = model_alloc((void**)&m->ps_roles, sizeof(int) * roles.size());
  if (!rc) rc = model_alloc((void**)&m->ps_pub_x, w8 * L * kPsMaxKs * H);
  if (!rc) rc = model_alloc((void**)&m->ps_pub_qkv, w8 * L * m->ps.kq * m->Nqkv);
  if (!rc) rc = model_alloc((void**)&m->ps_pub_o, w8 * L * m->QS);
  if (!rc) rc = model_alloc((void**)&m->ps_pub_xm, w8 * L * m->ps.ko * H);
  if (!rc) rc = model_alloc((void**)&m->ps_pub_h, w8 * L * L0.gu->T * 32);
  if (!rc) rc = model_alloc((void**)&m->ps_xcc, sizeof(int) * m->ps_blocks);
  if (rc) return rc;
  HIP_TRY(hipMemcpy(m->ps_xcc, xcc.data(), sizeof(int) * m->ps_blocks, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(m->ps_layers, tab.data(), sizeof(PsLayer) * L, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(m->ps_roles, roles.data(), sizeof(int) * roles.size(), hipMemcpyHostToDevice));
  const int seq = 1;  // the buffers are zero: token number 0 never matches
  HIP_TRY(hipMemcpy(m->ctrl + C_SEQ, &seq, sizeof(int), hipMemcpyHostToDevice));
  m->ps_on = true;
  rc = model_alloc((void**)&m->ps_args_dev, sizeof(PsArgs));
  if (rc) return rc;
  const PsArgs a = ps_args(m);
  HIP_TRY(hipMemcpy(m->ps_args_dev, &a, sizeof a, hipMemcpyHostToDevice));
  return ps_register(m, true);
}

int tlm_model_create(tlm_ctx* ctx, const tlm_model_desc* d, tlm_model** out) {
  if (!ctx || !d || !out) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  if (d->hidden_size <= 0 || d->intermediate_size <= 0 || d->num_layers <= 0 || d->vocab_size <= 0 ||
      d->max_tokens <= 0)
    return fail(TLM_ERR_INVALID, "TLMModel: invalid dimensions");
  if (d->hidden_size > 4096) return fail(TLM_ERR_INVALID, "TLMModel: hidden size above 4096 is not supported");
  if (d->linear_fmt != TLM_FMT_Q4 && d->linear_fmt != TLM_FMT_F16)
    return fail(TLM_ERR_INVALID, "TLMModel: linear_fmt must be q4 or fp16");
  if (d->embed_fmt != TLM_FMT_F16 && d->embed_fmt != TLM_FMT_F32)
    return fail(TLM_ERR_INVALID, "TLMModel: embed_fmt must be fp16 or fp32");
  if (d->tied && d->embed_fmt != TLM_FMT_F16)
    return fail(TLM_ERR_INVALID, "TLMModel: a tied head needs an fp16 embedding table");
  if (!d->tied && d->head_fmt != TLM_FMT_F16 && d->head_fmt != TLM_FMT_Q4)
    return fail(TLM_ERR_INVALID, "TLMModel: head_fmt must be fp16 or q4");
  if (d->hidden_size % 4 != 0)
    return fail(TLM_ERR_INVALID, "TLMModel: hidden_size %d must be a multiple of 4", d->hidden_size);
  if (d->sliding_window < 0) return fail(TLM_ERR_INVALID, "TLMModel: negative sliding window");
  for (int l = 0; d->layer_windows && l < d->num_layers; l++)
    if (d->layer_windows[l] < 0) return fail(TLM_ERR_INVALID, "TLMModel: negative sliding window of layer %d", l);
  tlm_model* m = new tlm_model();
  m->ctx = ctx;
  m->d = *d;
  m->d.layer_windows = nullptr;  // borrowed by the call only: copied here
  m->windows.assign(d->num_layers, d->sliding_window);
  if (d->layer_windows) m->windows.assign(d->layer_windows, d->layer_windows + d->num_layers);
  // the model-wide attention mode and chunk plans follow the widest window (0: full)
  bool full = false;
  int wmax = 0;
  for (int w : m->windows) full |= w == 0, wmax = std::max(wmax, w);
  const int widest = full ? 0 : wmax;
  const int H = d->hidden_size, I = d->intermediate_size, D = d->head_dim;
  m->QS = d->num_heads * D;
  m->Nqkv = m->QS + 2 * d->num_kv_heads * D;
  tlm_attn_desc ad{};
  ad.heads = d->num_heads;
  ad.kv_heads = d->num_kv_heads;
  ad.head_dim = D;
  ad.max_tokens = d->max_tokens;
  ad.rotary_dim = d->rotary_dim;
  ad.sliding_window = widest;
  ad.kv_fmt = d->kv_fmt == TLM_FMT_F32 ? TLM_FMT_F32 : TLM_FMT_F16;
  ad.inv_freq = d->inv_freq;
  ad.attention_factor = d->attention_factor;
  ad.attn_scale = d->attn_scale;  // DecoderCPURunner.ts:152 (recipe.attnScale)
  int rc = attn_init(ctx, &ad, &m->attn, false);
#define M_TRY(x)               \
  do {                         \
    if (rc == TLM_OK) rc = (x); \
  } while (0)
  const int lf = d->linear_fmt;
  m->layers.resize(d->num_layers);
  const size_t esz = ad.kv_fmt == TLM_FMT_F32 ? 4 : 2;
  const size_t cache = (size_t)d->num_kv_heads * d->max_tokens * D * esz;
  for (auto& L : m->layers) {
    M_TRY(linear_alloc(ctx, lf, m->Nqkv, H, false, &L.qkv));
    M_TRY(linear_alloc(ctx, lf, H, m->QS, false, &L.o));
    M_TRY(linear_alloc(ctx, lf, 2 * I, H, false, &L.gu, true));
    M_TRY(linear_alloc(ctx, lf, H, I, false, &L.down));
    if (rc == TLM_OK) rms_waves(L.qkv);
    M_TRY(model_alloc((void**)&L.attn_norm, sizeof(float) * H));
    M_TRY(model_alloc((void**)&L.ffn_norm, sizeof(float) * H));
    if (d->qkv_bias) M_TRY(model_alloc((void**)&L.bqkv, sizeof(float) * m->Nqkv));
    M_TRY(model_alloc(&L.kc, cache));
    M_TRY(model_alloc(&L.vc, cache));
  }
  M_TRY(model_alloc(&m->emb, (size_t)d->vocab_size * H * (d->embed_fmt == TLM_FMT_F32 ? 4 : 2)));
  M_TRY(linear_alloc(ctx, d->tied ? TLM_FMT_F16 : d->head_fmt, d->vocab_size, H, true, &m->head));
  M_TRY(model_alloc((void**)&m->final_norm, sizeof(float) * H));
  M_TRY(model_alloc((void**)&m->ctrl, sizeof(int) * 8));
  M_TRY(model_alloc((void**)&m->tokens_out, sizeof(int) * d->max_tokens));
  M_TRY(model_alloc((void**)&m->prompt, sizeof(int) * d->max_tokens));
  if (rc == TLM_OK && hipHostMalloc((void**)&m->host_pin, sizeof(int) * (kPinPrompt + d->max_tokens),
                                    hipHostMallocDefault) != hipSuccess) {
    m->host_pin = nullptr;
    rc = fail(TLM_ERR_HIP, "TLMModel: pinned host buffer allocation failed");
  }
  M_TRY(model_alloc((void**)&m->xa, sizeof(float) * H));
  m->nrep = rep_count(H);
  M_TRY(model_alloc((void**)&m->x0, sizeof(unsigned long long) * kRep * H));
  M_TRY(model_alloc((void**)&m->rb, sizeof(unsigned long long) * kRep * H * d->num_layers));
  M_TRY(model_alloc((void**)&m->xf, sizeof(float) * H));
  M_TRY(model_alloc((void**)&m->attn_out, sizeof(float) * m->QS));
  if (rc == TLM_OK) {
    const Layer& L0 = m->layers[0];
    M_TRY(model_alloc((void**)&m->pq, sizeof(float) * L0.qkv->plan.splits * m->Nqkv));
    M_TRY(model_alloc((void**)&m->po, sizeof(float) * L0.o->plan.splits * H));
    // fused MLP: kMlpWaves waves; gate|up chunks and down (tile, chunk) items
    // a wave loads per batch.  Small batches: each wave then gets past its
    // loads (the memory pipeline stalls a wave that issues more than it takes)
    // and into the norm sooner, and the rest of its chunks stream through the
    // loop.  Measured (tok/s), gate|up batch + down batch: Llama-3.2-3B at
    // 16384 positions 713 with 8 + 4, 744 with 2 + 1, 749 with 1 + 1 (A/B
    // again: 1339.7 against 1344.5 us per token); Llama-3.2-1B at 4096 1908
    // with 4 + 4, 1960 with 2 + 1 or 1 + 1; Qwen2.5-0.5B per-stage graph 2263
    // with 2 + 1, 2249 with 1 + 1.  One chunk from six chunks per wave up.
    const int per = (L0.gu->C + kMlpWaves - 1) / kMlpWaves;
    m->mlp_nch = per <= 1 || per >= 6 ? 1 : 2;
    m->mlp_ndb = 1;
    if (mlp_smem_bytes(wfmt(lf), L0.gu->C, H) > 65536)
      rc = fail(TLM_ERR_INVALID, "TLMModel: hidden size %d too large for the fused MLP block", H);
    m->lm_plan = plan_gemv(m->head->T, m->head->C, ctx->cus, chunk_k(m->head->fmt), true);
    m->lm_plan.gx = lm_head_grid(m->head->T, ctx->cus);
    {  // a wave's row slice in batches of 4 chunks: a wave that issues more
      // loads than the memory pipeline takes stalls at issue.  Per launch
      // against the whole slice in one batch: Llama-3.2-1B (32 chunks, batches
      // of 16) 91.1 -> 83.1 us, 87.3 at 8; Qwen2.5-0.5B (14 chunks) 44.3 ->
      // 43.4-43.7 us; Llama-3.2-3B (48 chunks) 120 us at 4, 8 or 16
      const int per = (m->head->C + m->lm_plan.waves - 1) / m->lm_plan.waves;
      m->lm_plan.nch = per <= 1 ? 1 : per <= 2 ? 2 : 4;
    }
    if (gemv_smem_bytes(wfmt(m->head->fmt), m->lm_plan.cps, m->lm_plan.waves) > 65536)
      rc = fail(TLM_ERR_INVALID, "TLMModel: hidden size %d too large for one LM head block", H);
  }
  M_TRY(model_alloc((void**)&m->logits, sizeof(float) * d->vocab_size));
  M_TRY(model_alloc((void**)&m->arg_val, sizeof(float) * 4096));
  M_TRY(model_alloc((void**)&m->arg_idx, sizeof(int) * 4096));
  M_TRY(model_alloc((void**)&m->arg_key, sizeof(unsigned long long)));
  M_TRY(model_alloc((void**)&m->arg_arrived, sizeof(unsigned)));
  M_TRY(model_alloc((void**)&m->cand_v, sizeof(float) * kTopkMax));
  M_TRY(model_alloc((void**)&m->cand_i, sizeof(int) * kTopkMax));
  if (rc == TLM_OK) rc = ps_setup(m);
#undef M_TRY
  if (rc) {
    std::string msg = g_error;
    tlm_model_destroy(m);
    g_error = msg;
    return rc;
  }
  *out = m;
  return TLM_OK;
}

void tlm_model_destroy(tlm_model* m) {
  if (!m) return;
  hipStreamSynchronize(m->ctx->stream);
  ps_register(m, false);
  for (auto* gm : {&m->pf_graphs, &m->replay_graphs})
    for (auto& kv : *gm) {
      hipGraphExecDestroy(kv.second.second);
      hipGraphDestroy(kv.second.first);
    }
  for (int i = 0; i < 2; i++) {
    if (m->g_logits[i]) hipGraphExecDestroy(m->g_logits[i]);
    if (m->g_prefill[i]) hipGraphExecDestroy(m->g_prefill[i]);
    if (m->g_layers[i]) hipGraphExecDestroy(m->g_layers[i]);
    if (m->graph_layers[i]) hipGraphDestroy(m->graph_layers[i]);
    if (m->graph_logits[i]) hipGraphDestroy(m->graph_logits[i]);
    if (m->graph_prefill[i]) hipGraphDestroy(m->graph_prefill[i]);
  }
  for (auto& L : m->layers) {
    tlm_linear_destroy(L.qkv);
    tlm_linear_destroy(L.o);
    tlm_linear_destroy(L.gu);
    tlm_linear_destroy(L.down);
    hipFree(L.attn_norm);
    hipFree(L.ffn_norm);
    hipFree(L.bqkv);
    hipFree(L.kc);
    hipFree(L.vc);
  }
  tlm_linear_destroy(m->head);
  attn_free(&m->attn, false);
  void* bufs[] = {m->emb, m->final_norm, m->ctrl, m->tokens_out, m->prompt, m->xa, m->x0, m->xf, m->attn_out,
                  m->pq, m->po, m->rb, m->logits, m->arg_val, m->arg_idx, m->arg_key, m->arg_arrived, m->cand_v, m->cand_i, m->pf_x, m->pf_part, m->pf_xn,
                  m->pf_q, m->pf_att, m->pf_h, m->pf_ex, m->pf_ss, m->pf_ovf, m->ps_layers, m->ps_roles, m->ps_pub_x, m->ps_pub_qkv,
                  m->ps_pub_o, m->ps_pub_xm, m->ps_pub_h, m->ps_args_dev, m->ps_xcc};
  for (void* p : bufs) hipFree(p);
  if (m->host_pin) hipHostFree(m->host_pin);
  delete m;
}

static int upload_f32(float* dst, const void* host, size_t bytes, size_t expect, const char* what) {
  if (bytes != expect) return fail(TLM_ERR_INVALID, "TLMModel: %s expects %zu bytes, got %zu", what, expect, bytes);
  HIP_TRY(hipMemcpy(dst, host, bytes, hipMemcpyHostToDevice));
  return TLM_OK;
}

static int upload_linear(tlm_linear* L, int r0, int rows, int cols, bool scales, const void* host, size_t bytes,
                         const char* what) {
  if (L->fmt == TLM_FMT_Q4) {
    const size_t expect = scales ? (size_t)rows * (cols / 32) * 2 : (size_t)rows * cols / 2;
    if (bytes != expect) return fail(TLM_ERR_INVALID, "TLMModel: %s expects %zu bytes, got %zu", what, expect, bytes);
    return scales ? linear_write_rows(L, r0, rows, nullptr, (const uint16_t*)host)
                  : linear_write_rows(L, r0, rows, host, nullptr);
  }
  if (scales) return fail(TLM_ERR_INVALID, "TLMModel: %s: fp16 linears have no scales", what);
  const size_t expect = (size_t)rows * cols * 2;
  if (bytes != expect) return fail(TLM_ERR_INVALID, "TLMModel: %s expects %zu bytes, got %zu", what, expect, bytes);
  return linear_write_rows(L, r0, rows, host, nullptr);
}

int tlm_model_upload(tlm_model* m, int tensor, int layer, const void* host, size_t bytes) {
  if (!m || !host) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  const tlm_model_desc& d = m->d;
  const int H = d.hidden_size, I = d.intermediate_size, V = d.vocab_size;
  const bool per_layer = tensor >= TLM_T_ATTN_NORM;
  if (per_layer && (layer < 0 || layer >= d.num_layers))
    return fail(TLM_ERR_INVALID, "TLMModel: layer %d outside [0, %d)", layer, d.num_layers);
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  Layer* L = per_layer ? &m->layers[layer] : nullptr;
  switch (tensor) {
    case TLM_T_EMBED: {
      const size_t esz = d.embed_fmt == TLM_FMT_F32 ? 4 : 2;
      if (bytes != (size_t)V * H * esz)
        return fail(TLM_ERR_INVALID, "TLMModel: embedding expects %zu bytes, got %zu", (size_t)V * H * esz, bytes);
      HIP_TRY(hipMemcpy(m->emb, host, bytes, hipMemcpyHostToDevice));
      if (d.tied) return linear_write_rows(m->head, 0, V, host, nullptr);
      return TLM_OK;
    }
    case TLM_T_LM_HEAD:
    case TLM_T_LM_HEAD_SCALES:
      if (d.tied) return fail(TLM_ERR_STATE, "TLMModel: the LM head is tied to the embedding");
      return upload_linear(m->head, 0, V, H, tensor == TLM_T_LM_HEAD_SCALES, host, bytes, "lm_head");
    case TLM_T_FINAL_NORM: return upload_f32(m->final_norm, host, bytes, sizeof(float) * H, "final norm");
    case TLM_T_ATTN_NORM: return upload_f32(L->attn_norm, host, bytes, sizeof(float) * H, "attn norm");
    case TLM_T_FFN_NORM: return upload_f32(L->ffn_norm, host, bytes, sizeof(float) * H, "ffn norm");
    case TLM_T_WQKV:
    case TLM_T_WQKV_SCALES:
      return upload_linear(L->qkv, 0, m->Nqkv, H, tensor == TLM_T_WQKV_SCALES, host, bytes, "wqkv");
    case TLM_T_BQKV:
      if (!d.qkv_bias) return fail(TLM_ERR_STATE, "TLMModel: model was created without a QKV bias");
      return upload_f32(L->bqkv, host, bytes, sizeof(float) * m->Nqkv, "bqkv");
    case TLM_T_WO:
    case TLM_T_WO_SCALES: return upload_linear(L->o, 0, H, m->QS, tensor == TLM_T_WO_SCALES, host, bytes, "wo");
    case TLM_T_WGATE:
    case TLM_T_WGATE_SCALES:
      return upload_linear(L->gu, 0, I, H, tensor == TLM_T_WGATE_SCALES, host, bytes, "wgate");
    case TLM_T_WUP:
    case TLM_T_WUP_SCALES: return upload_linear(L->gu, I, I, H, tensor == TLM_T_WUP_SCALES, host, bytes, "wup");
    case TLM_T_WDOWN:
    case TLM_T_WDOWN_SCALES:
      return upload_linear(L->down, 0, H, I, tensor == TLM_T_WDOWN_SCALES, host, bytes, "wdown");
  }
  return fail(TLM_ERR_INVALID, "TLMModel: unknown tensor id %d", tensor);
}

// ----------------------------------------------------- the per-token schedule

static EmbStage emb_stage(const tlm_model* m) {
  return EmbStage{m->emb, m->d.embed_fmt == TLM_FMT_F32 ? 1 : 0, m->d.hidden_size, m->x0};
}

// The host's token/position write (step 0), which also stages the token's
// embedding row.
static void set_ctrl(tlm_model* m, int token, int pos, int base, int len, hipStream_t st) {
  launch_set_ctrl(m->ctrl, token, pos, 0, base, len, emb_stage(m), st);
  m->x0_stale = false;
}

// Before a step on the per-stage graph: the embedding row of the token that a
// persistent step chose (its LM head and prefill advance do not stage it).
static void stage_x0(tlm_model* m, hipStream_t st) {
  if (!m->x0_stale) return;
  launch_stage_ctrl(m->ctrl, emb_stage(m), st);
  m->counts.kernel_launches++;
  m->x0_stale = false;
}

// Kernels of one layer.  which: -1 all; otherwise a single stage (timing).
static bool enqueue_layer(tlm_model* m, int l, hipStream_t st, int which, bool long_win) {
  bool ok = true;
  const tlm_model_desc& d = m->d;
  const int H = d.hidden_size, I = d.intermediate_size;
  Layer& L = m->layers[l];
  const int nl = d.num_layers;
  const size_t rstride = (size_t)kRep * H;
  // this layer's window (DecoderCPURunner.ts:150): at a long-window position a
  // layer whose own window spans at most kLongWindow positions stays on the
  // short-window kernels
  const int win = m->windows[l];
  long_win = long_win && (win == 0 || win > kLongWindow);
  // 1. x = residual accumulator (layer 0: the staged embedding row); RMSNorm;
  //    QKV GEMV.  Block (0,0) stores x for the MLP.
  if (which < 0 || which == 4) {
    GemvArgs a;
    fill_gemv_args(a, L.qkv, m->pq);
    a.acc_in = l == 0 ? m->x0 : m->rb + (size_t)(l - 1) * rstride;
    a.ctrl = m->ctrl;
    a.norm_w = L.attn_norm;
    a.eps = (float)d.rms_eps;
    a.xout = m->xa;
    ok &= launch_linear(L.qkv, m->nrep == 2 ? PRO_RMSFH : PRO_RMSF, a, st);
    m->counts.kernel_launches++;
  }
  // 2. RoPE + KV append + split-K attention
  if (which < 0 || which == 1) {
    AttnArgs a = attn_args(&m->attn, m->pq, L.qkv->plan.splits, m->Nqkv, L.bqkv, m->ctrl, L.kc, L.vc, m->attn_out,
                           long_win);
    a.window = win;
    ok &= launch_attention(d.kv_fmt == TLM_FMT_F32, m->attn.gmax, a, false, long_win, st);
    m->counts.kernel_launches++;
  }
  // 3. O projection; its prologue combines the attention chunk partials
  if (which < 0 || which == 5) {
    GemvArgs a;
    fill_gemv_args(a, L.o, m->po);
    a.ctrl = m->ctrl;
    a.pacc = m->attn.pacc;
    a.pml = m->attn.pml;
    a.att_D = d.head_dim;
    a.att_nsplit = long_win ? m->attn.nsplit_long : m->attn.nsplit;
    a.att_chmin = long_win ? m->attn.chmin_long : m->attn.chmin;
    a.att_window = win;
    a.att_max_tokens = d.max_tokens;
    // the accumulator layer l - 1 produced was last read by this layer's QKV
    // (layer 0: the previous token's final norm): clear it for its next use
    a.zero_ptr = m->rb + (size_t)((l + nl - 1) % nl) * rstride;
    a.zero_n = m->nrep * H;
    // more than 16 long-window chunks: the 32-slot combine keeps it to one round trip
    ok &= launch_linear(L.o, long_win && a.att_nsplit > 16 ? PRO_ATTN3 : PRO_ATTN, a, st);
    m->counts.kernel_launches++;
  }
  // 4. x_mid = x + O partials; RMSNorm; gate|up; SwiGLU; down, accumulated
  //    with x_mid into rb[l]
  if (which < 0 || which == 2) {
    MlpArgs a;
    fill_gemv_args(a.g, L.gu, nullptr);
    a.g.base = m->xa;
    a.g.pin = m->po;
    a.g.n_pin = L.o->plan.splits;
    a.g.pin_stride = H;
    a.g.norm_w = L.ffn_norm;
    a.g.eps = (float)d.rms_eps;
    a.g.ctrl = m->ctrl;
    a.wd = L.down->w;
    a.sd = L.down->s;
    a.Td = L.down->T;
    a.Cd = L.down->C;
    a.H = H;
    a.acc = m->rb + (size_t)l * rstride;
    a.nrep = m->nrep;
    ok &= launch_mlp(wfmt(L.gu->fmt), m->mlp_nch, m->mlp_ndb, L.gu->T, a, st);
    m->counts.kernel_launches++;
  }
  (void)I;
  return ok;
}

// LM head with the final RMSNorm in its prologue (every block normalises the
// last layer's residual accumulator; block 0 stores the result for
// readHidden) and the first argmax pass fused in, then the argmax merge.
// `ev` (optional) brackets the LM head kernel with two events.
static bool enqueue_head(tlm_model* m, hipStream_t st, bool advance, hipEvent_t* ev = nullptr, bool ps = false) {
  const tlm_model_desc& d = m->d;
  GemvArgs a;
  fill_gemv_args(a, m->head, nullptr);
  a.cps = m->lm_plan.cps;
  a.acc_in = m->rb + (size_t)(d.num_layers - 1) * kRep * d.hidden_size;
  int pro = m->nrep == 2 ? PRO_RMSFH : PRO_RMSF;
  if (ps) {  // the persistent schedule's last residual: the published down partials
    static_assert(kPsMaxKs == kRep, "the LM head prologue folds kRep partials");
    a.acc_in = m->ps_pub_x + (size_t)(d.num_layers - 1) * kPsMaxKs * d.hidden_size;
    pro = PRO_RMSF;
    a.ps_words = 1;
  }
  a.norm_w = m->final_norm;
  a.eps = (float)d.rms_eps;
  a.ctrl = m->ctrl;  // fixed-point range flag of the residual it reads
  a.xnorm = m->xf;
  a.logits = m->logits;
  a.arg_val = m->arg_val;
  a.arg_idx = m->arg_idx;
  a.arg_key = m->arg_key;  // the blocks fold their bests as they finish
  // after a persistent step the head's last block also does the merge
  // (TLM_HEAD_MERGE=0: greedy_pick_kernel, comparisons)
  static const bool merge_in_head = [] {
    const char* e = getenv("TLM_HEAD_MERGE");
    return !(e && e[0] == '0');
  }();
  const bool in_head = ps && advance && merge_in_head;
  if (in_head) {
    a.arrived = m->arg_arrived;
    a.mctrl = m->ctrl;
    a.tokens_out = m->tokens_out;
    a.max_steps = d.max_tokens;
  }
  if (ev) hipEventRecord(ev[0], st);
  if (!launch_lm_head(wfmt(m->head->fmt), pro, m->lm_plan.waves, m->lm_plan.nch, dim3(m->lm_plan.gx), a, st))
    return false;
  if (ev) hipEventRecord(ev[1], st);
  if (in_head) {
    m->x0_stale = true;  // the persistent kernel reads its token's row itself
    m->counts.kernel_launches++;
    return true;
  }
  // the persistent kernel reads its token's embedding row itself: the row is
  // staged only before a step on the per-stage graph (stage_x0)
  launch_greedy_pick(m->arg_key, m->ctrl, advance ? m->tokens_out : nullptr, advance ? 1 : 0, d.max_tokens,
                     ps ? EmbStage{} : emb_stage(m), st, ps ? 1 : 0);
  m->x0_stale = ps;
  m->counts.kernel_launches += 2;
  return true;
}

// One token of the persistent schedule, then its tail: the LM head and the
// argmax merge, or the prefill advance.
static bool enqueue_ps(tlm_model* m, hipStream_t st, int tail) {
  if (!launch_ps_token(m->ps, m->ps_blocks, m->ps_smem, m->ps_args_dev, st)) return false;
  m->counts.kernel_launches++;
  if (tail == 1) return enqueue_head(m, st, true, nullptr, true);
  launch_prefill_advance(m->ctrl, m->prompt, EmbStage{}, st, 1);
  m->x0_stale = true;
  m->counts.kernel_launches++;
  return true;
}

// Graph tails: the decode/logits step, the prefill step, or the layers alone
// (LM head timing).
enum GraphTail { TAIL_PREFILL = 0, TAIL_LOGITS = 1, TAIL_NONE = 2 };

// (Kernels recorded into a graph are not handed to the stream: the capture
// functions leave the model's counts and x0 state as they found them.)
static int capture(tlm_model* m, int tail, bool long_win, hipGraph_t* g, hipGraphExec_t* ge) {
  hipStream_t st = m->ctx->stream;
  const tlm_model_counts kept = m->counts;
  const bool stale = m->x0_stale;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  bool ok = true;
  for (int l = 0; l < m->d.num_layers; l++) ok &= enqueue_layer(m, l, st, -1, long_win);
  if (tail == TAIL_LOGITS)
    ok &= enqueue_head(m, st, true);
  else if (tail == TAIL_PREFILL)
    launch_prefill_advance(m->ctrl, m->prompt, emb_stage(m), st);
  m->counts = kept;
  m->x0_stale = stale;
  hipError_t le = hipGetLastError();
  HIP_TRY(hipStreamEndCapture(st, g));
  if (le != hipSuccess) return fail(TLM_ERR_HIP, "TLMModel: launch during capture failed: %s", hipGetErrorString(le));
  if (!ok) return fail(TLM_ERR_STATE, "TLMModel: no kernel variant for a stage of this model");
  HIP_TRY(hipGraphInstantiate(ge, *g, nullptr, nullptr, 0));
  return TLM_OK;
}

int tlm_model_finalize(tlm_model* m) {
  if (!m) return fail(TLM_ERR_INVALID, "TLMModel: null model");
  if (m->finalized) return TLM_OK;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  const char* env = getenv("TLM_GRAPHS");
  m->use_graphs = !(env && env[0] == '0');
  if (!m->use_graphs) {
    m->finalized = true;
    return TLM_OK;
  }
  int rc = TLM_OK;
  for (int lw = 0; lw < 2 && !rc; lw++) {
    rc = capture(m, TAIL_LOGITS, lw, &m->graph_logits[lw], &m->g_logits[lw]);
    if (rc == TLM_OK) rc = capture(m, TAIL_PREFILL, lw, &m->graph_prefill[lw], &m->g_prefill[lw]);
  }
  if (rc) return rc;
  m->finalized = true;
  return TLM_OK;
}

// One token of the schedule at position pos: the captured graph of its
// attention mode, or the same kernels enqueued directly.
static int run_token(tlm_model* m, bool logits, int pos) {
  hipStream_t st = m->ctx->stream;
  const bool lw = long_window(&m->attn, pos);
  m->host_pos = pos;
  kv_touch(m, (long)pos + 1);
  if (m->ps_on && !m->ps_suspend && !lw) {  // the persistent schedule
    // its two kernels enqueued directly: a graph launch of the same pair costs
    // ~4.6 us more per token here (Qwen2.5-0.5B decode: 328.3 -> 323.7 us)
    m->counts.persistent_tokens++;
    return ps_ordered(m, [&]() -> int {
      if (!enqueue_ps(m, st, logits ? 1 : 0)) return fail(TLM_ERR_STATE, "TLMModel: no persistent kernel variant");
      CHECK_LAUNCH("TLMModel");
      return TLM_OK;
    });
  }
  stage_x0(m, st);
  if (m->use_graphs) {
    HIP_TRY(hipGraphLaunch(logits ? m->g_logits[lw] : m->g_prefill[lw], st));
    m->counts.graph_launches++;
    return TLM_OK;
  }
  bool ok = true;
  for (int l = 0; l < m->d.num_layers; l++) ok &= enqueue_layer(m, l, st, -1, lw);
  if (logits) {
    ok &= enqueue_head(m, st, true);
  } else {
    launch_prefill_advance(m->ctrl, m->prompt, emb_stage(m), st);
    m->counts.kernel_launches++;
  }
  if (!ok) return fail(TLM_ERR_STATE, "TLMModel: no kernel variant for a stage of this model");
  CHECK_LAUNCH("TLMModel");
  return TLM_OK;
}

static int check_token(tlm_model* m, int32_t token, int32_t position) {
  if (token < 0 || token >= m->d.vocab_size)
    return fail(TLM_ERR_RANGE, "TLMModel: token %d outside [0, %d)", token, m->d.vocab_size);
  if (position < 0 || position >= m->d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMModel: position %d outside [0, %d)", position, m->d.max_tokens);
  return TLM_OK;
}

// Logs a run of n tokens from (token, pos) for ps_recover (models with the
// persistent schedule only; not while recomputing).
static void redo_log(tlm_model* m, int32_t token, int32_t pos, int32_t n, bool logits, bool device) {
  if (!m->ps_on || m->ps_suspend || m->redo_lost || n <= 0) return;
  if (m->redo.size() >= kRedoMax) {
    m->redo.clear();
    m->redo_lost = true;
    return;
  }
  m->redo.push_back(RedoEntry{token, pos, n, logits, device});
}

int tlm_compute_token(tlm_model* m, int32_t token, int32_t position, int flags) {
  if (!m) return fail(TLM_ERR_INVALID, "TLMModel: null model");
  int rc = check_token(m, token, position);
  if (rc) return rc;
  rc = tlm_model_finalize(m);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  set_ctrl(m, token, position, 0, 0, st);  // the token/position write
  m->counts.kernel_launches++;
  CHECK_LAUNCH("TLMModel");
  redo_log(m, token, position, 1, (flags & TLM_LOGITS) != 0, false);
  return run_token(m, (flags & TLM_LOGITS) != 0, position);
}

// Why the batched prefill cannot serve this model (null: it can).
static const char* prefill_unsupported(const tlm_model* m) {
  const tlm_model_desc& d = m->d;
  const int H = d.hidden_size, I = d.intermediate_size;
  if (d.linear_fmt != TLM_FMT_Q4 && d.linear_fmt != TLM_FMT_F16) return "linears are neither q4 nor fp16";
  if (d.kv_fmt == TLM_FMT_F32) return "the fp32 KV cache";
  if (d.head_dim != 64 && d.head_dim != 128) return "head_dim other than 64 or 128";
  if (H % 32 || I % 32 || m->QS % 32) return "hidden, intermediate and q sizes must be multiples of 32";
  // fp16 dequantised weights: (code - 8) * s must stay finite, 8 s <= 65504
  for (const Layer& L : m->layers)
    for (const tlm_linear* lin : {L.qkv, L.o, L.gu, L.down})
      if (lin->fmt == TLM_FMT_Q4 && lin->smax > 0x6FFF) return "a q4 scale above 8188 (fp16 overflow)";
  return nullptr;
}

// Row buffers for `rows` positions and `part` floats of split-K slices.
static int prefill_alloc(tlm_model* m, int rows, size_t part) {
  if (!m->pf_ovf) {
    int rc = model_alloc((void**)&m->pf_ovf, sizeof(int));
    if (rc) return rc;
  }
  if (m->pf_cap >= rows && m->pf_part_n >= part) return TLM_OK;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (m->pf_part_n < part) {
    hipFree(m->pf_part);
    m->pf_part = nullptr;
    m->pf_part_n = 0;
    int rc = model_alloc((void**)&m->pf_part, sizeof(float) * part);
    if (rc) return rc;
    m->pf_part_n = part;
  }
  if (m->pf_cap >= rows) return TLM_OK;
  rows = std::max(rows, m->pf_chunk);  // one allocation serves every later chunk
  void* bufs[] = {m->pf_x, m->pf_xn, m->pf_q, m->pf_att, m->pf_h, m->pf_ex, m->pf_ss};
  for (void* q : bufs) hipFree(q);
  m->pf_x = nullptr;
  m->pf_xn = m->pf_q = m->pf_att = m->pf_h = nullptr;
  m->pf_ex = nullptr;
  m->pf_ss = nullptr;
  m->pf_cap = 0;
  const size_t R = (size_t)rows, H = m->d.hidden_size, I = m->d.intermediate_size;
  int rc = TLM_OK;
  if (!rc) rc = model_alloc((void**)&m->pf_x, sizeof(float) * R * H);
  if (!rc) rc = model_alloc((void**)&m->pf_xn, 2 * R * H);
  if (!rc) rc = model_alloc((void**)&m->pf_q, 2 * R * m->QS);
  if (!rc) rc = model_alloc((void**)&m->pf_att, 2 * R * m->QS);
  if (!rc) rc = model_alloc((void**)&m->pf_h, 2 * R * I);
  if (!rc) rc = model_alloc((void**)&m->pf_ex, sizeof(int) * R);
  if (!rc) rc = model_alloc((void**)&m->pf_ss, sizeof(float) * R * ((H + kTile - 1) / kTile));
  if (!rc) m->pf_cap = rows;
  return rc;
}

static GemmArgs gemm_args(const tlm_linear* L, const uint16_t* A, int lda, int M) {
  GemmArgs g;
  memset(&g, 0, sizeof g);
  g.A = A;
  g.lda = lda;
  g.M = M;
  g.N = L->N;
  g.K = L->K;
  g.w = L->w;
  g.s = L->s;
  g.C = L->C;
  return g;
}

static RowsArgs rows_args(float* X, const float* part, int n_part, size_t pstride, int H, const float* w, double eps,
                          uint16_t* Y, int* ovf) {
  RowsArgs r;
  r.ovf = ovf;
  r.X = X;
  r.part = part;
  r.n_part = n_part;
  r.pstride = pstride;
  r.H = H;
  r.w = w;
  r.eps = (float)eps;
  r.Y = Y;
  r.ex = nullptr;
  r.emb = nullptr;
  r.emb_f32 = 0;
  r.tokens = nullptr;
  r.ctrl = nullptr;
  return r;
}

// Positions [p0, p0 + M) through every layer as row batches; the K and V rows
// land in the cache, nothing else of the model's decode state changes.
// tokens: device array of the M token ids.  Per layer: fold + RMSNorm rows ->
// QKV GEMM (split-K slices) -> RoPE/cache append (folds the slices) -> flash
// attention -> O GEMM (slices) -> fold + RMSNorm -> gate|up GEMM with SwiGLU ->
// down GEMM (slices, folded by the next layer's first kernel).  Small chunks
// fuse the QKV GEMM with RoPE and the O GEMM with its fold (PfPlan).
// Shapes of a batched chunk of M rows, with its row buffers allocated (on
// first use; never while a graph is being captured).
struct PfPlan {
  GemmShape sq, sr, so, sf, sg, sd;
  bool rope_epi;
  bool fold;  // the O GEMM folds its rows into the residual (GEMM_FOLD): no row kernel after it
};
// TLM_PF_FOLD=0: the row kernel after the O GEMM for every chunk (comparisons)
static const bool g_pf_fold = [] {
  const char* e = getenv("TLM_PF_FOLD");
  return !(e && e[0] == '0');
}();
static int prefill_plan(tlm_model* m, int M, PfPlan* pp) {
  const tlm_model_desc& d = m->d;
  const int H = d.hidden_size, I = d.intermediate_size, D = d.head_dim;
  const int lf = wfmt(d.linear_fmt), cus = m->ctx->cus;
  const Layer& L0 = m->layers[0];
  pp->sq = gemm_shape(lf, GEMM_PART, M, m->Nqkv, H, cus);
  // small chunks (the K-wave QKV GEMM), head_dim 64, full rotary: RoPE and the
  // cache append run in the QKV GEMM's epilogue (no split-K slices, no rope_kv)
  pp->sr = gemm_shape(lf, GEMM_ROPE, M, m->Nqkv, H, cus);
  pp->rope_epi = pp->sr.ring && pp->sr.kw && D == 64 && d.rotary_dim == 64;
  pp->so = gemm_shape(lf, GEMM_PART, M, H, m->QS, cus);
  pp->sg = gemm_shape(lf, GEMM_SWIGLU, M, L0.gu->T * kTile, H, cus);
  pp->sd = gemm_shape(lf, GEMM_PART, M, H, I, cus);
  // small chunks (K-wave O and gate|up GEMMs): the O GEMM, unsplit, adds its
  // rows to the residual and writes the FFN norm's operand as fp16(x w 2^e),
  // e from the attention norm of the same rows (which keeps it near unit
  // scale), with each 64-column tile's sum of squares; the gate|up GEMM then
  // applies the row's rsqrt(mean(x^2) + eps) 2^-e after the dot.  The row
  // kernel between them drops out (127-row Qwen2.5-0.5B chunk: its 24
  // launches were 3.6 us each; the unsplit O GEMM costs 0.4 us more).
  pp->sf = gemm_shape(lf, GEMM_FOLD, M, H, m->QS, cus);
  pp->fold = g_pf_fold && lf == WF_Q4 && pp->sf.ring && pp->sf.kw && pp->sg.ring && pp->sg.kw && H % kTile == 0 &&
             H / kTile <= 32;
  const size_t part = std::max({(size_t)pp->sq.splits * M * m->Nqkv, (size_t)pp->so.splits * M * H,
                                (size_t)pp->sd.splits * M * H});
  return prefill_alloc(m, M, part);
}

// Kernels of one batched chunk of M rows (the counterpart of the reference's
// chunk of replays, DecoderTSLRunner.ts:504-530): the chunk starts at
// position ctrl[C_POS] and its ids are m->prompt[ctrl[C_POS] - ctrl[C_BASE] ...],
// so one captured sequence serves every chunk of M rows.  Returns the kernel
// count (0: no kernel for a layer).
static int prefill_enqueue(tlm_model* m, const PfPlan& pp, int M, hipStream_t st) {
  const tlm_model_desc& d = m->d;
  const int H = d.hidden_size, I = d.intermediate_size, D = d.head_dim;
  const int lf = wfmt(d.linear_fmt);
  const size_t rowsH = (size_t)M * H;
  // per layer: two row kernels (one when the O GEMM folds its rows; layer 0's
  // first one also gathers the embedding rows), the QKV GEMM (+ rope_kv unless
  // RoPE runs in its epilogue), attention and three GEMMs; then the last fold
  for (int l = 0; l < d.num_layers; l++) {
    const Layer& L = m->layers[l];
    bool ok = true;
    RowsArgs ra = rows_args(m->pf_x, m->pf_part, l ? pp.sd.splits : 0, rowsH, H, L.attn_norm, d.rms_eps, m->pf_xn,
                            m->pf_ovf);
    if (pp.fold) ra.ex = m->pf_ex;
    if (l == 0) {  // the residual rows start as the chunk's embedding rows
      ra.emb = m->emb;
      ra.emb_f32 = d.embed_fmt == TLM_FMT_F32;
      ra.tokens = m->prompt;
      ra.ctrl = m->ctrl;
    }
    launch_rms_rows(ra, M, st);
    GemmArgs g = gemm_args(L.qkv, m->pf_xn, H, M);
    g.ovf = m->pf_ovf;
    if (pp.rope_epi) {
      g.bias = L.bqkv;
      g.Ch = m->pf_q;
      g.ldc = m->QS;
      g.rope_cos = m->attn.rope_cos;
      g.rope_sin = m->attn.rope_sin;
      g.ctrl = m->ctrl;
      g.Hq = d.num_heads;
      g.Hkv = d.num_kv_heads;
      g.max_tokens = d.max_tokens;
      g.kc = static_cast<uint16_t*>(L.kc);
      g.vc = static_cast<uint16_t*>(L.vc);
      ok = ok && launch_gemm(lf, GEMM_ROPE, pp.sr, g, st);
    } else {
      g.Cf = m->pf_part;
      g.ldc = m->Nqkv;
      ok = ok && launch_gemm(lf, GEMM_PART, pp.sq, g, st);
      RopeKvArgs r;
      memset(&r, 0, sizeof r);
      r.qkv = m->pf_part;
      r.n_part = pp.sq.splits;
      r.pstride = (size_t)M * m->Nqkv;
      r.bias = L.bqkv;
      r.M = M;
      r.ctrl = m->ctrl;
      r.Hq = d.num_heads;
      r.Hkv = d.num_kv_heads;
      r.D = D;
      r.rd = d.rotary_dim;
      r.max_tokens = d.max_tokens;
      r.rope_cos = m->attn.rope_cos;
      r.rope_sin = m->attn.rope_sin;
      r.q = m->pf_q;
      r.kc = L.kc;
      r.vc = L.vc;
      r.kv_f32 = 0;
      r.ovf = m->pf_ovf;
      launch_rope_kv(r, st);
    }
    PrefillAttnArgs pa;
    memset(&pa, 0, sizeof pa);
    pa.q = m->pf_q;
    pa.kc = L.kc;
    pa.vc = L.vc;
    pa.out = m->pf_att;
    pa.M = M;
    pa.ctrl = m->ctrl;
    pa.Hq = d.num_heads;
    pa.Hkv = d.num_kv_heads;
    pa.D = D;
    pa.G = m->attn.G;
    pa.max_tokens = d.max_tokens;
    pa.window = m->windows[l];
    pa.scale_log2 = m->attn.scale * 1.4426950408889634f;
    ok = ok && launch_prefill_attention(pa, st);
    g = gemm_args(L.o, m->pf_att, m->QS, M);
    g.ldc = H;
    if (pp.fold) {
      g.Cf = m->pf_x;
      g.Ch = m->pf_xn;
      g.nw = L.ffn_norm;
      g.ex = m->pf_ex;
      g.ss = m->pf_ss;
      g.ss_ld = H / kTile;
      g.ovf = m->pf_ovf;
      ok = ok && launch_gemm(lf, GEMM_FOLD, pp.sf, g, st);
    } else {
      g.Cf = m->pf_part;
      ok = ok && launch_gemm(lf, GEMM_PART, pp.so, g, st);
      launch_rms_rows(rows_args(m->pf_x, m->pf_part, pp.so.splits, rowsH, H, L.ffn_norm, d.rms_eps, m->pf_xn,
                                m->pf_ovf),
                      M, st);
    }
    g = gemm_args(L.gu, m->pf_xn, H, M);
    g.ovf = m->pf_ovf;
    if (pp.fold) {
      g.ss = m->pf_ss;
      g.ex = m->pf_ex;
      g.ss_ld = H / kTile;
      g.n_norm = H;
      g.eps = (float)d.rms_eps;
    }
    g.N = L.gu->T * kTile;
    g.Ch = m->pf_h;
    g.ldc = I;
    g.n_out = I;
    ok = ok && launch_gemm(lf, GEMM_SWIGLU, pp.sg, g, st);
    g = gemm_args(L.down, m->pf_h, I, M);
    g.Cf = m->pf_part;
    g.ldc = H;
    ok = ok && launch_gemm(lf, GEMM_PART, pp.sd, g, st);
    if (!ok) return 0;
  }
  // the last layer's MLP output joins the residual rows
  launch_rms_rows(rows_args(m->pf_x, m->pf_part, pp.sd.splits, rowsH, H, nullptr, d.rms_eps, nullptr, nullptr), M, st);
  return d.num_layers * ((pp.rope_epi ? 7 : 8) - (pp.fold ? 1 : 0)) + 1;
}

// One batched chunk [p, p + M) of the prompt [start, end): the control block
// names the chunk, then its captured graph (one per chunk size, captured on
// first use) or, with graphs off, its kernels.
static int prefill_rows(tlm_model* m, const int32_t* tokens, int start, int end, int p, int M) {
  PfPlan pp;
  int rc = prefill_plan(m, M, &pp);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  set_ctrl(m, tokens[p], p, start, end - start, st);
  m->counts.kernel_launches++;
  if (!m->use_graphs) {
    const int k = prefill_enqueue(m, pp, M, st);
    if (!k) return fail(TLM_ERR_STATE, "TLMModel: no batched prefill kernel for a layer");
    m->counts.kernel_launches += k;
    CHECK_LAUNCH("TLMModel");
    return TLM_OK;
  }
  auto it = m->pf_graphs.find(M);
  if (it == m->pf_graphs.end()) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const int k = prefill_enqueue(m, pp, M, st);
    hipError_t le = hipGetLastError();
    HIP_TRY(hipStreamEndCapture(st, &g));
    if (le != hipSuccess || !k) {
      hipGraphDestroy(g);
      if (!k) return fail(TLM_ERR_STATE, "TLMModel: no batched prefill kernel for a layer");
      return fail(TLM_ERR_HIP, "TLMModel: launch during capture failed: %s", hipGetErrorString(le));
    }
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) {
      hipGraphDestroy(g);
      return fail(TLM_ERR_HIP, "TLMModel: prefill graph instantiation failed");
    }
    it = m->pf_graphs.emplace(M, std::make_pair(g, ge)).first;
  }
  HIP_TRY(hipGraphLaunch(it->second.second, st));
  m->counts.graph_launches++;
  return TLM_OK;
}

// Kernels one replay graph records at most: a chunk whose token steps would
// record more is replayed as several graphs.  (Unbounded, a 2047-position
// chunk of the Llama-3.2-1B shape's long-window steps, some 80 kernels each,
// was captured as one linear graph of over 160,000 nodes, and the process took
// a segmentation fault.)
constexpr int kReplayGraphKernels = 2048;

// The decode graph replayed over the n prompt positions [p, p + n) (set_ctrl
// already named p; each step's prefill tail advances the position and stages
// the next id): captured graphs of up to kReplayGraphKernels kernels' worth of
// token steps per schedule and size -- one graph per chunk for most models
// (the reference encodes a chunk's replays into one submission,
// DecoderTSLRunner.ts:472-480,504-530) -- or one launch per position when the
// chunk crosses into the long-window kernels or graphs are off.
static int replay_chunk(tlm_model* m, int p, int n) {
  auto mode = [&](int pos) {
    const bool lw = long_window(&m->attn, pos);
    return m->ps_on && !m->ps_suspend && !lw ? 2 : lw ? 1 : 0;
  };
  const int md = mode(p);
  bool same = true;
  for (int i = 1; i < n && same; i++) same = mode(p + i) == md;
  if (!m->use_graphs || !same || n < 2) {
    int rc = TLM_OK;
    for (int i = 0; i < n && !rc; i++) rc = run_token(m, false, p + i);
    return rc;
  }
  // kernels per token step: the persistent kernel and the prefill advance, or
  // the per-stage prefill graph's nodes
  size_t per_step = 2;
  if (md != 2) HIP_TRY(hipGraphGetNodes(m->graph_prefill[md], nullptr, &per_step));
  const int per = (int)std::max<size_t>(1, kReplayGraphKernels / std::max<size_t>(per_step, 1));
  hipStream_t st = m->ctx->stream;
  if (md != 2) stage_x0(m, st);
  for (int done = 0; done < n;) {
    const int cnt = std::min(per, n - done);
    const int key = md * 65536 + cnt;
    auto it = m->replay_graphs.find(key);
    if (it == m->replay_graphs.end()) {
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      const tlm_model_counts kept = m->counts;
      const bool stale = m->x0_stale;
      HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      bool ok = true;
      for (int i = 0; i < cnt; i++) {
        if (md == 2) {
          ok &= enqueue_ps(m, st, 0);
        } else {
          for (int l = 0; l < m->d.num_layers; l++) ok &= enqueue_layer(m, l, st, -1, md == 1);
          launch_prefill_advance(m->ctrl, m->prompt, emb_stage(m), st);
        }
      }
      m->counts = kept;
      m->x0_stale = stale;
      hipError_t le = hipGetLastError();
      HIP_TRY(hipStreamEndCapture(st, &g));
      if (le != hipSuccess || !ok) {
        hipGraphDestroy(g);
        if (!ok) return fail(TLM_ERR_STATE, "TLMModel: no kernel variant for a stage of this model");
        return fail(TLM_ERR_HIP, "TLMModel: launch during capture failed: %s", hipGetErrorString(le));
      }
      if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) {
        hipGraphDestroy(g);
        return fail(TLM_ERR_HIP, "TLMModel: replay graph instantiation failed");
      }
      it = m->replay_graphs.emplace(key, std::make_pair(g, ge)).first;
    }
    m->host_pos = p + done + cnt - 1;
    auto launch = [&]() -> int {
      HIP_TRY(hipGraphLaunch(it->second.second, st));
      m->counts.graph_launches++;
      if (md == 2) m->counts.persistent_tokens += (uint64_t)cnt;
      m->x0_stale = md == 2;  // the persistent advance does not stage the row
      return TLM_OK;
    };
    const int rc = md == 2 ? ps_ordered(m, launch) : launch();
    if (rc) return rc;
    done += cnt;
  }
  return TLM_OK;
}

int tlm_model_set_prefill(tlm_model* m, int32_t min_rows, int32_t chunk) {
  if (!m) return fail(TLM_ERR_INVALID, "TLMModel: null model");
  if (chunk < 1) return fail(TLM_ERR_INVALID, "TLMModel: prefill chunk %d must be positive", chunk);
  if (min_rows > 0) {
    const char* why = prefill_unsupported(m);
    if (why) return fail(TLM_ERR_INVALID, "TLMModel: batched prefill unavailable: %s", why);
  }
  m->pf_min_rows = std::max(0, min_rows);
  m->pf_chunk = std::min(chunk, m->d.max_tokens);
  return TLM_OK;
}

int tlm_prefill(tlm_model* m, const int32_t* tokens, int32_t start, int32_t end) {
  if (!m || (!tokens && end > start)) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  if (start < 0 || end > m->d.max_tokens || start > end)
    return fail(TLM_ERR_RANGE, "TLMModel: prefill range [%d, %d) outside [0, %d)", start, end, m->d.max_tokens);
  if (start == end) return TLM_OK;
  for (int i = start; i < end; i++)
    if (tokens[i] < 0 || tokens[i] >= m->d.vocab_size)
      return fail(TLM_ERR_RANGE, "TLMModel: token %d outside [0, %d)", tokens[i], m->d.vocab_size);
  int rc = tlm_model_finalize(m);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  HIP_TRY(hipStreamSynchronize(st));
  rc = model_check(m);  // the earlier tokens are final before batched chunks overwrite cache rows
  if (rc) return rc;
  kv_touch(m, end);
  // the ids go to the device in stream order (no staging wait on the host);
  // the pinned words are free again: the stream finished its work above
  memcpy(m->host_pin + kPinPrompt, tokens + start, sizeof(int32_t) * (end - start));
  HIP_TRY(hipMemcpyAsync(m->prompt, m->host_pin + kPinPrompt, sizeof(int32_t) * (end - start), hipMemcpyHostToDevice,
                         st));
  const bool batched = m->pf_min_rows > 0 && !prefill_unsupported(m);
  for (int p = start; p < end;) {
    const int n = std::min(end - p, batched ? m->pf_chunk : end - p);
    bool replay = !(batched && n >= m->pf_min_rows);
    if (!replay) {
      rc = prefill_rows(m, tokens, start, end, p, n);
      if (rc) return rc;
      // an fp16 activation of the chunk overflowed (or was NaN): the chunk's
      // cache rows are rewritten by the fp32 decode path
      HIP_TRY(hipMemcpyAsync(m->host_pin + 8, m->pf_ovf, sizeof(int), hipMemcpyDeviceToHost, st));
      HIP_TRY(hipStreamSynchronize(st));
      if (m->host_pin[8]) {
        const int zero = 0;
        HIP_TRY(hipMemcpy(m->pf_ovf, &zero, sizeof(int), hipMemcpyHostToDevice));
        m->pf_replayed++;
        replay = true;
        rc = kv_clear(m, p, n);  // the chunk's rows may hold inf or NaN
        if (rc) return rc;
      }
      if (!replay) m->counts.prefill_chunks++;
    }
    if (replay) {  // the decode graph replayed per position
      set_ctrl(m, tokens[p], p, start, end - start, st);
      m->counts.kernel_launches++;
      m->counts.replayed_positions += n;
      CHECK_LAUNCH("TLMModel");
      for (int i = 0; i < n; i++) redo_log(m, tokens[p + i], p + i, 1, false, false);
      rc = replay_chunk(m, p, n);
    }
    if (rc) return rc;
    p += n;
  }
  return TLM_OK;
}

// Zeroes the cache rows [pos0, pos0 + n) of every layer before they are
// recomputed: the per-stage attention fills the padding slots of its last V
// tile with the row at the position (times a zero probability), so a stale
// NaN there (a failed token, an overflowed prefill chunk) would reach it.
static int kv_clear(tlm_model* m, int pos0, int n) {
  n = std::min(n, m->d.max_tokens - pos0);
  if (pos0 < 0 || n <= 0) return TLM_OK;
  const size_t esz = m->d.kv_fmt == TLM_FMT_F32 ? 4 : 2, row = (size_t)m->d.head_dim * esz;
  for (auto& L : m->layers)
    for (int h = 0; h < m->d.num_kv_heads; h++) {
      const size_t off = ((size_t)h * m->d.max_tokens + pos0) * row;
      HIP_TRY(hipMemsetAsync((char*)L.kc + off, 0, n * row, m->ctx->stream));
      HIP_TRY(hipMemsetAsync((char*)L.vc + off, 0, n * row, m->ctx->stream));
    }
  return TLM_OK;
}

// Recomputes the logged tokens on the per-stage graph after a persistent-
// schedule token failed (err: its ctrl[C_ERR] bits), in their order, so the
// cache rows, logits and greedy tokens are those of the per-stage kernels.
// A token whose last residual was not finite (an input of a q4 linear
// overflowed its fp16 copy) turns the schedule off for the model: its
// activations reach that range.
static int ps_recover(tlm_model* m, int err) {
  if (m->redo_lost) {
    m->redo_lost = false;
    return fail(TLM_ERR_HIP, "TLMModel: a token of the persistent decode schedule %s after more than %zu tokens "
                             "without a read; the tokens computed since the last read are invalid",
                err & kPsErrTimeout ? "timed out" : "overflowed fp16", kRedoMax);
  }
  if ((err & kPsErrTimeout) && m->ps_l2_items > 0) {
    // a block may have run on another XCD than its roles were placed for, where
    // a plain store never reaches its consumers: every handoff device-scope
    m->ps_l2_items = 0;
    m->ps.l2 = 0;
    PsArgs a;  // the launch's arguments as they are, without the XCD table
    HIP_TRY(hipMemcpy(&a, m->ps_args_dev, sizeof a, hipMemcpyDeviceToHost));
    a.xcc = nullptr;
    HIP_TRY(hipMemcpy(m->ps_args_dev, &a, sizeof a, hipMemcpyHostToDevice));
  }
  if (err & kPsErrRange) {
    int rc = ps_register(m, false);
    if (rc) return rc;
    m->ps_on = false;
    m->ps_range_off = true;
  }
  std::vector<RedoEntry> log;
  log.swap(m->redo);
  hipStream_t st = m->ctx->stream;
  m->ps_suspend = true;
  int rc = TLM_OK;
  for (const RedoEntry& e : log) {
    rc = kv_clear(m, e.pos, e.n);
    if (rc) break;
    set_ctrl(m, e.token, e.pos, 0, 0, st);
    m->counts.kernel_launches++;
    for (int i = 0; i < e.n && rc == TLM_OK; i++) rc = run_token(m, e.logits, e.pos + i);
    if (rc) break;
    m->counts.recomputed_positions += e.n;
  }
  m->ps_suspend = false;
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(st));
  return TLM_OK;
}

// After a sync: the flags of the tokens since the last check.  C_FXR (a
// residual value of the per-stage kernels left their fixed-point range): an
// error, the results are invalid.  C_ERR (a persistent-schedule token: a
// bounded wait ran out, the late block left; or its last residual was not
// finite): the logged tokens are recomputed (ps_recover) before the caller
// reads anything.  Clean: the logged tokens are final.
// The control block, read after the model's stream has finished its work
// (through the pinned words: a direct copy, no staging).
static int read_ctrl(tlm_model* m, int* c) {
  HIP_TRY(hipMemcpyAsync(m->host_pin, m->ctrl, sizeof(int) * 8, hipMemcpyDeviceToHost, m->ctx->stream));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  memcpy(c, m->host_pin, sizeof(int) * 8);
  return TLM_OK;
}

static int model_check(tlm_model* m, const int* ctrl_host) {
  int c[8];
  if (ctrl_host) memcpy(c, ctrl_host, sizeof c);
  else if (int rc = read_ctrl(m, c)) return rc;
  if (m->ps_on && c[C_ERR]) {
    const int zero = 0;
    HIP_TRY(hipMemcpy(m->ctrl + C_ERR, &zero, sizeof(int), hipMemcpyHostToDevice));
    if (int rc = ps_recover(m, c[C_ERR])) return rc;
    if (int rc = read_ctrl(m, c)) return rc;
  }
  m->redo.clear();
  m->redo_lost = false;
  if (c[C_FXR]) {
    const int zero = 0;
    HIP_TRY(hipMemcpy(m->ctrl + C_FXR, &zero, sizeof(int), hipMemcpyHostToDevice));
    return fail(TLM_ERR_RANGE, "TLMModel: a residual value of the per-stage kernels reached 2^30 in magnitude "
                               "(or NaN), past their fixed-point range; the tokens computed since the last read "
                               "are invalid");
  }
  return TLM_OK;
}

int tlm_read_logits(tlm_model* m, float* out, size_t n) {
  if (!m || !out || n > (size_t)m->d.vocab_size) return fail(TLM_ERR_INVALID, "TLMModel: invalid logits read");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (int rc = model_check(m)) return rc;
  HIP_TRY(hipMemcpy(out, m->logits, sizeof(float) * n, hipMemcpyDeviceToHost));
  return TLM_OK;
}

int tlm_read_candidates(tlm_model* m, int k, double softcap, int32_t* tokens, float* scores) {
  if (!m || !tokens || !scores) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  int rc = model_check(m);  // the logits are final (recomputed if a token was flagged)
  if (rc) return rc;
  rc = tlm_op_topk(m->ctx, m->logits, m->d.vocab_size, k, softcap, m->cand_i, m->cand_v);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(tokens, m->cand_i, sizeof(int32_t) * k, hipMemcpyDeviceToHost, m->ctx->stream));
  HIP_TRY(hipMemcpyAsync(scores, m->cand_v, sizeof(float) * k, hipMemcpyDeviceToHost, m->ctx->stream));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  return TLM_OK;
}

int tlm_read_hidden(tlm_model* m, float* out, size_t n) {
  if (!m || !out || n > (size_t)m->d.hidden_size) return fail(TLM_ERR_INVALID, "TLMModel: invalid hidden read");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (int rc = model_check(m)) return rc;
  HIP_TRY(hipMemcpy(out, m->xf, sizeof(float) * n, hipMemcpyDeviceToHost));
  return TLM_OK;
}

int tlm_read_token(tlm_model* m, int32_t* token) {
  if (!m || !token) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  int ctrl[8];
  if (int rc = read_ctrl(m, ctrl)) return rc;
  const bool recompute = m->ps_on && ctrl[C_ERR];
  if (int rc = model_check(m, ctrl)) return rc;
  if (recompute)  // the token is now the per-stage graph's
    if (int rc = read_ctrl(m, ctrl)) return rc;
  *token = ctrl[C_TOKEN];
  return TLM_OK;
}

int tlm_decode_greedy(tlm_model* m, int32_t token, int32_t position, int n, int32_t* out) {
  if (!m || (!out && n > 0) || n < 0) return fail(TLM_ERR_INVALID, "TLMModel: invalid decode argument");
  int rc = check_token(m, token, position);
  if (rc) return rc;
  if ((long)position + n > m->d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMModel: decode of %d tokens from %d passes max_tokens %d", n, position,
                m->d.max_tokens);
  rc = tlm_model_finalize(m);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  set_ctrl(m, token, position, 0, 0, st);
  m->counts.kernel_launches++;
  CHECK_LAUNCH("TLMModel");
  redo_log(m, token, position, n, true, true);
  for (int i = 0; i < n; i++) {
    rc = run_token(m, true, position + i);
    if (rc) return rc;
  }
  HIP_TRY(hipStreamSynchronize(st));
  if (int rc = model_check(m)) return rc;
  if (n > 0) HIP_TRY(hipMemcpy(out, m->tokens_out, sizeof(int32_t) * n, hipMemcpyDeviceToHost));
  return TLM_OK;
}

int tlm_reset_cache(tlm_model* m) {
  if (!m) return fail(TLM_ERR_INVALID, "TLMModel: null model");
  {  // the tokens since the last read are discarded with the cache: so are their flags
    HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    const int zero[2] = {0, 0};
    HIP_TRY(hipMemcpy(m->ctrl + C_FXR, zero, sizeof zero, hipMemcpyHostToDevice));
    m->redo.clear();
    m->redo_lost = false;
  }
  // only the rows that can hold values (positions below kv_hi): clearing all
  // max_tokens rows (402 MB at the Qwen2.5-0.5B shape's 32768) took ~80 us and
  // evicted the weights from the 256 MB last-level cache, which the next
  // prefill or decode then read from HBM (a 127-id prefill after it: 1.07 ms
  // against 0.99)
  const size_t esz = m->d.kv_fmt == TLM_FMT_F32 ? 4 : 2;
  const size_t row = (size_t)m->d.head_dim * esz, pitch = row * m->d.max_tokens;
  if (m->kv_hi > 0)
    for (auto& L : m->layers) {
      HIP_TRY(hipMemset2DAsync(L.kc, pitch, 0, row * m->kv_hi, m->d.num_kv_heads, m->ctx->stream));
      HIP_TRY(hipMemset2DAsync(L.vc, pitch, 0, row * m->kv_hi, m->d.num_kv_heads, m->ctx->stream));
    }
  m->kv_hi = 0;
  return TLM_OK;
}

static int kv_copy(tlm_model* m, int layer, int pos0, int count, void* k, void* v, bool write) {
  if (!m || !k || !v) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  if (layer < 0 || layer >= m->d.num_layers || pos0 < 0 || count < 0 || pos0 + count > m->d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMModel: KV range outside the cache");
  const size_t esz = m->d.kv_fmt == TLM_FMT_F32 ? 4 : 2;
  const int Hkv = m->d.num_kv_heads, D = m->d.head_dim, M = m->d.max_tokens;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (int rc = model_check(m)) return rc;  // the enqueued tokens' rows are final
  if (write) kv_touch(m, (long)pos0 + count);
  for (int h = 0; h < Hkv; h++) {
    // canonical rows are [t][h][d]; device rows are [h][t][d]
    HIP_TRY(hipMemcpy2D(
        write ? (char*)m->layers[layer].kc + ((size_t)h * M + pos0) * D * esz : (char*)k + (size_t)h * D * esz,
        write ? D * esz : (size_t)Hkv * D * esz,
        write ? (const char*)k + (size_t)h * D * esz : (const char*)m->layers[layer].kc + ((size_t)h * M + pos0) * D * esz,
        write ? (size_t)Hkv * D * esz : D * esz, D * esz, count, write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy2D(
        write ? (char*)m->layers[layer].vc + ((size_t)h * M + pos0) * D * esz : (char*)v + (size_t)h * D * esz,
        write ? D * esz : (size_t)Hkv * D * esz,
        write ? (const char*)v + (size_t)h * D * esz : (const char*)m->layers[layer].vc + ((size_t)h * M + pos0) * D * esz,
        write ? (size_t)Hkv * D * esz : D * esz, D * esz, count, write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost));
  }
  return TLM_OK;
}

int tlm_kv_write(tlm_model* m, int layer, int pos0, int count, const void* k, const void* v) {
  return kv_copy(m, layer, pos0, count, const_cast<void*>(k), const_cast<void*>(v), true);
}

int tlm_kv_read(tlm_model* m, int layer, int pos0, int count, void* k, void* v) {
  return kv_copy(m, layer, pos0, count, k, v, false);
}

int tlm_kv_fill_normal(tlm_model* m, uint64_t seed, int count) {
  if (!m || count < 0 || count > m->d.max_tokens) return fail(TLM_ERR_RANGE, "TLMModel: invalid fill count");
  kv_touch(m, count);
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  if (int rc = model_check(m)) return rc;
  for (int l = 0; l < m->d.num_layers; l++) {
    launch_kv_fill(m->layers[l].kc, m->layers[l].vc, m->d.kv_fmt == TLM_FMT_F32, 0, m->d.num_kv_heads,
                   m->d.max_tokens, m->d.head_dim, count, seed + (uint64_t)l * 0x100000000ull, m->ctx->stream);
    CHECK_LAUNCH("TLMModel");
  }
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  return TLM_OK;
}

// ------------------------------------------------------------------- timing --

int tlm_time_decode(tlm_model* m, int32_t token, int32_t position, int warmup, int n, double* ms) {
  if (!m || !ms || n <= 0 || warmup < 0) return fail(TLM_ERR_INVALID, "TLMModel: invalid timing argument");
  int rc = check_token(m, token, position);
  if (rc) return rc;
  if ((long)position + warmup + n > m->d.max_tokens)
    return fail(TLM_ERR_RANGE, "TLMModel: timed decode passes max_tokens");
  kv_touch(m, (long)position + warmup + n);
  rc = tlm_model_finalize(m);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  set_ctrl(m, token, position, 0, 0, st);
  m->counts.kernel_launches++;
  redo_log(m, token, position, warmup + n, true, true);
  for (int i = 0; i < warmup; i++) {
    rc = run_token(m, true, position + i);
    if (rc) return rc;
  }
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  HIP_TRY(hipStreamSynchronize(st));
  HIP_TRY(hipEventRecord(e0, st));
  for (int i = 0; i < n; i++) {
    rc = run_token(m, true, position + warmup + i);
    if (rc) return rc;
  }
  HIP_TRY(hipEventRecord(e1, st));
  HIP_TRY(hipEventSynchronize(e1));
  float f = 0.f;
  HIP_TRY(hipEventElapsedTime(&f, e0, e1));
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  *ms = f;
  return model_check(m);
}

// n decode steps from (token, position) with HIP events on the model stream
// around the layer part (the persistent kernel, or the layer graph / per-stage
// kernels) and around the LM head of each step; averages in ms.
static int time_step_parts(tlm_model* m, int32_t token, int32_t position, int n, double* layers_ms,
                           double* head_ms) {
  if (!m || n <= 0) return fail(TLM_ERR_INVALID, "TLMModel: invalid timing argument");
  int rc = check_token(m, token, position);
  if (rc) return rc;
  if ((long)position + n > m->d.max_tokens) return fail(TLM_ERR_RANGE, "TLMModel: timed decode passes max_tokens");
  kv_touch(m, (long)position + n);
  rc = tlm_model_finalize(m);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  for (int lw = 0; lw < 2 && m->use_graphs; lw++)
    if (!m->g_layers[lw]) {
      rc = capture(m, TAIL_NONE, lw, &m->graph_layers[lw], &m->g_layers[lw]);
      if (rc) return rc;
    }
  std::vector<hipEvent_t> ev(4 * (size_t)n, nullptr);
  for (auto& e : ev) HIP_TRY(hipEventCreate(&e));
  set_ctrl(m, token, position, 0, 0, st);
  m->counts.kernel_launches++;
  redo_log(m, token, position, n, true, true);
  bool ok = true;
  for (int i = 0; i < n && ok; i++) {
    const bool lw = long_window(&m->attn, position + i);
    const bool ps = m->ps_on && !lw;
    m->host_pos = position + i;
    auto step = [&]() -> int {
      if (!ps) stage_x0(m, st);
      hipEventRecord(ev[4 * (size_t)i], st);
      if (ps) {
        ok &= launch_ps_token(m->ps, m->ps_blocks, m->ps_smem, m->ps_args_dev, st);
        m->counts.kernel_launches++;
        m->counts.persistent_tokens++;
      } else if (m->use_graphs) {
        HIP_TRY(hipGraphLaunch(m->g_layers[lw], st));
        m->counts.graph_launches++;
      } else {
        for (int l = 0; l < m->d.num_layers; l++) ok &= enqueue_layer(m, l, st, -1, lw);
      }
      hipEventRecord(ev[4 * (size_t)i + 1], st);
      ok &= enqueue_head(m, st, true, &ev[4 * (size_t)i + 2], ps);
      return TLM_OK;
    };
    rc = ps ? ps_ordered(m, step) : step();
    if (rc) return rc;
  }
  if (!ok) return fail(TLM_ERR_STATE, "TLMModel: no kernel variant for a stage of this model");
  CHECK_LAUNCH("TLMModel");
  HIP_TRY(hipStreamSynchronize(st));
  double tl = 0.0, th = 0.0;
  for (int i = 0; i < n; i++) {
    float f = 0.f, g = 0.f;
    HIP_TRY(hipEventElapsedTime(&f, ev[4 * i], ev[4 * i + 1]));
    HIP_TRY(hipEventElapsedTime(&g, ev[4 * i + 2], ev[4 * i + 3]));
    tl += f;
    th += g;
  }
  for (auto& e : ev) hipEventDestroy(e);
  if (layers_ms) *layers_ms = tl / n;
  if (head_ms) *head_ms = th / n;
  return model_check(m);
}

int tlm_time_head(tlm_model* m, int32_t token, int32_t position, int n, double* avg_ms) {
  if (!avg_ms) return fail(TLM_ERR_INVALID, "TLMModel: invalid timing argument");
  return time_step_parts(m, token, position, n, nullptr, avg_ms);
}

int tlm_time_layers(tlm_model* m, int32_t token, int32_t position, int n, double* avg_ms) {
  if (!avg_ms) return fail(TLM_ERR_INVALID, "TLMModel: invalid timing argument");
  return time_step_parts(m, token, position, n, avg_ms, nullptr);
}

int tlm_time_kernel(tlm_model* m, int which, int iters, double* avg_ms) {
  if (!m || !avg_ms || iters <= 0 || which < 0 || which > 6 || which == 3)
    return fail(TLM_ERR_INVALID, "TLMModel: invalid kernel timing argument");
  int rc = tlm_model_finalize(m);
  if (rc) return rc;
  kv_touch(m, m->d.max_tokens);  // a stage timing writes the row at whatever position the control block names
  hipStream_t st = m->ctx->stream;
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  auto one = [&]() {
    if (which == 6)  // top-8 candidates over the logits
      return launch_topk(m->logits, m->d.vocab_size, 8, 0.f, m->ctx->topk_v, m->ctx->topk_i, kTopkWork, m->cand_v,
                         m->cand_i, st);
    return which == 0 ? enqueue_head(m, st, false)
                      : enqueue_layer(m, 0, st, which, long_window(&m->attn, m->host_pos));
  };
  if (!one()) return fail(TLM_ERR_STATE, "TLMModel: no kernel variant for stage %d", which);  // warm
  CHECK_LAUNCH("TLMModel");
  HIP_TRY(hipStreamSynchronize(st));
  HIP_TRY(hipEventRecord(e0, st));
  for (int i = 0; i < iters; i++) one();
  HIP_TRY(hipEventRecord(e1, st));
  HIP_TRY(hipEventSynchronize(e1));
  CHECK_LAUNCH("TLMModel");
  float f = 0.f;
  HIP_TRY(hipEventElapsedTime(&f, e0, e1));
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  *avg_ms = f / iters;
  // repeated single stages break the accumulators' zero-before-use order:
  // clear them (the cache and ctrl state are left as the stages wrote them)
  HIP_TRY(hipMemsetAsync(m->rb, 0, sizeof(unsigned long long) * kRep * m->d.hidden_size * m->d.num_layers, st));
  HIP_TRY(hipStreamSynchronize(st));
  return TLM_OK;
}

int tlm_trace_decode(tlm_model* m, int32_t token, int32_t position, int n, uint64_t* out, size_t n_out) {
  if (!m || !out || n <= 0) return fail(TLM_ERR_INVALID, "TLMModel: invalid trace argument");
  int rc = check_token(m, token, position);
  if (rc) return rc;
  if ((long)position + n > m->d.max_tokens) return fail(TLM_ERR_RANGE, "TLMModel: traced decode passes max_tokens");
  kv_touch(m, (long)position + n);
  if (!m->ps_on) return fail(TLM_ERR_STATE, "TLMModel: this model has no persistent schedule");
  if (long_window(&m->attn, position + n - 1))
    return fail(TLM_ERR_STATE, "TLMModel: position %d needs the long-window kernels", position + n - 1);
  const size_t need = (size_t)m->ps_blocks * kPsWaves * (m->d.num_layers + 1) * PS_STAGES * kPsEvents;
  if (n_out != need) return fail(TLM_ERR_INVALID, "TLMModel: trace buffer holds %zu stamps, need %zu", n_out, need);
  rc = tlm_model_finalize(m);
  if (rc) return rc;
  unsigned long long* tr = nullptr;
  PsArgs* ad = nullptr;
  HIP_TRY(hipMalloc(&tr, need * sizeof(unsigned long long)));
  if (hipMalloc(&ad, sizeof(PsArgs)) != hipSuccess) {
    hipFree(tr);
    return fail(TLM_ERR_OOM, "TLMModel: trace arguments");
  }
  PsArgs a = ps_args(m);
  a.trace = tr;
  hipStream_t st = m->ctx->stream;
  bool ok = hipMemcpy(ad, &a, sizeof a, hipMemcpyHostToDevice) == hipSuccess;
  set_ctrl(m, token, position, 0, 0, st);
  m->counts.kernel_launches++;
  redo_log(m, token, position, n, true, true);
  for (int i = 0; i < n && ok; i++) {
    ok &= hipMemsetAsync(tr, 0, need * sizeof(unsigned long long), st) == hipSuccess;
    rc = ps_ordered(m, [&]() -> int {
      ok &= launch_ps_token(m->ps, m->ps_blocks, m->ps_smem, ad, st);
      ok &= enqueue_head(m, st, true, nullptr, true);
      m->counts.kernel_launches++;
      m->counts.persistent_tokens++;
      return TLM_OK;
    });
    if (rc) break;
  }
  hipError_t e = hipStreamSynchronize(st);
  if (ok && e == hipSuccess) e = hipMemcpy(out, tr, need * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(tr);
  hipFree(ad);
  if (rc) return rc;
  if (!ok) return fail(TLM_ERR_STATE, "TLMModel: traced launch failed");
  if (e != hipSuccess) return fail(TLM_ERR_HIP, "TLMModel: %s", hipGetErrorString(e));
  return model_check(m);
}

int tlm_model_describe(tlm_model* m, char* out, size_t len) {
  if (!m || !out) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  const Layer& L = m->layers[0];
  auto p = [](const tlm_linear* x) {
    char b[128];
    snprintf(b, sizeof b, "%dx%d T=%d C=%d waves=%d cps=%d splits=%d", x->N, x->K, x->T, x->C, x->plan.waves,
             x->plan.cps, x->plan.splits);
    return std::string(b);
  };
  char mlp[160];
  snprintf(mlp, sizeof mlp, "gate|up %dx%d paired, down %dx%d; %d blocks x %d waves, %d+%d chunks/wave",
           L.gu->N, L.gu->K, L.down->N, L.down->K, L.gu->T, kMlpWaves, m->mlp_nch, m->mlp_ndb);
  std::string s = "qkv[" + p(L.qkv) + "] o[" + p(L.o) + "] mlp[" + mlp + "] head[" +
                  p(m->head) + " grid=" + std::to_string(m->lm_plan.gx) + " waves=" +
                  std::to_string(m->lm_plan.waves) + "] attn[nsplit=" + std::to_string(m->attn.nsplit) + "/" + std::to_string(m->attn.nsplit_long) +
                  " G=" + std::to_string(m->attn.G) + (m->attn.gqa ? " long=mfma" : "") + "]";
  if (m->ps_on) {
    const PsArgs a = ps_args(m);
    const int To = a.To, nq = 2 * a.Hkv * a.kq, ng = (a.Tgu + a.mw - 1) / a.mw;
    const int items = nq + a.Hq + To * a.ko + ng + To * a.ks;
    char b[320];
    snprintf(b, sizeof b, " persistent[%d blocks, %d items: %d k|v (%d splits), %d q+att, %d o (%d splits), %d gate|up "
             "(32x%d), %d down (%d splits); %zu B LDS; variant nx=%d no=%d nd=%d; %d publish through their XCD's L2]",
             m->ps_blocks, items, nq, a.kq, a.Hq, To * a.ko, a.ko, ng, a.mw, To * a.ks, a.ks, m->ps_smem, m->ps.nx,
             m->ps.no, m->ps.nd, m->ps_l2_items);
    s += b;
  } else {
    s += m->ps_range_off ? " persistent[off after an fp16 range overflow]" : " persistent[off]";
  }
  s += " prefill[batched from " + std::to_string(m->pf_min_rows) + " rows, chunk " + std::to_string(m->pf_chunk) +
       ", " + std::to_string(m->pf_replayed) + " replayed after fp16 overflow]";
  bool mixed = false;
  for (int w : m->windows) mixed |= w != m->windows[0];
  if (mixed) {  // per-layer windows, e.g. "windows[0,512,0,512]"
    s += " windows[";
    for (size_t l = 0; l < m->windows.size(); l++) s += (l ? "," : "") + std::to_string(m->windows[l]);
    s += "]";
  }
  snprintf(out, len, "%s", s.c_str());
  return TLM_OK;
}

int tlm_model_counts_read(tlm_model* m, tlm_model_counts* out) {
  if (!m || !out) return fail(TLM_ERR_INVALID, "TLMModel: null argument");
  *out = m->counts;
  return TLM_OK;
}

}  // extern "C"

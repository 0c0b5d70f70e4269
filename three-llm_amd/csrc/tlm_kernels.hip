// Hand-written gfx950 kernels of the per-token decoder path.
//
// Layouts (device):
//   linear weights  [T tiles of 64 rows][C chunks][64 lanes][16 B]; a chunk is
//                   32 k of q4 nibbles (canonical byte order) or 8 k of fp16.
//                   One wave64 streams 1 KB per load instruction, one output
//                   row per lane, so no cross-lane reduction is needed.
//   q4 scales       [T][C][64] fp16.
//   KV cache        [Hkv][max_tokens][D] per layer (head-major: a chunk of
//                   positions of one head is contiguous).
//   partial sums    [S][N] fp32: split-K GEMVs leave S partial vectors that the
//                   consuming kernel folds into its prologue.
#include <float.h>

#include <algorithm>
#include <hip/hip_fp16.h>

#include "tlm_device.h"

namespace tlm {


// ------------------------------------------------------------------ GEMV --

// Sum of n <= kMaxPart partial vectors at element k.  The loads are
// unconditional (indices clamped to valid rows) and only the adds are masked,
// so all of them are in flight before the first use: a consumer pays one
// memory round trip however many splits its producer used.  n == 0 reads nothing.
__device__ __forceinline__ float sum_parts(const float* p, int n, int stride, int k) {
  if (n <= 0) return 0.f;
  float v[kMaxPart];
#pragma unroll
  for (int j = 0; j < kMaxPart; j++) v[j] = p[(size_t)min(j, n - 1) * stride + k];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPart; j++) s += j < n ? v[j] : 0.f;
  return s;
}

__device__ __forceinline__ float4 f4add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// Flash-decoding combine of one output element (query head `row`, dim d) over
// the attention chunk partials, 16 chunks per round trip (nact >= 1).
__device__ float attn_combine_elem(const float* pacc, const float* pml, int row, int d, int D, int nsplit, int nact) {
  const float* ml = pml + (size_t)row * nsplit * 2;
  const float* ac = pacc + (size_t)row * nsplit * D + d;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int jb = 0; jb < nact; jb += 16) {
    float mm[16], ll[16], aa[16];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const int j = min(jb + u, nact - 1);
      mm[u] = ml[2 * j];
      ll[u] = ml[2 * j + 1];
      aa[u] = ac[(size_t)j * D];
    }
    float Mb = M;
#pragma unroll
    for (int u = 0; u < 16; u++) Mb = fmaxf(Mb, mm[u]);
    const float sc = M == -INFINITY ? 0.f : __expf(M - Mb);
    L *= sc;
    O *= sc;
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const float e = (jb + u < nact && mm[u] != -INFINITY) ? __expf(mm[u] - Mb) : 0.f;
      L = fmaf(ll[u], e, L);
      O = fmaf(aa[u], e, O);
    }
    M = Mb;
  }
  return O / L;
}

// Stores 4 prologue outputs at slice offset i (a multiple of 4) and, for q4,
// adds them into the group sums sum_k x_k of the 32-element groups: the 8
// lanes covering a group reduce with shuffles.  Every lane of the wave must
// call it (in_slice false contributes nothing).
template <int FMT>
__device__ __forceinline__ void put4(float* xl, float* xsum, int i, float4 y, bool in_slice) {
  if (in_slice) *reinterpret_cast<float4*>(xl + i) = y;
  if (FMT == WF_Q4) {
    const float g = sum8(in_slice ? (y.x + y.y) + (y.z + y.w) : 0.f);
    if (in_slice && (i & 31) == 0) xsum[i >> 5] = g;
  }
}

// Input slice x[k0, k1) of a GEMV in LDS (xl, zero-padded to klen_pad) plus,
// for q4, its 32-element group sums.  Each thread owns 4 consecutive elements
// (K % 4 == 0).  issue() puts the thread's first loads in flight and runs
// before the kernel issues its weight loads: a wave's loads complete in issue
// order, so the prologue's data (split-K partials of the previous kernel,
// L2/MALL-resident) must not queue behind the weights streamed from HBM.
// Every load in issue() is unconditional (indices clamped, results masked
// arithmetically) so the compiler can wait for exactly the prologue's loads
// while the weight loads stay outstanding.
template <int PRO, int FMT>
struct GemvPrologue {
  static constexpr bool kRmsFH = PRO == PRO_RMSFH || PRO == PRO_RMSF2H;  // 2 replicas
  static constexpr bool kRmsF = PRO == PRO_RMSF || PRO == PRO_RMSF2 || kRmsFH;
  static constexpr int NREP = kRmsFH ? 2 : kRep;  // replicas of the fixed-point residual
  static constexpr bool kRms = PRO == PRO_RMS || PRO == PRO_RMS2 || kRmsF;
  static constexpr int R = (PRO == PRO_RMS2 || PRO == PRO_RMSF2 || PRO == PRO_RMSF2H) ? 2 : 1;  // float4s of the residual row per thread
  float4 x[R], w[R];
  ulonglong2 fx[kRmsF ? R : 1][NREP][2];  // RMSF: the 4 elements' replicas
  float4 p[2][kMaxPart];  // RMS: partials per float4 (R rows); SWIGLU: [0] gate, [1] up partials
  static constexpr int kSlotLanes = 8;  // ATTN: lanes sharing one float4, splitting its chunk slots
  static constexpr bool kAttn = PRO == PRO_ATTN || PRO == PRO_ATTN3;
  // chunk slots per lane: 16 per float4 and round trip, or 32 for the long-
  // window combine (up to 32 chunks per head in one round trip; the short
  // windows keep the smaller first load)
  static constexpr int kSlotsPerLane = PRO == PRO_ATTN3 ? 4 : 2;
  float2 ml[kSlotsPerLane];  // ATTN: (m, l) and accumulators of this lane's chunk slots
  float4 ac[kSlotsPerLane];
  int nact;
  bool fast;  // float4 path (else element-wise, for odd fp16 shapes)

  __device__ __forceinline__ void load_parts(const float* base, int n, int stride, int k, float4* dst) {
#pragma unroll
    for (int j = 0; j < kMaxPart; j++)
      dst[j] = *reinterpret_cast<const float4*>(base + (size_t)max(min(j, n - 1), 0) * stride + k);
  }
  __device__ __forceinline__ float4 sum_loaded(const float4* src, int n) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kMaxPart; j++) {
      const float m = j < n ? 1.f : 0.f;
      s = make_float4(fmaf(src[j].x, m, s.x), fmaf(src[j].y, m, s.y), fmaf(src[j].z, m, s.z), fmaf(src[j].w, m, s.w));
    }
    return s;
  }
  // Loads of the float4 at slice index f (clamped into the slice and the
  // input); ATTN: chunks [jb, jb + 8), clamped to `lim` chunks.
  __device__ __forceinline__ void load_slice4(const GemvArgs& a, int f, int k0, int n4, int jb, int lim) {
    const int kc = min(k0 + 4 * min(f, n4 - 1), a.K - 4);
    if (PRO == PRO_COPY) {
      x[0] = *reinterpret_cast<const float4*>(a.in + kc);
    } else if (PRO == PRO_SWIGLU) {
      load_parts(a.pin, a.n_pin, a.pin_stride, kc, p[0]);
      load_parts(a.pin + a.up_off, a.n_pin, a.pin_stride, kc, p[1]);
    } else if (kAttn) {
      // slots jb + (lane & 7) + 8u of the float4 at f
      const int row = kc / a.att_D, d = kc % a.att_D;
      const float* mlp = a.pml + (size_t)row * a.att_nsplit * 2;
      const float* acp = a.pacc + (size_t)row * a.att_nsplit * a.att_D + d;
      const int sl = threadIdx.x & (kSlotLanes - 1);
#pragma unroll
      for (int u = 0; u < kSlotsPerLane; u++) {
        const int j = min(jb + sl + kSlotLanes * u, lim - 1);
        ml[u] = *reinterpret_cast<const float2*>(mlp + 2 * j);
        ac[u] = *reinterpret_cast<const float4*>(acp + (size_t)j * a.att_D);
      }
    }
  }

  __device__ __forceinline__ void issue(const GemvArgs& a, int k0, int klen_pad) {
    const int tid = threadIdx.x, nt = blockDim.x;
    fast = (a.K & 3) == 0 && (!kAttn || (a.att_D & 3) == 0);
    if (kRms) {
      const int K4 = a.K >> 2;
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int f = min(tid + r * nt, K4 - 1);
        // a wave holding no element of the row issues no loads (wave-uniform):
        // each vector load instruction costs the CU's memory pipeline the same
        // time whether its lanes read one cache line or sixteen
        const bool held = (tid & ~63) + r * nt < K4;
        if (held) {
          w[r] = *reinterpret_cast<const float4*>(a.norm_w + 4 * f);
          if (kRmsF) {
#pragma unroll
            for (int q = 0; q < NREP; q++) {
              const ulonglong2* src = reinterpret_cast<const ulonglong2*>(a.acc_in + (size_t)q * a.K + 4 * f);
              fx[kRmsF ? r : 0][q][0] = src[0];
              fx[kRmsF ? r : 0][q][1] = src[1];
            }
          } else {
            x[r] = *reinterpret_cast<const float4*>(a.base + 4 * f);
            load_parts(a.pin, a.n_pin, a.pin_stride, 4 * f, p[r]);
          }
        } else {
          w[r] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (kRmsF) {
#pragma unroll
            for (int q = 0; q < NREP; q++) fx[kRmsF ? r : 0][q][0] = fx[kRmsF ? r : 0][q][1] = make_ulonglong2(0, 0);
          } else {
            x[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int j = 0; j < kMaxPart; j++) p[r][j] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
      }
    } else if (fast) {
      // ATTN: the first chunk slots are read before the position is known
      // (slots past the active count are masked in attn_finish)
      load_slice4(a, kAttn ? tid / kSlotLanes : tid, k0, klen_pad / 4, 0, a.att_nsplit);
    }
  }

  // silu(gate) * up (TSLSiLUMul.ts:15-29) or the flash-decoding combine of the
  // attention chunk partials for the float4 loaded by load_slice4.
  __device__ __forceinline__ float4 value4(const GemvArgs& a, int f, int k0, int n4) {
    if (PRO == PRO_COPY) return x[0];
    if (PRO == PRO_SWIGLU) {
      const float4 g = sum_loaded(p[0], a.n_pin), u = sum_loaded(p[1], a.n_pin);
      return make_float4(g.x / (1.f + __expf(-g.x)) * u.x, g.y / (1.f + __expf(-g.y)) * u.y,
                         g.z / (1.f + __expf(-g.z)) * u.z, g.w / (1.f + __expf(-g.w)) * u.w);
    }
    return x[0];  // not reached for the attention prologues (attn_finish)
  }

  // Flash-decoding combine of the attention chunk partials: eight lanes share
  // one float4 (4 dims of one head) and split its active chunk slots; each
  // lane merges its slots online, then the eight merge with DPP (max, then the
  // rescaled sums).  Every lane of the wave takes part.
  __device__ __forceinline__ void attn_finish(const GemvArgs& a, float* xl, float* xsum, int k0, int klen_pad) {
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, sl = tid & (kSlotLanes - 1);
    const int n4 = klen_pad / 4, per = nt / kSlotLanes;
    constexpr int SB = kSlotLanes * kSlotsPerLane;  // slots per batch
    for (int fb = 0; fb < n4; fb += per) {
      const int f = fb + tid / kSlotLanes;
      if (fb > 0) load_slice4(a, f, k0, n4, 0, a.att_nsplit);
      float M = -INFINITY, L = 0.f;
      float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int jb = 0; jb < nact; jb += SB) {
        if (jb > 0) load_slice4(a, f, k0, n4, jb, nact);
        float Mb = M;
#pragma unroll
        for (int u = 0; u < kSlotsPerLane; u++)
          Mb = jb + sl + kSlotLanes * u < nact ? fmaxf(Mb, ml[u].x) : Mb;
        const float sc = M == -INFINITY ? 0.f : __expf(M - Mb);
        L *= sc;
        O = make_float4(O.x * sc, O.y * sc, O.z * sc, O.w * sc);
#pragma unroll
        for (int u = 0; u < kSlotsPerLane; u++) {
          // selects, not products: slots past nact may hold anything
          const bool use = jb + sl + kSlotLanes * u < nact && ml[u].x != -INFINITY;
          const float e = use ? __expf(ml[u].x - Mb) : 0.f;
          L = use ? fmaf(ml[u].y, e, L) : L;
          O.x = use ? fmaf(ac[u].x, e, O.x) : O.x;
          O.y = use ? fmaf(ac[u].y, e, O.y) : O.y;
          O.z = use ? fmaf(ac[u].z, e, O.z) : O.z;
          O.w = use ? fmaf(ac[u].w, e, O.w) : O.w;
        }
        M = Mb;
      }
      // merge the eight lanes of the float4
      float Mg = fmaxf(M, dpp<kDppXor1>(M));
      Mg = fmaxf(Mg, dpp<kDppXor2>(Mg));
      Mg = fmaxf(Mg, dpp<kDppHalfMirror>(Mg));
      const float sc = M == -INFINITY ? 0.f : __expf(M - Mg);
      const float Lg = sum8(L * sc);
      float4 y = make_float4(sum8(O.x * sc), sum8(O.y * sc), sum8(O.z * sc), sum8(O.w * sc));
      const float il = 1.f / Lg;
      y = make_float4(y.x * il, y.y * il, y.z * il, y.w * il);
      const bool valid = f < n4 && k0 + 4 * f < a.K;
      if (!valid) y = make_float4(0.f, 0.f, 0.f, 0.f);
      if (sl == 0 && f < n4) *reinterpret_cast<float4*>(xl + 4 * f) = y;
      if (FMT == WF_Q4) {
        // a wave's eight float4s are one aligned 32-element group
        const float gsum = wave_sum(sl == 0 ? (y.x + y.y) + (y.z + y.w) : 0.f);
        const int f0 = fb + (tid >> 6) * (64 / kSlotLanes);
        if (lane == 0 && f0 < n4) xsum[f0 / 8] = gsum;
      }
    }
  }

  // Residual row float4 r: base + partials, or the sum of the fixed-point replicas.
  __device__ __forceinline__ float4 residual4(const GemvArgs& a, int r) {
    if (kRmsF) {
      if (a.ps_words) {  // published words: the fp32 value in the low half, partials summed in order
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int q = 0; q < NREP; q++) {
          y.x += __uint_as_float((unsigned)fx[kRmsF ? r : 0][q][0].x);
          y.y += __uint_as_float((unsigned)fx[kRmsF ? r : 0][q][0].y);
          y.z += __uint_as_float((unsigned)fx[kRmsF ? r : 0][q][1].x);
          y.w += __uint_as_float((unsigned)fx[kRmsF ? r : 0][q][1].y);
        }
        return y;
      }
      unsigned long long s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
      for (int q = 0; q < NREP; q++) {
        s0 += fx[kRmsF ? r : 0][q][0].x;
        s1 += fx[kRmsF ? r : 0][q][0].y;
        s2 += fx[kRmsF ? r : 0][q][1].x;
        s3 += fx[kRmsF ? r : 0][q][1].y;
      }
      const float4 y = make_float4(from_fx(s0), from_fx(s1), from_fx(s2), from_fx(s3));
      fx_guard(fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w))), a.ctrl);
      return y;
    }
    return f4add(x[r], sum_loaded(p[r], a.n_pin));
  }

  // xm (optional, RMS prologues): receives the un-normalised residual row.
  __device__ void finish(const GemvArgs& a, float* xl, float* xsum, float* scratch, int k0, int k1, int klen_pad,
                         float* xm = nullptr) {
    const int tid = threadIdx.x, nt = blockDim.x;
    // the position is read here, after the weight loads are issued
    if (kAttn) nact = chunk_plan(a.ctrl[C_POS], a.att_window, a.att_nsplit, a.att_chmin).nact;
    if (kRms) {
      // residual stream x = base + sum(pin), then TSLRMSNorm.ts:50-74 over all K
      const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && a.xout != nullptr;
      const int K4 = a.K >> 2;
      float4 v[R];
      float ss = 0.f;
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int f = tid + r * nt;
        v[r] = residual4(a, r);
        const float m = f < K4 ? 1.f : 0.f;
        ss = fmaf(v[r].x * m, v[r].x, ss);
        ss = fmaf(v[r].y * m, v[r].y, ss);
        ss = fmaf(v[r].z * m, v[r].z, ss);
        ss = fmaf(v[r].w * m, v[r].w, ss);
        if (writer && f < K4) *reinterpret_cast<float4*>(a.xout + 4 * f) = v[r];
        if (xm && f < K4) *reinterpret_cast<float4*>(xm + 4 * f) = v[r];
      }
      const float inv = rsqrtf(block_sum(ss, scratch) / (float)a.K + a.eps);
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int k = 4 * (tid + r * nt);
        const float4 y = make_float4(v[r].x * inv * w[r].x, v[r].y * inv * w[r].y, v[r].z * inv * w[r].z,
                                     v[r].w * inv * w[r].w);
        put4<FMT>(xl, xsum, k - k0, y, k >= k0 && k < k1);
      }
      for (int i = (k1 - k0) + tid; i < klen_pad; i += nt) xl[i] = 0.f;  // slice padding past K
    } else if (!fast) {
      // element-wise path for shapes the float4 path cannot cover (fp16 weights
      // only: q4 needs K % 32 == 0, so no group sums here)
      for (int i = tid; i < klen_pad; i += nt) {
        const int k = k0 + i;
        float y = 0.f;
        if (k < a.K) {
          if (PRO == PRO_COPY) {
            y = a.in[k];
          } else if (PRO == PRO_SWIGLU) {
            const float g = sum_parts(a.pin, a.n_pin, a.pin_stride, k);
            y = g / (1.f + __expf(-g)) * sum_parts(a.pin + a.up_off, a.n_pin, a.pin_stride, k);
          } else {
            y = attn_combine_elem(a.pacc, a.pml, k / a.att_D, k % a.att_D, a.att_D, a.att_nsplit, nact);
          }
        }
        xl[i] = y;
      }
    } else if (kAttn) {
      attn_finish(a, xl, xsum, k0, klen_pad);
    } else {
      const int n4 = klen_pad / 4;
      for (int fb = 0; fb < n4; fb += nt) {
        const int f = fb + tid;
        if (fb > 0) load_slice4(a, f, k0, n4, 0, 1);
        float4 y = value4(a, f, k0, n4);
        if (!(f < n4 && k0 + 4 * f < a.K)) y = make_float4(0.f, 0.f, 0.f, 0.f);
        put4<FMT>(xl, xsum, 4 * f, y, f < n4);
      }
    }
  }
};


// NCH: chunks a wave keeps in flight per batch (>= its chunk count when that
// fits, so no load is a clamped duplicate).  STREAM: weights read once per
// token with nothing to gain from caching (the LM head) are loaded
// non-temporally.  The LM head's 273 MB would otherwise evict the layers'
// weights (201 MB at the Qwen2.5-0.5B shape) from the 256 MB last-level cache
// that keeps them between tokens: measured 496 -> 455 us per decode token.
template <int FMT, int NCH, bool STREAM = false>
struct GemvCore {
  static constexpr int CK = FMT == WF_Q4 ? 32 : 8;  // k per 16-byte chunk
  uint4 d[NCH];
  uint16_t sc[NCH];

  // Loads of batch b: unconditional (chunk index clamped to this wave's last
  // chunk, or to the slice's last chunk for a wave without chunks), so the
  // whole batch is in flight at once and the compiler can count exactly which
  // loads each use waits for.
  __device__ __forceinline__ void load(const GemvArgs& a, int t, int c0, int ncl, int wave, int W, int nw, int b) {
    const int lane = threadIdx.x & 63;
    const uint4* wt = a.w + (size_t)t * a.C * kTile;
#pragma unroll
    for (int u = 0; u < NCH; u++) {
      const int c = c0 + min(wave + min(b + u, max(nw, 1) - 1) * W, ncl - 1);
      if (STREAM) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + (size_t)c * kTile + lane));
        d[u] = make_uint4(v.x, v.y, v.z, v.w);
        if (FMT == WF_Q4) sc[u] = __builtin_nontemporal_load(a.s + ((size_t)t * a.C + c) * kTile + lane);
      } else {
        d[u] = wt[(size_t)c * kTile + lane];
        if (FMT == WF_Q4) sc[u] = a.s[((size_t)t * a.C + c) * kTile + lane];
      }
    }
  }

  __device__ __forceinline__ float compute(const float* xl, const float* xsum, int wave, int W, int nw, int b) const {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < NCH; u++) {
      if (b + u < nw) {  // wave-uniform
        const int cl = wave + (b + u) * W;
        if (FMT == WF_Q4)
          acc += dot_q4(d[u], xl + cl * CK, xsum[cl], h2f(sc[u]));
        else
          acc += dot_f16(d[u], xl + cl * CK);
      }
    }
    return acc;
  }
};

// Shared LDS carve-up of the GEMV kernels: x slice, q4 group sums, the
// cross-wave reduction and block-reduce scratch.
struct GemvSmem {
  float* xl;
  float* xsum;
  float* red;
  float* scratch;
  __device__ GemvSmem(float* sm, int cps, int CK, int W) {
    xl = sm;
    xsum = xl + cps * CK;
    red = xsum + cps;
    scratch = red + W * kTile;
  }
};

template <int FMT, int PRO, int W, int NCH>
__global__ __launch_bounds__(W * 64) void gemv_kernel(GemvArgs a) {
  extern __shared__ float sm[];
  constexpr int CK = GemvCore<FMT, NCH>::CK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s = blockIdx.y;
  const int c0 = s * a.cps, c1 = min(a.C, c0 + a.cps);
  const int ncl = c1 - c0;
  const int k0 = c0 * CK, k1 = min(a.K, c1 * CK);
  GemvSmem L(sm, a.cps, CK, W);
  const int nw = wave < ncl ? (ncl - wave + W - 1) / W : 0;

  GemvPrologue<PRO, FMT> pro;
  pro.issue(a, k0, ncl * CK);
  GemvCore<FMT, NCH> core;
  int t = blockIdx.x;
  if (a.zero_ptr) {  // clears an accumulator for a later kernel: each block a slice
    const int nb = gridDim.x * gridDim.y, bid = blockIdx.y * gridDim.x + blockIdx.x;
    const int per = (a.zero_n + nb - 1) / nb;
    for (int i = bid * per + threadIdx.x; i < min(a.zero_n, (bid + 1) * per); i += blockDim.x) a.zero_ptr[i] = 0ull;
  }
  core.load(a, t, c0, ncl, wave, W, nw, 0);  // weights in flight during the prologue (t < T: gridDim.x <= T)
  __builtin_amdgcn_sched_barrier(0);  // keep every load issued before the prologue's first wait
  pro.finish(a, L.xl, L.xsum, L.scratch, k0, k1, ncl * CK);
  lds_barrier();
  auto reduce_store = [&](int tt, float acc) {
    L.red[wave * kTile + lane] = acc;
    lds_barrier();
    if (wave == 0) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; w++) v += L.red[w * kTile + lane];
      const int row = tt * kTile + lane;
      if (row < a.N) {
        if (a.bias && s == 0) v += a.bias[row];
        a.out[(size_t)s * a.N + row] = v;
      }
    }
    lds_barrier();
  };
  // The first tile's first batch (in flight since before the prologue) in
  // straight-line code: each dot then waits for its own chunk only (inside
  // the loops the compiler's waits merge over the back edges).
  {
    float acc = core.compute(L.xl, L.xsum, wave, W, nw, 0);
    for (int b = NCH; b < nw; b += NCH) {
      core.load(a, t, c0, ncl, wave, W, nw, b);
      acc += core.compute(L.xl, L.xsum, wave, W, nw, b);
    }
    reduce_store(t, acc);
  }
  for (t += gridDim.x; t < a.T; t += gridDim.x) {
    float acc = 0.f;
    for (int b = 0; b < nw; b += NCH) {
      core.load(a, t, c0, ncl, wave, W, nw, b);
      acc += core.compute(L.xl, L.xsum, wave, W, nw, b);
    }
    reduce_store(t, acc);
  }
}

// The persistent schedule's token number advances once its token is done
// (never 0: zeroed words never match).
__device__ __forceinline__ int ps_next_seq(int cur) {
  const unsigned seq = (unsigned)cur + 1u;
  return (int)(seq ? seq : 1u);
}
// LM head: GEMV over the vocabulary (PRO_COPY input) with the first pass of
// the greedy sampler fused in (createChunkPartialMaxNode, TSLLogits.ts:201-248):
// each block keeps its best (score, id) over its tiles.
template <int FMT, int PRO, int W, int NCH>
__global__ __launch_bounds__(W * 64) void lm_head_kernel(GemvArgs a) {
  extern __shared__ float sm[];
  constexpr int CK = GemvCore<FMT, NCH>::CK;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ncl = a.C;
  GemvSmem L(sm, a.cps, CK, W);
  const int nw = wave < ncl ? (ncl - wave + W - 1) / W : 0;

  GemvPrologue<PRO, FMT> pro;
  pro.issue(a, 0, ncl * CK);
  GemvCore<FMT, NCH, true> core;
  int t = blockIdx.x;
  core.load(a, t, 0, ncl, wave, W, nw, 0);  // gridDim.x <= T
  __builtin_amdgcn_sched_barrier(0);
  pro.finish(a, L.xl, L.xsum, L.scratch, 0, a.K, ncl * CK);
  __syncthreads();
  if (a.xnorm && blockIdx.x == 0)  // the final hidden state (readHidden)
    for (int k = threadIdx.x; k < a.K; k += blockDim.x) a.xnorm[k] = L.xl[k];
  float best_v = kLowest;
  int best_i = 0x7fffffff;
  for (; t < a.T; t += gridDim.x) {
    float acc = 0.f;
    for (int b = 0; b < nw; b += NCH) {
      if (b > 0 || t != (int)blockIdx.x) core.load(a, t, 0, ncl, wave, W, nw, b);
      acc += core.compute(L.xl, L.xsum, wave, W, nw, b);
    }
    L.red[wave * kTile + lane] = acc;
    __syncthreads();
    if (wave == 0) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; w++) v += L.red[w * kTile + lane];
      const int row = t * kTile + lane;
      if (row < a.N) {
        if (a.logits) a.logits[row] = v;
        if (better(v, row, best_v, best_i)) {
          best_v = v;
          best_i = row;
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    wave_argmax(best_v, best_i);
    if (lane == 0) {
      a.arg_val[blockIdx.x] = best_v;
      a.arg_idx[blockIdx.x] = best_i;
      // the merge as it goes: one device-scope atomic max per block
      if (a.arg_key) {
        const unsigned long long prev =
            __hip_atomic_fetch_max(a.arg_key, greedy_key(best_v, best_i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.arrived) {
          // the count goes out only once the max has returned (performed), so
          // the block that counts last finds every block's best in the key
          asm volatile("" ::"v"((unsigned)prev), "v"((unsigned)(prev >> 32)) : "memory");
          const unsigned n = __hip_atomic_fetch_add(a.arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (n == gridDim.x - 1) {
            int* ctrl = a.mctrl;
            const int step = ctrl[C_STEP], posv = ctrl[C_POS], seqv = ctrl[C_SEQ];
            const unsigned long long k = __hip_atomic_load(a.arg_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // nothing above LOWEST (or nothing folded) -> token 0, as the merge
            const int token = k != 0 && greedy_key_value(k) > kLowest ? greedy_key_id(k) : 0;
            if (a.tokens_out && step >= 0 && step < a.max_steps) a.tokens_out[step] = token;
            ctrl[C_TOKEN] = token;
            ctrl[C_POS] = posv + 1;
            ctrl[C_STEP] = step + 1;
            ctrl[C_SEQ] = ps_next_seq(seqv);
            __hip_atomic_store(a.arg_key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
  }
}

// Second pass of the greedy sampler (createGreedyMergeNode, TSLLogits.ts:250-274):
// one block reduces the per-block partials; a separate launch, so the kernel
// boundary (not a device-scope fence per block) publishes the partials.  In the
// decode graph it also advances the token/position state for the next step.
// Writes the embedding row of `token`, in fixed point, to replica 0 of es.x0
// (all threads of the block take part).
__device__ __forceinline__ void stage_embedding(const EmbStage& es, int token) {
  if (!es.x0) return;
  for (int i = threadIdx.x; i < es.H; i += blockDim.x)
    es.x0[i] = to_fx(es.f32 ? ((const float*)es.emb)[(size_t)token * es.H + i]
                            : h2f(((const uint16_t*)es.emb)[(size_t)token * es.H + i]));
}

__device__ __forceinline__ void ps_next_token(int* ctrl) { ctrl[C_SEQ] = ps_next_seq(ctrl[C_SEQ]); }

__global__ __launch_bounds__(1024) void argmax_merge_kernel(const float* pval, const int* pidx, int n, int* ctrl,
                                                            int* tokens_out, int advance, int max_steps,
                                                            EmbStage es, int ps) {
  __shared__ float sv[16];
  __shared__ int si[16];
  __shared__ int tok_s;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // the control words this block updates, requested with the partials (no
  // other kernel of the step writes them)
  int step = 0, posv = 0, seqv = 0;
  if (threadIdx.x == 0) {
    step = ctrl[C_STEP];
    posv = ctrl[C_POS];
    seqv = ctrl[C_SEQ];
  }
  float bv = kLowest;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    if (better(pval[i], pidx[i], bv, bi)) {
      bv = pval[i];
      bi = pidx[i];
    }
  wave_argmax(bv, bi);
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < nw; w++)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    // the merge starts from (LOWEST, 0): nothing above LOWEST -> token 0
    const int token = bv > kLowest ? bi : 0;
    if (tokens_out && step >= 0 && step < max_steps) tokens_out[step] = token;
    ctrl[C_TOKEN] = token;
    if (advance) {
      ctrl[C_POS] = posv + 1;
      ctrl[C_STEP] = step + 1;
    }
    if (ps) ctrl[C_SEQ] = ps_next_seq(seqv);
    tok_s = token;
  }
  __syncthreads();
  stage_embedding(es, tok_s);
}

void launch_argmax_merge(const float* pval, const int* pidx, int n, int* ctrl, int* tokens_out, int advance,
                         int max_steps, const EmbStage& es, hipStream_t st, int ps) {
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(1), dim3(1024), 0, st, pval, pidx, n, ctrl, tokens_out, advance,
                     max_steps, es, ps);
}

// argmax_merge_kernel's work when the LM head blocks already folded their
// partials into one key (greedy_key): decode it, advance the control words,
// clear the key for the next launch.
__global__ __launch_bounds__(256) void greedy_pick_kernel(unsigned long long* key, int* ctrl, int* tokens_out,
                                                          int advance, int max_steps, EmbStage es, int ps) {
  __shared__ int tok_s;
  if (threadIdx.x == 0) {
    const int step = ctrl[C_STEP], posv = ctrl[C_POS], seqv = ctrl[C_SEQ];
    const unsigned long long k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // nothing above LOWEST (or nothing folded) -> token 0, as the merge
    const int token = k != 0 && greedy_key_value(k) > kLowest ? greedy_key_id(k) : 0;
    if (tokens_out && step >= 0 && step < max_steps) tokens_out[step] = token;
    ctrl[C_TOKEN] = token;
    if (advance) {
      ctrl[C_POS] = posv + 1;
      ctrl[C_STEP] = step + 1;
    }
    if (ps) ctrl[C_SEQ] = ps_next_seq(seqv);
    __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    tok_s = token;
  }
  __syncthreads();
  stage_embedding(es, tok_s);
}

void launch_greedy_pick(unsigned long long* key, int* ctrl, int* tokens_out, int advance, int max_steps,
                        const EmbStage& es, hipStream_t st, int ps) {
  hipLaunchKernelGGL(greedy_pick_kernel, dim3(1), dim3(256), 0, st, key, ctrl, tokens_out, advance, max_steps, es,
                     ps);
}

size_t gemv_smem_bytes(int fmt, int cps, int waves) {
  const int CK = fmt == WF_Q4 ? 32 : 8;
  return sizeof(float) * ((size_t)cps * CK + cps + waves * kTile + 64);
}

bool launch_gemv(int fmt, int pro, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st) {
  const size_t smem = gemv_smem_bytes(fmt, a.cps, waves);
  // the RMS prologue keeps one (PRO_RMS) or two (PRO_RMS2) float4s of the
  // residual row per thread
  if (pro == PRO_RMSF && a.K > 4 * 64 * waves) pro = PRO_RMSF2;
  if (pro == PRO_RMSFH && a.K > 4 * 64 * waves) pro = PRO_RMSF2H;
  if ((pro == PRO_RMSF2 || pro == PRO_RMSF2H) && a.K > 8 * 64 * waves) return false;
  if (pro == PRO_RMS || pro == PRO_RMS2) return false;  // residual + partials: the fused MLP kernel only
#define GEMV_CASE(F, P, Wv, N)                                                          \
  if (fmt == F && pro == P && waves == Wv && nch == N) {                                \
    hipLaunchKernelGGL((gemv_kernel<F, P, Wv, N>), grid, dim3(Wv * 64), smem, st, a);   \
    return true;                                                                        \
  }
#define GEMV_N(F, P, Wv) GEMV_CASE(F, P, Wv, 1) GEMV_CASE(F, P, Wv, 2) GEMV_CASE(F, P, Wv, 4) GEMV_CASE(F, P, Wv, 8)
#define GEMV_W(F, P) GEMV_N(F, P, 4) GEMV_N(F, P, 8)
  GEMV_W(WF_Q4, PRO_COPY)
  GEMV_W(WF_Q4, PRO_RMSF)
  GEMV_W(WF_Q4, PRO_RMSF2)
  GEMV_W(WF_Q4, PRO_RMSFH)
  GEMV_W(WF_Q4, PRO_RMSF2H)
  GEMV_W(WF_Q4, PRO_SWIGLU)
  GEMV_W(WF_Q4, PRO_ATTN)
  GEMV_W(WF_F16, PRO_ATTN)
  GEMV_W(WF_Q4, PRO_ATTN3)
  GEMV_W(WF_F16, PRO_ATTN3)
  GEMV_W(WF_F16, PRO_COPY)
  GEMV_W(WF_F16, PRO_RMSF)
  GEMV_W(WF_F16, PRO_RMSF2)
  GEMV_W(WF_F16, PRO_RMSFH)
  GEMV_W(WF_F16, PRO_RMSF2H)
  GEMV_W(WF_F16, PRO_SWIGLU)
#undef GEMV_W
#undef GEMV_N
#undef GEMV_CASE
  return false;
}

bool launch_lm_head(int fmt, int pro, int waves, int nch, dim3 grid, const GemvArgs& a, hipStream_t st) {
  const size_t smem = gemv_smem_bytes(fmt, a.cps, waves);
  if (pro == PRO_RMSF && a.K > 4 * 64 * waves) pro = PRO_RMSF2;
  if (pro == PRO_RMSFH && a.K > 4 * 64 * waves) pro = PRO_RMSF2H;
  if ((pro == PRO_RMSF2 || pro == PRO_RMSF2H) && a.K > 8 * 64 * waves) return false;
#define LM_CASE(F, P, Wv, N)                                                               \
  if (fmt == F && pro == P && waves == Wv && nch == N) {                                   \
    hipLaunchKernelGGL((lm_head_kernel<F, P, Wv, N>), grid, dim3(Wv * 64), smem, st, a);   \
    return true;                                                                           \
  }
#define LM_N(F, P, Wv) LM_CASE(F, P, Wv, 1) LM_CASE(F, P, Wv, 2) LM_CASE(F, P, Wv, 4) LM_CASE(F, P, Wv, 8) \
  LM_CASE(F, P, Wv, 16)
#define LM_P(F, Wv) LM_N(F, PRO_COPY, Wv) LM_N(F, PRO_RMSF, Wv) LM_N(F, PRO_RMSF2, Wv) LM_N(F, PRO_RMSFH, Wv) \
  LM_N(F, PRO_RMSF2H, Wv)
  LM_P(WF_F16, 4) LM_P(WF_F16, 8) LM_P(WF_Q4, 4) LM_P(WF_Q4, 8)
#undef LM_P
#undef LM_N
#undef LM_CASE
  return false;
}

// ------------------------------------------------------------------- MLP --

// Row tile of a block's i-th down item: rotated by the block index, so the
// blocks adding into one accumulator replica do not walk its rows in lockstep
// (the fixed-point sums do not depend on the order).  Llama-3.2-3B shape at
// 16384 positions: 1420 -> 1402 us per token; Llama-3.2-1B at 4096: 540 -> 534.
__device__ __forceinline__ int mlp_down_tile(int i, int blk, int Td) { return (i + blk) % Td; }

// Down-projection slice of one block: (tile, chunk) items over the block's 32
// intermediate indices; item = tile * CPG + chunk, this wave's items are
// wave, wave + W, ...  Loads are unconditional (items clamped).
template <int FMT, int DB>
struct MlpDown {
  static constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  static constexpr int CPG = 32 / CK;  // chunks per 32-index group
  uint4 d[DB];
  uint16_t sc[DB];
  __device__ __forceinline__ void load(const MlpArgs& m, int blk, int wave, int W, int nd, int nitems, int ib) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < DB; u++) {
      const int item = min(wave + min(ib + u, max(nd, 1) - 1) * W, nitems - 1);
      const int td = mlp_down_tile(item / CPG, blk, m.Td), c = min(blk * CPG + item % CPG, m.Cd - 1);
      const size_t at = ((size_t)td * m.Cd + c) * kTile + lane;
      d[u] = m.wd[at];
      if (FMT == WF_Q4) sc[u] = m.sd[at];
    }
  }
};

// One block per 32 intermediate indices i0 = 32 * blockIdx.x:
//   x_mid = base + sum of the O partials (TSLAdd.ts:10-33), RMSNorm
//   (TSLRMSNorm.ts:50-74), [g | u] = rows of the paired gate|up tile,
//   h = silu(g) * u (TSLSiLUMul.ts:15-29), then the down columns i0..i0+31:
//   y[n] += sum_i Wd[n][i0 + i] h[i], added in fixed point to replica
//   (block % nrep, nrep a power of two) of the accumulator; block 0 also adds x_mid (the residual).
// TSLGatedMLP.ts:17-90 computes the same product as three dispatches.
template <int FMT, int PRO, int NCH, int DB>
__global__ __launch_bounds__(kMlpWaves * 64) void mlp_kernel(MlpArgs m) {
  extern __shared__ float sm[];
  constexpr int W = kMlpWaves;
  constexpr int CK = GemvCore<FMT, NCH>::CK;
  using Down = MlpDown<FMT, DB>;
  const GemvArgs& a = m.g;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = blockIdx.x, C = a.C;
  float* xl = sm;               // [C * CK] normed x
  float* xsum = xl + C * CK;    // [C] q4 group sums
  float* red = xsum + ((C + 3) & ~3);  // [W][64] (keeps h and xm 16-byte aligned)
  float* scratch = red + W * kTile;
  float* h = scratch + 64;      // [32] silu(g) * u, then their sum
  float* xm = h + 64;           // [K] x_mid (block 0)
  const int nw = wave < C ? (C - wave + W - 1) / W : 0;
  const int nitems = m.Td * Down::CPG;
  const int nd = wave < nitems ? (nitems - wave + W - 1) / W : 0;

  GemvPrologue<PRO, FMT> pro;
  pro.issue(a, 0, C * CK);
  GemvCore<FMT, NCH> core;
  core.load(a, blk, 0, C, wave, W, nw, 0);
  Down dn;
  dn.load(m, blk, wave, W, nd, nitems, 0);
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the prologue's first wait
  pro.finish(a, xl, xsum, scratch, 0, a.K, C * CK, blk == 0 ? xm : nullptr);
  lds_barrier();

  // first batch in straight-line code: each dot waits for its own chunk only
  float acc = core.compute(xl, xsum, wave, W, nw, 0);
  for (int b = NCH; b < nw; b += NCH) {
    core.load(a, blk, 0, C, wave, W, nw, b);
    acc += core.compute(xl, xsum, wave, W, nw, b);
  }
  red[wave * kTile + lane] = acc;
  lds_barrier();
  if (wave == 0) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < W; w++) v += red[w * kTile + lane];
    // lanes 0..31 hold g, lanes 32..63 the matching u: h = silu(g) * u in
    // lanes 32..63 (padded indices have zero rows, so their h is 0)
    const float g = __shfl(v, lane & 31, 64);
    const float hv = g / (1.f + __expf(-g)) * v;
    if (lane >= 32) h[lane - 32] = hv;
    const float hs = wave_sum(lane >= 32 ? hv : 0.f);
    if (lane == 0) h[32] = hs;
  }
  lds_barrier();

  const float hsum = h[32];
  auto down_batch = [&](int ib) {
#pragma unroll
    for (int u = 0; u < DB; u++) {
      if (ib + u < nd) {  // wave-uniform
        const int item = wave + (ib + u) * W;
        const int td = mlp_down_tile(item / Down::CPG, blk, m.Td), cc = item % Down::CPG;
        const float p = FMT == WF_Q4 ? dot_q4(dn.d[u], h, hsum, h2f(dn.sc[u])) : dot_f16(dn.d[u], h + cc * CK);
        const int n = td * kTile + lane;
        if (n < m.H) {
          fx_guard(p, a.ctrl);
          atomicAdd(m.acc + (size_t)(blk & (m.nrep - 1)) * m.H + n, to_fx(p));
        }
      }
    }
  };
  down_batch(0);  // straight-line: its loads were issued before the prologue
  for (int ib = DB; ib < nd; ib += DB) {
    dn.load(m, blk, wave, W, nd, nitems, ib);
    down_batch(ib);
  }
  if (blk == 0)
    for (int n = threadIdx.x; n < m.H; n += blockDim.x) {
      fx_guard(xm[n], a.ctrl);
      atomicAdd(m.acc + n, to_fx(xm[n]));
    }
}

size_t mlp_smem_bytes(int fmt, int C, int K) {
  const int CK = fmt == WF_Q4 ? 32 : 8;
  return sizeof(float) * ((size_t)C * CK + ((C + 3) & ~3) + kMlpWaves * kTile + 64 + 64 + K);
}

bool launch_mlp(int fmt, int nch, int ndb, int blocks, const MlpArgs& m, hipStream_t st) {
  const size_t smem = mlp_smem_bytes(fmt, m.g.C, m.g.K);
  int pro = m.g.K > 4 * 64 * kMlpWaves ? PRO_RMS2 : PRO_RMS;
  if (m.g.K > 8 * 64 * kMlpWaves) return false;
#define MLP_CASE(F, P, N, D)                                                                          \
  if (fmt == F && pro == P && nch == N && ndb == D) {                                                 \
    hipLaunchKernelGGL((mlp_kernel<F, P, N, D>), dim3(blocks), dim3(kMlpWaves * 64), smem, st, m);    \
    return true;                                                                                      \
  }
#define MLP_D(F, P, N) MLP_CASE(F, P, N, 1) MLP_CASE(F, P, N, 2) MLP_CASE(F, P, N, 4)
#define MLP_N(F, P) MLP_D(F, P, 1) MLP_D(F, P, 2) MLP_D(F, P, 4) MLP_D(F, P, 8)
  MLP_N(WF_Q4, PRO_RMS)
  MLP_N(WF_Q4, PRO_RMS2)
  MLP_N(WF_F16, PRO_RMS)
  MLP_N(WF_F16, PRO_RMS2)
#undef MLP_N
#undef MLP_D
#undef MLP_CASE
  return false;
}

// ------------------------------------------------------------- attention --

int attn_lpp(int D, bool kv_f32) { return head_tiling(attn_dt(D), kv_f32 ? 4 : 2).lpp; }

// LDS of a head_kernel block: one wave region per wave, then (long windows)
// the merge area [kAttnWaves][2 + DT] (max, sum, unnormalised output of each wave).
size_t attn_smem_bytes(int gmax, int D, bool kv_f32, bool long_win) {
  (void)gmax;
  const int dt = attn_dt(D), esz = kv_f32 ? 4 : 2, nw = long_win ? kAttnWaves : 1;
  return sizeof(float) * ((size_t)nw * head_wave_floats(dt, esz) + (long_win ? (size_t)nw * (2 + dt) : 0));
}


// One block = one query head x one chunk of positions (split-K over the
// sequence, flash decoding; TSLAttention.ts:306-428 computes the same scores
// and softmax over the whole window).  Short windows (LONG false): one wave
// per block, block b = head b % Hq, chunk b / Hq.  Long windows (LONG): a
// chunk longer than 32 positions is split over up to kAttnWaves waves that
// merge (max, sum, output) in LDS at the end, so the combine downstream folds
// kAttnWaves times fewer partials, and the block numbering is XCD-aware
// (below).  The host captures one graph per mode and picks it per position.
// Each wave
//   * forms its q head and the KV head's new k and v from the QKV partial sums
//     + bias and applies RoPE (rotate-half, TSLAttention.ts:168-250),
//   * in the chunk holding `pos`, appends k and v to the cache (head g == 0 of
//     the group writes; TSLAttention.ts:252-286) and uses the rounded row,
//   * per pass of SUB positions: scores from the K rows in registers, an online
//     softmax with DPP wave reductions, P.V from the V rows staged in LDS,
//   * writes (max, sum, unnormalised output) for the combine.
// All global loads of the first pass are unconditional and issued before the
// first use; until the merge a wave touches only its own LDS region.
template <typename KT, int DT, bool LONG>
__global__ __launch_bounds__(64 * (LONG ? kAttnWaves : 1)) void head_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  constexpr int ESZ = sizeof(KT);
  constexpr HeadTiling TL = head_tiling(DT, ESZ);
  constexpr int LPP = TL.lpp, SUB = TL.sub, DL = TL.dl;
  constexpr bool GEN = DT == 32;  // runtime head_dim <= 32
  constexpr int EPL = DT > 64 ? DT / 64 : 1;  // q/k/v elements per lane (d = lane + 64 e)
  constexpr int KW = DL * ESZ / 4;            // K dwords per lane
  // fp16 cache, head_dim 128: the output dims of a lane are adjacent (P.V)
  constexpr bool PAIRD = !GEN && ESZ == 2 && DT == 128;
  constexpr int NW = LONG ? kAttnWaves : 1;
  const int G = a.G, b = blockIdx.x;
  int hk, c, h, g;
  if (LONG) {
    // Block -> (query head, chunk): workgroups go to the 8 XCDs round robin
    // (block b to XCD b % 8), so the G query heads of one (kv head, chunk)
    // pair take blocks 8 apart on one XCD and its L2 serves their shared K/V
    // rows: HBM reads each cached row once instead of once per query head.
    const int slot = b >> 3, pair = (slot / G) * 8 + (b & 7);
    if (pair >= a.Hkv * a.nsplit) return;
    g = slot % G;
    hk = pair % a.Hkv;
    c = pair / a.Hkv;
    h = hk * G + g;
  } else {
    if (b >= a.Hq * a.nsplit) return;
    h = b % a.Hq;
    c = b / a.Hq;
    hk = h / G;
    g = h % G;
  }
  const int lane = threadIdx.x & 63, wv = LONG ? threadIdx.x >> 6 : 0;
  const int D = GEN ? a.D : DT;
  const int pos = a.ctrl[C_POS];
  if (pos < 0 || pos >= a.max_tokens) return;
  const ChunkPlan cp = chunk_plan(pos, a.window, a.nsplit, a.chmin);
  if (c >= cp.nact) return;
  // the block's chunk [b0, b1), split over nwu <= kAttnWaves waves of at least
  // 32 positions (block-uniform); this wave's part [t0, t1) may be empty
  const int b0 = cp.first + c * cp.chunk, b1 = min(b0 + cp.chunk, pos + 1);
  const int nwu = LONG ? min(NW, (b1 - b0 + 31) / 32) : 1;
  if (nwu == 1 && wv != 0) return;  // one wave does the whole chunk, no merge
  const int sc = (b1 - b0 + nwu - 1) / nwu;
  const int t0 = min(b0 + wv * sc, b1), t1 = min(t0 + sc, b1);
  const bool own = pos >= t0 && pos < t1;
  float* q_l = sm + wv * head_wave_floats(DT, ESZ);  // [DT]
  float* kn = q_l + DT;       // [DT] new k (rounded like the cache)
  float* vn = kn + DT;        // [DT]
  float* raw = vn + DT;       // [3][DT] pre-RoPE q, k, v
  float* p_l = raw + 3 * DT;  // [SUB]
  KT* vt = reinterpret_cast<KT*>(p_l + SUB);  // [SUB][DT] V rows of the pass (4 KiB)
  const KT* kh = reinterpret_cast<const KT*>(a.kc) + (size_t)hk * a.max_tokens * D;
  const KT* vh = reinterpret_cast<const KT*>(a.vc) + (size_t)hk * a.max_tokens * D;
  const int pl = lane / LPP, part = lane % LPP;
  const int half = a.rd > 0 ? a.rd / 2 : 1;  // RoPE table row width

  // q (row 0), new k (row 1), new v (row 2): partial sums + bias, element d = lane + 64 e
  const int QS = a.Hq * D, KS = a.Hkv * D;
  float gp[3][EPL][kMaxPart], gb[3][EPL];
#pragma unroll
  for (int r = 0; r < 3; r++) {
    const int base = r == 0 ? h * D : r == 1 ? QS + hk * D : QS + KS + hk * D;
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const int col = base + min(lane + 64 * e, D - 1);
#pragma unroll
      for (int j = 0; j < kMaxPart; j++)
        gp[r][e][j] = a.src[(size_t)max(min(j, a.n_src - 1), 0) * a.src_stride + col];
      gb[r][e] = a.bias[col];
    }
  }
  float rc[EPL], rs[EPL];  // cos / sin of element d's rotation pair
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = min(lane + 64 * e, D - 1);
    const int j = d < half ? d : d - half;
    rc[e] = a.rope_cos[(size_t)pos * half + min(j, half - 1)];
    rs[e] = a.rope_sin[(size_t)pos * half + min(j, half - 1)];
  }
  // first pass: this lane's K slice and its 64 bytes of the V rows
  HeadLoads<KT, KW, GEN, DL> ld;
  const int row_bytes = D * ESZ;
  // unconditional (the compiler then waits for the prologue loads alone): an
  // empty part is [b1, b1) with b1 >= 1, so its clamped row b1 - 1 is cached
  ld.issue(kh, vh, t0, t1, pl, part, D, row_bytes, lane);
  __builtin_amdgcn_sched_barrier(0);

  // finish q/k/v: sums, RoPE through LDS pairs, cache rounding
#pragma unroll
  for (int r = 0; r < 3; r++)
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      float s = gb[r][e];
#pragma unroll
      for (int j = 0; j < kMaxPart; j++) s = fmaf(gp[r][e][j], j < a.n_src ? 1.f : 0.f, s);
      const int d = lane + 64 * e;
      if (d < D) raw[r * DT + d] = s;
    }
  wave_lds_sync();
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = lane + 64 * e;
    if (d < D) {
      float qv = raw[d], kv = raw[DT + d];
      if (d < a.rd) {
        const int pd = d < half ? d + half : d - half;
        const float sg = d < half ? -1.f : 1.f;
        qv = raw[d] * rc[e] + sg * raw[pd] * rs[e];
        kv = raw[DT + d] * rc[e] + sg * raw[DT + pd] * rs[e];
      }
      q_l[d] = qv;
      const KT kq = kv_store<KT>(kv), vq = kv_store<KT>(raw[2 * DT + d]);
      kn[d] = kv_load<KT>(&kq);
      vn[d] = kv_load<KT>(&vq);
      if (own && g == 0) {
        reinterpret_cast<KT*>(a.kc)[((size_t)hk * a.max_tokens + pos) * D + d] = kq;
        reinterpret_cast<KT*>(a.vc)[((size_t)hk * a.max_tokens + pos) * D + d] = vq;
      }
    }
  }
  for (int d = D + lane; d < DT; d += 64) q_l[d] = kn[d] = 0.f;  // padded dims (generic path)
  wave_lds_sync();

  float m = -INFINITY, l = 0.f, o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) o[e] = 0.f;
  float qr[DL];
#pragma unroll
  for (int e = 0; e < DL; e++) qr[e] = q_l[part * DL + e];
  for (int tb = t0; tb < t1; tb += SUB) {
    // V rows to LDS (the fresh row from vn), K slice of this lane (fresh row from kn)
    if (!GEN) {
#pragma unroll
      for (int j = 0; j < 4; j++) reinterpret_cast<uint4*>(vt)[j * 64 + lane] = ld.vs[j];
    } else {
      for (int i = lane; i < SUB * D; i += 64) vt[i] = vh[(size_t)min(tb + i / D, t1 - 1) * D + i % D];
    }
    const int t = tb + pl;
    const bool valid = t < t1;
    float kf[DL];
#pragma unroll
    for (int e = 0; e < DL; e++)
      kf[e] = ESZ == 2 ? h2f((ld.kw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) : __uint_as_float(ld.kw[e]);
    if (own && t == pos) {
#pragma unroll
      for (int e = 0; e < DL; e++) kf[e] = kn[min(part * DL + e, DT - 1)];
    }
    wave_lds_sync();
    if (own && pos >= tb && pos < tb + SUB)
      for (int d = lane; d < D; d += 64) vt[(size_t)(pos - tb) * D + d] = kv_store<KT>(vn[d]);
    // the next pass's loads overlap this pass's math
    if (tb + SUB < t1) ld.issue(kh, vh, tb + SUB, t1, pl, part, D, row_bytes, lane);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < DL; e++) s = fmaf(qr[e], kf[e], s);
    if (LPP > 1) s += dpp<kDppXor1>(s);
    if (LPP > 2) s += dpp<kDppXor2>(s);
    if (LPP > 4) s += __shfl_xor(s, 4, 64);
    const float sc = valid ? s * a.scale : -INFINITY;
    const float mn = fmaxf(m, wave_max(sc));
    const float p = (valid && mn != -INFINITY) ? __expf(sc - mn) : 0.f;
    const float corr = m == -INFINITY ? 0.f : __expf(m - mn);
    l = l * corr + wave_sum(part == 0 ? p : 0.f);
    m = mn;
    if (part == 0) p_l[pl] = p;
    wave_lds_sync();
    if constexpr (PAIRD) {  // lane owns dims 2 lane, 2 lane + 1: one 4-byte V read per position
      float a0 = o[0] * corr, a1 = o[1] * corr;
#pragma unroll
      for (int u = 0; u < SUB; u++) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(vt + (size_t)u * DT + 2 * lane);
        const float pu = p_l[u];
        a0 = fmaf(pu, h2f(w & 0xFFFFu), a0);
        a1 = fmaf(pu, h2f(w >> 16), a1);
      }
      o[0] = a0;
      o[1] = a1;
    } else {
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const int d = lane + 64 * e;
        float acc = o[e] * corr;
        if (d < D) {
#pragma unroll 8
          for (int u = 0; u < SUB; u++) acc = fmaf(p_l[u], kv_load<KT>(vt + (size_t)u * D + d), acc);
        }
        o[e] = acc;
      }
    }
    wave_lds_sync();
  }
  const size_t row = (size_t)h * a.nsplit + c;
  if (nwu == 1) {  // wave 0 alone: its result is the chunk's partial
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      const int d = PAIRD ? 2 * lane + e : lane + 64 * e;
      if (d < D) a.pacc[row * D + d] = o[e];
    }
    if (lane == 0) {
      a.pml[row * 2] = m;
      a.pml[row * 2 + 1] = l;
    }
    return;
  }
  // merge the waves' (max, sum, output) in wave order; wave 0 writes the chunk's partial
  float* mg = sm + NW * head_wave_floats(DT, ESZ);  // [NW][2 + DT]
  float* mine = mg + wv * (2 + DT);
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = PAIRD ? 2 * lane + e : lane + 64 * e;
    if (d < D) mine[2 + d] = o[e];
  }
  if (lane == 0) {
    mine[0] = m;
    mine[1] = l;
  }
  __syncthreads();  // every wave of the block reaches this once
  if (wv != 0) return;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; w++) M = fmaxf(M, mg[w * (2 + DT)]);
  float wsc[NW], L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; w++) {
    const float mw = mg[w * (2 + DT)];
    wsc[w] = mw == -INFINITY ? 0.f : __expf(mw - M);
    L = fmaf(mg[w * (2 + DT) + 1], wsc[w], L);
  }
  for (int d = lane; d < D; d += 64) {
    float od = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) od = fmaf(mg[w * (2 + DT) + 2 + d], wsc[w], od);
    a.pacc[row * D + d] = od;
  }
  if (lane == 0) {
    a.pml[row * 2] = M;
    a.pml[row * 2 + 1] = L;
  }
}

__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int row = blockIdx.x;
  const int pos = a.ctrl[C_POS];
  if (pos < 0 || pos >= a.max_tokens) return;
  const ChunkPlan cp = chunk_plan(pos, a.window, a.nsplit, a.chmin);
  for (int d = threadIdx.x; d < a.D; d += blockDim.x)
    a.out[(size_t)row * a.D + d] = attn_combine_elem(a.pacc, a.pml, row, d, a.D, a.nsplit, cp.nact);
}

bool launch_attention(bool kv_f32, int gmax, const AttnArgs& a, bool combine, bool long_win, hipStream_t st) {
  if (long_win && a.gqa) {
    const bool ok = !kv_f32 && launch_gqa_attention(a, st);
    if (ok && combine) hipLaunchKernelGGL(attn_combine_kernel, dim3(a.Hq), dim3(128), 0, st, a);
    return ok;
  }
  // long windows: XCD-aware numbering, groups of 8 (kv head, chunk) pairs x G heads
  const dim3 grid(long_win ? (unsigned)(((a.Hkv * a.nsplit + 7) / 8) * 8 * a.G) : (unsigned)(a.Hq * a.nsplit));
  const dim3 block(64 * (long_win ? kAttnWaves : 1));
  const size_t smem = attn_smem_bytes(gmax, a.D, kv_f32, long_win);
  const int dt = attn_dt(a.D);
#define HEAD_CASE(KT, DTV)                                                                        \
  if (dt == DTV) {                                                                                \
    if (long_win) hipLaunchKernelGGL((head_kernel<KT, DTV, true>), grid, block, smem, st, a);     \
    else hipLaunchKernelGGL((head_kernel<KT, DTV, false>), grid, block, smem, st, a);             \
    ok = true;                                                                                    \
  }
  bool ok = false;
  if (kv_f32) {
    HEAD_CASE(float, 32) HEAD_CASE(float, 64) HEAD_CASE(float, 128)
  } else {
    HEAD_CASE(uint16_t, 32) HEAD_CASE(uint16_t, 64) HEAD_CASE(uint16_t, 128)
  }
#undef HEAD_CASE
  if (ok && combine) hipLaunchKernelGGL(attn_combine_kernel, dim3(a.Hq), dim3(128), 0, st, a);
  return ok;
}

// --------------------------------------------------------- small kernels --

// Final norm: x = base + sum(pin); y = rmsnorm(x) * w (one block).
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* x, const float* w, int n, float eps, int offset,
                                                       float* y) {
  __shared__ float scratch[16];
  float ss = 0.f;
  for (int k = threadIdx.x; k < n; k += blockDim.x) ss = fmaf(x[k], x[k], ss);
  const float inv = rsqrtf(block_sum(ss, scratch) / (float)n + eps);
  for (int k = threadIdx.x; k < n; k += blockDim.x) {
    const float s = w == nullptr ? 1.f : offset ? 1.f + w[k] : w[k];
    y[k] = x[k] * inv * s;
  }
}

void launch_rmsnorm(const float* x, const float* w, int n, float eps, int offset, float* y, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, st, x, w, n, eps, offset, y);
}

__global__ void silu_mul_kernel(const float* g, const float* u, int n, float* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = g[i] / (1.f + __expf(-g[i])) * u[i];
}

void launch_silu_mul(const float* g, const float* u, int n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, st, g, u, n, out);
}

__global__ void reduce_kernel(const float* part, int n_part, int stride, const float* bias, int n, float* y) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = bias ? bias[i] : 0.f;
  for (int j = 0; j < n_part; j++) v += part[(size_t)j * stride + i];
  y[i] = v;
}

void launch_reduce(const float* part, int n_part, int stride, const float* bias, int n, float* y, hipStream_t st) {
  hipLaunchKernelGGL(reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, st, part, n_part, stride, bias, n, y);
}

// Greedy argmax of an fp32 vector: block partials, then argmax_merge_kernel.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* logits, int n, float* pval, int* pidx) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float bv = kLowest;
  int bi = 0x7fffffff;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    if (better(logits[i], i, bv, bi)) {
      bv = logits[i];
      bi = i;
    }
  wave_argmax(bv, bi);
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    pval[blockIdx.x] = bv;
    pidx[blockIdx.x] = bi;
  }
}

void launch_argmax(const float* logits, int n, float* pval, int* pidx, int* token, int blocks, hipStream_t st) {
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(blocks), dim3(256), 0, st, logits, n, pval, pidx);
  launch_argmax_merge(pval, pidx, blocks, token, nullptr, 0, 0, EmbStage{}, st);
}

// ---------------------------------------------------------------- top-k --
// Top-k candidates of TSLLogitSampler (TSLLogits.ts:276-330): the k best
// (score, id) in the greedy order (higher score, ties to the lower id),
// scores after the optional softcap cap * tanh(x / cap) (TSLLogits.ts:185-191).
// An entry takes part only if its score is above LOWEST_FLOAT (so -inf and NaN
// never do); slots past the last such entry are (id 0, LOWEST_FLOAT), as the
// reference's selection loops leave them.
// One block selects from up to kTopkSlice entries held in registers (8 per
// lane) as 64-bit order keys: every wave finds its k best by k passes (pass r
// takes the largest key below pass r-1's), then one wave merges the four
// lists the same way.  Deterministic; levels of blocks until one remains.
constexpr int kTopkPer = 8;
constexpr int kTopkSlice = 256 * kTopkPer;

// 64-bit order key of (score, id): the score mapped to an unsigned integer
// with the same order (-0 counts as +0, so equal scores stay equal) in the
// high word, the inverted id in the low word: a larger key is better in the
// greedy order.  0 marks "no candidate".
__device__ __forceinline__ unsigned long long topk_key(float v, int id) {
  const uint32_t u = __float_as_uint(v + 0.f);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ord << 32) | (uint32_t)(~(uint32_t)id);
}
__device__ __forceinline__ float topk_score(unsigned long long key) {
  const uint32_t ord = (uint32_t)(key >> 32);
  return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}
template <int CTRL>
__device__ __forceinline__ void max_u64_step(uint32_t& lo, uint32_t& hi) {
  const uint32_t olo = (uint32_t)dpp<CTRL>((int)lo), ohi = (uint32_t)dpp<CTRL>((int)hi);
  if (ohi > hi || (ohi == hi && olo > lo)) {
    lo = olo;
    hi = ohi;
  }
}
// Largest key of the wave, in every lane: DPP steps within rows of 16, then
// the four rows' results through readlane.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
  uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  max_u64_step<kDppXor1>(lo, hi);
  max_u64_step<kDppXor2>(lo, hi);
  max_u64_step<kDppHalfMirror>(lo, hi);
  max_u64_step<kDppMirror>(lo, hi);
  unsigned long long best = 0;
#pragma unroll
  for (int r = 0; r < 64; r += 16) {
    const unsigned long long v = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)hi, r) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)lo, r);
    best = v > best ? v : best;
  }
  return best;
}

// IDS: the entries are (vals[e], ids[e]) (a merge level) instead of (vals[e], e).
template <bool IDS>
__global__ __launch_bounds__(256) void topk_select_kernel(const float* __restrict__ vals, const int* __restrict__ ids,
                                                          int n, int k, float softcap, float* out_v, int* out_i) {
  __shared__ unsigned long long wk[4][kTopkMax];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t base = (size_t)blockIdx.x * kTopkSlice + wave * 64 * kTopkPer;
  // every load issued before the first use (clamped indices: no branches)
  float x[kTopkPer];
  int xi[kTopkPer];
#pragma unroll
  for (int u = 0; u < kTopkPer; u++) x[u] = vals[min(base + lane + 64 * u, (size_t)n - 1)];
#pragma unroll
  for (int u = 0; u < kTopkPer; u++)
    xi[u] = IDS ? ids[min(base + lane + 64 * u, (size_t)n - 1)] : (int)(base + lane + 64 * u);
  if (softcap > 0.f) {
#pragma unroll
    for (int u = 0; u < kTopkPer; u++) x[u] = softcap * tanhf(x[u] / softcap);
  }
  unsigned long long key[kTopkPer];
#pragma unroll
  for (int u = 0; u < kTopkPer; u++) {
    const bool ok = base + lane + 64 * u < (size_t)n && x[u] > kLowest;  // LOWEST, -inf, NaN: never a candidate
    key[u] = ok ? topk_key(x[u], xi[u]) : 0ull;
  }
  // each wave: its k best in k passes, pass r taking the best key below pass r-1's
  unsigned long long prev = ~0ull;
  for (int r = 0; r < k; r++) {
    unsigned long long best = 0;
#pragma unroll
    for (int u = 0; u < kTopkPer; u++) {
      const unsigned long long c = key[u] < prev ? key[u] : 0ull;
      best = c > best ? c : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) wk[wave][r] = best;
    prev = best;
  }
  __syncthreads();
  if (wave != 0) return;
  // wave 0 merges the 4 lists (4 k <= 64 keys, one per lane)
  const unsigned long long mine = lane < 4 * k ? wk[lane / k][lane % k] : 0ull;
  prev = ~0ull;
  for (int r = 0; r < k; r++) {
    const unsigned long long best = wave_max_u64(mine < prev ? mine : 0ull);
    if (lane == 0) {
      out_v[(size_t)blockIdx.x * k + r] = best ? topk_score(best) : kLowest;
      out_i[(size_t)blockIdx.x * k + r] = best ? (int)~(uint32_t)best : 0;
    }
    prev = best ? best : 0ull;
  }
}

bool launch_topk(const float* logits, int n, int k, float softcap, float* wv, int* wi, size_t wcap, float* out_v,
                 int* out_i, hipStream_t st) {
  if (n <= 0 || k <= 0 || k > kTopkMax) return false;
  int blocks = (n + kTopkSlice - 1) / kTopkSlice;
  if ((size_t)blocks * k > wcap) return false;
  const float* v = logits;
  const int* ids = nullptr;
  float cap = softcap;
  float* bufv[2] = {wv, wv + wcap};
  int* bufi[2] = {wi, wi + wcap};
  for (int level = 0;; level++) {
    const bool last = blocks == 1;
    float* ov = last ? out_v : bufv[level & 1];
    int* oi = last ? out_i : bufi[level & 1];
    if (ids)
      hipLaunchKernelGGL(topk_select_kernel<true>, dim3(blocks), dim3(256), 0, st, v, ids, n, k, cap, ov, oi);
    else
      hipLaunchKernelGGL(topk_select_kernel<false>, dim3(blocks), dim3(256), 0, st, v, ids, n, k, cap, ov, oi);
    if (last) return true;
    v = ov;
    ids = oi;
    cap = 0.f;
    n = blocks * k;
    blocks = (n + kTopkSlice - 1) / kTopkSlice;
  }
}

__global__ void set_ctrl_kernel(int* ctrl, int token, int pos, int step, int base, int len, EmbStage es) {
  if (threadIdx.x == 0) {
    ctrl[C_TOKEN] = token;
    ctrl[C_POS] = pos;
    ctrl[C_STEP] = step;
    ctrl[C_BASE] = base;
    ctrl[C_LEN] = len;
  }
  stage_embedding(es, token);
}

void launch_set_ctrl(int* ctrl, int token, int pos, int step, int base, int len, const EmbStage& es,
                     hipStream_t st) {
  hipLaunchKernelGGL(set_ctrl_kernel, dim3(1), dim3(256), 0, st, ctrl, token, pos, step, base, len, es);
}

__global__ __launch_bounds__(256) void stage_ctrl_kernel(const int* ctrl, EmbStage es) {
  stage_embedding(es, ctrl[C_TOKEN]);
}

void launch_stage_ctrl(const int* ctrl, const EmbStage& es, hipStream_t st) {
  hipLaunchKernelGGL(stage_ctrl_kernel, dim3(1), dim3(256), 0, st, ctrl, es);
}

// prefillChunkComputeNodes' advance node (DecoderTSLRunner.ts:216-225): next
// position, next prompt token.
__global__ void prefill_advance_kernel(int* ctrl, const int* prompt, EmbStage es, int ps) {
  const int pos = ctrl[C_POS] + 1;
  const int i = pos - ctrl[C_BASE];
  const bool next = i >= 0 && i < ctrl[C_LEN];
  const int token = next ? prompt[i] : 0;
  __syncthreads();  // every thread has read ctrl before thread 0 updates it
  if (threadIdx.x == 0) {
    ctrl[C_POS] = pos;
    if (next) ctrl[C_TOKEN] = token;
    if (ps) ps_next_token(ctrl);
  }
  if (next) stage_embedding(es, token);
}

void launch_prefill_advance(int* ctrl, const int* prompt, const EmbStage& es, hipStream_t st, int ps) {
  hipLaunchKernelGGL(prefill_advance_kernel, dim3(1), dim3(256), 0, st, ctrl, prompt, es, ps);
}

// Streaming copy, 16 bytes per lane per iteration.
__global__ __launch_bounds__(256) void copy_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

void launch_copy(uint4* dst, const uint4* src, size_t n16, hipStream_t st) {
  const size_t blocks = std::min<size_t>((n16 + 255) / 256, 8192);
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, src, n16);
}

__global__ void dequant_kernel(int fmt, const uint4* w, const uint16_t* s, int N, int C, int K, float* out) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)N * K) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  const int t = n / kTile, lane = n % kTile;
  if (fmt == WF_Q4) {
    const int c = k / 32;
    const uint8_t* chunk = reinterpret_cast<const uint8_t*>(w + ((size_t)t * C + c) * kTile + lane);
    const uint8_t b = chunk[(k % 32) / 2];
    const int nib = (k & 1) ? (b >> 4) : (b & 15);
    out[idx] = h2f(s[((size_t)t * C + c) * kTile + lane]) * (float)(nib - 8);
  } else {
    const int c = k / 8;
    const uint16_t* chunk = reinterpret_cast<const uint16_t*>(w + ((size_t)t * C + c) * kTile + lane);
    out[idx] = h2f(chunk[k % 8]);
  }
}

void launch_dequant(int fmt, const uint4* w, const uint16_t* s, int N, int T, int C, int K, float* out,
                    hipStream_t st) {
  (void)T;
  const size_t total = (size_t)N * K;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, fmt, w, s, N, C, K,
                     out);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// N(0,1) cache contents for long-context runs (values are not compared with
// anything; they only have to be finite and deterministic).
template <typename KT>
__global__ void kv_fill_kernel(KT* kc, KT* vc, int Hkv, int max_tokens, int D, int count, uint64_t seed) {
  const size_t per = (size_t)Hkv * count * D;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= 2 * per) return;
  const bool is_v = idx >= per;
  const size_t r = is_v ? idx - per : idx;
  const int h = (int)(r / ((size_t)count * D));
  const size_t rem = r % ((size_t)count * D);
  const int t = (int)(rem / D), d = (int)(rem % D);
  const uint64_t a = splitmix64(seed + 2 * idx), b = splitmix64(seed + 2 * idx + 1);
  const float u1 = ((a >> 40) + 0.5f) * (1.f / 16777216.f);
  const float u2 = (b >> 40) * (1.f / 16777216.f);
  const float z = sqrtf(-2.f * __logf(u1)) * __cosf(6.283185307f * u2);
  KT* dst = (is_v ? vc : kc) + ((size_t)h * max_tokens + t) * D + d;
  *dst = kv_store<KT>(z);
}

void launch_kv_fill(void* kc, void* vc, bool f32, size_t heads_stride, int Hkv, int max_tokens, int D, int count,
                    uint64_t seed, hipStream_t st) {
  (void)heads_stride;
  const size_t total = 2 * (size_t)Hkv * count * D;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (f32)
    hipLaunchKernelGGL(kv_fill_kernel<float>, grid, dim3(256), 0, st, (float*)kc, (float*)vc, Hkv, max_tokens, D,
                       count, seed);
  else
    hipLaunchKernelGGL(kv_fill_kernel<uint16_t>, grid, dim3(256), 0, st, (uint16_t*)kc, (uint16_t*)vc, Hkv,
                       max_tokens, D, count, seed);
}

}  // namespace tlm

// Persistent per-token decode schedule for gfx950: every layer of one token in
// one launch, one 1024-thread block per CU (stages and the wire format are
// described with PsArgs in tlm_kernels.h).
//
// Reference counterparts: the stages compute DecoderCPURunner.ts:102-132 for
// one position, i.e. TSLRMSNorm.ts:18-81 (both norms), TSLLinear.ts:13-82 (q|k|v
// with bias, O, gate|up, down), TSLAttention.ts:168-286 (RoPE, K/V append) and
// :306-428 (scores, softmax, P.V), TSLSiLUMul.ts:10-36 and TSLAdd.ts:10-33 (the
// two residual adds).
//
// Each block runs its (stage, item) roles for layer 0, then layer 1, ...; a
// role first issues its weight loads, then polls its inputs, so the weights
// arrive while the block waits.  Every role depends only on roles of earlier
// stages (or of the previous layer), and every block is resident, so all waits
// end; each is bounded anyway.
#include <algorithm>
#include <type_traits>

#include "tlm_device.h"

namespace tlm {

using u64 = unsigned long long;

// Device-scope relaxed loads and stores: global_load / global_store with sc1,
// i.e. past the (per-XCD) L2, with no cache-wide write-back or invalidate.
__device__ __forceinline__ u64 ld_dev(const u64* p) {
  return __hip_atomic_load(gl(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(u64* p, u64 v) {
  __hip_atomic_store(glw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 word(float v, unsigned seq) { return ((u64)seq << 32) | __float_as_uint(v); }
__device__ __forceinline__ float word_value(u64 w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ bool word_is(u64 w, unsigned seq) { return (unsigned)(w >> 32) == seq; }

// Bound of a spin: tick() is true once per 256 unsuccessful polls; late() then
// reads the wall clock (the first call starts it) and tells whether the wait
// has run out.  The clock is read that rarely because its read is a scalar
// memory access that LDS waits would also wait for.
struct PsSpin {
  int it = 0;
  long long t0 = 0;
  __device__ __forceinline__ bool tick() { return (++it & 255) == 0; }
  __device__ __forceinline__ bool late() {
    const long long now = wall_clock64();
    if (!t0) t0 = now;
    return now - t0 > kPsTimeoutTicks;
  }
};

// Timeline stamp e of (layer l, stage) by this wave's first lane (slot
// (L, 0) holds the kernel's start and end).
__device__ __forceinline__ void ps_stamp(const PsArgs& a, int l, int stage, int e) {
  if (a.trace && (threadIdx.x & 63) == 0)
    glw(a.trace)[((((size_t)blockIdx.x * kPsWaves + (threadIdx.x >> 6)) * (a.L + 1) + l) * PS_STAGES + stage) *
                     kPsEvents + e] = wall_clock64();
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Block-wide gather of n published words into LDS: word i is read from
// addr(i) and its value stored at dst[i].  Word i belongs to wave
// (i / 64) % 16, lane i % 64, so the 16 waves poll disjoint slices and no word
// is requested twice; a wave keeps all its (at most NW) loads in flight and
// spins until its whole slice carries seq, then the block meets at one
// barrier.  Detecting the data and loading it is one round trip.
// Block-uniform; false on time-out.
template <int NW, typename F>
__device__ bool ps_gather(int n, unsigned seq, F addr, float* dst, int* wflags) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int nu = 0;  // this wave's loads (wave-uniform)
#pragma unroll
  for (int u = 0; u < NW; u++)
    if (u * 1024 + wave * 64 < n) nu = u + 1;
  bool ok = true;
  if (nu > 0) {
    PsSpin spin;
    for (;;) {
      u64 w[NW];
#pragma unroll
      for (int u = 0; u < NW; u++)
        if (u < nu) w[u] = ld_dev(addr(min(u * 1024 + wave * 64 + lane, n - 1)));
      bool got = true;
#pragma unroll
      for (int u = 0; u < NW; u++) {
        const int i = u * 1024 + wave * 64 + lane;
        if (u < nu && i < n) {
          got &= word_is(w[u], seq);
          dst[i] = word_value(w[u]);
        }
      }
      if (__all(got)) break;
      if (spin.tick() && spin.late()) {
        ok = false;
        break;
      }
    }
  }
  if (lane == 0) wflags[wave] = ok ? 1 : 0;
  __syncthreads();
  bool all = true;
#pragma unroll
  for (int w = 0; w < kPsWaves; w++) all &= wflags[w] != 0;
  return all;
}

// v = thread t's elements 4t..4t+3 (t < H / 4, zeros elsewhere) of the sum of
// ks LDS rows of H floats (partials of one vector).
__device__ __forceinline__ float4 ps_row4(const float* x, int H, int ks) {
  const int tid = threadIdx.x;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tid < (H >> 2)) {
    float4 y[kPsMaxKs];  // all rows requested before the first add
#pragma unroll
    for (int s = 0; s < kPsMaxKs; s++) y[s] = *reinterpret_cast<const float4*>(x + (size_t)min(s, ks - 1) * H + 4 * tid);
#pragma unroll
    for (int s = 0; s < kPsMaxKs; s++)
      if (s < ks) v = make_float4(v.x + y[s].x, v.y + y[s].y, v.z + y[s].z, v.w + y[s].w);
  }
  return v;
}

// Sum over the n <= kPsMaxKs LDS values x[0], x[stride], ..., all requested
// before the first add.
__device__ __forceinline__ float ps_sum_rows(const float* x, int stride, int n) {
  float y[kPsMaxKs];
#pragma unroll
  for (int s = 0; s < kPsMaxKs; s++) y[s] = x[min(s, n - 1) * stride];
  float v = 0.f;
#pragma unroll
  for (int s = 0; s < kPsMaxKs; s++)
    if (s < n) v += y[s];
  return v;
}

// Sum over the block's 16 waves (every thread gets it); scratch: 16 floats,
// 16-byte aligned.
__device__ __forceinline__ float ps_block_sum(float v, float* scratch) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  const float4* s4 = reinterpret_cast<const float4*>(scratch);
  const float4 a = s4[0], b = s4[1], c = s4[2], d = s4[3];
  return (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w))) +
         (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
}

// xn = v * rsqrt(mean(x^2) + eps) * w (thread t owns elements 4t..4t+3 of the
// H-element row; H % 64 == 0, H <= 4096); q4: xsum[g] = sum of the 32-element
// group g of xn.  Ends with a block barrier.
template <int FMT>
__device__ __forceinline__ void ps_norm(float4 v, float4 w, int H, float eps, float* xn, float* xsum, float* scratch) {
  const int tid = threadIdx.x;
  const bool mine = tid < (H >> 2);
  float ss = v.x * v.x;
  ss = fmaf(v.y, v.y, ss);
  ss = fmaf(v.z, v.z, ss);
  ss = fmaf(v.w, v.w, ss);
  const float inv = rsqrtf(ps_block_sum(ss, scratch) / (float)H + eps);
  const float4 y = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
  if (mine) *reinterpret_cast<float4*>(xn + 4 * tid) = y;
  if (FMT == WF_Q4) {
    const float g = sum8(mine ? (y.x + y.y) + (y.z + y.w) : 0.f);
    if (mine && (tid & 7) == 0) xsum[tid >> 3] = g;
  }
  __syncthreads();
}

// q4: xsum[g] = sum of the 32-element group g of the n LDS values x (n a
// multiple of 32).  Every lane of the block calls it.
template <int FMT>
__device__ __forceinline__ void ps_groups(const float* x, float* xsum, int n) {
  if (FMT != WF_Q4) return;
  const int tid = threadIdx.x;
  const bool mine = tid < (n >> 2);
  float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
  if (mine) y = *reinterpret_cast<const float4*>(x + 4 * tid);
  const float g = sum8((y.x + y.y) + (y.z + y.w));
  if (mine && (tid & 7) == 0) xsum[tid >> 3] = g;
}

__device__ __forceinline__ float4 ld_f4(const float* p, int H) {
  const int tid = threadIdx.x;
  if (tid >= (H >> 2)) return make_float4(0.f, 0.f, 0.f, 0.f);
  return ldg_f4(p + 4 * tid);
}

// One 16-byte chunk of a weight row against the matching slice of x.
template <int FMT>
__device__ __forceinline__ float chunk_dot(uint4 d, uint16_t s, const float* x, const float* xsum, int c) {
  if (FMT == WF_Q4) return dot_q4(d, x + 32 * c, xsum[c], h2f(s));
  return dot_f16(d, x + 8 * c);
}

// Weights of NT consecutive 64-row tiles (t0.., clamped to T - 1), chunks
// c0 + wave + 16 u (u < NU) of a row of C chunks, for an input slice of n
// chunks from c0: a wave's share of a row-tile GEMV.  Loads are
// unconditional (indices clamped) and masked in dot().
template <int FMT, int NU, int NT>
struct PsRows {
  uint4 d[NT][NU];
  uint16_t s[NT][NU];
  __device__ __forceinline__ void load(const uint4* w, const uint16_t* sc, int C, int T, int t0, int c0, int n,
                                       int wave) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int u = 0; u < NU; u++) {
        const size_t at = ((size_t)min(t0 + t, T - 1) * C + c0 + min(wave + 16 * u, n - 1)) * kTile + lane;
        d[t][u] = ldg_u4(w + at);
        if (FMT == WF_Q4) s[t][u] = gl(sc)[at];
      }
  }
  // x: the slice's input (x[0] = element c0 * chunk); xsum: its group sums
  __device__ __forceinline__ float dot(int t, const float* x, const float* xsum, int n, int wave) const {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < NU; u++)
      if (wave + 16 * u < n) acc += chunk_dot<FMT>(d[t][u], s[t][u], x, xsum, wave + 16 * u);
    return acc;
  }
};

// ---------------------------------------------------------------- QKV head --
// Item i: head i / kq (rows of q head h, k head h - Hq or v head h - Hq - Hkv)
// over the input chunks of split i % kq.  Publishes the partial sums with RoPE
// applied (a rotation is linear) and the bias in split 0.
template <int FMT, typename KT, int DT, int NX>
__device__ __forceinline__ bool ps_qkv(const PsArgs& a, int l, int i, int pos, int token, unsigned seq, float* sm) {
  constexpr int NT = DT / 64;
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  constexpr int NW = (kPsMaxKs * 16 * NX * CK + 1023) / 1024;  // gathered words per lane: ks partials of H
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int H = a.H;
  float* red = sm;                        // [16][NT][64]
  float* xn = red + kPsWaves * NT * 64;   // [H]
  float* xsum = xn + H;                   // [H / 32, rounded to 4]
  float* out = xsum + ((H / 32 + 3) & ~3);  // [DT]
  float* scratch = out + DT;              // [16]
  int* wflags = reinterpret_cast<int*>(scratch + 16);  // [16]
  float* xb = scratch + 32;               // [ks][H] the residual's published partials
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int hd = i / a.kq, j = i % a.kq;
  const int r0 = hd * DT;
  const int kind = hd < a.Hq ? 0 : hd < a.Hq + a.Hkv ? 1 : 2;
  const int c0 = j * a.cq, cn = min(a.cq, a.Cx - c0);  // this split's input chunks
  PsRows<FMT, NX, NT> wr;
  wr.load(Ly.wqkv, Ly.sqkv, a.Cx, a.Tq, r0 / kTile, c0, cn, wave);
  const float bias = tid < DT && j == 0 ? gl(Ly.bqkv)[r0 + tid] : 0.f;
  const float4 nw = ld_f4(Ly.attn_norm, H);
  // rotate-half RoPE of element d = tid with its partner (TSLAttention.ts:168-250)
  const int half = a.rd > 0 ? a.rd / 2 : 1;
  float rc = 1.f, rs = 0.f, sg = 0.f;
  int pd = 0;
  if (tid < DT && kind < 2 && tid < a.rd) {
    const int jj = tid < half ? tid : tid - half;
    rc = gl(a.rope_cos)[(size_t)pos * half + jj];
    rs = gl(a.rope_sin)[(size_t)pos * half + jj];
    pd = tid < half ? tid + half : tid - half;
    sg = tid < half ? -1.f : 1.f;
  }
  if (wave == 0) ps_stamp(a, l, PS_QKV, 0);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (l == 0) {  // the token's embedding row (DecoderWeights.ts:355-383)
    if (tid < (H >> 2)) {
      if (a.emb_f32) {
        v = ldg_f4(reinterpret_cast<const float*>(a.emb) + (size_t)token * H + 4 * tid);
      } else {
        const uint2 e = ldg_u2(reinterpret_cast<const uint16_t*>(a.emb) + (size_t)token * H + 4 * tid);
        v = make_float4(h2f(e.x & 0xFFFFu), h2f(e.x >> 16), h2f(e.y & 0xFFFFu), h2f(e.y >> 16));
      }
    }
  } else {
    const u64* px = a.pub_x + (size_t)(l - 1) * kPsMaxKs * H;
    if (!ps_gather<NW>(a.ks * H, seq, [&](int k) { return px + k; }, xb, wflags)) return false;
    v = ps_row4(xb, H, a.ks);
  }
  if (wave == 0) ps_stamp(a, l, PS_QKV, 1);
  ps_norm<FMT>(v, nw, H, a.eps, xn, xsum, scratch);
#pragma unroll
  for (int t = 0; t < NT; t++)
    red[(wave * NT + t) * 64 + lane] = wr.dot(t, xn + c0 * CK, xsum + (FMT == WF_Q4 ? c0 : 0), cn, wave);
  __syncthreads();
  if (tid < DT) {
    float s = bias;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) s += red[(w * NT + (tid >> 6)) * 64 + (tid & 63)];
    out[tid] = s;
  }
  __syncthreads();
  if (wave == 0) ps_stamp(a, l, PS_QKV, 2);
  if (tid < DT) {
    float val = out[tid];
    if (kind < 2 && tid < a.rd) val = out[tid] * rc + sg * out[pd] * rs;
    st_dev(a.pub_qkv + ((size_t)l * a.kq + j) * a.Nqkv + r0 + tid, word(val, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_QKV, 3);
  return true;
}

// -------------------------------------------------------------- attention --
// Floats of one wave's LDS region: q, new k, new v, the pass's probabilities
// and its V tile (4 KiB).
template <typename KT, int DT>
constexpr int ps_wave_floats() {
  return (head_tiling(DT, sizeof(KT)).sub + 1024 + 3) & ~3;  // p_l, then a pass of V rows
}

// Item h: query head h over the window [first, pos].  Wave w takes the
// contiguous positions [first + w per, + per) (per: a multiple of 32); its
// first pass of cached K/V rows is requested before q is polled.  The row at
// pos comes from the published k and v (this token's cache write is not
// ordered before these reads).  The 16 waves merge (max, sum, output) in LDS
// in wave order.
template <typename KT, int DT>
__device__ __forceinline__ bool ps_att(const PsArgs& a, int l, int h, int first, int pos, unsigned seq, float* sm) {
  constexpr int ESZ = sizeof(KT);
  constexpr HeadTiling TL = head_tiling(DT, ESZ);
  constexpr int LPP = TL.lpp, SUB = TL.sub, DL = TL.dl;
  constexpr int EPL = DT / 64;
  constexpr int KW = DL * ESZ / 4;
  constexpr bool PAIRD = ESZ == 2 && DT == 128;
  constexpr int WF = ps_wave_floats<KT, DT>();
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int hk = h / a.G;
  const int n = pos - first + 1;
  const int per = max(32, ((n + kPsWaves - 1) / kPsWaves + 31) & ~31);
  const int t0 = min(first + wave * per, pos + 1), t1 = min(t0 + per, pos + 1);
  const bool active = t0 < t1;
  const bool own = active && pos < t1;  // this wave's range holds pos
  float* p_l = sm + wave * WF;
  KT* vt = reinterpret_cast<KT*>(p_l + SUB);
  float* mg = sm + kPsWaves * WF;  // [16][2 + DT] per-wave (max, sum, output)
  int* good = reinterpret_cast<int*>(mg + kPsWaves * (2 + DT));  // [16]
  float* gat = reinterpret_cast<float*>(good + kPsWaves);  // [kq][3][DT] published partials of q, k, v
  float* q_l = gat + kPsMaxKs * 3 * DT;  // [3][DT] their sums: q, then k and v rounded like the cache
  float* kn = q_l + DT;
  float* vn = kn + DT;
  int* wflags = reinterpret_cast<int*>(vn + DT);  // [16]
  const KT* kh = reinterpret_cast<const KT*>(Ly.kc) + (size_t)hk * a.max_tokens * DT;
  const KT* vh = reinterpret_cast<const KT*>(Ly.vc) + (size_t)hk * a.max_tokens * DT;
  const int pl = lane / LPP, part = lane % LPP;
  HeadLoads<KT, KW, false, DL> ld;
  const int tc0 = active ? t0 : first, tc1 = active ? t1 : first + 1;  // in-range rows for idle waves
  ld.issue(kh, vh, tc0, tc1, pl, part, DT, DT * ESZ, lane);
  ps_stamp(a, l, PS_ATT, 0);
  float m = -INFINITY, lsum = 0.f, o[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) o[e] = 0.f;
  // q of head h and this position's k and v: the sums of the kq partials
  const u64* pq = a.pub_qkv + (size_t)l * a.kq * a.Nqkv;
  constexpr int NWG = (kPsMaxKs * 3 * DT + 1023) / 1024;
  const bool ok = ps_gather<NWG>(a.kq * 3 * DT, seq,
                                 [&](int k) {
                                   const int j = k / (3 * DT), r = k - j * 3 * DT, c = r / DT, d = r - c * DT;
                                   const int off = c == 0 ? h * DT : a.QS + (c - 1) * a.Hkv * DT + hk * DT;
                                   return pq + (size_t)j * a.Nqkv + off + d;
                                 },
                                 gat, wflags);
  if (ok && tid < 3 * DT) {
    float sum = ps_sum_rows(gat + tid, 3 * DT, a.kq);
    if (tid >= DT) {  // k and v: rounded like the cache
      const KT r = kv_store<KT>(sum);
      sum = kv_load<KT>(&r);
      // the first query head of the group appends this position's k and v
      // (TSLAttention.ts:252-286); every head of the group rounds the same sums
      if (h % a.G == 0) {
        KT* cache = reinterpret_cast<KT*>(tid < 2 * DT ? Ly.kc : Ly.vc);
        glw(cache)[((size_t)hk * a.max_tokens + pos) * DT + (tid < 2 * DT ? tid - DT : tid - 2 * DT)] = r;
      }
    }
    q_l[tid] = sum;
  }
  __syncthreads();
  if (active) {
    ps_stamp(a, l, PS_ATT, 1);
    if (ok) {
      wave_lds_sync();
      const float* qp = q_l + part * DL;  // this lane's q slice (LDS broadcast reads)
      for (int tb = t0; tb < t1; tb += SUB) {
#pragma unroll
        for (int j = 0; j < 4; j++) reinterpret_cast<uint4*>(vt)[j * 64 + lane] = ld.vs[j];
        const int t = tb + pl;
        const bool valid = t < t1;
        uint32_t kw[KW];  // this lane's K slice; the row at pos is the published (cache-rounded) k
#pragma unroll
        for (int j = 0; j < KW; j++) kw[j] = ld.kw[j];
        if (own && t == pos) {
#pragma unroll
          for (int j = 0; j < KW; j++) {
            if (ESZ == 2) {
              const KT lo = kv_store<KT>(kn[part * DL + 2 * j]), hi = kv_store<KT>(kn[part * DL + 2 * j + 1]);
              kw[j] = (uint32_t)lo | ((uint32_t)hi << 16);
            } else {
              kw[j] = __float_as_uint(kn[part * DL + j]);
            }
          }
        }
        wave_lds_sync();
        if (own && pos >= tb && pos < tb + SUB)
          for (int d = lane; d < DT; d += 64) vt[(size_t)(pos - tb) * DT + d] = kv_store<KT>(vn[d]);
        if (tb + SUB < t1) ld.issue(kh, vh, tb + SUB, t1, pl, part, DT, DT * ESZ, lane);
        float s = 0.f;
#pragma unroll
        for (int e4 = 0; e4 < DL; e4 += 4) {
          const float4 q4 = *reinterpret_cast<const float4*>(qp + e4);
          const float qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
          for (int e = e4; e < e4 + 4; e++)
            s = fmaf(qv[e - e4], ESZ == 2 ? h2f((kw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) : __uint_as_float(kw[e]),
                     s);
        }
        if (LPP > 1) s += dpp<kDppXor1>(s);
        if (LPP > 2) s += dpp<kDppXor2>(s);
        if (LPP > 4) s += __shfl_xor(s, 4, 64);
        const float sc = valid ? s * a.scale : -INFINITY;
        const float mn = fmaxf(m, wave_max(sc));
        const float p = (valid && mn != -INFINITY) ? __expf(sc - mn) : 0.f;
        const float corr = m == -INFINITY ? 0.f : __expf(m - mn);
        lsum = lsum * corr + wave_sum(part == 0 ? p : 0.f);
        m = mn;
        if (part == 0) p_l[pl] = p;
        wave_lds_sync();
        if constexpr (PAIRD) {  // lane owns dims 2 lane, 2 lane + 1
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
#pragma unroll 8
            for (int u = 0; u < SUB; u++) acc = fmaf(p_l[u], kv_load<KT>(vt + (size_t)u * DT + d), acc);
            o[e] = acc;
          }
        }
        wave_lds_sync();
      }
    }
  }
  // merge the waves in order (an idle wave contributes max -inf, sum 0)
  float* mine = mg + wave * (2 + DT);
#pragma unroll
  for (int e = 0; e < EPL; e++) mine[2 + (PAIRD ? 2 * lane + e : lane + 64 * e)] = o[e];
  if (lane == 0) {
    mine[0] = m;
    mine[1] = lsum;
    good[wave] = ok ? 1 : 0;
  }
  __syncthreads();
  bool all_good = true;
#pragma unroll
  for (int w = 0; w < kPsWaves; w++) all_good &= good[w] != 0;
  if (!all_good) return false;  // block-uniform
  if (wave == 0) ps_stamp(a, l, PS_ATT, 2);
  if (tid < DT) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) M = fmaxf(M, mg[w * (2 + DT)]);
    float L = 0.f, od = 0.f;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) {
      const float mw = mg[w * (2 + DT)];
      const float sc = mw == -INFINITY ? 0.f : __expf(mw - M);
      L = fmaf(mg[w * (2 + DT) + 1], sc, L);
      od = fmaf(mg[w * (2 + DT) + 2 + tid], sc, od);
    }
    st_dev(a.pub_o + (size_t)l * a.QS + h * DT + tid, word(od / L, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_ATT, 3);
  return true;
}

// -------------------------------------------------------------- O row tile --
// Item i: rows 64 t .. 64 t + 63 (t = i % To) of the O projection over the
// attention-output chunks of split j = i / To; split 0 adds the residual rows:
// the partials of x_mid.
template <int FMT, int NO>
__device__ __forceinline__ bool ps_o(const PsArgs& a, int l, int i, int token, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  constexpr int NW = (16 * NO * CK + kPsMaxKs * 64 + 1023) / 1024;  // gathered words per lane
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int H = a.H, QS = a.QS;
  float* red = sm;                                 // [16][64]
  float* xo = red + kPsWaves * 64;                 // [QS] attention output, then [ks][64] residual rows
  float* xos = xo + QS + kPsMaxKs * 64;            // [QS / 32, rounded to 4]
  int* wflags = reinterpret_cast<int*>(xos + ((QS / 32 + 3) & ~3));  // [16]
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int t = i % a.To, j = i / a.To;
  const int c0 = j * a.co, cn = min(a.co, a.Co - c0), kn = cn * CK;  // this split's input chunks
  PsRows<FMT, NO, 1> wr;
  wr.load(Ly.wo, Ly.so, a.Co, a.To, t, c0, cn, wave);
  const int row = t * kTile + tid;  // threads tid < 64: the residual rows
  const bool rt = tid < kTile && row < H;
  float xr = 0.f;
  if (l == 0 && rt && j == 0)
    xr = a.emb_f32 ? gl(reinterpret_cast<const float*>(a.emb))[(size_t)token * H + row]
                   : h2f(gl(reinterpret_cast<const uint16_t*>(a.emb))[(size_t)token * H + row]);
  if (wave == 0) ps_stamp(a, l, PS_O, 0);
  const u64* po = a.pub_o + (size_t)l * QS + c0 * CK;
  const u64* px = a.pub_x + (size_t)(l > 0 ? l - 1 : 0) * kPsMaxKs * H + t * kTile;
  const int nx = l > 0 && j == 0 ? a.ks * kTile : 0;
  if (!ps_gather<NW>(kn + nx, seq,
                     [&](int k) { return k < kn ? po + k : px + (size_t)((k - kn) >> 6) * H + ((k - kn) & 63); },
                     xo, wflags))
    return false;
  if (wave == 0) ps_stamp(a, l, PS_O, 1);
  ps_groups<FMT>(xo, xos, kn);
  if (l > 0 && j == 0 && tid < kTile) xr = ps_sum_rows(xo + kn + tid, kTile, a.ks);
  __syncthreads();
  red[wave * 64 + lane] = wr.dot(0, xo, xos, cn, wave);
  __syncthreads();
  if (wave == 0) ps_stamp(a, l, PS_O, 2);
  if (rt) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) s += red[w * 64 + tid];
    st_dev(a.pub_xm + ((size_t)l * a.ko + j) * H + row, word(xr + s, seq));  // TSLAdd.ts:10-33
  }
  if (wave == 0) ps_stamp(a, l, PS_O, 3);
  return true;
}

// ------------------------------------------------------------ gate|up tiles --
// Item g: paired tiles g mw .. g mw + mw - 1 (tile t: gate rows 32 t.. in lanes
// 0..31, the matching up rows in lanes 32..63); publishes h = silu(g) * u for
// intermediate indices 32 t .. 32 t + 31.
template <int FMT, int NX, int MW>
__device__ __forceinline__ bool ps_gu(const PsArgs& a, int l, int g, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  constexpr int NW = (kPsMaxKs * 16 * NX * CK + 1023) / 1024;  // gathered words per lane: ko partials of H
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int H = a.H;
  float* red = sm;                          // [16][MW][64]
  float* xn = red + kPsWaves * MW * 64;     // [H]
  float* xsum = xn + H;                     // [H / 32, rounded to 4]
  float* scratch = xsum + ((H / 32 + 3) & ~3);  // [16]
  int* wflags = reinterpret_cast<int*>(scratch + 16);  // [16]
  float* xb = scratch + 32;                 // [ko][H] x_mid partials
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  PsRows<FMT, NX, MW> wr;
  wr.load(Ly.wgu, Ly.sgu, a.Cx, a.Tgu, g * MW, 0, a.Cx, wave);
  const float4 nw = ld_f4(Ly.ffn_norm, H);
  if (wave == 0) ps_stamp(a, l, PS_GU, 0);
  const u64* pm = a.pub_xm + (size_t)l * a.ko * H;
  if (!ps_gather<NW>(a.ko * H, seq, [&](int k) { return pm + k; }, xb, wflags)) return false;
  const float4 v = ps_row4(xb, H, a.ko);
  if (wave == 0) ps_stamp(a, l, PS_GU, 1);
  ps_norm<FMT>(v, nw, H, a.eps, xn, xsum, scratch);
#pragma unroll
  for (int s = 0; s < MW; s++)
    red[(wave * MW + s) * 64 + lane] = g * MW + s < a.Tgu ? wr.dot(s, xn, xsum, a.Cx, wave) : 0.f;
  __syncthreads();
  if (wave == 0) ps_stamp(a, l, PS_GU, 2);
  if (wave < MW && g * MW + wave < a.Tgu) {  // wave s finishes tile g mw + s
    float gs = 0.f, us = 0.f;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) {
      gs += red[(w * MW + wave) * 64 + (lane & 31)];
      us += red[(w * MW + wave) * 64 + (lane | 32)];
    }
    const float hv = gs / (1.f + __expf(-gs)) * us;  // TSLSiLUMul.ts:15-29
    if (lane < 32) st_dev(a.pub_h + (size_t)l * a.Tgu * 32 + (g * MW + wave) * 32 + lane, word(hv, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_GU, 3);
  return true;
}

// -------------------------------------------------------------- down tiles --
// Item (t, s): rows 64 t .. 64 t + 63 of the down projection over the input
// chunks [s cs, (s + 1) cs); split 0 adds x_mid (the MLP residual).
template <int FMT, int ND>
__device__ __forceinline__ bool ps_down(const PsArgs& a, int l, int t, int s, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  constexpr int NW = (16 * ND * CK + kPsMaxKs * 64 + 1023) / 1024;  // gathered words per lane
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int H = a.H;
  const int c0 = s * a.cs, cn = min(a.cs, a.Cd - c0);
  const int kn = cn * CK;  // input elements of the split
  float* red = sm;                          // [16][64]
  float* hs = red + kPsWaves * 64;          // [cs CK] the split's h, then [ko][64] x_mid rows (split 0)
  float* hss = hs + a.cs * CK + kPsMaxKs * 64;  // [cs CK / 32, rounded to 4]
  int* wflags = reinterpret_cast<int*>(hss + ((a.cs * CK / 32 + 3) & ~3));  // [16]
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  PsRows<FMT, ND, 1> wr;
  wr.load(Ly.wd, Ly.sd, a.Cd, a.To, t, c0, cn, wave);
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 0);
  const u64* ph = a.pub_h + (size_t)l * a.Tgu * 32 + (size_t)c0 * CK;
  const u64* pm = a.pub_xm + (size_t)l * a.ko * H + t * kTile;
  const int row = t * kTile + tid;
  const bool rt = tid < kTile && row < H;
  const int nm = s == 0 ? a.ko * kTile : 0;
  if (!ps_gather<NW>(kn + nm, seq,
                     [&](int k) { return k < kn ? ph + k : pm + (size_t)((k - kn) >> 6) * H + ((k - kn) & 63); }, hs,
                     wflags))
    return false;
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 1);
  ps_groups<FMT>(hs, hss, kn);
  float xm = 0.f;
  if (s == 0 && tid < kTile) xm = ps_sum_rows(hs + kn + tid, kTile, a.ko);
  __syncthreads();
  red[wave * 64 + lane] = wr.dot(0, hs, hss, cn, wave);
  __syncthreads();
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 2);
  if (rt) {
    const float v = s == 0 ? xm : 0.f;  // split 0 carries x_mid (TSLAdd.ts:10-33)
    float d = 0.f;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) d += red[w * 64 + tid];
    st_dev(a.pub_x + ((size_t)l * kPsMaxKs + s) * H + row, word(v + d, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 3);
  return true;
}

// -------------------------------------------------------------------- kernel --
template <int FMT, typename KT, int DT, int NX, int NO, int ND, int MW>
__global__ __launch_bounds__(kPsWaves * 64) void ps_token_kernel(const PsArgs* __restrict__ ap) {
  extern __shared__ float sm[];
  const PsArgs& a = *ap;  // in device memory: field reads are scalar loads
  const int pos = gl(a.ctrl)[C_POS], token = gl(a.ctrl)[C_TOKEN];
  const unsigned seq = (unsigned)gl(a.ctrl)[C_SEQ];
  if (pos < 0 || pos >= a.max_tokens) return;
  ps_stamp(a, a.L, 0, 0);
  const int first = a.window > 0 ? max(pos - a.window + 1, 0) : 0;
  const TLM_GLOBAL int* rl = gl(a.roles) + blockIdx.x * kPsRoles * 2;
  for (int l = 0; l < a.L; l++) {
#pragma unroll 1
    for (int r = 0; r < kPsRoles; r++) {
      const int st = rl[2 * r], it = rl[2 * r + 1];
      bool ok = true;
      if (st == PS_QKV)
        ok = ps_qkv<FMT, KT, DT, NX>(a, l, it, pos, token, seq, sm);
      else if (st == PS_ATT)
        ok = ps_att<KT, DT>(a, l, it, first, pos, seq, sm);
      else if (st == PS_O)
        ok = ps_o<FMT, NO>(a, l, it, token, seq, sm);
      else if (st == PS_GU)
        ok = ps_gu<FMT, NX, MW>(a, l, it, seq, sm);
      else if (st == PS_DOWN)
        ok = ps_down<FMT, ND>(a, l, it % a.To, it / a.To, seq, sm);
      if (!ok) {  // a bounded wait ran out: report and leave (block-uniform)
        if (threadIdx.x == 0) __hip_atomic_fetch_or(glw(a.ctrl + C_ERR), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      __syncthreads();  // LDS reused by the next role
    }
  }
  ps_stamp(a, a.L, 0, 1);
}

// ------------------------------------------------------------------- host --
struct PsVariant {
  int fmt, kv_f32, dt, nx, no, nd, mw;
};
// Compiled shapes (chunks per wave: nx of the H-input linears, no of O, nd of a
// down split; mw gate|up tiles per item).
static const PsVariant kPsVariants[] = {
    {WF_Q4, 0, 64, 2, 1, 3, 1},   // hidden 896, 14 x 64 heads, inter 4864 (Qwen2.5-0.5B shape)
    {WF_Q4, 0, 64, 4, 1, 4, 1},   // hidden 2048, 32 x 64 heads, inter 8192 (Llama-3.2-1B shape)
    {WF_Q4, 0, 128, 6, 2, 4, 2},  // hidden 3072, 24 x 128 heads, inter 8192 (Llama-3.2-3B shape)
    {WF_Q4, 0, 64, 1, 1, 1, 1},   // hidden <= 512 q4
    {WF_F16, 0, 64, 2, 1, 3, 1},  // hidden 256 fp16
};

// Items of each stage for a shape's splits.
static void ps_counts(int H, int Hq, int Hkv, int Tgu, int kq, int ko, int mw, int ks, int* c) {
  const int To = H / 64;
  c[PS_QKV] = (Hq + 2 * Hkv) * kq;
  c[PS_ATT] = Hq;
  c[PS_O] = To * ko;
  c[PS_GU] = (Tgu + mw - 1) / mw;
  c[PS_DOWN] = To * ks;
}

// Places the items on blocks (roles[b][r] = {stage, item}, stage -1: none) and
// returns the roles per block, 0 if they do not fit kPsRoles.  With one or two
// roles, a block's two stages are two or three apart, so that each role's
// weights load while the stages between its inputs and the block's other role
// run (the cycle continues into the next layer); with more, item k goes to
// block k % blocks as its role k / blocks.
static int ps_place(const int* counts, int blocks, int* roles) {
  int total = 0;
  for (int st = 0; st < PS_STAGES; st++) total += counts[st];
  if (total > kPsRoles * blocks) return 0;
  if (roles)
    for (int i = 0; i < 2 * kPsRoles * blocks; i++) roles[i] = i % 2 == 0 ? -1 : 0;
  auto put = [&](int b, int r, int st, int it) {
    if (roles) {
      roles[2 * (kPsRoles * b + r)] = st;
      roles[2 * (kPsRoles * b + r) + 1] = it;
    }
  };
  if (total <= 2 * blocks) {
    static const int kPairs[][2] = {{PS_QKV, PS_GU}, {PS_ATT, PS_DOWN}, {PS_O, PS_DOWN}, {PS_ATT, PS_GU}, {PS_QKV, PS_O}};
    int left[PS_STAGES], next[PS_STAGES] = {};
    for (int st = 0; st < PS_STAGES; st++) left[st] = counts[st];
    int need = std::max(0, total - blocks), b = 0;
    for (const auto& pr : kPairs)
      while (need > 0 && left[pr[0]] > 0 && left[pr[1]] > 0) {
        put(b, 0, pr[0], next[pr[0]]++);
        put(b, 1, pr[1], next[pr[1]]++);
        left[pr[0]]--, left[pr[1]]--, need--, b++;
      }
    if (need == 0) {
      for (int st = 0; st < PS_STAGES; st++)
        while (left[st] > 0) put(b++, 0, st, next[st]++), left[st]--;
      return total > blocks ? 2 : 1;
    }
    if (roles)
      for (int i = 0; i < 2 * kPsRoles * blocks; i++) roles[i] = i % 2 == 0 ? -1 : 0;
  }
  int k = 0;
  for (int st = 0; st < PS_STAGES; st++)
    for (int it = 0; it < counts[st]; it++, k++) put(k % blocks, k / blocks, st, it);
  return (total + blocks - 1) / blocks;
}

PsShape ps_shape(int fmt, int kv_f32, int H, int I, int D, int Hq, int Hkv, int cus) {
  PsShape none{};
  const int QS = Hq * D;
  if (D != 64 && D != 128) return none;
  if (H % 64 != 0 || H > 4096 || QS > 4096 || Hq % Hkv != 0) return none;
  const int CK = fmt == WF_Q4 ? 32 : 8;
  const int Cx = H / CK, Co = QS / CK, Cd = (I + CK - 1) / CK, Tgu = (I + 31) / 32;
  const int nx = (Cx + 15) / 16;
  // Over the compiled variants and the K-splits of QKV (kq), O (ko) and down
  // (ks): the least multiply-adds along one item of each linear stage, plus
  // the cost of a third role per block (about two microseconds of a CU's
  // multiply-adds, serial behind the previous role)
  PsShape best = none;
  long best_cost = 0;
  for (const PsVariant& v : kPsVariants) {
    if (v.fmt != fmt || v.kv_f32 != kv_f32 || v.dt != D || v.nx < nx) continue;
    for (int kq = 1; kq <= kPsMaxKs; kq++)
      for (int ko = 1; ko <= kPsMaxKs; ko++)
        for (int ks = 1; ks <= kPsMaxKs; ks++) {
          const int cq = (Cx + kq - 1) / kq, co = (Co + ko - 1) / ko, cs = (Cd + ks - 1) / ks;
          if ((co + 15) / 16 > v.no || (cs + 15) / 16 > v.nd) continue;
          int counts[PS_STAGES];
          ps_counts(H, Hq, Hkv, Tgu, kq, ko, v.mw, ks, counts);
          const int r = ps_place(counts, cus, nullptr);
          if (!r) continue;
          const long macs = (long)D * cq * CK + 64L * co * CK + 64L * v.mw * H + 64L * cs * CK;
          const long cost = macs + (r > 2 ? 128L * 1024 : 0);
          if (!best.dt || cost < best_cost) {
            best = PsShape{v.fmt, v.kv_f32, v.dt, v.nx, v.no, v.nd, v.mw, kq, ko, ks};
            best_cost = cost;
          }
        }
  }
  return best;
}

bool ps_roles(const PsShape& sh, int blocks, int H, int Hq, int Hkv, int Tgu, int* roles) {
  int counts[PS_STAGES];
  ps_counts(H, Hq, Hkv, Tgu, sh.kq, sh.ko, sh.mw, sh.ks, counts);
  return ps_place(counts, blocks, roles) > 0;
}

size_t ps_smem_bytes(const PsShape& sh, int H, int QS) {
  const int CK = sh.fmt == WF_Q4 ? 32 : 8;
  const size_t esz = sh.kv_f32 ? 4 : 2;
  const int sub = head_tiling(sh.dt, (int)esz).sub;
  auto r4 = [](size_t n) { return (n + 3) & ~(size_t)3; };
  const size_t att = (size_t)kPsWaves * ((sub + 1024 + 3) & ~3) + kPsWaves * (2 + sh.dt) + kPsWaves +
                     (size_t)(kPsMaxKs + 1) * 3 * sh.dt + kPsWaves;
  const size_t qkv = (size_t)kPsWaves * (sh.dt / 64) * 64 + H + r4(H / 32) + sh.dt + 32 + (size_t)kPsMaxKs * H;
  const size_t o = (size_t)kPsWaves * 64 + QS + kPsMaxKs * 64 + r4(QS / 32) + kPsWaves;
  const size_t gu = (size_t)kPsWaves * sh.mw * 64 + H + r4(H / 32) + 32 + (size_t)kPsMaxKs * H;
  const size_t cs = (size_t)sh.nd * 16 * CK;  // a down split's input elements, at most
  const size_t down = (size_t)kPsWaves * 64 + cs + kPsMaxKs * 64 + r4(cs / 32) + kPsWaves;
  return sizeof(float) * std::max({att, qkv, o, gu, down});
}

// The compiled kernel of a shape (null: none).
static const void* ps_kernel(const PsShape& sh) {
#define PS_CASE(F, KV, DTV, NXV, NOV, NDV, MWV)                                                             \
  if (sh.fmt == F && sh.kv_f32 == KV && sh.dt == DTV && sh.nx == NXV && sh.no == NOV && sh.nd == NDV &&   \
      sh.mw == MWV)                                                                                       \
    return (const void*)ps_token_kernel<F, std::conditional_t<KV, float, uint16_t>, DTV, NXV, NOV, NDV, MWV>;
  PS_CASE(WF_Q4, 0, 64, 2, 1, 3, 1)
  PS_CASE(WF_Q4, 0, 64, 4, 1, 4, 1)
  PS_CASE(WF_Q4, 0, 128, 6, 2, 4, 2)
  PS_CASE(WF_Q4, 0, 64, 1, 1, 1, 1)
  PS_CASE(WF_F16, 0, 64, 2, 1, 3, 1)
#undef PS_CASE
  return nullptr;
}

bool ps_prepare(const PsShape& sh, size_t smem) {
  const void* k = ps_kernel(sh);
  return k && hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) == hipSuccess;
}

bool launch_ps_token(const PsShape& sh, int blocks, size_t smem, const PsArgs* a_dev, hipStream_t st) {
  const void* k = ps_kernel(sh);
  if (!k) return false;
  const PsArgs* arg = a_dev;
  void* params[] = {&arg};
  return hipLaunchKernel(k, dim3(blocks), dim3(kPsWaves * 64), params, smem, st) == hipSuccess;
}

}  // namespace tlm

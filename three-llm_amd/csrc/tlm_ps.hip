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
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>
#include <vector>

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
// A handoff word whose consumers all run on this XCD: a plain store, which
// stays in the XCD's L2 where their device-scope loads find it (0.95 against
// 1.5 us per producer-consumer round trip through device-scope stores).
__device__ __forceinline__ void st_pub(bool l2, u64* p, u64 v) {
  if (l2)
    __hip_atomic_store(glw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    st_dev(p, v);
}
// This wave's XCD (hardware register XCC_ID).
__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg(20 | (0 << 6) | ((16 - 1) << 11)) & 0xF; }
__device__ __forceinline__ u64 word(float v, unsigned seq) { return ((u64)seq << 32) | __float_as_uint(v); }
__device__ __forceinline__ float word_value(u64 w) { return __uint_as_float((unsigned)w); }
__device__ __forceinline__ bool word_is(u64 w, unsigned seq) { return (unsigned)(w >> 32) == seq; }

// Bound of a spin: tick() is true once per 256 unsuccessful polls; late() then
// reads the wall clock (the first call starts it) and tells whether the wait
// has run out.  The clock is read that rarely because its read is a scalar
// memory access that LDS waits would also wait for.
struct PsSpin {
  long long limit;
  int it = 0;
  long long t0 = 0;
  __device__ __forceinline__ explicit PsSpin(long long ticks) : limit(ticks) {}
  __device__ __forceinline__ bool tick() { return (++it & 255) == 0; }
  __device__ __forceinline__ bool late() {
    const long long now = wall_clock64();
    if (!t0) t0 = now;
    return now - t0 > limit;
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


// ------------------------------------------------------- wave-level inputs --
// A linear stage's wave owns input chunks cbase + wave + 16 u (u < NU) and
// reads just their CK elements: no block barrier before its dot products.
// Element k of the input is the sum of np published partial vectors, word
// addr(p, k) for partial p.  Lane l reads element e = l % CK of each chunk
// for partials p = l / CK + j (64 / CK), j < PPL, and the lanes of one
// element add their sums, so every lane with l % CK == e ends with x[u] =
// element e of chunk u.  Chunks at or past cend read as zero.  Polls until
// every word carries seq; false on time-out (wave-uniform).
template <int CK, int NU, typename F>
__device__ __forceinline__ bool wl_gather(int cbase, int cend, int np, unsigned seq, F addr, int wave,
                                          float (&x)[NU], long long limit) {
  constexpr int S = 64 / CK;                          // lanes per element
  constexpr int PPL = (kPsMaxKs + S - 1) / S;         // partials per lane
  const int lane = threadIdx.x & 63, e = lane % CK, slot = lane / CK;
  PsSpin spin(limit);
  for (;;) {
    u64 w[NU][PPL];
#pragma unroll
    for (int u = 0; u < NU; u++)
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        const int c = cbase + wave + 16 * u, p = slot + j * S;
        w[u][j] = c < cend && p < np ? ld_dev(addr(p, c * CK + e)) : word(0.f, seq);
      }
    bool got = true;
#pragma unroll
    for (int u = 0; u < NU; u++) {
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        got &= word_is(w[u][j], seq);
        v += word_value(w[u][j]);
      }
      x[u] = v;
    }
    if (__all(got)) break;
    if (spin.tick() && spin.late()) return false;
  }
#pragma unroll
  for (int u = 0; u < NU; u++) {
    if (CK <= 8) x[u] += __shfl_xor(x[u], 8, 64);
    if (CK <= 16) x[u] += __shfl_xor(x[u], 16, 64);
    x[u] += lane_swap32(x[u]);
  }
  return true;
}

// The same chunks from the token's embedding row (layer 0's residual).
template <int CK, int NU>
__device__ __forceinline__ void wl_embedding(const PsArgs& a, int token, int cend, int wave, float (&x)[NU]) {
  const int e = (threadIdx.x & 63) % CK;
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const int c = wave + 16 * u;
    const size_t k = (size_t)token * a.H + (size_t)min(c, cend - 1) * CK + e;
    const float v = a.emb_f32 ? gl(reinterpret_cast<const float*>(a.emb))[k]
                              : h2f(gl(reinterpret_cast<const uint16_t*>(a.emb))[k]);
    x[u] = c < cend ? v : 0.f;
  }
}

// Residual rows of a row-tile item, lane = row: the sum of np published
// partials at addr(p) (lane's row), polled (wave-level).
template <typename F>
__device__ __forceinline__ bool wl_rows(int np, unsigned seq, F addr, float& xr, long long limit) {
  PsSpin spin(limit);
  for (;;) {
    u64 w[kPsMaxKs];
#pragma unroll
    for (int p = 0; p < kPsMaxKs; p++) w[p] = p < np ? ld_dev(addr(p)) : word(0.f, seq);
    bool got = true;
    float v = 0.f;
#pragma unroll
    for (int p = 0; p < kPsMaxKs; p++) {
      got &= word_is(w[p], seq);
      v += word_value(w[p]);
    }
    xr = v;
    if (__all(got)) return true;
    if (spin.tick() && spin.late()) return false;
  }
}

// Stage the wave's chunk inputs for its dot products: y = x[u] * nw (nw: the
// element's norm weight, 1 without a norm) in the wave's LDS slots; ss = the
// sum of squares of the raw x over the wave's chunks.
//
// fp16 weights (CK 8): xw[u][e] = y in fp32; xs unused.
// q4 weights (CK 32): y rounded to fp16, stored as the pairs that dot_q4h
// reads: dword 4 j + i of chunk u = (y[8 j + i], y[8 j + i + 4]); xs[u] =
// the chunk's sum of those fp16 values.  An input past the fp16 range
// becomes infinite and every dot product of its wave NaN, which reaches the
// last residual whatever the stage: the last layer's down items raise
// kPsErrRange from there (no check here, on the path to every dot).
// Ends with the wave's LDS writes visible to its lanes.
template <int FMT, int CK, int NU>
__device__ __forceinline__ void wl_stage(const float (&x)[NU], const float (&nw)[NU], float* xw, float (&xs)[NU],
                                         float& ss) {
  const int lane = threadIdx.x & 63;
  const bool mine = lane < CK;
  float q = 0.f;
  if constexpr (FMT == WF_Q4) {
    _Float16* xh = reinterpret_cast<_Float16*>(xw);
    // lane k (element k of each chunk) -> half (k / 4) & 1 of dword (k / 8) 4 + k % 4
    const int slot = ((lane >> 3) << 3) + ((lane & 3) << 1) + ((lane >> 2) & 1);
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const float y = x[u] * nw[u];
      q = fmaf(mine ? x[u] : 0.f, x[u], q);
      const _Float16 h = (_Float16)y;
      if (mine) xh[u * 32 + slot] = h;
      xs[u] = wave_sum(mine ? (float)h : 0.f);
    }
  } else {
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const float y = x[u] * nw[u];
      if (mine) xw[u * CK + lane] = y;
      q = fmaf(mine ? x[u] : 0.f, x[u], q);
      xs[u] = 0.f;
    }
  }
  ss = wave_sum(q);
  wave_lds_sync();
}

// One 16-byte chunk of a weight row against its CK staged inputs.
// (q4: x holds the chunk's 16 fp16-pair dwords staged by wl_stage.)
template <int FMT>
__device__ __forceinline__ float chunk_dot(uint4 d, uint16_t s, const float* x, float xs) {
  if (FMT == WF_Q4) return dot_q4h(d, reinterpret_cast<const uint32_t*>(x), xs, h2f(s));
  return dot_f16(d, x);
}

// Weights of NT consecutive 64-row tiles (t0.., clamped to T - 1): chunk
// cbase + wave + 16 u (u < NU) of each row of C chunks when it lies in
// [clo, chi) (the item's K range), else masked.  Loads are unconditional
// (indices clamped into the range).
template <int FMT, int NU, int NT>
struct PsRows {
  uint4 d[NT][NU];
  uint16_t s[NT][NU];
  __device__ __forceinline__ void load(const uint4* w, const uint16_t* sc, int C, int T, int t0, int cbase, int clo,
                                       int chi, int wave) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int u = 0; u < NU; u++) {
        const int c = min(max(cbase + wave + 16 * u, clo), chi - 1);
        const size_t at = ((size_t)min(t0 + t, T - 1) * C + c) * kTile + lane;
        d[t][u] = ldg_u4(w + at);
        if (FMT == WF_Q4) s[t][u] = gl(sc)[at];
      }
  }
  __device__ __forceinline__ float dot(int t, const float* xw, const float (&xs)[NU], int cbase, int clo, int chi,
                                       int wave) const {
    constexpr int XS = FMT == WF_Q4 ? 16 : 8;  // staged words per chunk
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int c = cbase + wave + 16 * u;
      if (c >= clo && c < chi) acc += chunk_dot<FMT>(d[t][u], s[t][u], xw + u * XS, xs[u]);
    }
    return acc;
  }
};

// Whether a stage widens its q4 weights ahead (PsRowsH): up to 3 chunks per
// wave (48 registers of pairs; with more, the kernel's registers spill).
template <int FMT, int NU>
constexpr bool ps_widen() {
  return FMT == WF_Q4 && NU <= 3;
}

// PsRows' q4 weights with the nibbles already widened to the fp16 pairs that
// dot_q4h forms (1 + n / 64): formed while the stage waits for its inputs,
// so that only the v_dot2 multiply-adds remain once they arrive.  The same
// operations in the same order as dot_q4h: the same results.
template <int NU, int NT>
struct PsRowsH {
  uint32_t p[NT][NU][16];
  float sc[NT][NU];
  __device__ __forceinline__ void from(const PsRows<WF_Q4, NU, NT>& r) {
    const uint32_t M = 0x00F000F0u, E = 0x3C003C00u;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int u = 0; u < NU; u++) {
        const uint32_t wv[4] = {r.d[t][u].x, r.d[t][u].y, r.d[t][u].z, r.d[t][u].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          p[t][u][4 * j] = and_or(wv[j] << 4, M, E);
          p[t][u][4 * j + 1] = and_or(wv[j], M, E);
          p[t][u][4 * j + 2] = and_or(wv[j] >> 4, M, E);
          p[t][u][4 * j + 3] = and_or(wv[j] >> 8, M, E);
        }
        sc[t][u] = h2f(r.s[t][u]);
      }
  }
  __device__ __forceinline__ float dot(int t, const float* xw, const float (&xs)[NU], int cbase, int clo, int chi,
                                       int wave) const {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const int c = cbase + wave + 16 * u;
      if (c < clo || c >= chi) continue;
      const uint32_t* xh = reinterpret_cast<const uint32_t*>(xw + u * 16);
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint4 xp = *reinterpret_cast<const uint4*>(xh + 4 * j);
        a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p[t][u][4 * j]), __builtin_bit_cast(f16x2, xp.x), a0, false);
        a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p[t][u][4 * j + 1]), __builtin_bit_cast(f16x2, xp.y), a1,
                                    false);
        a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p[t][u][4 * j + 2]), __builtin_bit_cast(f16x2, xp.z), a0,
                                    false);
        a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p[t][u][4 * j + 3]), __builtin_bit_cast(f16x2, xp.w), a1,
                                    false);
      }
      acc += sc[t][u] * fmaf(64.f, a0 + a1, -72.f * xs[u]);
    }
    return acc;
  }
};

// Block-uniform AND of the waves' flags (wf: 16 ints of LDS); a block barrier.
__device__ __forceinline__ bool ps_all(bool ok, int* wf) {
  if ((threadIdx.x & 63) == 0) wf[threadIdx.x >> 6] = ok ? 1 : 0;
  __syncthreads();
  const int4* f4 = reinterpret_cast<const int4*>(wf);
  const int4 a = f4[0], b = f4[1], c = f4[2], d = f4[3];
  return (a.x & a.y & a.z & a.w & b.x & b.y & b.z & b.w & c.x & c.y & c.z & c.w & d.x & d.y & d.z & d.w) != 0;
}

// Sum of the 16 waves' LDS values v[0], v[stride], ... (all requested first).
__device__ __forceinline__ float ps_sum16(const float* v, int stride) {
  float r[kPsWaves];
#pragma unroll
  for (int w = 0; w < kPsWaves; w++) r[w] = v[w * stride];
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kPsWaves; w++) s += r[w];
  return s;
}

// Norm weights of this lane's element of the wave's chunks (1 past cend).
template <int CK, int NU>
__device__ __forceinline__ void wl_norm_weights(const float* nw, int cend, int wave, float (&w)[NU]) {
  const int e = (threadIdx.x & 63) % CK;
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const int c = wave + 16 * u;
    w[u] = c < cend ? gl(nw)[c * CK + e] : 1.f;
  }
}

// LDS of a linear stage: per-wave input slots, then the wave partials.
struct PsLinLds {
  float* xw;   // [16][NU][CK] this wave's staged inputs
  float* red;  // [16][R][64] per-wave partial outputs
  float* ssw;  // [16] per-wave sums of squares
  int* wf;     // [16] per-wave flags
  float* out;  // [2][64] the item's outputs (QKV RoPE partner reads)
};
template <int CK, int NU, int R>
__device__ __forceinline__ PsLinLds ps_lin_lds(float* sm) {
  PsLinLds s;
  s.red = sm;
  s.ssw = s.red + kPsWaves * R * 64;
  s.wf = reinterpret_cast<int*>(s.ssw + kPsWaves);
  s.out = reinterpret_cast<float*>(s.wf + kPsWaves);
  s.xw = s.out + 128 + wave_id() * NU * CK;
  return s;
}
constexpr int ps_lin_floats(int ck, int nu, int r) { return kPsWaves * r * 64 + 2 * kPsWaves + 128 + kPsWaves * nu * ck; }

// ------------------------------------------------------------ k and v heads --
// Item i: k head i / kq or v head i / kq - Hkv (rows Hq + i / kq of q|k|v; the
// attention items compute q themselves) over the input chunks of split
// j = i % kq.  Each wave reads its chunks of the whole residual (the norm
// needs all of it) and dots those in the split; the norm's scale multiplies
// the summed dot products (a rotation and a scale are linear).  Publishes the
// partial sums with RoPE applied (k) and the bias in split 0.
template <int FMT, typename KT, int DT, int NX>
__device__ __forceinline__ bool ps_qkv(const PsArgs& a, int l, int i, int pos, int token, unsigned seq, bool l2,
                                       float* sm) {
  constexpr int NT = DT / 64;
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const PsLinLds s = ps_lin_lds<CK, NX, NT>(sm);
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int hd = a.Hq + i / a.kq, j = i % a.kq;
  const int r0 = hd * DT;
  const int kind = hd < a.Hq + a.Hkv ? 1 : 2;
  const int c0 = j * a.cq, c1 = min(c0 + a.cq, a.Cx);  // this split's input chunks
  PsRows<FMT, NX, NT> wr;
  wr.load(Ly.wqkv, Ly.sqkv, a.Cx, a.Tq, r0 / kTile, 0, c0, c1, wave);
  float nw[NX];
  wl_norm_weights<CK, NX>(Ly.attn_norm, a.Cx, wave, nw);
  float bias[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) bias[t] = j == 0 && wave == 0 ? gl(Ly.bqkv)[r0 + 64 * t + lane] : 0.f;
  // RoPE factors of wave 0's elements (the position is known before the wait;
  // rotate-half of element d with its partner, TSLAttention.ts:168-250)
  const int half = a.rd > 0 ? a.rd / 2 : 1;
  float rc[NT], rs[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int d = 64 * t + lane, jj = d < half ? d : d - half;
    const bool rot = wave == 0 && kind < 2 && d < a.rd;
    rc[t] = rot ? gl(a.rope_cos)[(size_t)pos * half + jj] : 1.f;
    rs[t] = rot ? gl(a.rope_sin)[(size_t)pos * half + jj] : 0.f;
  }
  if (wave == 0) ps_stamp(a, l, PS_QKV, 0);
  // q4: the weights widened to fp16 pairs while the residual is on its way
  PsRowsH<NX, NT> wh;
  if constexpr (ps_widen<FMT, NX>()) wh.from(wr);
  float x[NX];
  bool ok = true;
  if (l == 0) {
    wl_embedding<CK, NX>(a, token, a.Cx, wave, x);
  } else {
    const u64* px = a.pub_x + (size_t)(l - 1) * kPsMaxKs * a.H;
    ok = wl_gather<CK, NX>(0, a.Cx, a.ks, seq, [&](int p, int k) { return px + (size_t)p * a.H + k; }, wave, x, a.timeout);
  }
  if (l == a.fail_layer) ok = false;  // the forced failure path (tests)
  if (wave == 0) ps_stamp(a, l, PS_QKV, 1);
  float xs[NX], ss = 0.f;
  wl_stage<FMT, CK, NX>(x, nw, s.xw, xs, ss);
#pragma unroll
  for (int t = 0; t < NT; t++) {
    if constexpr (ps_widen<FMT, NX>()) s.red[(wave * NT + t) * 64 + lane] = wh.dot(t, s.xw, xs, 0, c0, c1, wave);
    else s.red[(wave * NT + t) * 64 + lane] = wr.dot(t, s.xw, xs, 0, c0, c1, wave);
  }
  if (lane == 0) s.ssw[wave] = ss;
  if (!ps_all(ok, s.wf)) return false;
  if (wave == 0) {
    ps_stamp(a, l, PS_QKV, 2);
    const float inv = rsqrtf(ps_sum16(s.ssw, 1) / (float)a.H + a.eps);
    if (NT == 1 && half == 32) {  // the rotation partner of lane d is lane d ^ 32
      const float val = bias[0] + inv * ps_sum16(s.red + lane, 64), partner = lane_swap32(val);
      const float y = kind < 2 ? val * rc[0] + (lane < 32 ? -partner : partner) * rs[0] : val;
      st_pub(l2, a.pub_qkv + ((size_t)l * a.kq + j) * a.Nqkv + r0 + lane, word(y, seq));
    } else {
#pragma unroll
      for (int t = 0; t < NT; t++) s.out[64 * t + lane] = bias[t] + inv * ps_sum16(s.red + t * 64 + lane, NT * 64);
      wave_lds_sync();
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int d = 64 * t + lane;
        float val = s.out[d];
        if (kind < 2 && d < a.rd) val = val * rc[t] + (d < half ? -s.out[d + half] : s.out[d - half]) * rs[t];
        st_pub(l2, a.pub_qkv + ((size_t)l * a.kq + j) * a.Nqkv + r0 + d, word(val, seq));
      }
    }
    ps_stamp(a, l, PS_QKV, 3);
  }
  return true;
}

// -------------------------------------------------------------- attention --
// Floats of one wave's LDS region: new k, new v, the pass's probabilities
// and its V tile (4 KiB).
template <typename KT, int DT>
constexpr int ps_wave_floats() {
  return (2 * DT + head_tiling(DT, sizeof(KT)).sub + 1024 + 3) & ~3;
}

// Floats of the attention item's LDS before its wave regions: the merge rows,
// the wave flags and q.  The merge rows come first so that every wave's row is
// one base address plus an immediate offset (below 64 KiB) for the merge's reads.
template <int DT>
constexpr int ps_att_head_floats() {
  return kPsWaves * (2 + DT) + kPsWaves + DT;
}

// Item h: query head h over the window [first, pos].  The item computes q
// itself, as a linear stage does (per-wave chunk dots of the residual, normed
// after the dot, reduced once in LDS; bias; RoPE), so the only handoff it
// waits for is the residual: the QKV items compute k and v alone.  Wave w
// takes the contiguous cached positions [first + w per, + per) below pos
// (per: a multiple of the pass length); its first pass of K/V rows is
// requested before the residual wait.  The last wave also takes the row at
// pos, after its range: it polls the new k and v (the sum of the kq published
// partials, computed meanwhile by the QKV items), appends them to the cache
// and adds their score to its softmax (this token's cache write is not
// ordered before the cache reads).  The 16 waves merge (max, sum, output) in
// LDS in wave order.
template <int FMT, typename KT, int DT, int NX>
__device__ __forceinline__ bool ps_att(const PsArgs& a, int l, int h, int first, int pos, int token, unsigned seq,
                                       bool l2, float* sm) {
  constexpr int ESZ = sizeof(KT);
  constexpr HeadTiling TL = head_tiling(DT, ESZ);
  constexpr int LPP = TL.lpp, SUB = TL.sub, DL = TL.dl;
  constexpr int EPL = DT / 64, NT = DT / 64;
  constexpr int KW = DL * ESZ / 4;
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  constexpr bool PAIRD = ESZ == 2 && DT == 128;
  // fp16 rows of 64: lane holds dims 2 (lane % 32), + 1 and sums half
  // lane / 32 of each pass's positions
  constexpr bool PAIR64 = ESZ == 2 && DT == 64;
  constexpr int NOE = PAIR64 ? 2 : EPL;
  constexpr int WF = ps_wave_floats<KT, DT>();
  static_assert(ps_att_head_floats<DT>() % 4 == 0, "wave regions hold 16-byte rows");
  static_assert(ps_lin_floats(CK, NX, NT) <= kPsWaves * WF, "q's dot products fit the wave regions");
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int hk = h / a.G;
  const int n = pos - first;  // cached rows
  const int per = max(SUB, ((n + kPsWaves - 1) / kPsWaves + SUB - 1) / SUB * SUB);
  const int t0 = min(first + wave * per, pos), t1 = min(t0 + per, pos);
  const bool active = t0 < t1;
  const bool own = wave == kPsWaves - 1;  // this wave takes the row at pos
  float* mg = sm;  // [16][2 + DT] per-wave (max, sum, output)
  int* good = reinterpret_cast<int*>(mg + kPsWaves * (2 + DT));  // [16]
  float* q_sh = reinterpret_cast<float*>(good + kPsWaves);  // [DT] q, read by every wave
  float* kn = sm + ps_att_head_floats<DT>() + wave * WF;
  float* vn = kn + DT;
  float* p_l = vn + DT;
  KT* vt = reinterpret_cast<KT*>(p_l + SUB);
  // q's dot products: their LDS overlaps the wave regions, used only after
  const PsLinLds s = ps_lin_lds<CK, NX, NT>(sm + ps_att_head_floats<DT>());
  PsRows<FMT, NX, NT> wr;
  wr.load(Ly.wqkv, Ly.sqkv, a.Cx, a.Tq, h * DT / kTile, 0, 0, a.Cx, wave);
  float nw[NX];
  wl_norm_weights<CK, NX>(Ly.attn_norm, a.Cx, wave, nw);
  float bias[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) bias[t] = wave == 0 ? gl(Ly.bqkv)[h * DT + 64 * t + lane] : 0.f;
  // RoPE factors of wave 0's elements (rotate-half of element d with its
  // partner, TSLAttention.ts:168-250)
  const int half = a.rd > 0 ? a.rd / 2 : 1;
  float rc[NT], rs[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int d = 64 * t + lane, jj = d < half ? d : d - half;
    const bool rot = wave == 0 && d < a.rd;
    rc[t] = rot ? gl(a.rope_cos)[(size_t)pos * half + jj] : 1.f;
    rs[t] = rot ? gl(a.rope_sin)[(size_t)pos * half + jj] : 0.f;
  }
  const KT* kh = reinterpret_cast<const KT*>(Ly.kc) + (size_t)hk * a.max_tokens * DT;
  const KT* vh = reinterpret_cast<const KT*>(Ly.vc) + (size_t)hk * a.max_tokens * DT;
  const int pl = lane / LPP, part = lane % LPP;
  HeadLoads<KT, KW, false, DL> ld;
  const int tc0 = active ? t0 : first, tc1 = active ? t1 : first + 1;  // in-range rows for idle waves
  ld.issue(kh, vh, tc0, tc1, pl, part, DT, DT * ESZ, lane);
  if (wave == 0) ps_stamp(a, l, PS_ATT, 0);
  // q4: q's weights widened to fp16 pairs while the residual is on its way
  PsRowsH<NX, NT> wh;
  if constexpr (ps_widen<FMT, NX>()) wh.from(wr);
  float x[NX];
  bool ok = true;
  if (l == 0) {
    wl_embedding<CK, NX>(a, token, a.Cx, wave, x);
  } else {
    const u64* px = a.pub_x + (size_t)(l - 1) * kPsMaxKs * a.H;
    ok = wl_gather<CK, NX>(0, a.Cx, a.ks, seq, [&](int p, int k) { return px + (size_t)p * a.H + k; }, wave, x, a.timeout);
  }
  if (wave == 0) ps_stamp(a, l, PS_ATT, 1);
  {  // q = norm(x) Wq + b (TSLRMSNorm.ts:50-74, TSLLinear.ts:56-75), rotated
    float xs[NX], ss = 0.f;
    wl_stage<FMT, CK, NX>(x, nw, s.xw, xs, ss);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if constexpr (ps_widen<FMT, NX>()) s.red[(wave * NT + t) * 64 + lane] = wh.dot(t, s.xw, xs, 0, 0, a.Cx, wave);
      else s.red[(wave * NT + t) * 64 + lane] = wr.dot(t, s.xw, xs, 0, 0, a.Cx, wave);
    }
    if (lane == 0) s.ssw[wave] = ss;
    if (!ps_all(ok, s.wf)) return false;
    if (wave == 0) {
      const float inv = rsqrtf(ps_sum16(s.ssw, 1) / (float)a.H + a.eps);
      if (NT == 1 && half == 32) {  // the rotation partner of lane d is lane d ^ 32
        const float val = bias[0] + inv * ps_sum16(s.red + lane, 64), partner = lane_swap32(val);
        q_sh[lane] = val * rc[0] + (lane < 32 ? -partner : partner) * rs[0];
      } else {
#pragma unroll
        for (int t = 0; t < NT; t++) s.out[64 * t + lane] = bias[t] + inv * ps_sum16(s.red + t * 64 + lane, NT * 64);
        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const int d = 64 * t + lane;
          float val = s.out[d];
          if (d < a.rd) val = val * rc[t] + (d < half ? -s.out[d + half] : s.out[d - half]) * rs[t];
          q_sh[d] = val;
        }
      }
    }
    lds_barrier();  // q visible to every wave; the dot products' LDS is free
  }
  float m = -INFINITY, lsum = 0.f, o[NOE];
#pragma unroll
  for (int e = 0; e < NOE; e++) o[e] = 0.f;
  if (active || own) {
    if (ok && active) {
      const float* qp = q_sh + part * DL;  // this lane's q slice (LDS broadcast reads)
      for (int tb = t0; tb < t1; tb += SUB) {
#pragma unroll
        for (int j = 0; j < 4; j++) reinterpret_cast<uint4*>(vt)[j * 64 + lane] = ld.vs[j];
        const int t = tb + pl;
        const bool valid = t < t1;
        uint32_t kw[KW];  // this lane's K slice
#pragma unroll
        for (int j = 0; j < KW; j++) kw[j] = ld.kw[j];
        wave_lds_sync();
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
        } else if constexpr (PAIR64) {
          // batches of 8 rows, their LDS reads issued together: one wait
          // per batch rather than one per row
          const int hh = lane >> 5;
          float a0 = hh == 0 ? o[0] * corr : 0.f, a1 = hh == 0 ? o[1] * corr : 0.f;
          const float4* p4 = reinterpret_cast<const float4*>(p_l + hh * (SUB / 2));
          const uint32_t* vw = reinterpret_cast<const uint32_t*>(vt + (size_t)hh * (SUB / 2) * DT) + (lane & 31);
#pragma unroll
          for (int g = 0; g < SUB / 2; g += 8) {
            const float4 pa = p4[g / 4], pb = p4[g / 4 + 1];
            uint32_t w[8];
#pragma unroll
            for (int u = 0; u < 8; u++) w[u] = vw[(size_t)(g + u) * (DT / 2)];
            const float pu[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
            for (int u = 0; u < 8; u++) {
              a0 = fmaf(pu[u], h2f(w[u] & 0xFFFFu), a0);
              a1 = fmaf(pu[u], h2f(w[u] >> 16), a1);
            }
          }
          o[0] = a0 + lane_swap32(a0);
          o[1] = a1 + lane_swap32(a1);
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
    if (ok && own) {  // the row at pos: its k and v, q · k over the wave, then one softmax step
      const u64* pq = a.pub_qkv + (size_t)l * a.kq * a.Nqkv;
      PsSpin spin(a.timeout);
      for (;;) {  // lane d: element d (+ 64 e) of k and v
        float sk[EPL], sv[EPL];
        bool got = true;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
          u64 wk[kPsMaxKs], wv[kPsMaxKs];
          const int d = lane + 64 * e;
#pragma unroll
          for (int j = 0; j < kPsMaxKs; j++) {
            const u64* pj = pq + (size_t)j * a.Nqkv;
            const bool in = j < a.kq;
            wk[j] = in ? ld_dev(pj + a.QS + hk * DT + d) : word(0.f, seq);
            wv[j] = in ? ld_dev(pj + a.QS + a.Hkv * DT + hk * DT + d) : word(0.f, seq);
          }
          sk[e] = sv[e] = 0.f;
#pragma unroll
          for (int j = 0; j < kPsMaxKs; j++) {
            got &= ((int)word_is(wk[j], seq) & (int)word_is(wv[j], seq)) != 0;
            sk[e] += word_value(wk[j]);
            sv[e] += word_value(wv[j]);
          }
        }
        if (__all(got)) {
#pragma unroll
          for (int e = 0; e < EPL; e++) {  // k and v rounded like the cache
            const int d = lane + 64 * e;
            const KT kr = kv_store<KT>(sk[e]), vr = kv_store<KT>(sv[e]);
            kn[d] = kv_load<KT>(&kr);
            vn[d] = kv_load<KT>(&vr);
            // the first query head of the group appends this position's k and
            // v (TSLAttention.ts:252-286); every head of the group rounds the
            // same sums
            if (h % a.G == 0) {
              glw(reinterpret_cast<KT*>(Ly.kc))[((size_t)hk * a.max_tokens + pos) * DT + d] = kr;
              glw(reinterpret_cast<KT*>(Ly.vc))[((size_t)hk * a.max_tokens + pos) * DT + d] = vr;
            }
          }
          break;
        }
        if (spin.tick() && spin.late()) {
          ok = false;
          break;
        }
      }
    }
    if (ok && own) {
      wave_lds_sync();
      float sp = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) sp = fmaf(q_sh[lane + 64 * e], kn[lane + 64 * e], sp);
      const float sc = wave_sum(sp) * a.scale;
      const float mn = fmaxf(m, sc);
      const float corr = m == -INFINITY ? 0.f : __expf(m - mn);
      const float p = __expf(sc - mn);
      lsum = lsum * corr + p;
      m = mn;
#pragma unroll
      for (int e = 0; e < NOE; e++) {
        const int d = PAIR64 ? 2 * (lane & 31) + e : PAIRD ? 2 * lane + e : lane + 64 * e;
        o[e] = fmaf(p, vn[d], o[e] * corr);
      }
    }
  }
  // merge the waves in order (an idle wave contributes max -inf, sum 0)
  float* mine = mg + wave * (2 + DT);
  if constexpr (PAIR64) {
    if (lane < 32) {
      mine[2 + 2 * lane] = o[0];
      mine[3 + 2 * lane] = o[1];
    }
  } else {
#pragma unroll
    for (int e = 0; e < EPL; e++) mine[2 + (PAIRD ? 2 * lane + e : lane + 64 * e)] = o[e];
  }
  if (lane == 0) {
    mine[0] = m;
    mine[1] = lsum;
  }
  if (!ps_all(ok, good)) return false;  // block-uniform
  if (wave == 0) ps_stamp(a, l, PS_ATT, 2);
  if (tid < DT) {
    // lane w (and w + 16, + 32, + 48) takes wave w's (max, sum) and its
    // scale exp(max_w - M): one exponential per lane instead of 16; the
    // scales reach every lane as scalar operands
    int w16 = lane & 15;
    asm volatile("" : "+v"(w16));  // computed here, not kept in a register from the kernel's start
    const float mw = mg[w16 * (2 + DT)], lw = mg[w16 * (2 + DT) + 1];
    float ow[kPsWaves];
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) ow[w] = mg[w * (2 + DT) + 2 + tid];
    const float M = wave_max(mw);
    const float f = mw == -INFINITY ? 0.f : __expf(mw - M);
    const float L = wave_sum(lane < 16 ? lw * f : 0.f);
    float od = 0.f;
#pragma unroll
    for (int w = 0; w < kPsWaves; w++) od = fmaf(ow[w], readlane(f, w), od);
    st_pub(l2, a.pub_o + (size_t)l * a.QS + h * DT + tid, word(od / L, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_ATT, 3);
  return true;
}

// -------------------------------------------------------------- O row tile --
// Item i: rows 64 t .. 64 t + 63 (t = i % To) of the O projection over the
// attention-output chunks of split j = i / To; split 0 adds the residual
// rows (the sum of the down partials, or layer 0's embedding row): the
// partials of x_mid.
template <int FMT, int NO>
__device__ __forceinline__ bool ps_o(const PsArgs& a, int l, int i, int token, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int H = a.H;
  const PsLinLds s = ps_lin_lds<CK, NO, 1>(sm);
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int t = i % a.To, j = i / a.To;
  const int c0 = j * a.co, c1 = min(c0 + a.co, a.Co);  // this split's input chunks
  PsRows<FMT, NO, 1> wr;
  wr.load(Ly.wo, Ly.so, a.Co, a.To, t, c0, c0, c1, wave);
  const int row = t * kTile + lane;
  if (wave == 0) ps_stamp(a, l, PS_O, 0);
  float x[NO], one[NO];
#pragma unroll
  for (int u = 0; u < NO; u++) one[u] = 1.f;
  // the residual rows first: they were published before this layer's QKV
  // stage, so their wait ends while the attention outputs are still on the
  // way (after the gather it would add a round trip to this item)
  bool ok = true;
  float xr = 0.f;
  if (wave == 0 && j == 0) {
    if (l == 0) {
      const size_t k = (size_t)token * H + min(row, H - 1);
      xr = a.emb_f32 ? gl(reinterpret_cast<const float*>(a.emb))[k]
                     : h2f(gl(reinterpret_cast<const uint16_t*>(a.emb))[k]);
    } else {
      const u64* px = a.pub_x + (size_t)(l - 1) * kPsMaxKs * H + min(row, H - 1);
      ok = wl_rows(a.ks, seq, [&](int p) { return px + (size_t)p * H; }, xr, a.timeout);
    }
  }
  // q4: the weights widened to fp16 pairs while the attention outputs are on their way
  PsRowsH<NO, 1> wh;
  if constexpr (ps_widen<FMT, NO>()) wh.from(wr);
  const u64* po = a.pub_o + (size_t)l * a.QS;
  ok &= wl_gather<CK, NO>(c0, c1, 1, seq, [&](int, int k) { return po + k; }, wave, x, a.timeout);
  if (wave == 0) ps_stamp(a, l, PS_O, 1);
  float xs[NO], ss;
  wl_stage<FMT, CK, NO>(x, one, s.xw, xs, ss);
  if constexpr (ps_widen<FMT, NO>()) s.red[wave * 64 + lane] = wh.dot(0, s.xw, xs, c0, c0, c1, wave);
  else s.red[wave * 64 + lane] = wr.dot(0, s.xw, xs, c0, c0, c1, wave);
  if (!ps_all(ok, s.wf)) return false;
  if (wave == 0) {
    ps_stamp(a, l, PS_O, 2);
    const float v = xr + ps_sum16(s.red + lane, 64);
    if (row < H) st_dev(a.pub_xm + ((size_t)l * a.ko + j) * H + row, word(v, seq));  // TSLAdd.ts:10-33
    ps_stamp(a, l, PS_O, 3);
  }
  return true;
}

// ------------------------------------------------------------ gate|up tiles --
// Item g: paired tiles g mw .. g mw + mw - 1 (tile t: gate rows 32 t.. in lanes
// 0..31, the matching up rows in lanes 32..63); publishes h = silu(g) * u for
// intermediate indices 32 t .. 32 t + 31.  The input is x_mid (the sum of the
// ko O partials), normed: the norm's scale multiplies the dot products.
template <int FMT, int NX, int MW>
__device__ __forceinline__ bool ps_gu(const PsArgs& a, int l, int g, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int H = a.H;
  const PsLinLds s = ps_lin_lds<CK, NX, MW>(sm);
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  PsRows<FMT, NX, MW> wr;
  wr.load(Ly.wgu, Ly.sgu, a.Cx, a.Tgu, g * MW, 0, 0, a.Cx, wave);
  float nw[NX];
  wl_norm_weights<CK, NX>(Ly.ffn_norm, a.Cx, wave, nw);
  if (wave == 0) ps_stamp(a, l, PS_GU, 0);
  // q4: the weights widened to fp16 pairs while x_mid is on its way
  PsRowsH<NX, MW> wh;
  if constexpr (ps_widen<FMT, NX>()) wh.from(wr);
  const u64* pm = a.pub_xm + (size_t)l * a.ko * H;
  float x[NX];
  const bool ok = wl_gather<CK, NX>(0, a.Cx, a.ko, seq, [&](int p, int k) { return pm + (size_t)p * H + k; }, wave, x, a.timeout);
  if (wave == 0) ps_stamp(a, l, PS_GU, 1);
  float xs[NX], ss;
  wl_stage<FMT, CK, NX>(x, nw, s.xw, xs, ss);
#pragma unroll
  for (int u = 0; u < MW; u++) {
    float dv = 0.f;
    if constexpr (ps_widen<FMT, NX>()) dv = wh.dot(u, s.xw, xs, 0, 0, a.Cx, wave);
    else dv = wr.dot(u, s.xw, xs, 0, 0, a.Cx, wave);
    s.red[(wave * MW + u) * 64 + lane] = g * MW + u < a.Tgu ? dv : 0.f;
  }
  if (lane == 0) s.ssw[wave] = ss;
  if (!ps_all(ok, s.wf)) return false;
  if (wave == 0) ps_stamp(a, l, PS_GU, 2);
  if (wave < MW && g * MW + wave < a.Tgu) {  // wave u finishes tile g mw + u
    const float inv = rsqrtf(ps_sum16(s.ssw, 1) / (float)H + a.eps);
    const float v = inv * ps_sum16(s.red + wave * 64 + lane, MW * 64);
    const float us = lane_swap32(v);  // lanes < 32: gate; their up rows sit in lanes + 32
    const float hv = v / (1.f + __expf(-v)) * us;  // TSLSiLUMul.ts:15-29
    if (lane < 32) st_dev(a.pub_h + (size_t)l * a.Tgu * 32 + (g * MW + wave) * 32 + lane, word(hv, seq));
  }
  if (wave == 0) ps_stamp(a, l, PS_GU, 3);
  return true;
}

// -------------------------------------------------------------- down tiles --
// Item (t, s): rows 64 t .. 64 t + 63 of the down projection over the input
// chunks [s cs, (s + 1) cs); split 0 adds x_mid (the MLP residual).
template <int FMT, int ND>
__device__ __forceinline__ bool ps_down(const PsArgs& a, int l, int t, int sp, unsigned seq, float* sm) {
  constexpr int CK = FMT == WF_Q4 ? 32 : 8;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int H = a.H;
  const PsLinLds s = ps_lin_lds<CK, ND, 1>(sm);
  const TLM_GLOBAL PsLayer& Ly = gl(a.layers)[l];
  const int c0 = sp * a.cs, c1 = min(c0 + a.cs, a.Cd);
  PsRows<FMT, ND, 1> wr;
  wr.load(Ly.wd, Ly.sd, a.Cd, a.To, t, c0, c0, c1, wave);
  const int row = t * kTile + lane;
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 0);
  const u64* ph = a.pub_h + (size_t)l * a.Tgu * 32;
  float x[ND], one[ND];
#pragma unroll
  for (int u = 0; u < ND; u++) one[u] = 1.f;
  // x_mid first: published before the gate|up stage, so its wait ends while
  // h is still on the way
  bool ok = true;
  float xm = 0.f;
  if (wave == 0 && sp == 0) {
    const u64* pm = a.pub_xm + (size_t)l * a.ko * H + min(row, H - 1);
    ok = wl_rows(a.ko, seq, [&](int p) { return pm + (size_t)p * H; }, xm, a.timeout);
  }
  // q4: the weights widened to fp16 pairs while h is on its way
  PsRowsH<ND, 1> wh;
  if constexpr (ps_widen<FMT, ND>()) wh.from(wr);
  ok &= wl_gather<CK, ND>(c0, c1, 1, seq, [&](int, int k) { return ph + k; }, wave, x, a.timeout);
  if (wave == 0) ps_stamp(a, l, PS_DOWN, 1);
  float xs[ND], ss;
  wl_stage<FMT, CK, ND>(x, one, s.xw, xs, ss);
  if constexpr (ps_widen<FMT, ND>()) s.red[wave * 64 + lane] = wh.dot(0, s.xw, xs, c0, c0, c1, wave);
  else s.red[wave * 64 + lane] = wr.dot(0, s.xw, xs, c0, c0, c1, wave);
  if (!ps_all(ok, s.wf)) return false;
  if (wave == 0) {
    ps_stamp(a, l, PS_DOWN, 2);
    const float v = xm + ps_sum16(s.red + lane, 64);  // split 0 carries x_mid (TSLAdd.ts:10-33)
    if (row < H) st_dev(a.pub_x + ((size_t)l * kPsMaxKs + sp) * H + row, word(v, seq));
    // a q4 input past the fp16 range made its wave's dot products NaN, and
    // NaN reaches every later stage: the last layer's rows tell the host
    if (l == a.L - 1 && row < H && !(fabsf(v) <= FLT_MAX))
      __hip_atomic_fetch_or(glw(a.ctrl + C_ERR), kPsErrRange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ps_stamp(a, l, PS_DOWN, 3);
  }
  return true;
}

// -------------------------------------------------------------------- kernel --
template <int FMT, typename KT, int DT, int NX, int NO, int ND, int MW, bool L2>
__global__ __launch_bounds__(kPsWaves * 64) void ps_token_kernel(const PsArgs* __restrict__ ap) {
  extern __shared__ float sm[];
  const PsArgs& a = *ap;  // in device memory: field reads are scalar loads
  const int pos = gl(a.ctrl)[C_POS], token = gl(a.ctrl)[C_TOKEN];
  const unsigned seq = (unsigned)gl(a.ctrl)[C_SEQ];
  if (pos < 0 || pos >= a.max_tokens) return;
  ps_stamp(a, a.L, 0, 0);
  const TLM_GLOBAL int* rl = gl(a.roles) + blockIdx.x * kPsRoles * 2;
  // handoffs through the L2 only on the XCD the roles were placed for
  const bool on_xcd = L2 && a.xcc && xcc_id() == gl(a.xcc)[blockIdx.x];
  for (int l = 0; l < a.L; l++) {
    const int win = gl(a.layers)[l].window;  // DecoderCPURunner.ts:150 (block.slidingWindow)
    const int first = win > 0 ? max(pos - win + 1, 0) : 0;
#pragma unroll 1
    for (int r = 0; r < kPsRoles; r++) {
      const int code = rl[2 * r], it = rl[2 * r + 1];
      const int st = code < 0 ? -1 : code & kPsStageMask;
      const bool l2 = on_xcd && (code & kPsLocal);
      bool ok = true;
      if (st == PS_QKV)
        ok = ps_qkv<FMT, KT, DT, NX>(a, l, it, pos, token, seq, l2, sm);
      else if (st == PS_ATT)
        ok = ps_att<FMT, KT, DT, NX>(a, l, it, first, pos, token, seq, l2, sm);
      else if (st == PS_O)
        ok = ps_o<FMT, NO>(a, l, it, token, seq, sm);
      else if (st == PS_GU)
        ok = ps_gu<FMT, NX, MW>(a, l, it, seq, sm);
      else if (st == PS_DOWN)
        ok = ps_down<FMT, ND>(a, l, it % a.To, it / a.To, seq, sm);
      if (!ok) {  // a bounded wait ran out: report and leave (block-uniform)
        if (threadIdx.x == 0)
          __hip_atomic_fetch_or(glw(a.ctrl + C_ERR), kPsErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// down split; mw gate|up tiles per item).  None for head_dim 128: at the
// Llama-3.2-3B shape (648 items, three roles on most blocks, registers spilled)
// the schedule took 1274 us per token at positions 127..382 against 1102 for the
// per-stage graph; the Llama-3.2-1B shape gains (447 against 512).
static const PsVariant kPsVariants[] = {
    {WF_Q4, 0, 64, 2, 1, 3, 1},   // hidden 896, 14 x 64 heads, inter 4864 (Qwen2.5-0.5B shape)
    {WF_Q4, 0, 64, 4, 1, 4, 1},   // hidden 2048, 32 x 64 heads, inter 8192 (Llama-3.2-1B shape)
    {WF_Q4, 0, 64, 1, 1, 1, 1},   // hidden <= 512 q4
    {WF_F16, 0, 64, 2, 1, 3, 1},  // hidden 256 fp16
};

// Items of each stage for a shape's splits.
static void ps_counts(int H, int Hq, int Hkv, int Tgu, int kq, int ko, int mw, int ks, int* c) {
  const int To = H / 64;
  c[PS_QKV] = 2 * Hkv * kq;  // k and v heads (the attention items compute q)
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
  // 16K per split (every split is one more set of producers a consumer waits
  // for and one more partial it adds: Qwen2.5-0.5B shape, 381 us/token at
  // kq = ko = 2 against 387.5 at 4 and 4, 383 at 1 and 2, 386.4 at 1 and 4),
  // plus the cost of a third role per block (about two microseconds of a
  // CU's multiply-adds, serial behind the previous role)
  PsShape best = none;
  long best_cost = 0;
  // TLM_PS_SPLITS=kq,ko,ks fixes the K-splits (comparisons)
  int fq = 0, fo = 0, fs = 0;
  if (const char* e = getenv("TLM_PS_SPLITS")) sscanf(e, "%d,%d,%d", &fq, &fo, &fs);
  for (const PsVariant& v : kPsVariants) {
    if (v.fmt != fmt || v.kv_f32 != kv_f32 || v.dt != D || v.nx < nx) continue;
    for (int kq = 1; kq <= kPsMaxKs; kq++)
      for (int ko = 1; ko <= kPsMaxKs; ko++)
        for (int ks = 1; ks <= kPsMaxKs; ks++) {
          if ((fq && kq != fq) || (fo && ko != fo) || (fs && ks != fs)) continue;
          const int cq = (Cx + kq - 1) / kq, co = (Co + ko - 1) / ko, cs = (Cd + ks - 1) / ks;
          if ((co + 15) / 16 > v.no || (cs + 15) / 16 > v.nd) continue;
          int counts[PS_STAGES];
          ps_counts(H, Hq, Hkv, Tgu, kq, ko, v.mw, ks, counts);
          const int r = ps_place(counts, cus, nullptr);
          if (!r) continue;
          const long macs = (long)D * cq * CK + 64L * co * CK + 64L * v.mw * H + 64L * cs * CK;
          const long cost = macs + 16384L * (kq + ko + ks) + (r > 2 ? 128L * 1024 : 0);
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

__global__ void ps_xcc_kernel(int* xcc) {
  if (threadIdx.x == 0) xcc[blockIdx.x] = xcc_id();
}

bool ps_xcc_probe(int blocks, int* xcc) {
  int* d = nullptr;
  if (hipMalloc(&d, sizeof(int) * blocks) != hipSuccess) return false;
  hipLaunchKernelGGL(ps_xcc_kernel, dim3(blocks), dim3(64), 0, 0, d);
  const bool ok = hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
                  hipMemcpy(xcc, d, sizeof(int) * blocks, hipMemcpyDeviceToHost) == hipSuccess;
  hipFree(d);
  return ok;
}

// The hardware hands a launch's workgroups to the XCDs in turn, so blocks with
// one value of b % 8 share an XCD (checked on xcc).  A group is the k|v items
// and attention items of one kv head, and, when every O split covers whole kv
// heads, those of all kv heads of one split together with the split's O items.
// Each group goes to one class of blocks; the k|v items publish through the
// L2 (their consumers are the group's attention items), and so do the
// attention items when the O items are in the group.
int ps_localize(const PsShape& sh, int blocks, int Hq, int Hkv, int To, const int* xcc, int* roles) {
  constexpr int kClasses = 8;
  if (!xcc || blocks % kClasses != 0 || Hkv <= 0 || Hq % Hkv != 0) return 0;
  for (int b = 0; b < blocks; b++)
    if (xcc[b] != xcc[b % kClasses]) return 0;
  for (int c = 0; c < kClasses; c++)
    for (int e = c + 1; e < kClasses; e++)
      if (xcc[c] == xcc[e]) return 0;
  const int G = Hq / Hkv, CK = sh.fmt == WF_Q4 ? 32 : 8, QS = Hq * sh.dt;
  const int co = (QS / CK + sh.ko - 1) / sh.ko;  // O chunks per split
  bool o_in = true;                               // every O split covers whole kv heads
  for (int j = 0; j < sh.ko; j++) {
    const int d0 = j * co * CK, d1 = std::min((j + 1) * co * CK, QS);
    if (d0 % (G * sh.dt) != 0 || (d1 % (G * sh.dt) != 0 && d1 != QS)) o_in = false;
  }
  const int groups = o_in ? sh.ko : Hkv;
  if (groups > kClasses) return 0;
  auto group_of_kv = [&](int g) { return o_in ? g * G * sh.dt / (co * CK) : g; };
  auto group_of = [&](int st, int it) {
    if (st == PS_QKV) return group_of_kv((it / sh.kq) % Hkv);
    if (st == PS_ATT) return group_of_kv(it / G);
    if (st == PS_O && o_in) return it / To;
    return -1;
  };
  const int per = blocks / kClasses;
  std::vector<int> used(kClasses, 0), dest(blocks, -1);
  std::vector<bool> taken(blocks, false);
  // blocks holding a group's item first, each to the next free block of its class
  for (int b = 0; b < blocks; b++) {
    int g = -1;
    for (int r = 0; r < kPsRoles; r++) {
      const int st = roles[2 * (kPsRoles * b + r)];
      if (st < 0) continue;
      const int gi = group_of(st, roles[2 * (kPsRoles * b + r) + 1]);
      if (gi < 0) continue;
      if (g >= 0 && gi != g) return 0;  // two groups on one block
      g = gi;
    }
    if (g < 0) continue;
    if (used[g] == per) return 0;  // the group does not fit its class
    const int nb = g + kClasses * used[g]++;
    dest[b] = nb;
    taken[nb] = true;
  }
  int next = 0;
  for (int b = 0; b < blocks; b++) {
    if (dest[b] >= 0) continue;
    while (taken[next]) next++;
    dest[b] = next;
    taken[next] = true;
  }
  std::vector<int> out((size_t)2 * kPsRoles * blocks);
  int marked = 0;
  for (int b = 0; b < blocks; b++)
    for (int r = 0; r < kPsRoles; r++) {
      int st = roles[2 * (kPsRoles * b + r)];
      const int it = roles[2 * (kPsRoles * b + r) + 1];
      if (st == PS_QKV || (st == PS_ATT && o_in)) {
        st |= kPsLocal;
        marked++;
      }
      out[2 * (kPsRoles * dest[b] + r)] = st;
      out[2 * (kPsRoles * dest[b] + r) + 1] = it;
    }
  std::copy(out.begin(), out.end(), roles);
  return marked;
}

size_t ps_smem_bytes(const PsShape& sh, int H, int QS) {
  (void)H;
  (void)QS;
  const int CK = sh.fmt == WF_Q4 ? 32 : 8;
  const size_t esz = sh.kv_f32 ? 4 : 2;
  const int sub = head_tiling(sh.dt, (int)esz).sub;
  // the attention item: merge rows, flags, q, then the wave regions
  const size_t att = (size_t)kPsWaves * (2 + sh.dt) + kPsWaves + sh.dt + (size_t)kPsWaves * ((2 * sh.dt + sub + 1024 + 3) & ~3);
  const size_t qkv = ps_lin_floats(CK, sh.nx, sh.dt / 64);
  const size_t o = ps_lin_floats(CK, sh.no, 1);
  const size_t gu = ps_lin_floats(CK, sh.nx, sh.mw);
  const size_t down = ps_lin_floats(CK, sh.nd, 1);
  return sizeof(float) * std::max({att, qkv, o, gu, down});
}

// The compiled kernel of a shape (null: none).
// (l2: the variant that publishes through an XCD's L2 where the roles say so;
// the other one has no such stores at all)
static const void* ps_kernel(const PsShape& sh, bool l2) {
#define PS_CASE(F, KV, DTV, NXV, NOV, NDV, MWV)                                                             \
  if (sh.fmt == F && sh.kv_f32 == KV && sh.dt == DTV && sh.nx == NXV && sh.no == NOV && sh.nd == NDV &&   \
      sh.mw == MWV)                                                                                       \
    return l2 ? (const void*)ps_token_kernel<F, std::conditional_t<KV, float, uint16_t>, DTV, NXV, NOV, NDV, MWV, true>  \
              : (const void*)ps_token_kernel<F, std::conditional_t<KV, float, uint16_t>, DTV, NXV, NOV, NDV, MWV, false>;
  PS_CASE(WF_Q4, 0, 64, 2, 1, 3, 1)
  PS_CASE(WF_Q4, 0, 64, 4, 1, 4, 1)
  PS_CASE(WF_Q4, 0, 64, 1, 1, 1, 1)
  PS_CASE(WF_F16, 0, 64, 2, 1, 3, 1)
#undef PS_CASE
  return nullptr;
}

bool ps_prepare(const PsShape& sh, size_t smem) {
  for (bool l2 : {false, true}) {
    const void* k = ps_kernel(sh, l2);
    if (!k || hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) return false;
  }
  return true;
}

bool launch_ps_token(const PsShape& sh, int blocks, size_t smem, const PsArgs* a_dev, hipStream_t st) {
  const void* k = ps_kernel(sh, sh.l2 != 0);
  if (!k) return false;
  const PsArgs* arg = a_dev;
  void* params[] = {&arg};
  return hipLaunchKernel(k, dim3(blocks), dim3(kPsWaves * 64), params, smem, st) == hipSuccess;
}

}  // namespace tlm

// Device helpers shared by the kernel files: fp16 and fixed-point
// conversions, DPP wave reductions, the q4 / fp16 16-byte chunk dots and the
// decode attention tiling.
#pragma once
#include <float.h>

#include <hip/hip_fp16.h>

#include "tlm_kernels.h"

namespace tlm {

// A pointer known to address global memory (address space 1): loads and
// stores through it are global_* instructions.  Pointers read from memory
// (argument tables) are otherwise generic, and flat instructions count in
// lgkmcnt too, so every LDS wait would also wait for them.
#define TLM_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const TLM_GLOBAL T* gl(const T* p) {
  return (const TLM_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ TLM_GLOBAL T* glw(T* p) {
  return (TLM_GLOBAL T*)p;
}

constexpr float kLowest = -3.4028234663852886e38f;  // TSLLogits.ts:21 LOWEST_FLOAT

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

// Fixed-point residual values (x * 2^32 as a two's-complement int64).
__device__ __forceinline__ unsigned long long to_fx(float v) {
  return (unsigned long long)__float2ll_rn(v * kFxScale);
}
__device__ __forceinline__ float from_fx(unsigned long long s) { return __ll2float_rn((long long)s) * kFxInv; }
// The accumulators add int64 replicas modulo 2^64, so a residual value is exact
// while the true sum stays below 2^31 in magnitude.  A term or a sum of 2^30
// or more (or NaN) sets ctrl[C_FXR]: the host then reports the results as
// invalid instead of reading wrapped values.
constexpr float kFxLimit = 1073741824.0f;  // 2^30
__device__ __forceinline__ void fx_guard(float v, const int* ctrl) {
  if (!(fabsf(v) < kFxLimit) && ctrl)
    __hip_atomic_fetch_or(const_cast<int*>(ctrl) + C_FXR, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-lane moves through DPP (data-parallel primitives: a VALU operand
// modifier, no LDS round trip).  Every reduction below pairs lanes
// symmetrically, so all lanes of a group end with the same bits.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float sum8(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  return v + dpp<kDppHalfMirror>(v);
}

// v of lane l ^ 16 / l ^ 32, through gfx950's VALU lane swaps
// (v_permlane16_swap / v_permlane32_swap) rather than an LDS round trip.
__device__ __forceinline__ float lane_swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Sum / max over the 64 lanes of a wave (wave-uniform result).
__device__ __forceinline__ float wave_sum(float v) {
  v = sum8(v);
  v += dpp<kDppMirror>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

// Block-wide sum (blockDim.x a multiple of 64); every thread gets the result.
// scratch holds one float per wave and must not be in use by another
// reduction of the same kernel (each kernel calls this once per scratch).
// Block barrier that orders LDS only.  __syncthreads() also orders global
// memory, so every wave first waits for all of its outstanding vector loads:
// a kernel that issues its weight (or cache) loads early and computes on LDS
// data in between would otherwise consume nothing until the last load lands.
// For kernels whose threads exchange data through LDS only (global outputs
// are read by later kernels).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over the block, in every thread; scratch: LDS, one float per wave.
__device__ inline float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) scratch[wave] = v;
  lds_barrier();
  float r = 0.f;
  for (int i = 0; i < nw; i++) r += scratch[i];
  return r;
}

// Greedy order of TSLLogits.ts:228-229: higher score, ties to the lower id.
// A strict total order on (score, id) for non-NaN scores; lanes start from
// (LOWEST, INT_MAX) and only take better candidates, so NaN never enters.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  const float ov = dpp<CTRL>(v);
  const int oi = dpp<CTRL>(i);
  if (better(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

// Best (score, id) of the wave, in every lane.
// A 64-bit key whose unsigned order is the greedy order of (score, id):
// the higher score, then the lower id (better()); -0 counts as +0.
__device__ __forceinline__ unsigned long long greedy_key(float v, int i) {
  const unsigned u = __float_as_uint(v == 0.f ? 0.f : v);
  const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)o << 32) | (0xffffffffu - (unsigned)i);
}
__device__ __forceinline__ float greedy_key_value(unsigned long long k) {
  const unsigned o = (unsigned)(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ int greedy_key_id(unsigned long long k) { return (int)(0xffffffffu - (unsigned)k); }

__device__ inline void wave_argmax(float& v, int& i) {
  argmax_step<kDppXor1>(v, i);
  argmax_step<kDppXor2>(v, i);
  argmax_step<kDppHalfMirror>(v, i);
  argmax_step<kDppMirror>(v, i);
  float bv = readlane(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float rv = readlane(v, r);
    const int ri = __builtin_amdgcn_readlane(i, r);
    if (better(rv, ri, bv, bi)) {
      bv = rv;
      bi = ri;
    }
  }
  v = bv;
  i = bi;
}

// 32 q4 weights of one row (one 16-byte chunk) against x[0..32).
// sum_k s*(n_k - 8)*x_k = s*(sum_k n_k x_k - 8*sum_k x_k); n_k in [0,15] via
// byte-lane conversions (v_cvt_f32_ubyte*).
__device__ __forceinline__ float dot_q4(const uint4 d, const float* __restrict__ x, float xsum, float s) {
  const uint32_t wv[4] = {d.x, d.y, d.z, d.w};
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t lo = wv[j] & 0x0F0F0F0Fu, hi = (wv[j] >> 4) & 0x0F0F0F0Fu;
    // opaque to the optimiser: otherwise it folds the masks into per-nibble
    // bit-field extracts (v_bfe_u32 + v_cvt_f32_ubyte0) instead of converting
    // byte k of lo / hi directly (v_cvt_f32_ubyte{0..3}), 24 more VALU per chunk
    asm("" : "+v"(lo), "+v"(hi));
    const float4 xa = *reinterpret_cast<const float4*>(x + 8 * j);
    const float4 xb = *reinterpret_cast<const float4*>(x + 8 * j + 4);
    a0 = fmaf((float)(lo & 0xFFu), xa.x, a0);
    a1 = fmaf((float)(hi & 0xFFu), xa.y, a1);
    a0 = fmaf((float)((lo >> 8) & 0xFFu), xa.z, a0);
    a1 = fmaf((float)((hi >> 8) & 0xFFu), xa.w, a1);
    a0 = fmaf((float)((lo >> 16) & 0xFFu), xb.x, a0);
    a1 = fmaf((float)((hi >> 16) & 0xFFu), xb.y, a1);
    a0 = fmaf((float)(lo >> 24), xb.z, a0);
    a1 = fmaf((float)(hi >> 24), xb.w, a1);
  }
  return s * ((a0 + a1) - 8.f * xsum);
}

// 32 q4 weights of one row (one 16-byte chunk) against fp16 inputs, two
// weights per v_dot2_f32_f16.  xh: 16 dwords, dword 4 j + i = (x[8 j + i],
// x[8 j + i + 4]); xsum = the sum of those 32 fp16 values.  Nibble m of
// dword j (weight k = 8 j + m) is moved to bits 4..7 of one half (m < 4: the
// low half, with m + 4 in the high half), and 0x3C00 or'ed in: the fp16
// value 1 + n / 64 (exact).  Products of two fp16 values are exact in fp32,
// so acc = sum_k (1 + n_k / 64) x_k, and
// sum_k (n_k - 8) x_k = 64 acc - 72 xsum.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// (a & m) | c in one v_and_or_b32 (the compiler otherwise emits an and and an
// or: VOP3 takes no literal on gfx950, so m and c sit in registers)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
  return r;
}
__device__ __forceinline__ float dot_q4h(const uint4 d, const uint32_t* __restrict__ xh, float xsum, float s) {
  const uint32_t wv[4] = {d.x, d.y, d.z, d.w};
  const uint32_t M = 0x00F000F0u, E = 0x3C003C00u;
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint4 xp = *reinterpret_cast<const uint4*>(xh + 4 * j);
    const uint32_t w = wv[j];
    const uint32_t p0 = and_or(w << 4, M, E), p1 = and_or(w, M, E), p2 = and_or(w >> 4, M, E),
                   p3 = and_or(w >> 8, M, E);
    a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p0), __builtin_bit_cast(f16x2, xp.x), a0, false);
    a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p1), __builtin_bit_cast(f16x2, xp.y), a1, false);
    a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p2), __builtin_bit_cast(f16x2, xp.z), a0, false);
    a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p3), __builtin_bit_cast(f16x2, xp.w), a1, false);
  }
  return s * fmaf(64.f, a0 + a1, -72.f * xsum);
}

// 8 fp16 weights of one row against x[0..8).
__device__ __forceinline__ float dot_f16(const uint4 d, const float* __restrict__ x) {
  const uint32_t wv[4] = {d.x, d.y, d.z, d.w};
  const float4 xa = *reinterpret_cast<const float4*>(x);
  const float4 xb = *reinterpret_cast<const float4*>(x + 4);
  float a0 = 0.f, a1 = 0.f;
  a0 = fmaf(h2f(wv[0] & 0xFFFFu), xa.x, a0);
  a1 = fmaf(h2f(wv[0] >> 16), xa.y, a1);
  a0 = fmaf(h2f(wv[1] & 0xFFFFu), xa.z, a0);
  a1 = fmaf(h2f(wv[1] >> 16), xa.w, a1);
  a0 = fmaf(h2f(wv[2] & 0xFFFFu), xb.x, a0);
  a1 = fmaf(h2f(wv[2] >> 16), xb.y, a1);
  a0 = fmaf(h2f(wv[3] & 0xFFFFu), xb.z, a0);
  a1 = fmaf(h2f(wv[3] >> 16), xb.w, a1);
  return a0 + a1;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Global-memory vector loads (through the native vector types: HIP's vector
// classes cannot bind an address-space-1 reference).
__device__ __forceinline__ uint4 ldg_u4(const uint4* p) {
  const u32x4 v = *gl(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg_u2(const void* p) {
  const u32x2 v = *gl(reinterpret_cast<const u32x2*>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float4 ldg_f4(const float* p) {
  const f32x4 v = *gl(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

template <typename KT>
__device__ __forceinline__ float kv_load(const KT* p);
template <>
__device__ __forceinline__ float kv_load<uint16_t>(const uint16_t* p) { return h2f(*p); }
template <>
__device__ __forceinline__ float kv_load<float>(const float* p) { return *p; }
template <typename KT>
__device__ __forceinline__ KT kv_store(float v);
template <>
__device__ __forceinline__ uint16_t kv_store<uint16_t>(float v) { return __half_as_ushort(__float2half_rn(v)); }
template <>
__device__ __forceinline__ float kv_store<float>(float v) { return v; }

// Tiling of head_kernel: LPP lanes per cached position, so each lane holds 64
// bytes of a K row; SUB = 64 / LPP positions per pass; the V rows of a pass
// (always 4 KiB) are staged in LDS with 64 bytes per lane.
struct HeadTiling {
  int lpp, sub, dl;
};
constexpr __host__ __device__ inline HeadTiling head_tiling(int dt, int esz) {
  HeadTiling t{};
  t.lpp = dt * esz <= 64 ? 1 : dt * esz / 64;
  t.sub = 64 / t.lpp;
  t.dl = dt / t.lpp;  // K elements per lane
  return t;
}

// Compiled head dimension: 64 and 128 exactly; 32 covers any even head_dim
// <= 32 through runtime bounds (element-wise, clamped loads).
inline int attn_dt(int D) { return D <= 32 ? 32 : D; }


// LDS of one head_kernel wave (floats): q, the new k and v, their pre-RoPE
// values, the pass's probabilities and the V tile (4 KiB); a multiple of 4
// floats so every wave's region stays 16-byte aligned.
constexpr __host__ __device__ inline int head_wave_floats(int dt, int esz) {
  return (6 * dt + head_tiling(dt, esz).sub + 1024 + 3) & ~3;
}


// Order a wave's own LDS writes before its later reads (regions private to
// one wave: no block barrier, whose waves may run different pass counts).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Global loads of one head_kernel pass, held in registers: this lane's K-row
// slice (DL elements) and its 64 bytes of the pass's V rows.  Unconditional:
// rows are clamped to t1 - 1.
template <typename KT, int KW, bool GEN, int DL>
struct HeadLoads {
  static constexpr int ESZ = sizeof(KT);
  uint32_t kw[KW];
  uint4 vs[4];
  __device__ __forceinline__ void issue(const KT* kh, const KT* vh, int tb, int t1, int pl, int part, int D,
                                        int row_bytes, int lane) {
    const int t = min(tb + pl, t1 - 1);
    if (!GEN) {
      const TLM_GLOBAL u32x4* kr = gl(reinterpret_cast<const u32x4*>(kh + (size_t)t * D + part * DL));
#pragma unroll
      for (int j = 0; j < KW / 4; j++) {
        const u32x4 v = kr[j];
        kw[4 * j] = v.x;
        kw[4 * j + 1] = v.y;
        kw[4 * j + 2] = v.z;
        kw[4 * j + 3] = v.w;
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int off = (j * 64 + lane) * 16;  // byte offset in the [SUB][D] tile
        const int r = min(tb + off / row_bytes, t1 - 1);
        const u32x4 v = *gl(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vh + (size_t)r * D) +
                                                          off % row_bytes));
        vs[j] = make_uint4(v.x, v.y, v.z, v.w);
      }
    } else {
      const KT* kr = kh + (size_t)t * D;
#pragma unroll
      for (int e = 0; e < DL; e++) {
        const int k = min(part * DL + e, D - 1);
        const uint32_t v = ESZ == 2 ? (uint32_t)((const uint16_t*)kr)[k] : ((const uint32_t*)kr)[k];
        if (ESZ == 2) {
          if (e & 1) kw[e >> 1] |= v << 16; else kw[e >> 1] = v;
        } else {
          kw[e] = v;
        }
      }
    }
  }
};

}  // namespace tlm

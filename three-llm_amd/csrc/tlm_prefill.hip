// Batched prefill: M prompt positions per layer pass.  The reference replays
// its one-token decode graph once per prompt position (DecoderTSLRunner.ts:
// 472-480, 504-530); here the linears of all M positions run as one q4 x fp16
// GEMM on MFMA (v_mfma_f32_32x32x16_f16) and causal attention as one MFMA
// flash-attention pass, which gives the token-by-token result up to fp16
// rounding of the activations.
#include "tlm_kernels.h"
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdlib.h>

namespace tlm {

// fp16 rounding of a prefill activation with the overflow report: values at
// or beyond 65520 in magnitude (they round to inf) and NaN set *ovf, and the
// host then replays the chunk on the fp32 decode path.
__device__ __forceinline__ _Float16 f16_guard(int* ovf, float v) {
  if (ovf && !(fabsf(v) < 65520.f)) __hip_atomic_fetch_or(ovf, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (_Float16)v;
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));

namespace {

// 8 q4 codes of one dword (k order: low then high nibble of each byte) as
// fp16 (code - 8) * s.  The fp16 bit pattern 0x6400 | n is 1024 + n, so
// subtracting 1032 gives n - 8 exactly; the product with s rounds once.
__device__ __forceinline__ half8_t dequant8(uint32_t w, half2_t s2) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  half8_t r;
#pragma unroll
  for (int b = 0; b < 4; b++) {
    // byte 0 <- lo byte b, byte 2 <- hi byte b, bytes 1 and 3 <- 0 (selector 0x0c)
    const uint32_t sel = 0x0c000c00u | (uint32_t)b | ((uint32_t)(4 + b) << 16);
    const uint32_t bits = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
    half2_t v = __builtin_bit_cast(half2_t, bits);
    v = (v - (half2_t){(_Float16)1032.f, (_Float16)1032.f}) * s2;
    r[2 * b] = v[0];
    r[2 * b + 1] = v[1];
  }
  return r;
}

__device__ __forceinline__ half8_t as_half8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

// silu(g) * u for a result rounded to fp16: the hardware reciprocal (1 ulp)
// instead of a full-precision division; g -> -inf gives exp = inf, rcp = 0.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)) * u;
}

// Cross-lane steps on the VALU (DPP, gfx950's v_permlane16/32_swap) instead of
// ds_bpermute, whose LDS round trips each cost a wait.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_amdgcn_update_dpp(0.f, v, CTRL, 0xF, 0xF, false);
}
// v of lane l ^ 32
__device__ __forceinline__ float swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
// Sum over each 32-lane half of the wave, the same bits in every lane of the half.
__device__ __forceinline__ float half_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_f<0x141>(v);  // row_half_mirror: lane i <-> 7 - i of its 8
  v += dpp_f<0x140>(v);  // row_mirror: lane i <-> 15 - i of its 16
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return v + __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}

__device__ __forceinline__ float block_sum_f(float v, float* scratch) {
  v = half_sum(v);
  v += swap32(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; i++) s += scratch[i];
  return s;
}

}  // namespace

// Global loads of one 32-k step: the thread's A pieces and the lane's weight
// chunks (q4: one 16-byte chunk + scale; fp16: the two 8-k chunks of its half).
template <int FMT, int MT, int NB>
struct GemmPtrs {
  const uint16_t* asrc[MT];
  const uint4* wp[NB];
  const uint16_t* sp[NB];
};
// Registers of one step in flight; members are named, not arrays, so that the
// compiler keeps every stage of the ring in registers.
template <int FMT, int MT, int NB>
struct GemmStage {
  static_assert(MT <= 2 && NB <= 2, "stage registers are spelled out for MT, NB <= 2");
  uint4 a0, a1;      // A pieces (a1 when MT == 2)
  uint4 w0, w1;      // column group 0: q4 chunk, or the two fp16 chunks
  uint4 v0, v1;      // column group 1 (NB == 2)
  uint16_t s0, s1;   // q4 scales of the groups
  __device__ __forceinline__ void load(const GemmPtrs<FMT, MT, NB>& p, int c, int kh) {
    a0 = *reinterpret_cast<const uint4*>(p.asrc[0] + c * 32);
    if constexpr (MT > 1) a1 = *reinterpret_cast<const uint4*>(p.asrc[1] + c * 32);
    if constexpr (FMT == WF_Q4) {
      w0 = p.wp[0][(size_t)c * kTile];
      s0 = p.sp[0][(size_t)c * kTile];
      if constexpr (NB > 1) {
        v0 = p.wp[1][(size_t)c * kTile];
        s1 = p.sp[1][(size_t)c * kTile];
      }
    } else {
      w0 = p.wp[0][(size_t)(4 * c + kh) * kTile];
      w1 = p.wp[0][(size_t)(4 * c + 2 + kh) * kTile];
      if constexpr (NB > 1) {
        v0 = p.wp[1][(size_t)(4 * c + kh) * kTile];
        v1 = p.wp[1][(size_t)(4 * c + 2 + kh) * kTile];
      }
    }
  }
  // B operands of column group j for the two 16-k halves of the step
  __device__ __forceinline__ void operands(int j, int kh, half8_t& b1, half8_t& b2) const {
    const uint4& x = j ? v0 : w0;
    if constexpr (FMT == WF_Q4) {
      const _Float16 s = __builtin_bit_cast(_Float16, j ? s1 : s0);
      const half2_t s2 = {s, s};
      b1 = dequant8(kh ? x.y : x.x, s2);
      b2 = dequant8(kh ? x.w : x.z, s2);
    } else {
      b1 = as_half8(x);
      b2 = as_half8(j ? v1 : w1);
    }
  }
};

// ----------------------------------------------------------------- GEMM --
// C = A W^T.  Block: 4 waves as 2 (rows) x 2 (columns); a wave owns 32 MT rows
// x 32 NB columns as MT x NB MFMA tiles of 32 x 32.  Per 32-k step the block's
// A rows [64 MT][32] go through LDS (double buffered, one barrier per step)
// and each lane forms its column's B operand in registers: q4 codes
// dequantised once per step, fp16 rows loaded as they are.  Global loads run
// kPf steps ahead of the MFMAs through a ring of register stages (the loop is
// unrolled by kPf so every stage is a fixed set of registers).
// Split-K: blockIdx.z takes steps [z spc, (z + 1) spc); GEMM_PART writes each
// split's sum to its own slice Cf + z M ldc, the consumer adds the slices.
// MFMA 32x32x16 f16 lane layouts: A: lane l holds A[l % 32][8 (l / 32) + 0..7];
// B: B[8 (l / 32) + 0..7][l % 32]; D: register v of lane l holds
// D[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].
// Columns are physical weight rows: with NB = 2 a wave's two groups are the
// two halves of one 64-row tile, which for the paired gate|up layout are the
// gate rows 32t.. and the matching up rows, so GEMM_SWIGLU finishes in-lane.
constexpr int kPf = 4;  // steps in flight (the four stages of gemm_kernel)

template <int FMT, int MT, int NB>
struct GemmMain {
  static constexpr int LS = 40;  // LDS halves per A row (32 + 8: conflict-free 16-byte reads)
  float16_t acc[MT][NB];

  // one step: stage -> LDS buffer and B registers, refill the stage, barrier, MFMAs
  // returns the stage refilled with step `next` (values, not references: the
  // ring then stays in registers)
  __device__ __forceinline__ GemmStage<FMT, MT, NB> step(GemmStage<FMT, MT, NB> st,
                                                         const GemmPtrs<FMT, MT, NB>& p, _Float16* buf,
                                                         const int* adst, int next, bool refill, int arow,
                                                         int kh) {
    *reinterpret_cast<uint4*>(buf + adst[0]) = st.a0;
    if constexpr (MT > 1) *reinterpret_cast<uint4*>(buf + adst[1]) = st.a1;
    half8_t b[NB][2];
#pragma unroll
    for (int j = 0; j < NB; j++) st.operands(j, kh, b[j][0], b[j][1]);
    // the stage's registers are free once the operands are formed: keep the
    // refill after them so the loads land in the same registers (otherwise the
    // loop needs copies that wait for the loads)
    __builtin_amdgcn_sched_barrier(0);
    if (refill) st.load(p, next, kh);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MT; i++) {
      const _Float16* ar = buf + (arow + 32 * i) * LS + 8 * kh;
      const half8_t a1 = *reinterpret_cast<const half8_t*>(ar);
      const half8_t a2 = *reinterpret_cast<const half8_t*>(ar + 16);
#pragma unroll
      for (int j = 0; j < NB; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b[j][0], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b[j][1], acc[i][j], 0, 0, 0);
      }
    }
    return st;
  }
};

template <int FMT, int MT, int NB, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  using Main = GemmMain<FMT, MT, NB>;
  constexpr int BM = 64 * MT, LS = Main::LS;
  __shared__ __align__(16) _Float16 as[2][BM * LS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, kh = lane >> 5;
  const int m0 = blockIdx.y * BM;
  const int cg0 = (blockIdx.x * 2 + wn) * 32 * NB;
  const int c0 = blockIdx.z * g.spc, n = min(g.spc, g.K / 32 - c0);

  GemmPtrs<FMT, MT, NB> p;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int r = min(cg0 + 32 * j + l32, g.N - 1);  // clamped: loads stay unconditional
    const size_t base = (size_t)(r / kTile) * g.C * kTile + r % kTile;
    p.wp[j] = g.w + base;
    p.sp[j] = FMT == WF_Q4 ? g.s + base : g.s;
  }
  int adst[MT];
#pragma unroll
  for (int u = 0; u < MT; u++) {
    const int q = tid + 256 * u, r = q >> 2, piece = q & 3;
    p.asrc[u] = g.A + (size_t)min(m0 + r, g.M - 1) * g.lda + piece * 8;
    adst[u] = r * LS + piece * 8;
  }

  Main mm;
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) mm.acc[i][j] = (float16_t){};

  // four named stages (not an array: the ring must stay in registers)
  GemmStage<FMT, MT, NB> s0, s1, s2, s3;
  s0.load(p, c0, kh);
  s1.load(p, c0 + min(1, n - 1), kh);
  s2.load(p, c0 + min(2, n - 1), kh);
  s3.load(p, c0 + min(3, n - 1), kh);
  const int arow = wm * 32 * MT + l32;
  const int nfull = n - n % kPf;
  for (int cb = 0; cb < nfull; cb += kPf) {
    s0 = mm.step(s0, p, as[0], adst, c0 + min(cb + 4, n - 1), true, arow, kh);
    s1 = mm.step(s1, p, as[1], adst, c0 + min(cb + 5, n - 1), true, arow, kh);
    s2 = mm.step(s2, p, as[0], adst, c0 + min(cb + 6, n - 1), true, arow, kh);
    s3 = mm.step(s3, p, as[1], adst, c0 + min(cb + 7, n - 1), true, arow, kh);
  }
  // tail: stage u holds step nfull + u
  if (nfull < n) mm.step(s0, p, as[0], adst, 0, false, arow, kh);
  if (nfull + 1 < n) mm.step(s1, p, as[1], adst, 0, false, arow, kh);
  if (nfull + 2 < n) mm.step(s2, p, as[0], adst, 0, false, arow, kh);

  const int rbase = m0 + wm * 32 * MT + 4 * kh;
  if (EPI == GEMM_SWIGLU) {
    const int oi = (cg0 / kTile) * 32 + l32;  // canonical gate index of this lane's column
    if (oi >= g.n_out) return;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
        if (row < g.M) {
          const float gt = mm.acc[i][0][v], up = mm.acc[i][NB - 1][v];
          const _Float16 hv = f16_guard(g.ovf, silu_mul(gt, up));
          g.Ch[(size_t)row * g.ldc + oi] = __builtin_bit_cast(uint16_t, hv);
        }
      }
    return;
  }
  float* out = g.Cf + (EPI == GEMM_PART ? (size_t)blockIdx.z * g.M * g.ldc : 0);
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int col = cg0 + 32 * j + l32;
    if (col >= g.N) continue;
    const float bias = (EPI == GEMM_STORE && g.bias) ? g.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = rbase + 32 * i + 8 * (v >> 2) + (v & 3);
        if (row < g.M) out[(size_t)row * g.ldc + col] = mm.acc[i][j][v] + bias;
      }
  }
}

// ------------------------------------------------------- q4 GEMM, LDS ring --
// The q4 GEMM with its operands streamed by direct global -> LDS loads
// (global_load_lds: no registers held while the loads are in flight).
// Block: 4 waves side by side over 256 columns (four 64-row weight tiles); a
// wave owns all 32 MT rows x its 64 columns (MT x 2 MFMA tiles of 32 x 32).
// Per 32-k step a stage of the LDS ring holds the block's A rows [32 MT][32]
// (16-byte pieces at a swizzled slot, see a_slot), the 256 weight chunks and
// their scales.  kRing stages: a step's loads are issued kRing - 1 steps
// before its MFMAs; every wave issues the same number of loads per stage
// (small blocks repeat a copy of identical bytes), so one immediate vmcnt
// bounds the loads still in flight.  Columns: for the paired gate|up layout
// a wave's two 32-column groups are the gate rows and the matching up rows.
// The depth is even: the operands of consecutive steps alternate between two
// register sets (a 6-stage ring measured slower).
constexpr int kRing = 4;
static_assert(kRing % 2 == 0, "even ring depth");

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding (n < 64) and leaves the other counters alone: vmcnt bits 3:0 in
// simm16 bits 3:0 and bits 5:4 in simm16 bits 15:14 (gfx9 encoding).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) & 3) << 14 | 0x70 | 0xF00; }
// the same with lgkmcnt(0): this wave's LDS reads are complete as well
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) & 3) << 14 | 0x70; }

// Slot (16 bytes) of piece q of A row r in a stage: piece q ^ f(r), where
// f(r) = ((r1 ^ r3), r2) makes the 16-byte reads of 8 consecutive rows (32
// banks) and of 16 consecutive rows (64 banks) hit distinct banks.
__device__ __forceinline__ int a_swz(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1); }
__device__ __forceinline__ int a_slot(int r, int q) { return r * 4 + (q ^ a_swz(r)); }

// lane-wise global -> LDS copies; `lds` is the wave's destination base (a
// byte address in the workgroup's LDS, the same for every lane), lane l
// writes lds + l * size.  Issued from asm so the compiler keeps no count of
// them: the kernel waits for them itself (vmcnt) before its barrier.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory", "m0");
}

template <int MT, int WN>
struct RingLayout {
  static constexpr int BM = 32 * MT;
  static constexpr int NA = 2 * MT;             // 1 KiB A copies per stage
  static constexpr int AW = (NA + WN - 1) / WN; // A copies per wave
  static constexpr int S_BYTES = WN * 128 > 256 ? WN * 128 : 256;
  static constexpr int W_OFF = BM * 64, S_OFF = W_OFF + WN * 1024, STAGE = S_OFF + S_BYTES;
  static constexpr int LPS = AW + 2;            // copies per wave per stage: A, one weight tile, scales
  static constexpr int NR = kRing;
  static_assert((NR - 1) * LPS <= 63, "copies in flight within vmcnt's range");
};

// One block's state: loop-invariant byte offsets of its copies and reads, the
// accumulators, and the step body with the stage index a template constant
// (LDS addresses become immediates).  k order inside a 32-k step: MFMA 1
// takes k = 16 kh + 0..7, MFMA 2 k = 16 kh + 8..15 (kh = lane / 32), so a
// lane's A pieces are 2 kh, 2 kh + 1 and its weight dwords 2 kh, 2 kh + 1
// (one 8-byte read).
template <int MT, int WN>
struct RingBlock {
  using RL = RingLayout<MT, WN>;
  const char* abase;  // A + 32 c halves, weight and scale bases advance per step
  const char* wbase;
  const char* sbase;
  int a_lds_stride;   // bytes per 32-k step in each operand
  uint32_t agoff[RL::AW], alds[RL::AW];  // global byte offsets / LDS offsets of this wave's A copies
  uint32_t wgoff, sgoff, wlds, slds;
  uint32_t lbase;
  int rd_a1[MT], rd_a2[MT];              // LDS read offsets of the A pieces (within a stage)
  int rd_w[2], rd_s[2];
  float16_t acc[MT][2];

  __device__ __forceinline__ void issue(int stage, int c) {
    const uint32_t sb = lbase + stage * RL::STAGE;
    const char* ab = abase + (size_t)c * 64;
    const char* wb = wbase + (size_t)c * kTile * 16;
    const char* sbs = sbase + (size_t)c * kTile * 2;
#pragma unroll
    for (int u = 0; u < RL::AW; u++) lds_dma16(ab, agoff[u], __builtin_amdgcn_readfirstlane(sb + alds[u]));
    lds_dma16(wb, wgoff, __builtin_amdgcn_readfirstlane(sb + wlds));
    lds_dma4(sbs, sgoff, __builtin_amdgcn_readfirstlane(sb + slds));
  }

  // One step's MFMA operands: the A pieces as read from LDS and the weights
  // of the lane's two 32-column groups dequantised to fp16.
  struct Ops {
    half8_t a1[MT], a2[MT];
    half8_t b[2][2];
  };

  template <int S>
  __device__ __forceinline__ void read_w(const unsigned char* lds, uint2 (&w)[2], _Float16 (&sc)[2]) const {
    const unsigned char* sb = lds + S * RL::STAGE;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      w[j] = *reinterpret_cast<const uint2*>(sb + rd_w[j]);
      sc[j] = *reinterpret_cast<const _Float16*>(sb + rd_s[j]);
    }
  }
  template <int S>
  __device__ __forceinline__ void read_a(const unsigned char* lds, Ops& o) const {
    const unsigned char* sb = lds + S * RL::STAGE;
#pragma unroll
    for (int t = 0; t < MT; t++) {
      o.a1[t] = *reinterpret_cast<const half8_t*>(sb + rd_a1[t]);
      o.a2[t] = *reinterpret_cast<const half8_t*>(sb + rd_a2[t]);
    }
  }
  static __device__ __forceinline__ void dequant(const uint2 (&w)[2], const _Float16 (&sc)[2], Ops& o) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const half2_t s2 = {sc[j], sc[j]};
      o.b[j][0] = dequant8(w[j].x, s2);
      o.b[j][1] = dequant8(w[j].y, s2);
    }
  }
  template <int S>
  __device__ __forceinline__ void read(const unsigned char* lds, Ops& o) const {
    uint2 w[2];
    _Float16 sc[2];
    read_w<S>(lds, w, sc);
    read_a<S>(lds, o);
    dequant(w, sc, o);
  }

  // Step i in stage S; `cur` holds its operands, read and dequantised during
  // step i - 1.  Wait until this wave's copies of step i + 1 have landed (at
  // most NR - 3 later stages in flight) and its LDS reads are complete; after
  // the barrier every wave's copies of step i + 1 have landed and every
  // wave's reads of stage i - 1 (made in step i - 2) are complete.  Then read
  // step i + 1, refill stage i - 1 with step i + NR - 1, and run step i's
  // MFMAs with the dequantisation of step i + 1 in their shadow (both waves
  // of a SIMD pass the barrier together, so VALU work left outside the MFMAs
  // would serialise with them).
  template <int S>
  __device__ __forceinline__ void step(const unsigned char* lds, int refill_c, const Ops& cur, Ops& nxt) {
    constexpr int NR = RL::NR;
    __builtin_amdgcn_sched_barrier(0);  // the previous step's MFMAs stay before this barrier
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0((NR - 3) * RL::LPS));
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // keep each step's MFMAs after its own barrier
    uint2 w[2];
    _Float16 sc[2];
    read_w<(S + 1) % NR>(lds, w, sc);
    read_a<(S + 1) % NR>(lds, nxt);
    issue((S + NR - 1) % NR, refill_c);
    __builtin_amdgcn_sched_barrier(0);  // the reads and copies go out before the MFMAs
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.a1[t], cur.b[j][0], acc[t][j], 0, 0, 0);
        acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.a2[t], cur.b[j][1], acc[t][j], 0, 0, 0);
      }
    dequant(w, sc, nxt);
    // order: a few MFMAs while the weight reads land, then one MFMA per
    // slice of the dequantisation
    __builtin_amdgcn_sched_group_barrier(0x008, MT, 0);
#define RING_MV __builtin_amdgcn_sched_group_barrier(0x002, 8, 0); __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    RING_MV RING_MV RING_MV RING_MV RING_MV RING_MV RING_MV RING_MV RING_MV RING_MV
#undef RING_MV
  }
};

// Steps S..E-1 of one pass over the ring, each with its stage a constant:
// full() refills each stage with the step NR - 1 ahead, tail() runs the steps
// left after the last full pass (their stages already hold them).  Even steps
// take their operands from o0 and read the next step's into o1, odd steps
// the other way round.
template <int MT, int WN, int S, int E>
struct RingSteps {
  using RB = RingBlock<MT, WN>;
  using Ops = typename RB::Ops;
  static __device__ __forceinline__ void full(RB& rb, const unsigned char* lds, int i, int n, Ops& o0, Ops& o1) {
    const int c = min(i + S + RingLayout<MT, WN>::NR - 1, n - 1);
    if constexpr (S % 2 == 0) rb.template step<S>(lds, c, o0, o1);
    else rb.template step<S>(lds, c, o1, o0);
    RingSteps<MT, WN, S + 1, E>::full(rb, lds, i, n, o0, o1);
  }
  static __device__ __forceinline__ void tail(RB& rb, const unsigned char* lds, int i, int n, Ops& o0, Ops& o1) {
    if (i + S < n) {
      if constexpr (S % 2 == 0) rb.template step<S>(lds, n - 1, o0, o1);
      else rb.template step<S>(lds, n - 1, o1, o0);
    }
    RingSteps<MT, WN, S + 1, E>::tail(rb, lds, i, n, o0, o1);
  }
};
template <int MT, int WN, int E>
struct RingSteps<MT, WN, E, E> {
  using Ops = typename RingBlock<MT, WN>::Ops;
  static __device__ __forceinline__ void full(RingBlock<MT, WN>&, const unsigned char*, int, int, Ops&, Ops&) {}
  static __device__ __forceinline__ void tail(RingBlock<MT, WN>&, const unsigned char*, int, int, Ops&, Ops&) {}
};

template <int MT, int WN, int EPI>
__global__ __launch_bounds__(64 * WN) __attribute__((amdgpu_waves_per_eu(2))) void gemm_q4_ring_kernel(GemmArgs g) {
  using RL = RingLayout<MT, WN>;
  constexpr int NR = RL::NR;
  __shared__ __align__(16) unsigned char lds[NR * RL::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, kh = lane >> 5;
  const int m0 = blockIdx.y * RL::BM, t0 = blockIdx.x * WN, T = (g.N + kTile - 1) / kTile;
  const int c0 = blockIdx.z * g.spc, n = min(g.spc, g.K / 32 - c0);

  RingBlock<MT, WN> rb;
  rb.lbase = (uint32_t)(uintptr_t)lds;
  rb.abase = reinterpret_cast<const char*>(g.A) + (size_t)c0 * 64;
  rb.wbase = reinterpret_cast<const char*>(g.w) + (size_t)c0 * kTile * 16;
  rb.sbase = reinterpret_cast<const char*>(g.s) + (size_t)c0 * kTile * 2;
#pragma unroll
  for (int u = 0; u < RL::AW; u++) {
    const int ai = (wave * RL::AW + u) % RL::NA, sl = ai * 64 + lane, r = sl >> 2;
    rb.agoff[u] = (uint32_t)(((size_t)min(m0 + r, g.M - 1) * g.lda + 8 * ((sl & 3) ^ a_swz(r))) * 2);
    rb.alds[u] = ai * 1024;
  }
  rb.wgoff = (uint32_t)(((size_t)min(t0 + wave, T - 1) * g.C * kTile + lane) * 16);
  const int sidx = WN >= 4 ? wave % (WN / 2) : 0;  // one scale copy covers two tiles
  rb.sgoff = (uint32_t)(((size_t)min(t0 + 2 * sidx + (lane >> 5), T - 1) * g.C * kTile + 2 * (lane & 31)) * 2);
  rb.wlds = RL::W_OFF + wave * 1024;
  rb.slds = RL::S_OFF + sidx * 256;
#pragma unroll
  for (int t = 0; t < MT; t++) {
    const int r = 32 * t + l32;
    rb.rd_a1[t] = a_slot(r, 2 * kh) * 16;
    rb.rd_a2[t] = a_slot(r, 2 * kh + 1) * 16;
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int cc = wave * 64 + 32 * j + l32;
    rb.rd_w[j] = RL::W_OFF + cc * 16 + 8 * kh;
    rb.rd_s[j] = RL::S_OFF + cc * 2;
  }
#pragma unroll
  for (int i = 0; i < MT; i++) rb.acc[i][0] = rb.acc[i][1] = (float16_t){};

  // steps are relative to c0 from here on
#pragma unroll
  for (int st = 0; st < NR - 1; st++) rb.issue(st, min(st, n - 1));
  typename RingBlock<MT, WN>::Ops o0, o1;
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((NR - 2) * RL::LPS));  // step 0 has landed (this wave's copies)
  asm volatile("s_barrier" ::: "memory");                        // ... and every wave's
  rb.template read<0>(lds, o0);
  int i = 0;
  for (; i + NR <= n; i += NR) RingSteps<MT, WN, 0, NR>::full(rb, lds, i, n, o0, o1);
  RingSteps<MT, WN, 0, NR - 1>::tail(rb, lds, i, n, o0, o1);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // the clamped trailing copies land before the block exits

  const int cg0 = (t0 + wave) * kTile;
  const int rbase = m0 + 4 * kh;
  if (EPI == GEMM_SWIGLU) {
    const int oi = (t0 + wave) * 32 + l32;
    if (oi >= g.n_out) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = rbase + 32 * t + 8 * (v >> 2) + (v & 3);
        if (row < g.M) {
          const float gt = rb.acc[t][0][v], up = rb.acc[t][1][v];
          const _Float16 hv = f16_guard(g.ovf, silu_mul(gt, up));
          g.Ch[(size_t)row * g.ldc + oi] = __builtin_bit_cast(uint16_t, hv);
        }
      }
    return;
  }
  float* out = g.Cf + (EPI == GEMM_PART ? (size_t)blockIdx.z * g.M * g.ldc : 0);
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = cg0 + 32 * j + l32;
    if (col >= g.N) continue;
    const float bias = (EPI == GEMM_STORE && g.bias) ? g.bias[col] : 0.f;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = rbase + 32 * t + 8 * (v >> 2) + (v & 3);
        if (row < g.M) out[(size_t)row * g.ldc + col] = rb.acc[t][j][v] + bias;
      }
  }
}

// ------------------------------------------------ q4 GEMM, waves split K --
// For grids too small to fill the CUs (short prompts): a block's 4 waves take
// the same 64 columns and 32 MT rows and split the block's K range in four.
// Each wave streams its own operands through a private LDS ring (global ->
// LDS copies as above, no block barrier in the loop); at the end waves 1..3
// hand their accumulators to wave 0 through LDS, which adds them in wave
// order (deterministic) and runs the epilogue.  Same epilogues as above.
__device__ __forceinline__ float f4_at(const float4& v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

template <int MT>
struct KwLayout {
  static constexpr int NR = 4;                           // ring stages per wave
  static constexpr int NA = 2 * MT;                      // 1 KiB A copies per stage
  static constexpr int W_OFF = MT * 2048, S_OFF = W_OFF + 1024, STAGE = S_OFF + 256;
  static constexpr int WAVE_BYTES = NR * STAGE;          // one wave's ring
  static constexpr int LPS = NA + 2;                     // copies per stage
  static constexpr int ACC_FLOATS = MT * 2 * 16 * 64;    // one wave's accumulators
  static_assert(4 * ACC_FLOATS * 4 <= 4 * WAVE_BYTES, "accumulator handoff fits in the rings");
  static_assert((NR - 1) * LPS <= 63, "copies in flight within vmcnt's range");
};

template <int MT>
struct KwWave {
  using KL = KwLayout<MT>;
  const char* abase;
  const char* wbase;
  const char* sbase;
  uint32_t agoff[KL::NA];
  uint32_t wgoff, sgoff, lbase;
  int rd_a1[MT], rd_a2[MT], rd_w[2], rd_s[2];
  float16_t acc[MT][2];

  __device__ __forceinline__ void issue(int stage, int c) {
    const uint32_t sb = lbase + stage * KL::STAGE;
    const char* ab = abase + (size_t)c * 64;
#pragma unroll
    for (int u = 0; u < KL::NA; u++) lds_dma16(ab, agoff[u], __builtin_amdgcn_readfirstlane(sb + u * 1024));
    lds_dma16(wbase + (size_t)c * kTile * 16, wgoff, __builtin_amdgcn_readfirstlane(sb + KL::W_OFF));
    lds_dma4(sbase + (size_t)c * kTile * 2, sgoff, __builtin_amdgcn_readfirstlane(sb + KL::S_OFF));
  }

  template <int S>
  __device__ __forceinline__ void step(const unsigned char* mine, int refill_c) {
    // this wave's copies of the step have landed when at most NR - 2 later
    // stages are in flight; the stage refilled below was last read by this
    // wave in its previous step, and those LDS reads must be complete before
    // the copies may overwrite it: the scheduler leaves the last of them
    // (an A operand) in flight past this point, so wait for lgkmcnt(0) too
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0((KL::NR - 2) * KL::LPS));
    asm volatile("" ::: "memory");
    issue((S + KL::NR - 1) % KL::NR, refill_c);
    const unsigned char* sb = mine + S * KL::STAGE;
    half8_t b[2][2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint2 wv = *reinterpret_cast<const uint2*>(sb + rd_w[j]);
      const _Float16 sc = *reinterpret_cast<const _Float16*>(sb + rd_s[j]);
      const half2_t s2 = {sc, sc};
      b[j][0] = dequant8(wv.x, s2);
      b[j][1] = dequant8(wv.y, s2);
    }
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const half8_t a1 = *reinterpret_cast<const half8_t*>(sb + rd_a1[t]);
      const half8_t a2 = *reinterpret_cast<const half8_t*>(sb + rd_a2[t]);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b[j][0], acc[t][j], 0, 0, 0);
        acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b[j][1], acc[t][j], 0, 0, 0);
      }
    }
  }
};

template <int MT, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_q4_kw_kernel(GemmArgs g) {
  using KL = KwLayout<MT>;
  __shared__ __align__(16) unsigned char lds[4 * KL::WAVE_BYTES];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, kh = lane >> 5;
  const int m0 = blockIdx.y * 32 * MT, t0 = blockIdx.x, T = (g.N + kTile - 1) / kTile;
  const int cb = blockIdx.z * g.spc, nb = min(g.spc, g.K / 32 - cb);
  const int q = (nb + 3) / 4, c0 = cb + wave * q, n = max(0, min(q, nb - wave * q));
  const unsigned char* mine = lds + wave * KL::WAVE_BYTES;

  KwWave<MT> kw;
  kw.lbase = (uint32_t)(uintptr_t)mine;
  kw.abase = reinterpret_cast<const char*>(g.A) + (size_t)c0 * 64;
  kw.wbase = reinterpret_cast<const char*>(g.w) + (size_t)c0 * kTile * 16;
  kw.sbase = reinterpret_cast<const char*>(g.s) + (size_t)c0 * kTile * 2;
#pragma unroll
  for (int u = 0; u < KL::NA; u++) {
    const int sl = u * 64 + lane, r = sl >> 2;
    kw.agoff[u] = (uint32_t)(((size_t)min(m0 + r, g.M - 1) * g.lda + 8 * ((sl & 3) ^ a_swz(r))) * 2);
  }
  kw.wgoff = (uint32_t)(((size_t)min(t0, T - 1) * g.C * kTile + lane) * 16);
  kw.sgoff = (uint32_t)(((size_t)min(t0 + (lane >> 5), T - 1) * g.C * kTile + 2 * (lane & 31)) * 2);
#pragma unroll
  for (int t = 0; t < MT; t++) {
    kw.rd_a1[t] = a_slot(32 * t + l32, 2 * kh) * 16;
    kw.rd_a2[t] = a_slot(32 * t + l32, 2 * kh + 1) * 16;
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    kw.rd_w[j] = KL::W_OFF + (32 * j + l32) * 16 + 8 * kh;
    kw.rd_s[j] = KL::S_OFF + (32 * j + l32) * 2;
  }
#pragma unroll
  for (int i = 0; i < MT; i++) kw.acc[i][0] = kw.acc[i][1] = (float16_t){};
  // the epilogue's per-row inputs (GEMM_FOLD: residual values, exponents and
  // norm weights; GEMM_SWIGLU after a GEMM_FOLD: exponents and tile sums),
  // requested before the K loop, whose waits then cover them.  Lane (l32, kh)
  // of wave w ends with rows m0 + 32 t + 8 w + 4 kh + e, columns 32 j + l32.
  const int rbase = m0 + 4 * kh + 8 * wave;
  const bool post_norm = EPI == GEMM_SWIGLU && g.ss != nullptr;
  float xv[MT][2][4], nwv[2], ssv[MT][4];
  int exv[MT][4];
  if (EPI == GEMM_FOLD) {
#pragma unroll
    for (int j = 0; j < 2; j++) nwv[j] = g.nw[t0 * kTile + 32 * j + l32];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = min(rbase + 32 * t + e, g.M - 1);
        exv[t][e] = g.ex[row];
#pragma unroll
        for (int j = 0; j < 2; j++) xv[t][j][e] = g.Cf[(size_t)row * g.ldc + t0 * kTile + 32 * j + l32];
      }
  }
  if (post_norm) {
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = min(rbase + 32 * t + e, g.M - 1);
        exv[t][e] = g.ex[row];
        ssv[t][e] = l32 < g.ss_ld ? g.ss[(size_t)row * g.ss_ld + l32] : 0.f;
      }
  }
  if (n > 0) {  // steps relative to c0
    kw.issue(0, 0);
    kw.issue(1, min(1, n - 1));
    kw.issue(2, min(2, n - 1));
    int i = 0;
    for (; i + 4 <= n; i += 4) {
      kw.template step<0>(mine, min(i + 3, n - 1));
      kw.template step<1>(mine, min(i + 4, n - 1));
      kw.template step<2>(mine, min(i + 5, n - 1));
      kw.template step<3>(mine, min(i + 6, n - 1));
    }
    if (i < n) kw.template step<0>(mine, n - 1);
    if (i + 1 < n) kw.template step<1>(mine, n - 1);
    if (i + 2 < n) kw.template step<2>(mine, n - 1);
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // every copy of this wave has landed
  __syncthreads();                           // every wave is done with its ring
  // Handoff: every wave puts its accumulators in LDS; wave w then owns
  // registers 4w..4w+3 of every tile (rows 8w..8w+7 of each 32-row band),
  // adds the four waves' values in wave order and runs the epilogue for them.
  float4* xch = reinterpret_cast<float4*>(lds);
  constexpr int Q = MT * 2 * 4;  // float4 per lane per wave
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int q = 0; q < 4; q++)
        xch[(wave * Q + (t * 2 + j) * 4 + q) * 64 + lane] =
            make_float4(kw.acc[t][j][4 * q], kw.acc[t][j][4 * q + 1], kw.acc[t][j][4 * q + 2], kw.acc[t][j][4 * q + 3]);
  __syncthreads();
  float4 r[MT][2];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      float4 v = xch[((t * 2 + j) * 4 + wave) * 64 + lane];
#pragma unroll
      for (int w = 1; w < 4; w++) {
        const float4 u = xch[(w * Q + (t * 2 + j) * 4 + wave) * 64 + lane];
        v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
      }
      r[t][j] = v;
    }

  if (EPI == GEMM_FOLD) {
    // x = residual + this tile's sum (one block per element: no split-K);
    // the norm's operand fp16(x w 2^ex) and the tile's sum of squares per row
    // (lanes l32 of a half-wave hold the row's 64 columns: half_sum)
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = rbase + 32 * t + e;
        float sq = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const float x = xv[t][j][e] + f4_at(r[t][j], e);
          sq = fmaf(x, x, sq);
          if (row < g.M) {
            const size_t at = (size_t)row * g.ldc + t0 * kTile + 32 * j + l32;
            g.Cf[at] = x;
            g.Ch[at] = __builtin_bit_cast(uint16_t, f16_guard(g.ovf, ldexpf(x * nwv[j], exv[t][e])));
          }
        }
        sq = half_sum(sq);
        if (l32 == 0 && row < g.M) g.ss[(size_t)row * g.ss_ld + t0] = sq;
      }
    return;
  }
  if (EPI == GEMM_ROPE) {
    // tile t0 is one head of 64: q heads, then k, then v.  Lane l32 holds dims
    // d = l32 and d + 32 of its rows, the rotate-half pair of RoPE
    // (TSLAttention.ts:168-250 for one row; the rope_kv kernel's arithmetic)
    const int d = l32, kind = t0 < g.Hq ? 0 : t0 < g.Hq + g.Hkv ? 1 : 2;
    const int p0 = g.ctrl ? g.ctrl[C_POS] : g.p0;
    const int hk = kind == 1 ? t0 - g.Hq : t0 - g.Hq - g.Hkv;
    const float b0 = g.bias ? g.bias[t0 * kTile + d] : 0.f, b1 = g.bias ? g.bias[t0 * kTile + d + 32] : 0.f;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = rbase + 32 * t + e;
        if (row >= g.M) continue;
        const int pos = p0 + row;
        const float x0 = f4_at(r[t][0], e) + b0, x1 = f4_at(r[t][1], e) + b1;
        float y0 = x0, y1 = x1;
        if (kind < 2) {
          const float c = g.rope_cos[(size_t)pos * 32 + d], sn = g.rope_sin[(size_t)pos * 32 + d];
          y0 = x0 * c - x1 * sn;
          y1 = x1 * c + x0 * sn;
        }
        if (kind == 0) {
          uint16_t* qr = g.Ch + (size_t)row * g.ldc + t0 * kTile;
          qr[d] = __builtin_bit_cast(uint16_t, f16_guard(g.ovf, y0));
          qr[d + 32] = __builtin_bit_cast(uint16_t, f16_guard(g.ovf, y1));
        } else {
          uint16_t* cr = (kind == 1 ? g.kc : g.vc) + ((size_t)hk * g.max_tokens + pos) * kTile;
          cr[d] = __builtin_bit_cast(uint16_t, f16_guard(g.ovf, y0));
          cr[d + 32] = __builtin_bit_cast(uint16_t, f16_guard(g.ovf, y1));
        }
      }
    return;
  }
  if (EPI == GEMM_SWIGLU) {
    // after a GEMM_FOLD the RMSNorm scale of each row comes here: the sum of
    // its tile sums (a butterfly over the half-wave, every lane the same bits)
    float sc[MT][4];
    const float inv_n = 1.f / (float)g.n_norm;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        sc[t][e] = post_norm ? ldexpf(rsqrtf(half_sum(ssv[t][e]) * inv_n + g.eps), -exv[t][e]) : 1.f;
    const int oi = t0 * 32 + l32;
    if (oi >= g.n_out) return;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = rbase + 32 * t + e;
        if (row < g.M) {
          const float gt = f4_at(r[t][0], e) * sc[t][e], up = f4_at(r[t][1], e) * sc[t][e];
          const _Float16 hv = f16_guard(g.ovf, silu_mul(gt, up));
          g.Ch[(size_t)row * g.ldc + oi] = __builtin_bit_cast(uint16_t, hv);
        }
      }
    return;
  }
  float* out = g.Cf + (EPI == GEMM_PART ? (size_t)blockIdx.z * g.M * g.ldc : 0);
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = t0 * kTile + 32 * j + l32;
    if (col >= g.N) continue;
    const float bias = (EPI == GEMM_STORE && g.bias) ? g.bias[col] : 0.f;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int row = rbase + 32 * t + e;
        if (row < g.M) out[(size_t)row * g.ldc + col] = f4_at(r[t][j], e) + bias;
      }
  }
}

// TLM_GEMM_RING=0 selects the register-prefetch kernel for q4 too (comparisons)
static const bool g_use_ring = [] {
  const char* e = getenv("TLM_GEMM_RING");
  return !(e && e[0] == '0');
}();
// TLM_GEMM_SPLIT_WAVES=n: split K while the grid holds at most n waves per CU
// (default 4: with 32-row K-wave tiles, 4 beat 8 by 2-7 % from 127 to 1100
// rows; every split adds an M x N fp32 slice that the consuming row kernel folds)
static const int g_split_waves = [] {
  const char* e = getenv("TLM_GEMM_SPLIT_WAVES");
  const int v = e ? atoi(e) : 0;
  return v > 0 && v <= 64 ? v : 4;
}();

GemmShape gemm_shape(int fmt, int epi, int M, int N, int K, int cus) {
  GemmShape s;
  s.ring = fmt == WF_Q4 && g_use_ring;
  s.wn = 1;
  s.kw = 0;
  const int steps = K >= 32 ? K / 32 : 1;  // K % 32 != 0 is rejected by launch_gemm
  int min_steps = 4;                       // 32-k steps per wave, at least
  int kdiv = 1;                            // waves sharing one block's K range
  if (s.ring) {
    s.mt = M > 64 ? 4 : M > 32 ? 2 : 1;
    s.nb = 2;
    s.gy = (M + 32 * s.mt - 1) / (32 * s.mt);
    if (((N + 255) / 256) * s.gy >= cus / 2) {  // four waves side by side over 256 columns
      s.wn = 4;
      s.gx = (N + 255) / 256;
    } else {  // too few tiles to fill the CUs: four waves split K on one tile
      // of 32 rows: 4x the blocks of 128-row tiles, and three blocks fit a CU
      // (53 KB of LDS against 151 KB), which the re-read weight tiles (L2 hits)
      // more than pay for (measured 5-25 % faster from 64 to 1100 rows)
      s.kw = 1;
      s.mt = 1;
      s.gy = (M + 31) / 32;
      s.gx = (N + kTile - 1) / kTile;
      kdiv = 4;
      min_steps = 2;
    }
  } else {
    s.mt = M > 64 ? 2 : 1;
    s.nb = (epi == GEMM_SWIGLU || N > 64) ? 2 : 1;
    s.gx = (N + 64 * s.nb - 1) / (64 * s.nb);
    s.gy = (M + 64 * s.mt - 1) / (64 * s.mt);
    s.wn = 4;
  }
  int splits = 1;
  if (epi == GEMM_PART && s.ring && !s.kw) {
    // four-wave ring blocks, two per CU: pick the split count with the least
    // (rounds of blocks x steps per block) + the split slices' write and read
    // (M N 8 bytes each at ~6 TB/s, in units of a ~1 us step), the latter
    // weighted 2x: the slice stores compete with the GEMM's own operand reads
    // (measured 1-2 % faster 2048-row chunks than at weight 1, none slower)
    const double slice_steps = 2.0 * (double)M * N * 8.0 / 6e6;
    double best = 1e30;
    for (int sp = 1; sp <= 32 && steps / sp >= min_steps; sp *= 2) {
      const int rounds = (s.gx * s.gy * sp + 2 * cus - 1) / (2 * cus);
      const double cost = (double)rounds * ((steps + sp - 1) / sp) + sp * slice_steps;
      if (cost < best) best = cost, splits = sp;
    }
  } else if (epi == GEMM_PART) {
    // split K while the grid stays within about g_split_waves waves per CU:
    // past one round of blocks a CU streams the same bytes either way and each
    // split only adds a slice for the next row kernel to fold (Qwen2.5-0.5B
    // shape, 64 to 300 rows: the down GEMM in 4 splits instead of 8, the chunk
    // 3-6 % faster; TLM_GEMM_SPLIT_FLOOR=0 splits until the grid reaches that
    // size instead)
    const int target = g_split_waves * cus;
    const int waves = s.gx * s.gy * (s.ring ? (s.kw ? 4 : s.wn) : 4);
    static const bool floor_rule = [] { const char* e = getenv("TLM_GEMM_SPLIT_FLOOR"); return !(e && e[0] == '0'); }();
    if (floor_rule)
      while (splits < 32 && waves * splits * 2 <= target && steps / (2 * splits * kdiv) >= min_steps) splits *= 2;
    else
      while (splits < 32 && waves * splits < target && steps / (2 * splits * kdiv) >= min_steps) splits *= 2;
  }
  s.spc = (steps + splits - 1) / splits;
  s.splits = (steps + s.spc - 1) / s.spc;
  return s;
}

bool launch_gemm(int fmt, int epi, const GemmShape& sh, const GemmArgs& ga, hipStream_t st) {
  if (ga.K % 32 != 0 || ga.lda % 8 != 0 || ga.M <= 0 || ga.N <= 0) return false;
  if (epi == GEMM_SWIGLU && (ga.N % kTile != 0 || sh.nb != 2)) return false;
  if (epi != GEMM_PART && sh.splits != 1) return false;
  if (epi == GEMM_ROPE && !(sh.ring && sh.kw && ga.N % kTile == 0)) return false;  // the K-wave kernel only
  if (epi == GEMM_FOLD && !(sh.ring && sh.kw && ga.N % kTile == 0 && ga.N / kTile <= ga.ss_ld)) return false;
  if (epi == GEMM_SWIGLU && ga.ss && !(sh.ring && sh.kw && ga.ss_ld <= 32)) return false;
  GemmArgs g = ga;
  g.spc = sh.spc;
  const dim3 grid(sh.gx, sh.gy, sh.splits);
  const int mt = sh.mt, nb = sh.nb;
  if (sh.ring && sh.kw) {
    if (fmt != WF_Q4) return false;
#define KW_CASE(MTV, E)                                                                          \
  if (mt == MTV && epi == E) {                                                                   \
    hipLaunchKernelGGL((gemm_q4_kw_kernel<MTV, E>), grid, dim3(256), 0, st, g);                  \
    return true;                                                                                 \
  }
#define KW_EPIS(MTV) KW_CASE(MTV, GEMM_STORE) KW_CASE(MTV, GEMM_PART) KW_CASE(MTV, GEMM_SWIGLU) KW_CASE(MTV, GEMM_ROPE) \
  KW_CASE(MTV, GEMM_FOLD)
    KW_EPIS(1)  // gemm_shape gives the K-wave blocks 32 rows
#undef KW_EPIS
#undef KW_CASE
    return false;
  }
  if (sh.ring) {
    if (fmt != WF_Q4) return false;
#define RING_CASE(MTV, WNV, E)                                                                   \
  if (mt == MTV && sh.wn == WNV && epi == E) {                                                   \
    hipLaunchKernelGGL((gemm_q4_ring_kernel<MTV, WNV, E>), grid, dim3(64 * WNV), 0, st, g);      \
    return true;                                                                                 \
  }
#define RING_EPIS(MTV, WNV) RING_CASE(MTV, WNV, GEMM_STORE) RING_CASE(MTV, WNV, GEMM_PART) RING_CASE(MTV, WNV, GEMM_SWIGLU)
    RING_EPIS(1, 4) RING_EPIS(2, 4) RING_EPIS(4, 4)
#undef RING_EPIS
#undef RING_CASE
    return false;
  }
#define GEMM_CASE(F, MTV, NBV, E)                                                         \
  if (fmt == F && mt == MTV && nb == NBV && epi == E) {                                   \
    hipLaunchKernelGGL((gemm_kernel<F, MTV, NBV, E>), grid, dim3(256), 0, st, g);         \
    return true;                                                                          \
  }
#define GEMM_EPIS(F, MTV, NBV) \
  GEMM_CASE(F, MTV, NBV, GEMM_STORE) GEMM_CASE(F, MTV, NBV, GEMM_PART) GEMM_CASE(F, MTV, NBV, GEMM_SWIGLU)
  GEMM_EPIS(WF_Q4, 1, 1) GEMM_EPIS(WF_Q4, 1, 2) GEMM_EPIS(WF_Q4, 2, 1) GEMM_EPIS(WF_Q4, 2, 2)
  GEMM_EPIS(WF_F16, 1, 1) GEMM_EPIS(WF_F16, 1, 2) GEMM_EPIS(WF_F16, 2, 1) GEMM_EPIS(WF_F16, 2, 2)
#undef GEMM_EPIS
#undef GEMM_CASE
  return false;
}

// ------------------------------------------------------------ row kernels --

// Residual fold + RMSNorm per row (TSLRMSNorm.ts:18-81): x = X[m] + sum of
// the split-K slices part[s][m] (written back to X when there are any), or
// (emb non-null, layer 0) the embedding row of the row's token in fp32, stored
// to X (DecoderWeights.ts:355-383 stages the same rows for the replayed decode
// graph); then Y[m] = fp16(x * rsqrt(mean(x^2) + eps) * w) unless Y is null.
// H % 4 == 0, H <= 4096: each of the 256 threads holds up to four float4 of the row.
constexpr int kRowVec = 4;
__global__ __launch_bounds__(256) void rms_rows_kernel(RowsArgs a) {
  __shared__ float scratch[4];
  const int m = blockIdx.x, H4 = a.H >> 2;
  float4* x = reinterpret_cast<float4*>(a.X + (size_t)m * a.H);
  const float4* part = reinterpret_cast<const float4*>(a.part + (size_t)m * a.H);
  const size_t ps4 = a.pstride >> 2;
  float4 xs[kRowVec];
  float ss = 0.f;
  size_t erow = 0;  // the embedding row's first element
  if (a.emb) erow = (size_t)a.tokens[(a.ctrl ? a.ctrl[C_POS] - a.ctrl[C_BASE] : 0) + m] * a.H;
#pragma unroll
  for (int j = 0; j < kRowVec; j++) {
    const int k = threadIdx.x + 256 * j;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < H4 && a.emb) {
      if (a.emb_f32) {
        v = reinterpret_cast<const float4*>(static_cast<const float*>(a.emb) + erow)[k];
      } else {
        const half4_t h = reinterpret_cast<const half4_t*>(static_cast<const _Float16*>(a.emb) + erow)[k];
        v = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
      }
      x[k] = v;
    } else if (k < H4) {
      v = x[k];
#pragma unroll 4
      for (int s = 0; s < a.n_part; s++) {
        const float4 p = part[s * ps4 + k];
        v.x += p.x, v.y += p.y, v.z += p.z, v.w += p.w;
      }
      if (a.n_part) x[k] = v;
    }
    xs[j] = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (!a.Y) return;
  const float inv = rsqrtf(block_sum_f(ss, scratch) / (float)a.H + a.eps);
  if (a.ex && threadIdx.x == 0) a.ex[m] = max(-64, min(64, ilogbf(inv)));
  half4_t* y = reinterpret_cast<half4_t*>(a.Y + (size_t)m * a.H);
  const float4* w = reinterpret_cast<const float4*>(a.w);
#pragma unroll
  for (int j = 0; j < kRowVec; j++) {
    const int k = threadIdx.x + 256 * j;
    if (k < H4) {
      const float4 wv = w[k], v = xs[j];
      y[k] = (half4_t){f16_guard(a.ovf, v.x * inv * wv.x), f16_guard(a.ovf, v.y * inv * wv.y),
                       f16_guard(a.ovf, v.z * inv * wv.z), f16_guard(a.ovf, v.w * inv * wv.w)};
    }
  }
}

void launch_rms_rows(const RowsArgs& a, int M, hipStream_t st) {
  hipLaunchKernelGGL(rms_rows_kernel, dim3(M), dim3(256), 0, st, a);
}

// Rotate-half RoPE of the q and k heads of row m at position p0 + m
// (TSLAttention.ts:252-286) on bias + the sum of the split-K slices; q to fp16
// rows, k and v appended to the cache.  A thread takes a rotation pair
// (d, d + rd/2) of a head, or one element outside the rotary part.
__device__ __forceinline__ float fold_slices(const float* row, const float* bias, int n_part, size_t pstride, int i) {
  float v = bias ? bias[i] : 0.f;
#pragma unroll 4
  for (int s = 0; s < n_part; s++) v += row[s * pstride + i];
  return v;
}

__device__ __forceinline__ void rope_store(const RopeKvArgs& a, int m, int pos, int i, float y) {
  const int nq = a.Hq * a.D, nk = a.Hkv * a.D;
  if (i < nq) {
    a.q[(size_t)m * nq + i] = __builtin_bit_cast(uint16_t, f16_guard(a.ovf, y));
    return;
  }
  const bool isv = i >= nq + nk;
  const int j = i - nq - (isv ? nk : 0), hk = j / a.D, d = j % a.D;
  const size_t dst = ((size_t)hk * a.max_tokens + pos) * a.D + d;
  void* cache = isv ? a.vc : a.kc;
  if (a.kv_f32)
    static_cast<float*>(cache)[dst] = y;
  else
    static_cast<uint16_t*>(cache)[dst] = __builtin_bit_cast(uint16_t, f16_guard(a.ovf, y));
}

// Pair pi of a q|k|v row: head pi / (D / 2), q = pi % (D / 2).  In a rotated
// head (q or k) q < rd / 2 is the rotate-half pair (d, d + rd / 2) and the
// rest covers dims rd.. two at a time; a v head takes dims 2 q, 2 q + 1.
__device__ __forceinline__ void rope_pair(const RopeKvArgs& a, int pi, int& i0, int& i1, bool& rot, int& dr) {
  const int hd = a.D / 2, h = pi / hd, q = pi - h * hd, half = a.rd / 2;
  rot = h < a.Hq + a.Hkv && q < half;
  dr = q;
  if (rot) {
    i0 = h * a.D + q;
    i1 = i0 + half;
  } else {
    const int d = h < a.Hq + a.Hkv ? a.rd + 2 * (q - half) : 2 * q;
    i0 = h * a.D + d;
    i1 = i0 + 1;
  }
}

// RoPE + cache append of the rows' q|k|v (the split-K slices summed with the
// bias first; TSLAttention.ts:168-286 for one row).  Thread = one element
// pair of RKV_ROWS consecutive rows (grid: row groups x 256-pair chunks): no
// idle threads, and the 2 RKV_ROWS n_part loads of a thread go out at once.
constexpr int RKV_ROWS = 2;
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeKvArgs a) {
  const int D = a.D, width = (a.Hq + 2 * a.Hkv) * D;
  const int pi = blockIdx.y * 256 + threadIdx.x;
  if (pi >= width / 2) return;
  int i0, i1, dr;
  bool rot;
  rope_pair(a, pi, i0, i1, rot, dr);
  const int half = a.rd / 2;
  const int p0 = a.ctrl ? a.ctrl[C_POS] : a.p0;
  float x0[RKV_ROWS], x1[RKV_ROWS], c[RKV_ROWS], sn[RKV_ROWS];
#pragma unroll
  for (int r = 0; r < RKV_ROWS; r++) {
    const int m = min(blockIdx.x * RKV_ROWS + r, a.M - 1), pos = p0 + m;
    const float* row = a.qkv + (size_t)m * width;
    x0[r] = fold_slices(row, a.bias, a.n_part, a.pstride, i0);
    x1[r] = fold_slices(row, a.bias, a.n_part, a.pstride, i1);
    c[r] = rot ? a.rope_cos[(size_t)pos * half + dr] : 1.f;
    sn[r] = rot ? a.rope_sin[(size_t)pos * half + dr] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < RKV_ROWS; r++) {
    const int m = blockIdx.x * RKV_ROWS + r;
    if (m >= a.M) break;
    const int pos = p0 + m;
    rope_store(a, m, pos, i0, rot ? x0[r] * c[r] - x1[r] * sn[r] : x0[r]);
    rope_store(a, m, pos, i1, rot ? x1[r] * c[r] + x0[r] * sn[r] : x1[r]);
  }
}

// The same per element, four elements per load: with full rotary (rd == D,
// D % 8 == 0) and an fp16 cache, thread g of a row takes dims 4j..4j+3 of a
// q or k head and their rotation partners D/2 + 4j.., or dims 8j..8j+7 of a v
// head (j = g mod D/8), so every slice, bias, cos and sin read is 16 bytes
// and every fp16 store 8 (the scalar kernel's 4- and 2-byte accesses took
// 17.5 us per layer of a 2048-row Llama-3.2-1B chunk).
__device__ __forceinline__ float4 fold_slices4(const float* row, const float* bias, int n_part, size_t pstride, int i) {
  float4 v = bias ? *reinterpret_cast<const float4*>(bias + i) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
  for (int s = 0; s < n_part; s++) {
    const float4 p = *reinterpret_cast<const float4*>(row + s * pstride + i);
    v.x += p.x, v.y += p.y, v.z += p.z, v.w += p.w;
  }
  return v;
}

__device__ __forceinline__ void rope_store4(const RopeKvArgs& a, int m, int pos, int i, float4 y) {
  const int nq = a.Hq * a.D, nk = a.Hkv * a.D;
  const half4_t h = {f16_guard(a.ovf, y.x), f16_guard(a.ovf, y.y), f16_guard(a.ovf, y.z), f16_guard(a.ovf, y.w)};
  uint16_t* dst;
  if (i < nq) {
    dst = a.q + (size_t)m * nq + i;
  } else {
    const bool isv = i >= nq + nk;
    const int j = i - nq - (isv ? nk : 0), hk = j / a.D, d = j % a.D;
    dst = static_cast<uint16_t*>(isv ? a.vc : a.kc) + ((size_t)hk * a.max_tokens + pos) * a.D + d;
  }
  *reinterpret_cast<half4_t*>(dst) = h;
}

__global__ __launch_bounds__(256) void rope_kv4_kernel(RopeKvArgs a) {
  const int D = a.D, g8 = D / 8, groups = (a.Hq + 2 * a.Hkv) * g8, half = D / 2;
  const int g = blockIdx.y * 256 + threadIdx.x;
  if (g >= groups) return;
  const int h = g / g8, j = g - h * g8;
  const bool rot = h < a.Hq + a.Hkv;
  const int i0 = h * D + (rot ? 4 * j : 8 * j), i1 = i0 + (rot ? half : 4);
  const int width = (a.Hq + 2 * a.Hkv) * D;
  const int p0 = a.ctrl ? a.ctrl[C_POS] : a.p0;
  float4 x0[RKV_ROWS], x1[RKV_ROWS], c[RKV_ROWS], sn[RKV_ROWS];
#pragma unroll
  for (int r = 0; r < RKV_ROWS; r++) {
    const int m = min(blockIdx.x * RKV_ROWS + r, a.M - 1), pos = p0 + m;
    const float* row = a.qkv + (size_t)m * width;
    x0[r] = fold_slices4(row, a.bias, a.n_part, a.pstride, i0);
    x1[r] = fold_slices4(row, a.bias, a.n_part, a.pstride, i1);
    c[r] = rot ? *reinterpret_cast<const float4*>(a.rope_cos + (size_t)pos * half + 4 * j) : make_float4(1.f, 1.f, 1.f, 1.f);
    sn[r] = rot ? *reinterpret_cast<const float4*>(a.rope_sin + (size_t)pos * half + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int r = 0; r < RKV_ROWS; r++) {
    const int m = blockIdx.x * RKV_ROWS + r;
    if (m >= a.M) break;
    const int pos = p0 + m;
    float4 y0 = x0[r], y1 = x1[r];
    if (rot) {
      const float4 u = x0[r], v = x1[r], cc = c[r], ss = sn[r];
      y0 = make_float4(u.x * cc.x - v.x * ss.x, u.y * cc.y - v.y * ss.y, u.z * cc.z - v.z * ss.z, u.w * cc.w - v.w * ss.w);
      y1 = make_float4(v.x * cc.x + u.x * ss.x, v.y * cc.y + u.y * ss.y, v.z * cc.z + u.z * ss.z, v.w * cc.w + u.w * ss.w);
    }
    rope_store4(a, m, pos, i0, y0);
    rope_store4(a, m, pos, i1, y1);
  }
}

// TLM_ROPE_VEC=0 keeps the scalar kernel for every shape (comparisons)
static const bool g_rope_vec = [] {
  const char* e = getenv("TLM_ROPE_VEC");
  return !(e && e[0] == '0');
}();

void launch_rope_kv(const RopeKvArgs& a, hipStream_t st) {
  const bool vec = g_rope_vec && !a.kv_f32 && a.rd == a.D && a.D % 8 == 0 && a.pstride % 4 == 0;
  if (vec) {
    const int groups = (a.Hq + 2 * a.Hkv) * a.D / 8;
    hipLaunchKernelGGL(rope_kv4_kernel, dim3((a.M + RKV_ROWS - 1) / RKV_ROWS, (groups + 255) / 256), dim3(256), 0, st,
                       a);
    return;
  }
  const int pairs = (a.Hq + 2 * a.Hkv) * a.D / 2;
  hipLaunchKernelGGL(rope_kv_kernel, dim3((a.M + RKV_ROWS - 1) / RKV_ROWS, (pairs + 255) / 256), dim3(256), 0, st, a);
}

// ------------------------------------------------------- flash attention --
// Causal attention of M query rows over the fp16 cache (TSLAttention.ts:
// 288-449 for one query).  Block: one kv head, 32 query rows and up to four
// query heads of the group (one wave each), times NG key groups: group z
// takes key tiles z, z + NG, ... and the groups merge their (max, sum, O) at
// the end, which halves the serial chain of the long (late) query tiles.
// Per tile of 64 keys: K rows and V^T sit in LDS (double buffered; the next
// tiles' rows are loaded into registers while this one is computed, one
// barrier per tile); S^T = K Q^T (lane = query, registers = keys), an online
// softmax in registers (the two half-waves of a query exchange one value;
// masks only on tiles that cross the causal diagonal or the window start; O
// is rescaled only when some row's max moved), then O^T += V^T P^T with P^T
// taken straight from the S^T registers: the key order of the contraction is
// permuted to match that register layout.  P is rounded to fp16 toward zero.
template <int DT, int NG>
struct AttnTile {
  static constexpr int KT = 64;            // keys per tile
  static constexpr int KS = DT + 8;        // halves per K row in LDS
  // halves per V row: the four rows a half-wave's transposing reads touch fall
  // on different banks (row strides of 40 and 80 dwords)
  static constexpr int VS = DT + (DT == 64 ? 16 : 32);
  static constexpr int PIECES = KT * DT / 8;  // 16-byte pieces of K (or V) per tile
  static constexpr int PPT = PIECES / 256;    // pieces per thread (256 threads per key group)
  static constexpr int TILE_HALVES = KT * KS + KT * VS;
};

typedef short short4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (gfx950): in each group of 16 lanes, lane j names 4
// halves in[j][0..3] and lane i receives in[4 k + i / 4][i % 4], k = 0..3.
// With lane j at V[key0 + j / 4][d0 + 4 (j % 4)], lane i receives
// V[key0 + k][d0 + i]: four consecutive keys of one dim (checked on the
// device with an index-valued LDS probe).
__device__ __forceinline__ half4_t lds_read_tr4(const _Float16* p) {
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (short4_t __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(half4_t, v);
}

// K and V pieces of one tile in registers: piece i is row i / (DT / 8), dims
// 8 (i % (DT / 8)) .. + 7; rows past qhi repeat row qhi (their keys are masked).
template <int DT, int NG>
struct AttnStage {
  using AT = AttnTile<DT, NG>;
  uint4 kr[AT::PPT], vr[AT::PPT];
  __device__ __forceinline__ void load(const _Float16* kb, const _Float16* vb, int kt0, int qhi, int t) {
#pragma unroll
    for (int u = 0; u < AT::PPT; u++) {
      const int i = t + 256 * u;
      const size_t src = (size_t)min(kt0 + i / (DT / 8), qhi) * DT + 8 * (i % (DT / 8));
      kr[u] = *reinterpret_cast<const uint4*>(kb + src);
      vr[u] = *reinterpret_cast<const uint4*>(vb + src);
    }
  }
  // K and V rows as they are (V is read transposed, lds_read_tr4)
  __device__ __forceinline__ void store(_Float16* tile, int t) const {
    _Float16* ks = tile;
    _Float16* vs = tile + AT::KT * AT::KS;
#pragma unroll
    for (int u = 0; u < AT::PPT; u++) {
      const int i = t + 256 * u, r = i / (DT / 8), c8 = i % (DT / 8);
      *reinterpret_cast<uint4*>(&ks[r * AT::KS + 8 * c8]) = kr[u];
      *reinterpret_cast<uint4*>(&vs[r * AT::VS + 8 * c8]) = vr[u];
    }
  }
};

template <int DT, int NG>
__global__ __launch_bounds__(256 * NG) __attribute__((amdgpu_waves_per_eu(2))) void prefill_attn_kernel(PrefillAttnArgs a) {
  using AT = AttnTile<DT, NG>;
  constexpr int KT = AT::KT, KS = AT::KS, VS = AT::VS, NDT = DT / 32;
  __shared__ __align__(16) _Float16 lds[2 * NG * AT::TILE_HALVES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = __builtin_amdgcn_readfirstlane(tid >> 8), t256 = tid & 255, wave = t256 >> 6;
  const int l32 = lane & 31, kh = lane >> 5;
  const int nqt = (a.M + 31) / 32;
  // Longest key ranges first in the lower half of the (head, group) blocks and
  // shortest first in the upper half: with two blocks per CU, blocks L and
  // L + half of the grid share a CU, so a long query tile pairs with a short one.
  const int yz = blockIdx.z * gridDim.y + blockIdx.y, nyz = gridDim.y * gridDim.z;
  const int qt = (2 * yz < nyz) ? nqt - 1 - (int)blockIdx.x : (int)blockIdx.x;
  const int hk = blockIdx.y;
  const int gw = (int)blockIdx.z * 4 + wave;
  const bool active = gw < a.G;
  const int h = hk * a.G + min(gw, a.G - 1);
  const int p0 = a.ctrl ? a.ctrl[C_POS] : a.p0;
  const int qr = qt * 32 + l32, qpos = p0 + qr;
  const int qlo = p0 + qt * 32, qhi = p0 + min(qt * 32 + 31, a.M - 1);
  const int kfirst = a.window > 0 ? max(0, qlo - a.window + 1) : 0;
  const int qfirst = a.window > 0 ? max(0, qpos - a.window + 1) : 0;
  const int QW = a.Hq * DT;

  half8_t qb[DT / 16];
  const _Float16* qrow = reinterpret_cast<const _Float16*>(a.q) + (size_t)min(qr, a.M - 1) * QW + h * DT;
#pragma unroll
  for (int j = 0; j < DT / 16; j++) qb[j] = *reinterpret_cast<const half8_t*>(qrow + 16 * j + 8 * kh);

  const _Float16* kb = reinterpret_cast<const _Float16*>(a.kc) + (size_t)hk * a.max_tokens * DT;
  const _Float16* vb = reinterpret_cast<const _Float16*>(a.vc) + (size_t)hk * a.max_tokens * DT;
  AttnStage<DT, NG> sg;

  float16_t o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; i++) o[i] = (float16_t){};
  float mrun = -INFINITY, lrun = 0.f;  // running max (log2 units) and this half-wave's sum
  const int kbeg = kfirst & ~(KT - 1);
  const int ntiles = (qhi - kbeg) / KT + 1;
  const int nsteps = (ntiles + NG - 1) / NG;
  _Float16* const mytile = lds + grp * AT::TILE_HALVES;  // buffer b at + b NG TILE_HALVES
  sg.load(kb, vb, kbeg + grp * KT, qhi, t256);
  sg.store(mytile, t256);
  __syncthreads();
  for (int it = 0; it < nsteps; it++) {
    const int buf = it & 1, tile = it * NG + grp, kt0 = kbeg + tile * KT;
    sg.load(kb, vb, kt0 + NG * KT, qhi, t256);  // this group's next tile, in flight during the math
    if (tile < ntiles) {
      const _Float16* kbuf = mytile + buf * NG * AT::TILE_HALVES;
      const _Float16* vbuf = kbuf + KT * KS;
      float16_t s[2];
#pragma unroll
      for (int b2 = 0; b2 < 2; b2++) {
        s[b2] = (float16_t){};
#pragma unroll
        for (int j = 0; j < DT / 16; j++) {
          const half8_t ak = *reinterpret_cast<const half8_t*>(kbuf + (32 * b2 + l32) * KS + 16 * j + 8 * kh);
          s[b2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ak, qb[j], s[b2], 0, 0, 0);
        }
      }
      if (kt0 + KT - 1 > qlo || (a.window > 0 && kt0 < qhi - a.window + 1)) {
#pragma unroll
        for (int b2 = 0; b2 < 2; b2++)
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int key = kt0 + 32 * b2 + 8 * (v >> 2) + 4 * kh + (v & 3);
            if (key > qpos || key < qfirst) s[b2][v] = -INFINITY;
          }
      }
      float mv[16];  // max over the 32 scores as a tree, not a chain
#pragma unroll
      for (int v = 0; v < 16; v++) mv[v] = fmaxf(s[0][v], s[1][v]);
#pragma unroll
      for (int w = 8; w > 0; w >>= 1)
#pragma unroll
        for (int v = 0; v < w; v++) mv[v] = fmaxf(mv[v], mv[v + w]);
      float mx = fmaxf(mv[0], swap32(mv[0])) * a.scale_log2;
      const float mn = fmaxf(mrun, mx);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float corr = __builtin_amdgcn_exp2f(mrun - mu);
      float ps = 0.f;
      uint32_t pk[2][8];
#pragma unroll
      for (int b2 = 0; b2 < 2; b2++)
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(s[b2][v], a.scale_log2, -mu));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(s[b2][v + 1], a.scale_log2, -mu));
          ps += p0 + p1;
          pk[b2][v >> 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0, p1));
        }
      lrun = lrun * corr + ps;
      mrun = mn;
      if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
        for (int i = 0; i < NDT; i++) o[i] *= corr;
      }
#pragma unroll
      for (int b2 = 0; b2 < 2; b2++) {
        const half8_t pb0 = __builtin_bit_cast(half8_t, make_uint4(pk[b2][0], pk[b2][1], pk[b2][2], pk[b2][3]));
        const half8_t pb1 = __builtin_bit_cast(half8_t, make_uint4(pk[b2][4], pk[b2][5], pk[b2][6], pk[b2][7]));
#pragma unroll
        for (int i = 0; i < NDT; i++) {
          // lane (16 g + j) names V[32 b2 + 4 kh + j / 4 + 8 s][32 i + 16 (g % 2) + 4 (j % 4)]
          // and receives keys 32 b2 + 4 kh + 8 s + 0..3 of dim 32 i + l32
          const _Float16* vr0 = vbuf + (32 * b2 + 4 * kh + (lane & 15) / 4) * VS + 32 * i + 16 * ((lane >> 4) & 1) +
                                4 * (lane & 3);
          const half4_t x0 = lds_read_tr4(vr0);
          const half4_t x1 = lds_read_tr4(vr0 + 8 * VS);
          const half4_t x2 = lds_read_tr4(vr0 + 16 * VS);
          const half4_t x3 = lds_read_tr4(vr0 + 24 * VS);
          const half8_t a1 = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
          const half8_t a2 = {x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]};
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, pb0, o[i], 0, 0, 0);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, pb1, o[i], 0, 0, 0);
        }
      }
    }
    sg.store(mytile + (buf ^ 1) * NG * AT::TILE_HALVES, t256);
    __syncthreads();
  }
  lrun += swap32(lrun);
  if (NG > 1) {  // group 1 hands (max, sum, O) to group 0 through LDS (the tiles are free now)
    float* xch = reinterpret_cast<float*>(lds) + (size_t)(wave * 64 + lane) * (2 + 16 * NDT);
    if (grp == 1) {
      xch[0] = mrun;
      xch[1] = lrun;
#pragma unroll
      for (int i = 0; i < NDT; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) xch[2 + 16 * i + v] = o[i][v];
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = xch[0], l1 = xch[1];
    const float mn = fmaxf(mrun, m1);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float c0 = __builtin_amdgcn_exp2f(mrun - mu), c1 = __builtin_amdgcn_exp2f(m1 - mu);
    lrun = lrun * c0 + l1 * c1;
#pragma unroll
    for (int i = 0; i < NDT; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) o[i][v] = o[i][v] * c0 + xch[2 + 16 * i + v] * c1;
  }
  if (!active || qr >= a.M) return;
  const float inv = lrun > 0.f ? 1.f / lrun : 0.f;
  _Float16* orow = reinterpret_cast<_Float16*>(a.out) + (size_t)qr * QW + h * DT;
#pragma unroll
  for (int i = 0; i < NDT; i++)
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
      const half4_t y = {(_Float16)(o[i][4 * g4] * inv), (_Float16)(o[i][4 * g4 + 1] * inv),
                         (_Float16)(o[i][4 * g4 + 2] * inv), (_Float16)(o[i][4 * g4 + 3] * inv)};
      *reinterpret_cast<half4_t*>(orow + 32 * i + 8 * g4 + 4 * kh) = y;
    }
}

bool launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t st) {
  // four query heads per block (waves past the group's heads only stage K/V)
  const dim3 grid((a.M + 31) / 32, a.Hkv, (a.G + 3) / 4);
  if (a.D == 64)
    hipLaunchKernelGGL((prefill_attn_kernel<64, 2>), grid, dim3(512), 0, st, a);
  else if (a.D == 128)
    hipLaunchKernelGGL((prefill_attn_kernel<128, 1>), grid, dim3(256), 0, st, a);
  else
    return false;
  return true;
}

// fp32 -> fp16 (round to nearest even)
__global__ void rows_to_f16_kernel(const float* x, size_t n, _Float16* y) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (_Float16)x[i];
}

void launch_rows_to_f16(const float* x, size_t n, uint16_t* y, hipStream_t st) {
  hipLaunchKernelGGL(rows_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n,
                     reinterpret_cast<_Float16*>(y));
}

}  // namespace tlm

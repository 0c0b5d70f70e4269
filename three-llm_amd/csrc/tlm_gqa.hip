// Long-window decode attention on the matrix cores: one block per (kv head,
// chunk of positions) serves all G query heads of the kv head from one read
// of the chunk's K and V rows (TSLAttention.ts:306-428 computes the same
// scores, softmax and weighted sum per query head over the whole window).
//
// fp16 cache, head_dim 64 or 128, G <= 16.  Each wave takes 32-position tiles
// of the block's chunk:
//   * scores S^T (positions x heads) = K Q^T with v_mfma_f32_16x16x32_f16:
//     the K rows are the A operand straight from global memory (16 bytes per
//     lane), the G query rows (padded to 16) the B operand;
//   * an online softmax per head in registers (base 2: the query carries
//     scale * log2 e);
//   * O^T (dims x heads) += V^T P^T: V rows staged in the wave's LDS region
//     and read transposed (ds_read_b64_tr_b16), P^T straight from the score
//     registers (the contraction's position order is permuted to match).
// q and P enter the matrix cores as hi + lo fp16 pairs (x = hi + lo to about
// 2^-22 relative; two MFMAs into one accumulator), so the scores and the
// weighted sum keep fp32-level accuracy while K and V are exact fp16.
//
// The block forms q (its G heads), the new k and v rows from the QKV partial
// sums + bias with RoPE (rotate-half), and the block whose chunk holds `pos`
// appends k and v to the cache and substitutes them for that row in its tile.
// The waves merge (max, sum, output) in LDS; the block writes one chunk
// partial per query head in the layout the O projection's combine reads.
#include <float.h>
#include <math.h>

#include <hip/hip_fp16.h>

#include "tlm_device.h"

namespace tlm {
namespace {

typedef _Float16 gh8_t __attribute__((ext_vector_type(8)));
typedef _Float16 gh4_t __attribute__((ext_vector_type(4)));
typedef short gs4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: in each group of 16 lanes, lane j names 4 halves
// in[j][0..3] and lane i receives in[4 k + i / 4][i % 4], k = 0..3.  With lane
// j at V[key0 + j / 4][d0 + 4 (j % 4)], lane i receives V[key0 + k][d0 + i].
__device__ __forceinline__ gh4_t tr4(const _Float16* p) {
  const gs4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((gs4_t __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(gh4_t, v);
}

template <int DT>
struct GqaShape {
  static constexpr int SLABS = DT / 32;              // 32-dim K steps of the score MFMAs
  static constexpr int NK = 2 * SLABS;               // K fragments per lane per tile
  static constexpr int NV = kGqaTile * DT / 8 / 64;  // 16-byte V pieces per lane per tile
  static constexpr int DTILES = DT / 16;             // 16-dim output tiles
  // halves per V row in LDS: a stride of 72 (DT 128) or 40 (DT 64) dwords puts
  // the 8 rows of one half-wave's transposing read on distinct bank groups
  static constexpr int VS = DT + 16;
  static constexpr int WAVE_HALVES = kGqaTile * VS;
  // halves per q row in LDS: the 16 rows one B-operand read touches start 4
  // banks apart (a stride of DT halves would put them all on the same banks)
  static constexpr int QS = DT + 8;
  // LDS: V regions (reused for the merge), q hi / lo [16][QS], new k / v rows,
  // the pre-RoPE q|k|v rows [G + 2][DT] in fp32 (RAW floats: every thread
  // stores all kGqaPro of its slots, used or not)
  static constexpr int RAW = kGqaPro * 64 * kGqaWaves;
  static constexpr int LDS_HALVES = kGqaWaves * WAVE_HALVES + 2 * 16 * QS + 2 * DT + 2 * RAW;
  static_assert(16 * (2 + DT) * 2 <= WAVE_HALVES, "a wave region holds its merge record");
  static_assert((64 * kGqaWaves) % DT == 0, "a thread's prologue elements share one dim");
};

// A tile's K rows in registers: lane (i, qd) = (lane % 16, lane / 16) holds
// dims 32 jj + 8 qd .. + 7 of rows t0 + i and t0 + 16 + i (the A operand of
// the score MFMAs).  Rows past `last` repeat row `last` (masked in the softmax).
template <int DT>
struct GqaK {
  using S = GqaShape<DT>;
  gh8_t k[S::NK];
  __device__ __forceinline__ void load(const _Float16* kb, int t0, int last, int lane) {
    const int i = lane & 15, qd = lane >> 4;
#pragma unroll
    for (int st = 0; st < 2; st++) {
      const TLM_GLOBAL gh8_t* kr = gl(reinterpret_cast<const gh8_t*>(kb + (size_t)min(t0 + 16 * st + i, last) * DT + 8 * qd));
#pragma unroll
      for (int jj = 0; jj < S::SLABS; jj++) k[st * S::SLABS + jj] = kr[4 * jj];
    }
  }
};

// A tile's V rows in registers on their way to LDS: 16-byte pieces lane + 64 u
// of the row-major [kGqaTile][DT] tile (rows past `last` repeat row `last`).
template <int DT>
struct GqaV {
  using S = GqaShape<DT>;
  uint4 v[S::NV];
  __device__ __forceinline__ void load(const _Float16* vb, int t0, int last, int lane) {
#pragma unroll
    for (int u = 0; u < S::NV; u++) {
      const int p = lane + 64 * u;
      const size_t off = (size_t)min(t0 + p / (DT / 8), last) * DT + 8 * (p % (DT / 8));
      const u32x4 w = *gl(reinterpret_cast<const u32x4*>(vb + off));
      v[u] = make_uint4(w.x, w.y, w.z, w.w);
    }
  }
};

template <int DT>
__global__ __launch_bounds__(64 * kGqaWaves) void gqa_attn_kernel(AttnArgs a) {
  using S = GqaShape<DT>;
  __shared__ __align__(16) _Float16 lds[S::LDS_HALVES];
  _Float16* const qhi = lds + kGqaWaves * S::WAVE_HALVES;  // [16][QS]
  _Float16* const qlo = qhi + 16 * S::QS;                  // [16][QS]
  _Float16* const kn = qlo + 16 * S::QS;                   // [DT] new k row (rounded like the cache)
  _Float16* const vn = kn + DT;                            // [DT]
  float* const raw = reinterpret_cast<float*>(vn + DT);    // [G + 2][DT] (RAW floats)

  const int G = a.G, Hkv = a.Hkv;
  const int hk = blockIdx.x % Hkv, c = blockIdx.x / Hkv;
  const int pos = a.ctrl[C_POS];
  if (pos < 0 || pos >= a.max_tokens) return;
  const ChunkPlan cp = chunk_plan(pos, a.window, a.nsplit, a.chmin);
  if (c >= cp.nact) return;  // block-uniform, before any barrier
  const int b0 = cp.first + c * cp.chunk, b1 = min(b0 + cp.chunk, pos + 1), last = b1 - 1;
  const int ntile = (b1 - b0 + kGqaTile - 1) / kGqaTile;
  const bool owner = pos <= last;  // this chunk holds the new row
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i16 = lane & 15, qd = lane >> 4;
  const _Float16* kb = reinterpret_cast<const _Float16*>(a.kc) + (size_t)hk * a.max_tokens * DT;
  const _Float16* vb = reinterpret_cast<const _Float16*>(a.vc) + (size_t)hk * a.max_tokens * DT;

  // Loads in the order they are needed (a wave's vector loads complete in
  // issue order): the q|k|v inputs of this thread's elements (at most
  // kGqaPro: (G + 2) DT <= kGqaPro * 64 kGqaWaves) and its RoPE factors, then
  // the wave's first tile.  The q, k, v rows are formed while that tile
  // streams in; the wave's second tile is requested after them (below).
  // Tile loads are unconditional (a wave past the chunk's tiles reads row
  // `last` only); a tile's registers are refilled with the wave's tile after
  // next.
  const int E = (G + 2) * DT, QW = a.Hq * DT, KW = Hkv * DT;
  auto col_of = [&](int e) {
    const int r = e / DT, d = e % DT;
    return r < G ? (hk * G + r) * DT + d : (r == G ? QW : QW + KW) + hk * DT + d;
  };
  float gp[kGqaPro][kMaxPart], gb[kGqaPro];
#pragma unroll
  for (int x = 0; x < kGqaPro; x++) {
    const int col = col_of(min(tid + 64 * kGqaWaves * x, E - 1));
#pragma unroll
    for (int j = 0; j < kMaxPart; j++) gp[x][j] = a.src[(size_t)max(min(j, a.n_src - 1), 0) * a.src_stride + col];
    gb[x] = a.bias[col];
  }
  // every element this thread rotates has dim d = tid % DT (64 kGqaWaves is a multiple of DT)
  const int half = a.rd > 0 ? a.rd / 2 : 1;
  const int dr = tid % DT, jr = dr < half ? dr : dr - half;
  const float rc = a.rope_cos[(size_t)pos * half + min(jr, half - 1)];
  const float rs = a.rope_sin[(size_t)pos * half + min(jr, half - 1)];
  GqaK<DT> k0, k1;
  GqaV<DT> v0, v1;
  __builtin_amdgcn_sched_barrier(0);  // the tile's loads go after the prologue's
  k0.load(kb, b0 + kGqaTile * w, last, lane);
  v0.load(vb, b0 + kGqaTile * w, last, lane);

  // q (G heads), new k, new v: partial sums + bias (stored unconditionally,
  // so the loads above are neither moved nor waited for behind the tile's),
  // then RoPE through LDS
#pragma unroll
  for (int x = 0; x < kGqaPro; x++) {
    float sum = gb[x];
#pragma unroll
    for (int j = 0; j < kMaxPart; j++) sum = fmaf(gp[x][j], j < a.n_src ? 1.f : 0.f, sum);
    raw[tid + 64 * kGqaWaves * x] = sum;
  }
  lds_barrier();
  const float qscale = a.scale * 1.4426950408889634f;  // log2 e: the softmax runs in base 2
  constexpr int NROT = (18 * DT + 64 * kGqaWaves - 1) / (64 * kGqaWaves);
#pragma unroll
  for (int x = 0; x < NROT; x++) {  // unrolled: no loop whose entry would wait for every load
    const int e = tid + 64 * kGqaWaves * x;
    if (e >= 18 * DT) break;
    const int r = e / DT, d = e % DT;  // d == dr
    if (r >= G && r < 16) {  // padding heads
      qhi[r * S::QS + d] = qlo[r * S::QS + d] = (_Float16)0.f;
      continue;
    }
    const int rr = r < G ? r : G + (r - 16);  // row of raw: q heads, then k, v
    float val = raw[rr * DT + d];
    if (rr <= G && d < a.rd) {
      const int pd = d < half ? d + half : d - half;
      const float sg = d < half ? -1.f : 1.f;
      val = raw[rr * DT + d] * rc + sg * raw[rr * DT + pd] * rs;
    }
    if (rr < G) {
      const float qs = val * qscale;
      const _Float16 hi = (_Float16)qs;
      qhi[r * S::QS + d] = hi;
      qlo[r * S::QS + d] = (_Float16)(qs - (float)hi);
    } else {
      const uint16_t bits = kv_store<uint16_t>(val);
      reinterpret_cast<uint16_t*>(rr == G ? kn : vn)[d] = bits;
      if (owner) {
        uint16_t* cache = reinterpret_cast<uint16_t*>(rr == G ? a.kc : a.vc);
        cache[((size_t)hk * a.max_tokens + pos) * DT + d] = bits;
      }
    }
  }
  lds_barrier();

  // B operands of the scores (read from LDS once per tile): lane (i16, qd)
  // takes dims 32 jj + 8 qd .. + 7 of head i16
  const _Float16* const bqp = qhi + i16 * S::QS + 8 * qd;
  const _Float16* const blp = qlo + i16 * S::QS + 8 * qd;

  _Float16* const vt = lds + w * S::WAVE_HALVES;  // [kGqaTile][VS]
  f32x4 o[S::DTILES];
#pragma unroll
  for (int r = 0; r < S::DTILES; r++) o[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lrun = 0.f;  // running max (base 2) and this lane's share of the sum

  // tile t0 with K in f and V in vr
  auto process = [&](GqaK<DT>& f, GqaV<DT>& vr, int t0) {
    // V rows to LDS; in the tile holding `pos`, that row and the clamped rows
    // after it come from the new v row
    const bool own = t0 <= pos && pos < t0 + kGqaTile;  // wave-uniform
    wave_lds_sync();  // the previous tile's transposing reads are done
#pragma unroll
    for (int u = 0; u < S::NV; u++) {
      const int p = lane + 64 * u, r = p / (DT / 8), c8 = p % (DT / 8);
      uint4 val = vr.v[u];
      if (own && t0 + r >= pos) val = *reinterpret_cast<const uint4*>(vn + 8 * c8);
      *reinterpret_cast<uint4*>(vt + r * S::VS + 8 * c8) = val;
    }
    if (own) {
#pragma unroll
      for (int st = 0; st < 2; st++)
        if (t0 + 16 * st + i16 >= pos) {
#pragma unroll
          for (int jj = 0; jj < S::SLABS; jj++)
            f.k[st * S::SLABS + jj] = *reinterpret_cast<const gh8_t*>(kn + 32 * jj + 8 * qd);
        }
    }
    wave_lds_sync();
    // scores: lane (head i16, qd) gets positions t0 + 16 st + 4 qd + v
    f32x4 acc[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int jj = 0; jj < S::SLABS; jj++) {
      const gh8_t bq = *reinterpret_cast<const gh8_t*>(bqp + 32 * jj);
      const gh8_t bl = *reinterpret_cast<const gh8_t*>(blp + 32 * jj);
#pragma unroll
      for (int st = 0; st < 2; st++) {
        acc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k[st * S::SLABS + jj], bq, acc[st], 0, 0, 0);
        acc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k[st * S::SLABS + jj], bl, acc[st], 0, 0, 0);
      }
    }
    float sv[8];
#pragma unroll
    for (int st = 0; st < 2; st++)
#pragma unroll
      for (int v = 0; v < 4; v++) sv[4 * st + v] = t0 + 16 * st + 4 * qd + v <= last ? acc[st][v] : -INFINITY;
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
    mx = fmaxf(mx, lane_swap16(mx));
    mx = fmaxf(mx, lane_swap32(mx));
    const float mn = fmaxf(mrun, mx);  // finite: the tile holds a position of the chunk
    const float corr = __builtin_amdgcn_exp2f(mrun - mn);
    float ps = 0.f;
    gh8_t ph, pl;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float p = __builtin_amdgcn_exp2f(sv[e] - mn);
      ps += p;
      const _Float16 h = (_Float16)p;
      ph[e] = h;
      pl[e] = (_Float16)(p - (float)h);
    }
    lrun = fmaf(lrun, corr, ps);
    mrun = mn;
    if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
      for (int r = 0; r < S::DTILES; r++) o[r] *= corr;
    }
    // O^T += V^T P^T: k = 8 qd + e is position 4 qd + e (e < 4) or 16 + 4 qd + e - 4
#pragma unroll
    for (int r = 0; r < S::DTILES; r++) {
      const _Float16* v0 = vt + (4 * qd + i16 / 4) * S::VS + 16 * r + 4 * (i16 & 3);
      const gh4_t x0 = tr4(v0), x1 = tr4(v0 + 16 * S::VS);
      const gh8_t av = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      o[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, ph, o[r], 0, 0, 0);
      o[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pl, o[r], 0, 0, 0);
    }
  };

  // The wave's tiles w, w + 8, w + 16, ...: the first two in straight-line
  // code (inside a loop the compiler's waits merge over the back edge and
  // the first tile would wait for the second's loads), any further ones in
  // the loop, each pair's registers refilled two tiles ahead.
  constexpr int NW = kGqaWaves;
  // The second tile's K goes out before the first tile's math and its V
  // after it: a wave blocks while the memory pipeline will not take more
  // loads, and issuing all of the second tile up front kept every wave from
  // computing its first tile until nearly all data had arrived (3B at 16384
  // positions: 1457 against 1420 us per token; K and V both after: 1445).
  k1.load(kb, b0 + kGqaTile * (w + NW), last, lane);
  if (w < ntile) process(k0, v0, b0 + kGqaTile * w);
  v1.load(vb, b0 + kGqaTile * (w + NW), last, lane);
  if (w + 2 * NW < ntile) {
    k0.load(kb, b0 + kGqaTile * (w + 2 * NW), last, lane);
    v0.load(vb, b0 + kGqaTile * (w + 2 * NW), last, lane);
  }
  if (w + NW < ntile) process(k1, v1, b0 + kGqaTile * (w + NW));
  if (w + 3 * NW < ntile) {
    k1.load(kb, b0 + kGqaTile * (w + 3 * NW), last, lane);
    v1.load(vb, b0 + kGqaTile * (w + 3 * NW), last, lane);
  }
  for (int it = w + 2 * NW; it < ntile; it += 2 * NW) {
    process(k0, v0, b0 + kGqaTile * it);
    if (it + 2 * NW < ntile) {
      k0.load(kb, b0 + kGqaTile * (it + 2 * NW), last, lane);
      v0.load(vb, b0 + kGqaTile * (it + 2 * NW), last, lane);
    }
    if (it + NW >= ntile) break;
    process(k1, v1, b0 + kGqaTile * (it + NW));
    if (it + 3 * NW < ntile) {
      k1.load(kb, b0 + kGqaTile * (it + 3 * NW), last, lane);
      v1.load(vb, b0 + kGqaTile * (it + 3 * NW), last, lane);
    }
  }

  // merge the waves' (max, sum, output) per head; every wave takes part
  lrun += lane_swap16(lrun);
  lrun += lane_swap32(lrun);
  wave_lds_sync();
  float* const mine = reinterpret_cast<float*>(vt);  // [G][2 + DT]
  if (i16 < G) {
    float* rec = mine + i16 * (2 + DT);
#pragma unroll
    for (int r = 0; r < S::DTILES; r++)
#pragma unroll
      for (int v = 0; v < 4; v++) rec[2 + 16 * r + 4 * qd + v] = o[r][v];
    if (qd == 0) {
      rec[0] = mrun;
      rec[1] = lrun;
    }
  }
  __syncthreads();
  for (int e = tid; e < G * DT; e += 64 * kGqaWaves) {
    const int j = e / DT, d = e % DT;
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < kGqaWaves; x++)
      M = fmaxf(M, reinterpret_cast<const float*>(lds + x * S::WAVE_HALVES)[j * (2 + DT)]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int x = 0; x < kGqaWaves; x++) {
      const float* rec = reinterpret_cast<const float*>(lds + x * S::WAVE_HALVES) + j * (2 + DT);
      const float sc = __builtin_amdgcn_exp2f(rec[0] - M);  // a wave without tiles: exp2(-inf) = 0
      L = fmaf(rec[1], sc, L);
      O = fmaf(rec[2 + d], sc, O);
    }
    const size_t row = (size_t)(hk * G + j) * a.nsplit + c;
    a.pacc[row * DT + d] = O;
    if (d == 0) {
      a.pml[row * 2] = M * 0.6931471805599453f;  // natural-log units, like the other attention kernels
      a.pml[row * 2 + 1] = L;
    }
  }
}

}  // namespace

bool launch_gqa_attention(const AttnArgs& a, hipStream_t st) {
  if (!gqa_attention_fits(a.G, a.D)) return false;
  const dim3 grid((unsigned)(a.Hkv * a.nsplit)), block(64 * kGqaWaves);
  if (a.D == 64) hipLaunchKernelGGL(gqa_attn_kernel<64>, grid, block, 0, st, a);
  else if (a.D == 128) hipLaunchKernelGGL(gqa_attn_kernel<128>, grid, block, 0, st, a);
  else return false;
  return true;
}

}  // namespace tlm

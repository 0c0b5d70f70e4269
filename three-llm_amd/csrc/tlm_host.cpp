// Host-side helpers of the C ABI: synthetic inputs, the q4 quantizer and fp16
// rounding.  Pure C++ (no device code); threads split index ranges, every
// element is computed independently, so results do not depend on the thread count.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/tlm.h"

namespace {

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

uint64_t stream_key(uint64_t seed, uint64_t stream) { return splitmix64(seed ^ splitmix64(stream + 0x5851F42D4C957F2Dull)); }

template <typename F>
void parallel_for(size_t n, F f) {
  unsigned hw = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
  if (n < (1u << 16) || hw == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> threads;
  size_t per = (n + hw - 1) / hw;
  for (unsigned i = 0; i < hw; i++) {
    size_t b = i * per, e = std::min(n, b + per);
    if (b >= e) break;
    threads.emplace_back([=] { f(b, e); });
  }
  for (auto& t : threads) t.join();
}

uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (absx < 0x38800000u) {
    if (absx < 0x33000000u) return (uint16_t)sign;
    uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    int shift = 126 - (int)(absx >> 23);
    uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (((absx >> 23) - 112u) << 10) | ((absx & 0x7fffffu) >> 13);
  uint32_t rem = absx & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float f16_bits_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ffu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int sh = 0;
      while (!(m & 0x400u)) {
        m <<= 1;
        sh++;
      }
      bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

int tlm_host_fail(int code, const char* msg);  // tlm_api.hip: sets tlm_last_error()

extern "C" {

int tlm_synth_normal(uint64_t seed, uint64_t stream, size_t n, float stddev, float* out) {
  if (!out && n) return tlm_host_fail(TLM_ERR_INVALID, "TLMSynth: null output");
  const uint64_t key = stream_key(seed, stream);
  const size_t pairs = (n + 1) / 2;
  parallel_for(pairs, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; i++) {
      const uint64_t a = splitmix64(key + 2 * i), c = splitmix64(key + 2 * i + 1);
      const double u1 = ((double)(a >> 11) + 0.5) * 0x1.0p-53;
      const double u2 = (double)(c >> 11) * 0x1.0p-53;
      const double r = sqrt(-2.0 * log(u1)) * stddev;
      out[2 * i] = (float)(r * cos(2.0 * M_PI * u2));
      if (2 * i + 1 < n) out[2 * i + 1] = (float)(r * sin(2.0 * M_PI * u2));
    }
  });
  return TLM_OK;
}

int tlm_synth_tokens(uint64_t seed, uint64_t stream, size_t n, int32_t vocab, int32_t* out) {
  if (vocab <= 0 || (!out && n)) return tlm_host_fail(TLM_ERR_INVALID, "TLMSynth: vocabulary must be positive and the output non-null");
  const uint64_t key = stream_key(seed, stream);
  for (size_t i = 0; i < n; i++) out[i] = (int32_t)(splitmix64(key + i) % (uint64_t)vocab);
  return TLM_OK;
}

// The canonical q4 format: per row and group of 32 k, s = fp16(fp32(max|w| / 7))
// (largest finite fp16 at most), q = clamp(rint(w / f32(s)), -8, 7), q = 0 when
// s == 0, nibble q + 8 with even k in the low nibble.
int tlm_quantize_q4(const float* w, int n_out, int k_in, uint8_t* packed, uint16_t* scales) {
  if (!w || !packed || !scales || n_out <= 0 || k_in <= 0 || k_in % 32 != 0)
    return tlm_host_fail(TLM_ERR_INVALID, "TLMQuantize: q4 needs non-null buffers, n_out > 0 and k_in a positive multiple of 32");
  const int G = k_in / 32;
  parallel_for((size_t)n_out * G, [&](size_t b, size_t e) {
    for (size_t idx = b; idx < e; idx++) {
      const size_t n = idx / G, g = idx % G;
      const float* src = w + n * k_in + g * 32;
      float maxabs = 0.f;
      for (int j = 0; j < 32; j++) maxabs = std::max(maxabs, fabsf(src[j]));
      uint16_t s16 = f32_to_f16_bits(maxabs / 7.0f);
      if ((s16 & 0x7c00u) == 0x7c00u) s16 = (uint16_t)((s16 & 0x8000u) | 0x7bffu);
      const float s = f16_bits_to_f32(s16);
      scales[idx] = s16;
      uint8_t* dst = packed + n * (k_in / 2) + g * 16;
      for (int j = 0; j < 32; j += 2) {
        int q[2];
        for (int u = 0; u < 2; u++) {
          float r = s == 0.f ? 0.f : rintf(src[j + u] / s);
          r = std::min(7.f, std::max(-8.f, r));
          q[u] = (int)r;
        }
        dst[j / 2] = (uint8_t)((q[0] + 8) | ((q[1] + 8) << 4));
      }
    }
  });
  return TLM_OK;
}

int tlm_f32_to_f16(const float* in, size_t n, uint16_t* out) {
  if ((!in || !out) && n) return tlm_host_fail(TLM_ERR_INVALID, "TLMQuantize: null buffer");
  parallel_for(n, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; i++) out[i] = f32_to_f16_bits(in[i]);
  });
  return TLM_OK;
}

}  // extern "C"

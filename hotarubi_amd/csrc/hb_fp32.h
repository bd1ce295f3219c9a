// Bit-exact FP32 arithmetic of the hotarubi NPU, for host and device.
//
// Semantics of tools/iss/fp32.hpp:24-104: round to nearest even, an exponent
// field of 0 on input reads as zero, results below the normal range become
// +0, results at biased exponent >= 255 become +-inf, and exponent 255 on
// input is an ordinary exponent (no NaN or infinity handling).
//
// The kernels compute with the hardware FP32 units wherever those give the
// same bits (normal operands and results, FTZ mode) and fall back to these
// integer routines for the rest: operands with exponent 255, products near
// the bottom of the normal range, and block scales outside the range the
// matrix-core path is proven exact for.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define HB_HD __host__ __device__ __forceinline__

namespace hb {

HB_HD uint32_t ExpField(uint32_t bits) { return (bits >> 23) & 0xFFu; }

HB_HD uint32_t Significand(uint32_t bits) {
  return ExpField(bits) ? ((bits & 0x7FFFFFu) | 0x800000u) : 0u;
}

HB_HD int BitWidth32(uint32_t v) { return v ? 32 - __builtin_clz(v) : 0; }
HB_HD int BitWidth64(uint64_t v) { return v ? 64 - __builtin_clzll(v) : 0; }

HB_HD uint32_t Pack(uint32_t sign, int32_t exponent, uint32_t fraction) {
  if (exponent <= 0) return 0u;
  if (exponent >= 255) return (sign << 31) | 0x7F800000u;
  return (sign << 31) | ((uint32_t)exponent << 23) | fraction;
}

HB_HD uint32_t Round(uint32_t sign, int32_t exponent, uint32_t sig24, bool guard,
                     bool sticky) {
  uint32_t r = sig24 + ((guard && (sticky || (sig24 & 1u))) ? 1u : 0u);
  if (r >> 24) {
    ++exponent;
    r >>= 1;
  }
  return Pack(sign, exponent, r & 0x7FFFFFu);
}

// Add with guard, round and sticky bits after alignment.
HB_HD uint32_t AddBits(uint32_t a, uint32_t b) {
  const uint32_t ea = ExpField(a), eb = ExpField(b);
  const uint32_t ma = Significand(a), mb = Significand(b);
  const bool a_larger = ((ea << 24) | ma) >= ((eb << 24) | mb);
  const uint32_t e_big = a_larger ? ea : eb;
  const uint32_t gap = a_larger ? ea - eb : eb - ea;
  const uint32_t m_big = a_larger ? ma : mb;
  const uint32_t m_small = a_larger ? mb : ma;
  uint32_t aligned = 0;
  if (m_small != 0) {
    if (gap > 26) {
      aligned = 1;
    } else {
      const uint32_t wide = m_small << 3;
      aligned = (wide >> gap) | ((wide & ((1u << gap) - 1u)) ? 1u : 0u);
    }
  }
  const bool subtract = ((a ^ b) >> 31) != 0;
  const uint32_t sum = subtract ? (m_big << 3) - aligned : (m_big << 3) + aligned;
  if (sum == 0) return 0u;
  const int shift = 28 - BitWidth32(sum);
  const uint32_t norm = sum << shift;
  return Round((a_larger ? a : b) >> 31, (int32_t)e_big + 1 - shift, norm >> 4,
               ((norm >> 3) & 1u) != 0, (norm & 7u) != 0);
}

HB_HD uint32_t MulBits(uint32_t a, uint32_t b) {
  if (ExpField(a) == 0 || ExpField(b) == 0) return 0u;
  const uint64_t product = (uint64_t)Significand(a) * Significand(b);
  const bool carry = (product >> 47) != 0;
  const int drop = carry ? 23 : 22;
  const uint64_t kept = product >> drop;
  const bool sticky = (product & ((1ull << drop) - 1ull)) != 0;
  const int32_t exponent = (int32_t)(ExpField(a) + ExpField(b)) - (carry ? 126 : 127);
  return Round((a ^ b) >> 31, exponent, (uint32_t)(kept >> 1), (kept & 1u) != 0, sticky);
}

// s * fraction / 2^16 with one rounding (the table interpolation multiply).
HB_HD uint32_t MulFractionBits(uint32_t s, uint32_t fraction) {
  if (ExpField(s) == 0 || fraction == 0) return 0u;
  const uint64_t product = (uint64_t)Significand(s) * fraction;
  const int shift = 40 - BitWidth64(product);
  const uint64_t norm = product << shift;
  return Round(s >> 31, (int32_t)ExpField(s) - shift, (uint32_t)(norm >> 16),
               ((norm >> 15) & 1u) != 0, (norm & 0x7FFFu) != 0);
}

// ---- GEMM block arithmetic (tools/iss/gemm_array.cpp:25-110) ----

enum : uint32_t { kModeFp4 = 0, kModeW8Hi = 1, kModeW8Lo = 2 };

HB_HD uint32_t DecodeMode(uint32_t wmode) {
  const uint32_t w = wmode & 3u;
  return w == 0 ? kModeFp4 : w == 1 ? kModeW8Hi : kModeW8Lo;
}

HB_HD int32_t ScaleBias(uint32_t mode) {
  return mode == kModeFp4 ? -7 : mode == kModeW8Hi ? -8 : -12;
}

// FP4: sign * 2 * E2M1 magnitude {0,1,2,3,4,6,8,12}; W8_HI: signed nibble;
// W8_LO: unsigned nibble.  The magnitudes are the nibbles of 0xC8643210.
HB_HD int32_t WeightValue(uint32_t nibble, uint32_t mode) {
  nibble &= 0xFu;
  if (mode == kModeFp4) {
    const int32_t mag = (int32_t)((0xC8643210u >> (4u * (nibble & 7u))) & 0xFu);
    return (nibble & 8u) ? -mag : mag;
  }
  if (mode == kModeW8Hi) return (nibble & 8u) ? (int32_t)nibble - 16 : (int32_t)nibble;
  return (int32_t)nibble;
}

// sum * 2^((a_scale - 127) + (w_scale - 127) + SBIAS), exact (|sum| < 2^24).
HB_HD uint32_t BlockValue(int32_t sum, uint32_t a_scale, uint32_t w_scale, uint32_t mode) {
  if (sum == 0) return 0u;
  const uint32_t mag = (uint32_t)(sum < 0 ? -sum : sum);
  const int msb = BitWidth32(mag) - 1;
  const int32_t exponent = (int32_t)(a_scale + w_scale) - 254 + ScaleBias(mode) + msb + 127;
  return Pack(sum < 0 ? 1u : 0u, exponent, (mag << (23 - msb)) & 0x7FFFFFu);
}

// ---- VEC requantize (tools/iss/lane.cpp:384-404) ----
// The reference's steps without branches: its shift is at least 17 (the
// element's exponent is at most the block's), and from 25 on it takes the
// magnitude as 0, which the same rounding arithmetic gives with the shift
// held at 31 (the significand has 24 bits); a zero significand rounds to 0.
HB_HD uint8_t QuantizeElement(uint32_t value, uint32_t emax) {
  const uint32_t sig = Significand(value);
  const uint32_t shift = emax - ExpField(value) + 17;
  const uint32_t s = shift < 31u ? shift : 31u;
  const uint32_t integer = sig >> s;
  const uint32_t guard = (sig >> (s - 1)) & 1u;
  const uint32_t sticky = (sig & ((1u << (s - 1)) - 1u)) != 0 ? 1u : 0u;
  const uint32_t mag = integer + (guard & (sticky | (integer & 1u)));
  const uint32_t pos = mag >= 128 ? 0x7Fu : mag;
  const uint32_t neg = mag >= 128 ? 0x80u : ((256u - mag) & 0xFFu);
  return (uint8_t)((value >> 31) ? neg : pos);
}

// ---- host encoder (tools/runtime/formats.cpp:35-56) ----
// RNE(x * 2^(6 - e)) saturated to [-128, 127]; subnormals keep their value.
// Inf/NaN (rejected by the reference) encodes as 0 with *bad set.
HB_HD int8_t QuantizeInt8(uint32_t bits, int32_t e, bool* bad) {
  const uint32_t field = ExpField(bits);
  if (field == 0xFFu) {
    *bad = true;
    return 0;
  }
  const uint64_t sig = field == 0 ? (bits & 0x7FFFFFu) : ((bits & 0x7FFFFFu) | 0x800000u);
  const int64_t shift = (field == 0 ? -149 : (int64_t)field - 150) + 6 - e;
  int64_t mag = 0;
  if (shift >= 0) {
    mag = shift > 8 ? 256 : (int64_t)(sig << shift);
  } else if (shift > -64) {
    const uint64_t kept = sig >> (-shift);
    const uint64_t rest = sig & ((1ull << (-shift)) - 1ull);
    const uint64_t half = 1ull << (-shift - 1);
    mag = (int64_t)(kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u));
  }
  int64_t v = (bits >> 31) ? -mag : mag;
  v = v < -128 ? -128 : (v > 127 ? 127 : v);
  return (int8_t)v;
}

// ---- MXFP8 E4M3 activations (no counterpart in the reference) ----
// An E4M3 code (OCP E4M3FN: bias 7, no infinities, max 448) as an integer
// in units of 2^-9: m for exponent field 0, (8 + m) << (e - 1) otherwise
// (the NaN codes 0x7F / 0xFF read as +-480; they are not valid input).
HB_HD int32_t Fp8Int(uint32_t code) {
  const uint32_t e = (code >> 3) & 15u, m = code & 7u;
  const int32_t u = e == 0 ? (int32_t)m : (int32_t)((8u + m) << (e - 1u));
  return (code & 0x80u) ? -u : u;
}

// A block's exact sum S = sum Fp8Int(a) * WeightValue(w) against MXFP4 (28
// bits at most), S * 2^(a_scale + w_scale - 264) rounded once to FP32 by
// the reference's Round / Pack (RNE; below normal -> +0; overflow -> inf).
HB_HD uint32_t BlockValueFp8(int32_t sum, uint32_t a_scale, uint32_t w_scale) {
  if (sum == 0) return 0u;
  const uint32_t sign = sum < 0 ? 1u : 0u;
  const uint32_t mag = (uint32_t)(sum < 0 ? -sum : sum);
  const int msb = BitWidth32(mag) - 1;
  const int32_t exponent = (int32_t)(a_scale + w_scale) - 264 + msb + 127;
  if (msb <= 23) return Pack(sign, exponent, (mag << (23 - msb)) & 0x7FFFFFu);
  const int sh = msb - 23;
  return Round(sign, exponent, mag >> sh, ((mag >> (sh - 1)) & 1u) != 0,
               (mag & ((1u << (sh - 1)) - 1u)) != 0);
}

// OCP MX encoding of one element at block exponent x: x-scaled value
// rounded to nearest even on the E4M3 grid, saturated to +-448; a zero
// magnitude encodes as 0.  Inf/NaN encodes as 0 with *bad set.
HB_HD uint8_t QuantizeFp8(uint32_t bits, int32_t x, bool* bad) {
  const uint32_t field = ExpField(bits);
  if (field == 0xFFu) {
    *bad = true;
    return 0;
  }
  const uint64_t sig = field == 0 ? (bits & 0x7FFFFFu) : ((bits & 0x7FFFFFu) | 0x800000u);
  if (sig == 0) return 0;
  const int bw = BitWidth64(sig);
  const int64_t ev = (field == 0 ? -149 : (int64_t)field - 150) - x;  // |y| = sig 2^ev
  int64_t qe = (int64_t)bw - 1 + ev - 3;                                // the grid step
  qe = qe < -9 ? -9 : qe;
  const int64_t s = qe - ev;
  uint64_t mant = 0;
  if (s <= 0) {
    mant = sig << (-s);
  } else if (s <= 40) {
    const uint64_t kept = sig >> s, rest = sig & ((1ull << s) - 1ull), half = 1ull << (s - 1);
    mant = kept + ((rest > half || (rest == half && (kept & 1u))) ? 1u : 0u);
  }
  uint64_t u = qe + 9 > 30 ? ~0ull : mant << (qe + 9);  // units of 2^-9
  if (mant != 0 && (qe + 9 > 30 || u > 229376u)) u = 229376u;
  if (u == 0) return 0;
  uint32_t code;
  if (u < 8) {
    code = (uint32_t)u;
  } else {
    const int top = BitWidth64(u) - 1;
    code = ((uint32_t)(top - 2) << 3) | ((uint32_t)(u >> (top - 3)) & 7u);
  }
  return (uint8_t)(code | ((bits >> 31) ? 0x80u : 0u));
}

}  // namespace hb

// C entry points over the reference's own FP32 code, compiled where it lies
// under /root/reference (see oracle/Makefile).  Used only by the tests to
// check the oracle's restatement; nothing here is copied from the reference.
//   tools/iss/fp32.hpp   : the ISS arithmetic (Fp32Add/Mul/MulFraction)
//   tb/fp32_ref.cpp      : the testbench arithmetic (Fp32Add/Mul/FromInt)
#include <cstdint>

#include "fp32.hpp"      // tools/iss
#include "fp32_ref.hpp"  // tb

extern "C" {
uint32_t ref_iss_fp32_add(uint32_t a, uint32_t b) { return hotarubi::iss::Fp32Add(a, b); }
uint32_t ref_iss_fp32_mul(uint32_t a, uint32_t b) { return hotarubi::iss::Fp32Mul(a, b); }
uint32_t ref_iss_fp32_mul_fraction(uint32_t s, uint32_t f) {
  return hotarubi::iss::Fp32MulFraction(s, f);
}
uint32_t ref_tb_fp32_add(uint32_t a, uint32_t b) { return hotarubi::tb::Fp32Add(a, b); }
uint32_t ref_tb_fp32_mul(uint32_t a, uint32_t b) { return hotarubi::tb::Fp32Mul(a, b); }
uint32_t ref_tb_fp32_from_int(int64_t v, int e) { return hotarubi::tb::Fp32FromInt(v, e); }

// Batched forms so the tests can sweep millions of operands quickly.
void ref_iss_fp32_add_n(const uint32_t* a, const uint32_t* b, uint32_t* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = hotarubi::iss::Fp32Add(a[i], b[i]);
}
void ref_iss_fp32_mul_n(const uint32_t* a, const uint32_t* b, uint32_t* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = hotarubi::iss::Fp32Mul(a[i], b[i]);
}
void ref_iss_fp32_mul_fraction_n(const uint32_t* s, const uint32_t* f, uint32_t* out,
                                 uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = hotarubi::iss::Fp32MulFraction(s[i], f[i]);
}
void ref_tb_fp32_add_n(const uint32_t* a, const uint32_t* b, uint32_t* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = hotarubi::tb::Fp32Add(a[i], b[i]);
}
void ref_tb_fp32_from_int_n(const int64_t* v, const int32_t* e, uint32_t* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = hotarubi::tb::Fp32FromInt(v[i], e[i]);
}
}

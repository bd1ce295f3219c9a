// Building blocks of the streaming kernels (hb_stream.hip, hb_w8.hip): loads
// from global memory straight into LDS with waits counted by hand, and the
// split of MXINT8 activation codes into two exact FP6 E2M3 operand planes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace hb {
namespace ring {

typedef uint32_t u32x6 __attribute__((ext_vector_type(6)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x32 __attribute__((ext_vector_type(32)));

// f(I) for I = 0 .. kN-1 as compile-time constants (std::integral_constant),
// for builtin arguments that must be constant.
template <typename Fn, int... kI>
__device__ __forceinline__ void UnrollImpl(Fn&& f, std::integer_sequence<int, kI...>) {
  (f(std::integral_constant<int, kI>{}), ...);
}
template <int kN, typename Fn>
__device__ __forceinline__ void Unroll(Fn&& f) {
  UnrollImpl(f, std::make_integer_sequence<int, kN>{});
}

// A pointer as a wave-uniform value (scalar registers).  The builtin returns
// int: each half is widened through uint32_t, not by sign extension.
__device__ __forceinline__ uint64_t UniformAddress(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (hi << 32) | lo;
}

// Direct load into LDS: lane l's 16 bytes at base + voff land at LDS byte
// lds + 16 l (lds is wave-uniform, passed in M0).  The load counts in the
// wave's vector memory counter like any load; the compiler does not see it,
// so the caller waits for it with WaitVm.
__device__ __forceinline__ void Dma16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(UniformAddress(base)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Wait until at most kN of this wave's vector memory operations are
// outstanding (s_waitcnt vmcnt(kN), the other counters left alone).
template <int kN>
__device__ __forceinline__ void WaitVm() {
  static_assert(kN >= 0 && kN < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((kN & 15) | ((kN >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Wait for this wave's LDS operations (s_waitcnt lgkmcnt(0)).
__device__ __forceinline__ void WaitLds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// 32 int8 codes q (8 dwords, K order; `mask` 0 zeroes them) -> the FP6 E2M3
// codes of h = q / 32 rounded to FP6 and of (q - 32 h) / 2.  Both are exact:
// |q / 32| <= 4 rounds to a multiple of 1/8 (1/4 from 2 on), so q - 32 h is
// an integer with |q - 32 h| <= 4, and (q - 32 h) / 2, a multiple of 1/2 in
// [-2, 2], is an E2M3 value.  h carries scale byte ea - 1 and the rest
// ea - 5: (h 2^(ea-128)) + ((q - 32 h) / 2) 2^(ea-132) = q 2^(ea-133).
// A byte u = q ^ 0x80 placed under the f16 exponent byte 0x64 is 1024 + u,
// so one v_perm and one packed subtract of 1152 give q exactly.
__device__ __forceinline__ void SplitA(const uint32_t* x, uint32_t mask, u32x6& h6, u32x6& r6) {
  const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  f16x32 q;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const uint32_t u = (x[d] & mask) ^ 0x80808080u;
    const f16x2 p0 =
        __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    const f16x2 p1 =
        __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
    q[4 * d] = p0[0];
    q[4 * d + 1] = p0[1];
    q[4 * d + 2] = p1[0];
    q[4 * d + 3] = p1[1];
  }
  h6 = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(q, 32.0f);
  const f16x32 hv = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6(h6, 1.0f);
  const f16x32 m32 = (_Float16)-32.0f;
  const f16x32 r = __builtin_elementwise_fma(hv, m32, q);
  r6 = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(r, 2.0f);
}

}  // namespace ring
}  // namespace hb

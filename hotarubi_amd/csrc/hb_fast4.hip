// Streaming MXFP4 kernel for gfx950 (HB_LINEAR_FAST, one FP4 weight plane,
// tiles of 128 rows x 256 columns, plain fp32 output).
//
// Same arithmetic as FastKernel (hb_fast.hip): v_mfma_scale_f32_32x32x64_f8f6f4
// with A as two exact FP6 E2M3 planes (scale bytes ea-1 and ea-5) and the
// WBUF column-blocks as the E2M1 B operand with their E8M0 scale bytes.  The
// A planes are formed differently: the int8 q (exact in f16) is rounded to
// FP6 at scale 32, h = fp6(q/32), and the residual r = q - 32h is again
// exact in FP6 as r/2 (|r| <= 4), so q = 32 h + 2 (r/2): h carries the
// weight of the hi plane (scale byte ea-1) and r/2 that of the lo plane (ea-5).
//   tools/iss/gemm_array.cpp:84-110 (FP4 value 2*E2M1, SBIAS -7):
//   q * 2e2m1 * 2^(ea+ew-261) = h e2m1 2^(ea-1+ew-254) + (r/2) e2m1 2^(ea-5+ew-254).
// Both planes come from one conversion per (row, block): 59 VALU operations
// for 32 values, against about 90 for nibble planes.
//
// Work split, one workgroup per CU (8 waves, 256 registers each):
//   4 producer waves (one per SIMD): thread t streams the raw bytes of one
//     (row, block) of A and of one column's two blocks of W per K-step (64)
//     through a ring of register sets, converts A, and stages both in LDS
//     in the MFMA lanes' operand layout (128-bit accesses throughout).
//   4 consumer waves: 64 x 128 outputs each (2 x 4 MFMA tiles, 128
//     accumulators); the operands of step s + 1 are read from LDS into a
//     second register set while the matrix cores run step s, so LDS latency
//     never stalls the matrix issue.
// One barrier per step; the LDS stage producers fill in iteration s (step
// s + 2) was read into registers in iteration s - 1 (step 0: before the
// loop, behind its own barrier), so two stages suffice.
// Epilogue: the consumers park the tile in LDS (row-major, padded pitch),
// then all 8 waves store whole rows with 16-byte stores; dword stores
// straight from the MFMA layout drain several times slower.
#include <utility>

#include "hb_device.h"
#include "hb_internal.h"

namespace hb {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x6 __attribute__((ext_vector_type(6)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x32 __attribute__((ext_vector_type(32)));

constexpr int kBM = 128, kBN = 256;
constexpr int kP = 256;    // producer threads
constexpr int kRing = 8;   // raw register sets per producer thread (= loop unroll, even)
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;

constexpr int kOutPitch = kBN + 8;  // floats: rows r and r + 4 fall on disjoint LDS banks

// One K-step (two blocks) of operands.  Lane l of an m-tile holds row l % 32
// and block l / 32; lane l of an n-tile holds column l % 32 and block l / 32.
struct Stage {
  uint4 a[4][64][3];   // [m-tile][lane]: h codes (dwords 0-5), r/2 codes (6-11)
  uint4 w[8][64];      // [n-tile][lane]: 32 E2M1 codes
  uint32_t sa[2][64];  // [m-tile / 2][lane]: byte (m-tile % 2) * 2 + plane
  uint32_t sw[2][64];  // [n-tile / 4][lane]: byte n-tile % 4
};

// f(I) for I = 0 .. kN-1 as compile-time constants.
template <typename Fn, int... kI>
__device__ __forceinline__ void UnrollImpl(Fn&& f, std::integer_sequence<int, kI...>) {
  (f(std::integral_constant<int, kI>{}), ...);
}
template <int kN, typename Fn>
__device__ __forceinline__ void Unroll(Fn&& f) {
  UnrollImpl(f, std::make_integer_sequence<int, kN>{});
}

template <bool kMulti>
__device__ __forceinline__ uint32_t BlockOf(const GemmArgs& g, uint32_t idx) {
  uint32_t base = g.piece_off[0];
  if (kMulti) {
    uint32_t start = 0;
#pragma unroll
    for (uint32_t p = 1; p < kMaxPieces; ++p) {
      start += g.piece_kb[p - 1];
      const bool in = p < g.n_pieces && idx >= start;
      base = in ? g.piece_off[p] - start : base;
    }
  }
  return base + idx;
}

// A producer thread's raw bytes of one step: its A (row, block) and its
// column's W column-blocks of both blocks, with the aligned dwords that hold
// their scale bytes.
struct Raw {
  uint32_t a[8];
  uint32_t sa;
  uint32_t w[2][4];
  uint32_t sw[2];
  uint32_t mask;  // 0xFFFFFFFF, or 0 where the A block is past the end
};

// 32 int8 (8 dwords, K order) -> FP6 E2M3 codes of h = q/32 rounded and of
// the residual (q - 32h)/2, both exact.  (q ^ 0x80) under the f16 exponent
// byte 0x64 is 1024 + q + 128, so one v_perm and one packed subtract give
// two f16 values q.
__device__ __forceinline__ void SplitA(const uint32_t* x, uint32_t mask, uint4* out) {
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
  const u32x6 h = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(q, 32.0f);  // codes of q/32
  const f16x32 hv = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6(h, 1.0f);
  const f16x32 m32 = (_Float16)-32.0f;
  const f16x32 r = __builtin_elementwise_fma(hv, m32, q);  // q - 32h, exact
  const u32x6 lo = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(r, 2.0f);  // codes of r/2
  out[0] = uint4{h[0], h[1], h[2], h[3]};
  out[1] = uint4{h[4], h[5], lo[0], lo[1]};
  out[2] = uint4{lo[2], lo[3], lo[4], lo[5]};
}

template <bool kMulti>
__global__ __launch_bounds__(512) void Fp4Kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) union {
    Stage stage[2];
    float out[kBM][kOutPitch];  // after the K loop: the tile's outputs
  } lds;
  __shared__ uint32_t lds_unsafe;

  const TileId tile = LogicalTile(g.gx, g.gy, g.gz);
  const uint32_t z = tile.z;
  const uint8_t* a = g.a + z * g.a_batch;
  const uint8_t* w0 = g.w[0] + z * g.w_batch;
  uint32_t* c = g.c + z * g.c_batch;

  const bool consumer = __builtin_amdgcn_readfirstlane(threadIdx.x >= kP);  // wave-uniform
  const uint32_t q0 = tile.y * (kBM / 4), g0 = tile.x * (kBN / 8);
  const uint32_t row0 = q0 * 4, col0 = g0 * 8;

  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < g.n_pieces; ++p) nblocks += g.piece_kb[p];
  const uint32_t steps = (nblocks + 1) / 2;  // both roles run this many iterations

  // Wave v of 8 stores tile rows v, v + 8, ...: lane l the 4 columns 4l ..
  // 4l + 3 (n is a multiple of 8, so 4 columns are all in or all out).
  auto store_rows = [&](uint32_t v) {
    const uint32_t l = threadIdx.x & 63, col = col0 + 4 * l;
    if (col >= g.n) return;
    for (uint32_t r = v; r < kBM; r += 8) {
      if (row0 + r >= g.m) break;
      const float4 val = *reinterpret_cast<const float4*>(&lds.out[r][4 * l]);
      *reinterpret_cast<float4*>(c + (size_t)(row0 + r) * g.n + col) = val;
    }
  };

  if (!consumer) {
    const uint32_t t = threadIdx.x, lane = t & 63, mt = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t h = lane >> 5;  // the A lane's block within the step
    const uint32_t word_row = g.kb_total * kDdrWord;
    const uint32_t r = mt * 32 + (lane & 31);
    const uint32_t quad = min(q0 + (r >> 2), g.quads - 1);
    const uint32_t o_a = quad * word_row + (r & 3) * 32, o_sa = quad * word_row + 128;
    const uint32_t grp = min(g0 + (t >> 3), g.groups - 1), cl = t & 7;
    const uint32_t o_w = grp * word_row + cl * 16, o_sw = grp * word_row + 128 + (cl & 4);

    // Steps at or past `steps` reload the last step's words (cache hits)
    // with A masked to zero.  Each load is one instruction on (uniform
    // base, 32-bit lane offset).
    auto load = [&](Raw& rw, uint32_t live) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t step = min(live, steps - 1);
      const uint32_t ub0 = BlockOf<kMulti>(g, 2 * step) * kDdrWord;
      const uint32_t ub1 = BlockOf<kMulti>(g, min(2 * step + 1, nblocks - 1)) * kDdrWord;
      // the lane's block: a step's two blocks need not be in memory order
      // (a piece list), so each lane addresses its own from the layer base
      const uint32_t ub = h ? ub1 : ub0;
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(a + (o_a + ub));
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(a + (o_a + ub) + 16);
      rw.sa = *reinterpret_cast<const uint32_t*>(a + (o_sa + ub));
      const u32x4 x0 = *reinterpret_cast<const u32x4*>(w0 + ub0 + o_w);
      rw.sw[0] = *reinterpret_cast<const uint32_t*>(w0 + ub0 + o_sw);
      const u32x4 x1 = *reinterpret_cast<const u32x4*>(w0 + ub1 + o_w);
      rw.sw[1] = *reinterpret_cast<const uint32_t*>(w0 + ub1 + o_sw);
      // applied at conversion time: a select on the loaded registers here
      // would make the compiler wait for the loads at once
      rw.mask = (live >= steps || (h && 2 * step + 1 >= nblocks)) ? 0u : 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[i] = v0[i];
        rw.a[4 + i] = v1[i];
        rw.w[0][i] = x0[i];
        rw.w[1][i] = x1[i];
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto store = [&](const Raw& rw, Stage& st) {
      uint4 codes[3];
      SplitA(rw.a, rw.mask, codes);
#pragma unroll
      for (int i = 0; i < 3; ++i) st.a[mt][lane][i] = codes[i];
      const uint32_t ea = __builtin_amdgcn_ubfe(rw.sa, 8 * (lane & 3), 8);  // row r % 4
      reinterpret_cast<uint16_t*>(&st.sa[mt >> 1][lane])[mt & 1] =
          (uint16_t)(((ea - 5u) << 8) | ((ea - 1u) & 0xFFu));
      bool bad = ea - kSafeLo > kSafeHi - kSafeLo;
      const uint32_t nt = t >> 5;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint32_t slot = (t & 31) + 32 * b;
        st.w[nt][slot] = uint4{rw.w[b][0], rw.w[b][1], rw.w[b][2], rw.w[b][3]};
        const uint32_t ew = __builtin_amdgcn_ubfe(rw.sw[b], 8 * (cl & 3), 8);
        reinterpret_cast<uint8_t*>(&st.sw[nt >> 2][slot])[nt & 3] = (uint8_t)ew;
        bad |= ew - kSafeLo > kSafeHi - kSafeLo;
      }
      return bad;
    };

    Raw ring[kRing];
    bool unsafe = false;
    if (t == 0) lds_unsafe = 0;
#pragma unroll
    for (int i = 0; i < kRing; ++i) load(ring[i], i);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      unsafe |= store(ring[i], lds.stage[i]);
      load(ring[i], i + kRing);
    }
    __syncthreads();  // steps 0 and 1 staged
    __syncthreads();  // the consumers hold step 0: its stage may be refilled
    for (uint32_t s = 0; s < steps; s += kRing) {
#pragma unroll
      for (int i = 0; i < kRing; ++i) {  // iteration s + i stages step s + i + 2
        if (s + i >= steps) break;
        unsafe |= store(ring[(i + 2) % kRing], lds.stage[i % 2]);
        load(ring[(i + 2) % kRing], s + i + 2 + kRing);
        __syncthreads();
      }
    }
    if (unsafe) lds_unsafe = 1;
    __syncthreads();  // the flags are in
    __syncthreads();  // the outputs are in LDS
    store_rows(t >> 6);
    return;
  }

  // Consumer wave cw: rows 64 * (cw % 2) .. + 64 (m-tiles 2 wm, 2 wm + 1),
  // columns 128 * (cw / 2) .. + 128 (n-tiles 4 wn .. 4 wn + 3).  MFMA tile
  // j = mi * 4 + nj.
  const uint32_t tid = threadIdx.x - kP, lane = tid & 63;
  const uint32_t cw = __builtin_amdgcn_readfirstlane(tid >> 6), wm = cw & 1, wn = cw >> 1;
  auto row_of = [&](uint32_t mi, uint32_t r) {
    return row0 + (2 * wm + mi) * 32 + 4 * (lane >> 5) + 8 * (r / 4) + (r & 3);
  };
  auto col_of = [&](uint32_t nj) { return col0 + (4 * wn + nj) * 32 + (lane & 31); };

  f32x16 acc[8];
  bool unsafe = false;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t row = row_of(j / 4, r), col = col_of(j % 4);
      uint32_t init = 0;
      if (g.acc && row < g.m && col < g.n) {
        init = c[(size_t)row * g.n + col];
        unsafe |= ExpField(init) > 252u;
      }
      acc[j][r] = __uint_as_float(init);
    }

  struct Ops {
    i32x8 a[2][2];  // [mi][plane]
    i32x8 b[4];
    int sa, sb;
  };
  auto read = [&](const Stage& st, Ops& o) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
      const uint4* p = st.a[2 * wm + mi][lane];
      const uint4 v0 = p[0], v1 = p[1], v2 = p[2];
      o.a[mi][0] = i32x8{(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, 0, 0};
      o.a[mi][1] = i32x8{(int)v1.z, (int)v1.w, (int)v2.x, (int)v2.y, (int)v2.z, (int)v2.w, 0, 0};
    }
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const uint4 v = st.w[4 * wn + nj][lane];
      o.b[nj] = i32x8{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
    }
    o.sa = (int)st.sa[wm][lane];
    o.sb = (int)st.sw[wn][lane];
  };
  auto matrix = [&](const Ops& o) {
    Unroll<2>([&](auto p) {
      Unroll<8>([&](auto j) {
        constexpr int kP2 = decltype(p)::value, kJ = decltype(j)::value;
        constexpr int kMi = kJ / 4, kNj = kJ % 4;
        acc[kJ] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            o.a[kMi][kP2], o.b[kNj], acc[kJ], 2, 4, kMi * 2 + kP2, o.sa, kNj, o.sb);
      });
    });
  };
  // Iteration s: read step s + 1 (stage st) into `nxt`, run step s from
  // `cur`, then the barrier (which waits for the reads).  The accumulators
  // are anchored on both sides of the barrier (the empty asm emits nothing),
  // so the compiler neither sinks the matrix work past it nor hoists the
  // next step's above it.
  auto iteration = [&](const Ops& cur, Ops& nxt, int st) {
    __builtin_amdgcn_sched_barrier(0);
    read(lds.stage[st], nxt);
    __builtin_amdgcn_sched_barrier(0);
    matrix(cur);
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(acc[j]));
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(acc[j]));
  };

  Ops x, y;
  __syncthreads();  // steps 0 and 1 staged; the flag is clear
  if (unsafe) lds_unsafe = 1;
  read(lds.stage[0], x);
  __syncthreads();  // step 0 is in registers before producers refill its stage
  for (uint32_t s = 0; s < steps; s += kRing) {
#pragma unroll
    for (int i = 0; i < kRing; i += 2) {
      if (s + i >= steps) break;
      iteration(x, y, 1);
      if (s + i + 1 >= steps) break;
      iteration(y, x, 0);
    }
  }
  __syncthreads();  // the producers' flags are in; the stages are free
  const bool slow = lds_unsafe != 0;
  // Output r of MFMA tile j of this lane is tile row 32 (2 wm + j / 4) +
  // 4 (lane / 32) + 8 (r / 4) + r % 4, column 32 (4 wn + j % 4) + lane % 32.
  if (slow) {  // a scale byte left the window: every output of the tile exactly
    for (uint32_t j = 0; j < 8; ++j)
      for (uint32_t r = 0; r < 16; ++r) {
        const uint32_t row = row_of(j / 4, r), col = col_of(j % 4);
        if (row >= g.m || col >= g.n) continue;
        const uint32_t init = g.acc ? c[(size_t)row * g.n + col] : 0u;
        lds.out[row - row0][col - col0] = __uint_as_float(SlowLinear(g, a, w0, w0, init, row, col));
      }
  } else {
    // Adding +0 maps -0 to +0 (and a denormal sum, in the kernel's
    // flush-to-zero mode, to +0).
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        lds.out[row_of(j / 4, r) - row0][col_of(j % 4) - col0] = acc[j][r] + 0.0f;
  }
  __syncthreads();  // the outputs are in LDS
  store_rows(4 + cw);
}

}  // namespace

bool Fp4Eligible(const GemmArgs& args, uint32_t tile_rows) {
  return args.n_planes == 1 && args.modes[0] == kModeFp4 && tile_rows == kBM &&
         args.n_ops == 0 && args.q_out == nullptr && args.ws == nullptr && args.splits <= 1;
}

hipError_t LaunchFp4(const GemmArgs& args, hipStream_t stream) {
  const dim3 grid(args.gx * args.gy * args.gz), block(512);
  if (args.n_pieces > 1) hipLaunchKernelGGL((Fp4Kernel<true>), grid, block, 0, stream, args);
  else hipLaunchKernelGGL((Fp4Kernel<false>), grid, block, 0, stream, args);
  return hipGetLastError();
}

}  // namespace hb

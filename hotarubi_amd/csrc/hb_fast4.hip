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
// Epilogue: each consumer wave passes its outputs, one 32 x 32 MFMA tile at
// a time, through a 4 KB LDS block of its own and stores rows of 4 columns
// per lane with 16-byte stores (dword stores straight from the MFMA layout
// drain several times slower).  No barrier is involved: the producers go on
// with the next tile's loads, and the tile's out-of-window flag reaches the
// consumers through the ordinary per-step barriers.
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
constexpr int kU = 4;      // raw register sets per producer thread = loop unroll (even)
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;

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

// Logical tiles of one workgroup: first + k * stride, k < count.  With more
// tiles than workgroups (one per CU), each XCD (workgroups b with b % 8 = x;
// the hardware deals workgroups round-robin over the 8 XCDs) takes one
// contiguous eighth of the tiles, so the tiles in flight on an XCD are
// neighbours (the column tiles of a layer share A in that XCD's L2).
struct Schedule {
  uint32_t first, stride, count;
};
__device__ __forceinline__ Schedule TilesOf(uint32_t total) {
  const uint32_t b = blockIdx.x, grid = gridDim.x;
  Schedule sc;
  if (grid >= total) {  // one tile each, remapped as LogicalTile does
    sc.first = total % kXcds == 0 ? (b % kXcds) * (total / kXcds) + b / kXcds : b;
    sc.stride = 1;
    sc.count = 1;
    return sc;
  }
  const uint32_t per = grid / kXcds, x = b % kXcds, idx = b / kXcds;  // grid % 8 == 0
  const uint32_t lo = (uint32_t)((uint64_t)x * total / kXcds);
  const uint32_t hi = (uint32_t)((uint64_t)(x + 1) * total / kXcds);
  sc.first = lo + idx;
  sc.stride = per;
  sc.count = hi > sc.first ? (hi - sc.first + per - 1) / per : 0u;
  return sc;
}

// Persistent: a workgroup runs its tiles back to back.  The K loop of every
// tile has `iters` iterations (the steps rounded up to kU; surplus steps add
// zeros), and the producers' ring streams straight across tile boundaries:
// global iteration u (tile u / iters) stages global step u + 2 and loads
// ahead in bursts, so the next tile's first steps are in LDS when a tile
// ends.  Both roles pass the same barriers: one per iteration and two
// before the loop.
//
// Out-of-window scale bytes are flagged per tile in lds_unsafe[k % 2]: the
// producers set it while staging tile k's last step (iteration
// (k + 1) iters - 3, at least two barriers before the consumers read it
// after iteration (k + 1) iters - 1), and consumer 0 clears the other slot
// in tile k's epilogue (tile k - 1's flag, read in its epilogue before
// barrier k iters; tile k + 1's flag is set no earlier than iteration
// (k + 1) iters + 1).
template <bool kMulti>
__global__ __launch_bounds__(512) void Fp4Kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) Stage lds_stage[2];
  __shared__ __attribute__((aligned(16))) float lds_xpose[4][32 * 32];  // one per consumer
  __shared__ uint32_t lds_unsafe[2];

  const Schedule sc = TilesOf(g.gx * g.gy * g.gz);
  const bool consumer = __builtin_amdgcn_readfirstlane(threadIdx.x >= kP);  // wave-uniform
  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < g.n_pieces; ++p) nblocks += g.piece_kb[p];
  const uint32_t steps = (nblocks + 1) / 2;
  const uint32_t iters = (steps + kU - 1) / kU * kU;  // per tile, both roles

  struct Tile {
    uint32_t row0, col0, z;
  };
  auto tile_of = [&](uint32_t k) {
    const uint32_t t = sc.first + k * sc.stride;
    Tile tl;
    tl.col0 = (t % g.gx) * kBN;
    tl.row0 = ((t / g.gx) % g.gy) * kBM;
    tl.z = t / (g.gx * g.gy);
    return tl;
  };
  if (!consumer) {
    const uint32_t t = threadIdx.x, lane = t & 63, mt = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t h = lane >> 5;  // the A lane's block within the step
    const uint32_t word_row = g.kb_total * kDdrWord, a_row = g.a_row * kDdrWord;
    const uint32_t r = mt * 32 + (lane & 31), cl = t & 7;

    // Load cursor: tile lk (clamped to the last), step ls; per-tile byte
    // offsets cached while the cursor stays on one tile.
    uint32_t lk = 0, ls = 0, cached = ~0u;
    const uint8_t *a = nullptr, *w0 = nullptr;
    uint32_t o_a = 0, o_sa = 0, o_w = 0, o_sw = 0;
    // Steps past a tile's end (and past the last tile) reload a valid step
    // with A masked to zero.  Each load is one instruction on (uniform base,
    // 32-bit lane offset).
    auto load = [&](Raw& rw) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t k = min(lk, sc.count - 1);
      if (k != cached) {  // uniform
        cached = k;
        const Tile tl = tile_of(k);
        a = g.a + tl.z * g.a_batch;
        w0 = g.w[0] + tl.z * g.w_batch;
        const uint32_t quad = min(tl.row0 / 4 + (r >> 2), g.quads - 1);
        o_a = quad * a_row + (r & 3) * 32;
        o_sa = quad * a_row + 128;
        const uint32_t grp = min(tl.col0 / 8 + (t >> 3), g.groups - 1);
        o_w = grp * word_row + cl * 16;
        o_sw = grp * word_row + 128 + (cl & 4);
      }
      const bool live = lk < sc.count && ls < steps;
      const uint32_t step = min(ls, steps - 1);
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
      rw.mask = (!live || (h && 2 * step + 1 >= nblocks)) ? 0u : 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[i] = v0[i];
        rw.a[4 + i] = v1[i];
        rw.w[0][i] = x0[i];
        rw.w[1][i] = x1[i];
      }
      if (++ls == iters) {
        ls = 0;
        ++lk;
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

    // Convert cursor: the tile of the step being staged, for its
    // out-of-window flag, raised with the tile's last step.
    uint32_t ck = 0, cs = 0;
    bool bad = false;
    auto stage = [&](const Raw& rw, Stage& st) {
      bad |= store(rw, st) && ck < sc.count;
      if (++cs == iters) {
        if (bad) lds_unsafe[ck & 1] = 1;
        bad = false;
        cs = 0;
        ++ck;
      }
    };
    // Ring of kU register sets, slot j % kU holding global step j: iteration
    // u stages step u + 2 and refills its slot with step u + 2 + kU.
    Raw ring[kU];
    if (t < 2) lds_unsafe[t] = 0;
#pragma unroll
    for (int i = 0; i < kU; ++i) load(ring[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      stage(ring[i], lds_stage[i]);
      load(ring[i]);
    }
    __syncthreads();  // global steps 0 and 1 staged
    __syncthreads();  // the consumers hold step 0: its stage may be refilled
    for (uint32_t u = 0; u < sc.count * iters; u += kU) {
#pragma unroll
      for (int i = 0; i < kU; ++i) {  // global iteration u + i stages step u + i + 2
        stage(ring[(i + 2) % kU], lds_stage[i % 2]);
        load(ring[(i + 2) % kU]);
        __syncthreads();
      }
    }
    return;
  }

  // Consumer wave cw: rows 64 * (cw % 2) .. + 64 (m-tiles 2 wm, 2 wm + 1),
  // columns 128 * (cw / 2) .. + 128 (n-tiles 4 wn .. 4 wn + 3).  MFMA tile
  // j = mi * 4 + nj.  Output r of tile j of this lane is tile row
  // 32 (2 wm + j / 4) + 4 (lane / 32) + 8 (r / 4) + r % 4, column
  // 32 (4 wn + j % 4) + lane % 32.
  const uint32_t tid = threadIdx.x - kP, lane = tid & 63;
  const uint32_t cw = __builtin_amdgcn_readfirstlane(tid >> 6), wm = cw & 1, wn = cw >> 1;
  auto trow = [&](uint32_t mi, uint32_t r) {
    return (2 * wm + mi) * 32 + 4 * (lane >> 5) + 8 * (r / 4) + (r & 3);
  };
  auto tcol = [&](uint32_t nj) { return (4 * wn + nj) * 32 + (lane & 31); };

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
  f32x16 acc[8];
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
  // Iteration: read the next step (stage st) into `nxt`, run this step
  // from `cur`, then the barrier (which waits for the reads).  The
  // accumulators are anchored on both sides of the barrier (the empty asm
  // emits nothing), so the compiler neither sinks the matrix work past it
  // nor hoists the next step's above it.
  auto iteration = [&](const Ops& cur, Ops& nxt, int st) {
    __builtin_amdgcn_sched_barrier(0);
    read(lds_stage[st], nxt);
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
  __syncthreads();  // global steps 0 and 1 staged; the flags are clear
  read(lds_stage[0], x);
  __syncthreads();  // step 0 is in registers before producers refill its stage
  float* const xp = lds_xpose[cw];
  for (uint32_t k = 0; k < sc.count; ++k) {
    const Tile tl = tile_of(k);
    const uint8_t* a = g.a + tl.z * g.a_batch;
    const uint8_t* w0 = g.w[0] + tl.z * g.w_batch;
    uint32_t* c = g.c + tl.z * g.c_batch;
    bool init_unsafe = false;  // this wave's outputs start from an exponent > 252
    if (g.acc) {  // uniform: start from C
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t row = tl.row0 + trow(j / 4, r), col = tl.col0 + tcol(j % 4);
          uint32_t init = 0;
          if (row < g.m && col < g.n) {
            init = c[(size_t)row * g.n + col];
            init_unsafe |= ExpField(init) > 252u;
          }
          acc[j][r] = __uint_as_float(init);
        }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32x16{};
    }
    for (uint32_t s = 0; s < iters; s += kU) {
#pragma unroll
      for (int i = 0; i < kU; i += 2) {
        iteration(x, y, 1);
        iteration(y, x, 0);
      }
    }
    // Epilogue, this wave's 64 x 128 outputs only.
    const bool slow = __builtin_amdgcn_readfirstlane(
        lds_unsafe[k & 1] != 0 || __builtin_amdgcn_ballot_w64(init_unsafe) != 0);
    if (tid == 0) lds_unsafe[(k + 1) & 1] = 0;
    if (slow) {  // a scale byte or an initial C left the window: every output exactly
      for (uint32_t j = 0; j < 8; ++j)
        for (uint32_t r = 0; r < 16; ++r) {
          const uint32_t row = tl.row0 + trow(j / 4, r), col = tl.col0 + tcol(j % 4);
          if (row >= g.m || col >= g.n) continue;
          uint32_t* out = c + (size_t)row * g.n + col;
          *out = SlowLinear(g, a, w0, w0, g.acc ? *out : 0u, row, col);
        }
      continue;
    }
    // Each MFMA tile goes through the wave's LDS block: output r of lane l
    // (block row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32) is written at
    // physical row p(row) = row ^ ((row >> 2) & 1), so the two half-waves of a
    // write (rows row and row + 4) and the 16-lane groups of a read (two
    // physical rows) use disjoint banks; read q gives lane l the 4 columns
    // 4 (l % 8) .. of physical row l / 8 + 8 q.  LDS accesses of one wave
    // execute in order, so a wave-scope fence orders the lanes' accesses.
    // Adding +0 maps -0 to +0 (and a denormal sum, in the kernel's
    // flush-to-zero mode, to +0).  (The lane index is read again here: held
    // over the K loop, its addresses spilled.)
    const uint32_t ln = LaneNow();
    Unroll<8>([&](auto jj) {
      constexpr int kJ = decltype(jj)::value;
      const uint32_t lane = ln;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t row = 8 * (r / 4) + 4 * (lane >> 5) + (r & 3);
        xp[(row ^ ((row >> 2) & 1)) * 32 + (lane & 31)] = acc[kJ][r] + 0.0f;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float4* rd = reinterpret_cast<const float4*>(xp) + (lane >> 3) * 8 + (lane & 7);
      const float4 v0 = rd[0], v1 = rd[64], v2 = rd[128], v3 = rd[192];  // q = 0 .. 3
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // n is a multiple of 8: the lane's 4 columns are all in or all out
      const uint32_t col = tl.col0 + (4 * wn + kJ % 4) * 32 + 4 * (lane & 7);
      const uint32_t prow = lane >> 3, row = tl.row0 + (2 * wm + kJ / 4) * 32 + (prow ^ ((prow >> 2) & 1));
      float4* out = reinterpret_cast<float4*>(c + (size_t)row * g.n + col);
      const size_t q_step = (size_t)2 * g.n;  // 8 rows, in float4 units
      if (col < g.n) {
        if (row < g.m) out[0] = v0;
        if (row + 8 < g.m) out[q_step] = v1;
        if (row + 16 < g.m) out[2 * q_step] = v2;
        if (row + 24 < g.m) out[3 * q_step] = v3;
      }
    });
  }
}

}  // namespace

bool Fp4Eligible(const GemmArgs& args, uint32_t tile_rows) {
  // C is stored 16 bytes at a time
  const bool aligned = reinterpret_cast<uintptr_t>(args.c) % 16 == 0 && args.c_batch % 4 == 0;
  return !args.w_panels && args.n_planes == 1 && args.modes[0] == kModeFp4 && tile_rows == kBM &&
         aligned &&
         args.n_ops == 0 && args.q_out == nullptr && args.ws == nullptr && args.splits <= 1;
}

hipError_t LaunchFp4(const GemmArgs& args, hipStream_t stream) {
  // one workgroup per CU (a multiple of the 8 XCDs), or one per tile
  static int cus[64] = {};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (cus[dev] == 0) {
    int n = 0;
    err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return err;
    cus[dev] = n / (int)kXcds * (int)kXcds;
    if (cus[dev] == 0) cus[dev] = (int)kXcds;
  }
  const uint32_t tiles = args.gx * args.gy * args.gz;
  const dim3 grid(tiles < (uint32_t)cus[dev] ? tiles : (uint32_t)cus[dev]), block(512);
  if (args.n_pieces > 1) hipLaunchKernelGGL((Fp4Kernel<true>), grid, block, 0, stream, args);
  else hipLaunchKernelGGL((Fp4Kernel<false>), grid, block, 0, stream, args);
  return hipGetLastError();
}

}  // namespace hb

// Streaming MXFP4 kernel over weight panels (HB_LINEAR_FAST | HB_LINEAR_PANELS,
// plain layers of more than 64 rows): tiles of 128 rows x 320 columns (five
// 64-column panels), 4 waves per workgroup, one workgroup per CU.
//
// Arithmetic as in the other fast kernels (hb_fast4.hip): A as two exact FP6
// E2M3 planes, h = fp6(q / 32) with scale byte ea - 1 and r / 2 = (q - 32 h) / 2
// with ea - 5; W's E2M1 codes and E8M0 bytes untouched, in
// v_mfma_scale_f32_32x32x64_f8f6f4 (tools/iss/gemm_array.cpp:84-110).
//
// Data flow.  Every operand byte of the K loop reaches LDS by the CU's
// direct global-to-LDS loads (global_load_lds_dwordx4 / _dword), through a
// ring of kD steps: per step, each wave's A rows (its 32 rows x 2 blocks: 32
// code bytes and the scale dword per lane) and the tile's W chunks (5
// panels x 2176 bytes, spread over the 4 waves, 16 bytes per lane).  The
// loads hold no registers while in flight, so kD - 1 = 5 steps (about 100 KB
// per CU) stream ahead of the matrix cores.
//   Wave w owns rows 32w..32w+31 of the tile (one m-tile) and all 10
// n-tiles: it converts only its own A rows (one (row, block) per lane per
// step), so converted A never passes through LDS; only W is shared, read
// by each wave from the ring (its B operands, 1 KiB per n-tile).  The
// conversion of step u + 1 runs on the VALU while the matrix cores run
// step u.
//
// Synchronisation: one barrier per step.  In iteration u a wave waits for
// its own loads of step u + 1 (the load counter, counted by hand: the loads
// are issued from inline asm, which the compiler's own waits do not see),
// then the barrier (every wave's loads of steps u, u + 1 are in LDS, and
// every wave has finished reading ring slot u - 1), then it refills slot
// u - 1 with step u + kD - 1.  Loads past the last step repeat a valid
// address, so every wave issues the same number of loads every step.
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

constexpr int kWaves = 4;                              // one per SIMD
constexpr int kBM = 32 * kWaves;                       // tile rows
constexpr int kTP = 5;                                 // panels per tile
constexpr int kBN = kTP * (int)kPanelCols;             // tile columns
constexpr int kNT = 2 * kTP;                           // 32-column n-tiles
constexpr int kD = 6;                                  // ring depth, steps
constexpr uint32_t kChunkPieces = kPanelChunk / 16;    // 136 16-byte pieces per chunk
constexpr uint32_t kPieces = kTP * kChunkPieces;       // W pieces per step
constexpr int kWRounds = (kPieces + 255) / 256;        // W loads per wave per step
constexpr uint32_t kABytes = 2304;                     // per wave: 2 x 1 KiB codes, 256 B scales
constexpr uint32_t kSlotA = kWaves * kABytes;
constexpr uint32_t kSlotW = kWRounds * 256 * 16;
constexpr uint32_t kSlot = kSlotA + kSlotW;
constexpr int kOps = 3 + kWRounds;                     // loads per wave per step
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;
static_assert((kD - 3) * kOps < 64, "load counter range");
static_assert(kSlot % 16 == 0, "16-byte slots");

template <typename Fn, int... kI>
__device__ __forceinline__ void UnrollImpl(Fn&& f, std::integer_sequence<int, kI...>) {
  (f(std::integral_constant<int, kI>{}), ...);
}
template <int kN, typename Fn>
__device__ __forceinline__ void Unroll(Fn&& f) {
  UnrollImpl(f, std::make_integer_sequence<int, kN>{});
}

// Direct loads into LDS: lane l's 16 (or 4) bytes at base + voff land at LDS
// byte lds + 16 l (4 l).  lds is wave-uniform (M0).
// (base and lds are made wave-uniform values in scalar registers.)
__device__ __forceinline__ uint64_t UniformAddress(const uint8_t* p) {
  // (the builtin returns int: widen through uint32_t, not by sign extension)
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (hi << 32) | lo;
}
__device__ __forceinline__ void Dma16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(UniformAddress(base)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void Dma4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(UniformAddress(base)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// Wait until at most kN of this wave's vector memory operations are
// outstanding (s_waitcnt vmcnt(kN), the other counters left alone).
template <int kN>
__device__ __forceinline__ void WaitVm() {
  __builtin_amdgcn_s_waitcnt((kN & 15) | ((kN >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void WaitLds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// 32 int8 (8 dwords, K order) -> FP6 E2M3 codes of h = q/32 rounded and of
// (q - 32h)/2, both exact (hb_fast4.hip).
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

struct Schedule {
  uint32_t first, stride, count;
};
__device__ __forceinline__ Schedule TilesOf(uint32_t total) {
  const uint32_t b = blockIdx.x, grid = gridDim.x;
  Schedule sc;
  if (grid >= total) {
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

// One step's operands for this lane: the B operands of the tile's 10
// n-tiles (t: panel t / 2, columns 32 (t % 2) ..) with the panels' scale
// bytes (bytes 0, 1 of sw[q]: n-tiles 2q, 2q + 1), and the converted A
// planes h, r/2 with their scale bytes (ea - 1 | (ea - 5) << 8); abad: the
// lane's A scale byte left the window.
struct Ops {
  u32x4 b[kNT];
  uint32_t sw[kTP];
  u32x6 h, r;
  int sa;
  uint32_t abad;
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void StreamKernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_ring[kD * kSlot];
  __shared__ __attribute__((aligned(16))) float lds_xpose[kWaves][32 * 32];

  const Schedule sc = TilesOf(g.gx * g.gy * g.gz);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t steps = g.w_steps, nblocks = g.kb_total;
  const uint32_t total = sc.count * steps;
  const uint32_t n_panels = (g.n + kPanelCols - 1) / kPanelCols;
  const uint32_t ring = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_ring));

  struct Tile {
    uint32_t row0, col0, p0, z;
  };
  auto tile_of = [&](uint32_t k) __attribute__((always_inline)) {
    const uint32_t t = sc.first + min(k, sc.count - 1) * sc.stride;
    Tile tl;
    const uint32_t x = t % g.gx;
    tl.col0 = x * kBN;
    tl.p0 = x * kTP;
    tl.row0 = ((t / g.gx) % g.gy) * kBM;
    tl.z = t / (g.gx * g.gy);
    return tl;
  };

  // Per-lane constants of the loads.  A: row r of the tile, block h of the
  // step.  W: piece i = (round * 4 + w) * 64 + lane of the step's kPieces
  // (panel i / 136 of the tile, byte (i % 136) * 16 of its chunk); pieces
  // past kPieces (padding of the last round) repeat piece 0's panel.
  const uint32_t r = w * 32 + (lane & 31), h = lane >> 5;
  uint32_t wq[kWRounds], woff[kWRounds];
#pragma unroll
  for (int k = 0; k < kWRounds; ++k) {
    const uint32_t i = (k * kWaves + w) * 64 + lane;
    wq[k] = i < kPieces ? i / kChunkPieces : 0u;
    woff[k] = i < kPieces ? (i % kChunkPieces) * 16 : 0u;
  }

  // Load cursor: the next global step to load (tile dk, step ds, slot
  // dslot), with the tile's bases cached.  Past the last step: the last
  // step again, so every wave issues kOps loads per step.
  uint32_t dk = 0, ds = 0, dslot = 0, dcached = ~0u;
  const uint8_t* da = nullptr;
  const uint8_t* dw = nullptr;
  uint32_t da_lane = 0, dw_lane[kWRounds];
  auto issue_next = [&]() __attribute__((always_inline)) {
    const uint32_t k = min(dk, sc.count - 1);
    if (k != dcached) {  // uniform: once per tile
      dcached = k;
      const Tile tl = tile_of(k);
      da = g.a + tl.z * g.a_batch;
      dw = g.w[0] + tl.z * g.w_batch;
      const uint32_t quad = min(tl.row0 / 4 + (r >> 2), g.quads - 1);
      da_lane = quad * g.a_row * kDdrWord + (r & 3) * 32;
#pragma unroll
      for (int k2 = 0; k2 < kWRounds; ++k2)
        dw_lane[k2] = min(tl.p0 + wq[k2], n_panels - 1) * steps * kPanelChunk + woff[k2];
    }
    const uint32_t s = dk < sc.count ? ds : steps - 1;
    const uint32_t blk = min(2 * s + h, nblocks - 1);
    const uint32_t slot = ring + dslot * kSlot;
    const uint32_t abase = __builtin_amdgcn_readfirstlane(slot + w * kABytes);
    const uint32_t aw = da_lane + blk * kDdrWord;
    Dma16(da, aw, abase);
    Dma16(da, aw + 16, abase + 1024);
    Dma4(da, aw + 128 - (r & 3) * 32, abase + 2048);
#pragma unroll
    for (int k2 = 0; k2 < kWRounds; ++k2)
      Dma16(dw, dw_lane[k2] + s * kPanelChunk,
            __builtin_amdgcn_readfirstlane(slot + kSlotA + (k2 * kWaves + w) * 1024));
    if (++ds == steps) {
      ds = 0;
      ++dk;
    }
    dslot = dslot + 1 == kD ? 0u : dslot + 1;
  };

  // Read step (k, s)'s operands from ring slot `slot`: the B operands and
  // W scale dwords, and this lane's A (converted).
  auto fetch = [&](Ops& o, uint32_t slot, uint32_t k, uint32_t s) __attribute__((always_inline)) {
    const uint8_t* base = lds_ring + slot * kSlot;
    const uint8_t* wslot = base + kSlotA;
#pragma unroll
    for (int q = 0; q < kTP; ++q) {
      const uint8_t* chunk = wslot + q * kPanelChunk;
      o.sw[q] = *reinterpret_cast<const uint32_t*>(chunk + kPanelScales + 4 * (lane >> 1));
#pragma unroll
      for (int t = 0; t < 2; ++t)
        o.b[2 * q + t] = *reinterpret_cast<const u32x4*>(
            chunk + ((lane >> 5) * kPanelCols + t * 32 + (lane & 31)) * 16);
    }
    const uint8_t* abuf = base + w * kABytes;
    const u32x4 x0 = *reinterpret_cast<const u32x4*>(abuf + lane * 16);
    const u32x4 x1 = *reinterpret_cast<const u32x4*>(abuf + 1024 + lane * 16);
    const uint32_t sd = *reinterpret_cast<const uint32_t*>(abuf + 2048 + lane * 4);
    const bool live = k < sc.count && 2 * s + h < nblocks;
    const uint32_t x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    SplitA(x, live ? 0xFFFFFFFFu : 0u, o.h, o.r);
    const uint32_t ea = __builtin_amdgcn_ubfe(sd, 8 * (r & 3), 8);
    o.sa = (int)(((ea - 5u) << 8) | ((ea - 1u) & 0xFFu));
    o.abad = live && ea - kSafeLo > kSafeHi - kSafeLo ? 1u : 0u;
  };

  float* const xp = lds_xpose[w];
  f32x16 acc[kNT];
  uint32_t bad = 0;        // this wave's tile saw a scale byte outside the window
  bool init_unsafe = false;
  Tile tl{};
  uint32_t row_w = 0, live_nt = 0;
  // Start tile k: its geometry and the accumulators (+0, or C).
  auto begin_tile = [&](uint32_t k) __attribute__((always_inline)) {
    tl = tile_of(k);
    row_w = tl.row0 + w * 32;
    live_nt = min((uint32_t)kNT, (g.n - min(tl.col0, g.n) + 31) / 32);
    bad = 0;
    init_unsafe = false;
    if (g.acc) {  // uniform: start from C (a compiler-visible load: drain the ring's first)
      WaitVm<0>();
      const uint32_t* c = g.c + tl.z * g.c_batch;
#pragma unroll
      for (int j = 0; j < kNT; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t row = row_w + 4 * (lane >> 5) + 8 * (e / 4) + (e & 3);
          const uint32_t col = tl.col0 + j * 32 + (lane & 31);
          uint32_t init = 0;
          if (row < g.m && col < g.n) {
            init = c[(size_t)row * g.n + col];
            init_unsafe |= ExpField(init) > 252u;
          }
          acc[j][e] = __uint_as_float(init);
        }
    } else {
#pragma unroll
      for (int j = 0; j < kNT; ++j) acc[j] = f32x16{};
    }
  };
  // Finish the current tile: exact recompute if flagged, else store C.
  auto end_tile = [&]() __attribute__((always_inline)) {
    const uint8_t* a = g.a + tl.z * g.a_batch;
    const uint8_t* w0 = g.w[0] + tl.z * g.w_batch;
    uint32_t* c = g.c + tl.z * g.c_batch;
    const bool slow = __builtin_amdgcn_readfirstlane(
        __builtin_amdgcn_ballot_w64(init_unsafe || bad != 0) != 0);
    if (slow) {  // a scale byte or an initial C left the window: every output exactly
      WaitVm<0>();
      for (uint32_t j = 0; j < kNT; ++j)
        for (uint32_t e = 0; e < 16; ++e) {
          const uint32_t row = row_w + 4 * (lane >> 5) + 8 * (e / 4) + (e & 3);
          const uint32_t col = tl.col0 + j * 32 + (lane & 31);
          if (row >= g.m || col >= g.n) continue;
          uint32_t* out = c + (size_t)row * g.n + col;
          *out = SlowLinear(g, a, w0, w0, g.acc ? *out : 0u, row, col);
        }
      return;
    }
    // Each MFMA tile through the wave's LDS block, stored as 16-byte rows
    // of 4 columns (rows at row ^ ((row >> 2) & 1): conflict-free writes and
    // reads); +0 maps -0 (and a flushed denormal) to +0.
    Unroll<kNT>([&](auto jj) {
      constexpr int kJ = decltype(jj)::value;
      if ((uint32_t)kJ >= live_nt) return;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row = 8 * (e / 4) + 4 * (lane >> 5) + (e & 3);
        xp[(row ^ ((row >> 2) & 1)) * 32 + (lane & 31)] = acc[kJ][e] + 0.0f;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float4* rd = reinterpret_cast<const float4*>(xp) + (lane >> 3) * 8 + (lane & 7);
      const float4 v0 = rd[0], v1 = rd[64], v2 = rd[128], v3 = rd[192];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t col = tl.col0 + kJ * 32 + 4 * (lane & 7);
      const uint32_t prow = lane >> 3;
      const uint32_t row = row_w + (prow ^ ((prow >> 2) & 1));
      float4* out = reinterpret_cast<float4*>(c + (size_t)row * g.n + col);
      const size_t q_step = (size_t)2 * g.n;  // 8 rows, in float4 units
      if (col < g.n) {
        if (row < g.m) out[0] = v0;
        if (row + 8 < g.m) out[q_step] = v1;
        if (row + 16 < g.m) out[2 * q_step] = v2;
        if (row + 24 < g.m) out[3 * q_step] = v3;
      }
    });
  };

  // Prologue: steps 0 .. kD - 2 in flight; steps 0, 1 landed; step 0 read.
#pragma unroll
  for (int v = 0; v < kD - 1; ++v) issue_next();
  WaitVm<(kD - 3) * kOps>();
  __syncthreads();
  Ops o0, o1;
  fetch(o0, 0, 0, 0);
  begin_tile(0);

  // Iteration u (tile k, step s, ring slot u % kD): wait for this wave's
  // loads of step u + 1, barrier, refill slot u - 1 with step u + kD - 1,
  // read step u + 1's operands into the other register set while the
  // matrix cores run step u.
  uint32_t u = 0, k = 0, s = 0, slot = 0;
  auto iteration = [&](const Ops& cur, Ops& nxt) __attribute__((always_inline)) {
    WaitVm<(kD - 3) * kOps>();
    WaitLds();
    __syncthreads();
    issue_next();
    const uint32_t nslot = slot + 1 == kD ? 0u : slot + 1;
    const bool wrap = s + 1 == steps;
    fetch(nxt, nslot, wrap ? k + 1 : k, wrap ? 0u : s + 1);
    // the window checks (a panel past the layer repeats the last one's bytes)
    uint32_t wb = cur.abad;
#pragma unroll
    for (int q = 0; q < kTP; ++q) {
      const uint32_t sq = cur.sw[q] >> (16 * (lane & 1));
      wb |= (uint32_t)((sq & 0xFFu) - kSafeLo > kSafeHi - kSafeLo) |
            (uint32_t)(((sq >> 8) & 0xFFu) - kSafeLo > kSafeHi - kSafeLo);
    }
    bad |= wb;
    const i32x8 ah = {(int)cur.h[0], (int)cur.h[1], (int)cur.h[2], (int)cur.h[3],
                      (int)cur.h[4], (int)cur.h[5], 0, 0};
    const i32x8 ar = {(int)cur.r[0], (int)cur.r[1], (int)cur.r[2], (int)cur.r[3],
                      (int)cur.r[4], (int)cur.r[5], 0, 0};
    // plane h over the n-tiles, then plane r (branch-free: n-tiles past the
    // layer compute outputs that are not stored)
    Unroll<kNT>([&](auto t_c) {
      constexpr int kT = decltype(t_c)::value;
      const i32x8 bt = {(int)cur.b[kT][0], (int)cur.b[kT][1], (int)cur.b[kT][2], (int)cur.b[kT][3],
                        0, 0, 0, 0};
      acc[kT] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          ah, bt, acc[kT], 2, 4, 0, cur.sa, kT % 2,
          (int)(cur.sw[kT / 2] >> (16 * (lane & 1))));
    });
    Unroll<kNT>([&](auto t_c) {
      constexpr int kT = decltype(t_c)::value;
      const i32x8 bt = {(int)cur.b[kT][0], (int)cur.b[kT][1], (int)cur.b[kT][2], (int)cur.b[kT][3],
                        0, 0, 0, 0};
      acc[kT] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          ar, bt, acc[kT], 2, 4, 1, cur.sa, kT % 2,
          (int)(cur.sw[kT / 2] >> (16 * (lane & 1))));
    });
    ++u;
    slot = nslot;
    if (wrap) {  // uniform: the tile's last step
      end_tile();
      s = 0;
      if (++k < sc.count) begin_tile(k);
    } else {
      ++s;
    }
  };
  while (u < total) {
    iteration(o0, o1);
    if (u >= total) break;
    iteration(o1, o0);
  }
  WaitVm<0>();  // no load into LDS outlives the workgroup
}

}  // namespace

bool StreamEligible(const GemmArgs& args) {
  // one piece over every block in order
  // C is stored, and A and W are loaded, 16 bytes at a time
  const bool aligned = reinterpret_cast<uintptr_t>(args.c) % 16 == 0 && args.c_batch % 4 == 0 &&
                       reinterpret_cast<uintptr_t>(args.a) % 16 == 0 && args.a_batch % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(args.w[0]) % 16 == 0 && args.w_batch % 16 == 0;
  return args.w_panels && args.n_planes == 1 && args.modes[0] == kModeFp4 && aligned &&
         args.n_ops == 0 && args.q_out == nullptr && args.n_pieces == 1 &&
         args.piece_off[0] == 0 && args.piece_kb[0] == args.kb_total && args.quads * 4 > 64;
}

hipError_t LaunchStream(const GemmArgs& in, uint32_t batch, hipStream_t stream) {
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
  GemmArgs args = in;
  args.gx = (args.n + kBN - 1) / kBN;
  args.gy = (args.quads * 4 + kBM - 1) / kBM;
  args.gz = batch;
  const uint32_t tiles = args.gx * args.gy * args.gz;
  const dim3 grid(tiles < (uint32_t)cus[dev] ? tiles : (uint32_t)cus[dev]), block(256);
  hipLaunchKernelGGL(StreamKernel, grid, block, 0, stream, args);
  return hipGetLastError();
}

}  // namespace hb

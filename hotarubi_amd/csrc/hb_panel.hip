// Weight panels: the GPU-native layout of a weight plane, and the streaming
// MXFP4 kernel over it (HB_LINEAR_FAST | HB_LINEAR_PANELS).
//
// Layout (hb_internal.h, kPanelChunk): a plane of n columns x kb_total
// blocks becomes ceil(n / 64) panels of 64 columns; a panel is
// ceil(kb_total / 2) consecutive 2176-byte chunks, one per K-step of two
// blocks: 2048 bytes of 16-byte column-blocks (block b of the step, column
// c: at (b * 64 + c) * 16, the DDR word's 16 bytes of that column
// unchanged), then the 128 scale bytes (at 2048 + 2 (b * 32 + c % 32) +
// c / 32).  Chunk order is panel-major, so one panel's K range is one
// contiguous run, and the lane order of a chunk is the B operand order of
// v_mfma_scale_f32_32x32x64_f8f6f4: lane l of n-tile t holds column
// 32 t + l % 32, block l / 32, so a wave loads one n-tile's operands as one
// contiguous KiB and its two n-tiles' scale bytes as one 16-bit load.
// hb_pack_weights / hb_unpack_weights convert from and to the DDR words
// (tools/compiler/tensors.cpp:66-90 PackWbuf), bit for bit.
//
// Streaming kernel.  Same arithmetic as the other fast kernels (A as two
// exact FP6 E2M3 planes h = fp6(q / 32), r / 2 = (q - 32 h) / 2 with scale
// bytes ea - 1, ea - 5; W's E2M1 codes and E8M0 bytes untouched; see
// hb_fast4.hip), a different data flow:
//   4 producer waves convert A: lane (row, block) per step, as in
//     hb_fast4.hip, into one of 3 LDS stages;
//   4 consumer waves each own one 64-column panel of the tile (all 128
//     rows: 4 m-tiles x 2 n-tiles, 128 accumulators) and stream its chunks
//     from HBM straight into their B operand registers through a ring of
//     kD steps: no W byte passes through LDS, and each wave's loads are one
//     sequential stream of 2176-byte chunks.
// One barrier per step: in iteration u the consumers read stage u % 3 and
// the producers write stage (u + 2) % 3 (step u + 2), which the consumers
// last read in iteration u - 1.  Persistent over tiles (one workgroup per
// CU, contiguous tile ranges per XCD); both rings stream across tile ends.
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

constexpr int kBM = 128, kTilePanels = 4, kBN = kTilePanels * (int)kPanelCols;
constexpr int kP = 256;     // producer threads
constexpr int kU = 4;       // producer raw ring = consumer W ring = unroll
constexpr int kStages = 3;  // LDS stages of converted A
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;

struct StageA {
  uint4 a[4][64][3];   // [m-tile][lane]: h codes (dwords 0-5), r/2 codes (6-11)
  uint32_t sa[2][64];  // [m-tile / 2][lane]: byte (m-tile % 2) * 2 + plane
};

template <typename Fn, int... kI>
__device__ __forceinline__ void UnrollImpl(Fn&& f, std::integer_sequence<int, kI...>) {
  (f(std::integral_constant<int, kI>{}), ...);
}
template <int kN, typename Fn>
__device__ __forceinline__ void Unroll(Fn&& f) {
  UnrollImpl(f, std::make_integer_sequence<int, kN>{});
}

// 32 int8 (8 dwords, K order) -> FP6 E2M3 codes of h = q/32 rounded and of
// (q - 32h)/2, both exact (as in hb_fast4.hip).
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
  const u32x6 h = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(q, 32.0f);
  const f16x32 hv = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6(h, 1.0f);
  const f16x32 m32 = (_Float16)-32.0f;
  const f16x32 r = __builtin_elementwise_fma(hv, m32, q);
  const u32x6 lo = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(r, 2.0f);
  out[0] = uint4{h[0], h[1], h[2], h[3]};
  out[1] = uint4{h[4], h[5], lo[0], lo[1]};
  out[2] = uint4{lo[2], lo[3], lo[4], lo[5]};
}

// Tiles of one workgroup: first + k * stride, k < count (contiguous ranges
// per XCD; the hardware deals workgroups round-robin over the 8 XCDs).
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

struct RawA {
  uint32_t a[8];
  uint32_t sa;
  uint32_t mask;  // 0xFFFFFFFF, or 0 for a step past the tile's end
};

struct RawW {
  u32x4 b[2];   // n-tiles 0, 1
  uint32_t sw;  // the dword holding their scale bytes (at bit scale_shift)
};

__global__ __launch_bounds__(512) void PanelKernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) StageA lds_stage[kStages];
  __shared__ __attribute__((aligned(16))) float lds_xpose[4][32 * 32];  // one per consumer
  __shared__ uint32_t lds_unsafe[2];

  const Schedule sc = TilesOf(g.gx * g.gy * g.gz);
  const bool consumer = __builtin_amdgcn_readfirstlane(threadIdx.x >= kP);
  const uint32_t nblocks = g.kb_total, steps = g.w_steps;
  const uint32_t iters = (steps + kU - 1) / kU * kU;  // per tile, both roles
  const uint32_t total = sc.count * iters;
  const uint32_t n_panels = (g.n + kPanelCols - 1) / kPanelCols;

  struct Tile {
    uint32_t row0, col0, z;
  };
  auto tile_of = [&](uint32_t k) {
    const uint32_t t = sc.first + min(k, sc.count - 1) * sc.stride;
    Tile tl;
    tl.col0 = (t % g.gx) * kBN;
    tl.row0 = ((t / g.gx) % g.gy) * kBM;
    tl.z = t / (g.gx * g.gy);
    return tl;
  };

  if (!consumer) {
    const uint32_t t = threadIdx.x, lane = t & 63, mt = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t h = lane >> 5;  // the lane's block within the step
    const uint32_t a_row = g.a_row * kDdrWord;
    const uint32_t r = mt * 32 + (lane & 31);
    // Load cursor: global step u = tile * iters + step.
    uint32_t lk = 0, ls = 0, cached = ~0u;
    const uint8_t* a = nullptr;
    uint32_t o_a = 0, o_sa = 0;
    auto load = [&](RawA& rw) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t k = min(lk, sc.count - 1);
      if (k != cached) {  // uniform
        cached = k;
        const Tile tl = tile_of(k);
        a = g.a + tl.z * g.a_batch;
        const uint32_t quad = min(tl.row0 / 4 + (r >> 2), g.quads - 1);
        o_a = quad * a_row + (r & 3) * 32;
        o_sa = quad * a_row + 128;
      }
      const bool live = lk < sc.count && ls < steps && 2 * ls + h < nblocks;
      const uint32_t blk = min(2 * min(ls, steps - 1) + h, nblocks - 1);
      const uint32_t ub = blk * kDdrWord;
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(a + (o_a + ub));
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(a + (o_a + ub) + 16);
      rw.sa = *reinterpret_cast<const uint32_t*>(a + (o_sa + ub));
      rw.mask = live ? 0xFFFFFFFFu : 0u;  // applied at conversion time
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[i] = v0[i];
        rw.a[4 + i] = v1[i];
      }
      if (++ls == iters) {
        ls = 0;
        ++lk;
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // Convert cursor, for the tile's out-of-window flag (raised with the
    // tile's last step, at least two barriers before the consumers read it).
    uint32_t ck = 0, cs = 0;
    bool bad = false;
    auto stage = [&](const RawA& rw, StageA& st) {
      uint4 codes[3];
      SplitA(rw.a, rw.mask, codes);
#pragma unroll
      for (int i = 0; i < 3; ++i) st.a[mt][lane][i] = codes[i];
      const uint32_t ea = __builtin_amdgcn_ubfe(rw.sa, 8 * (lane & 3), 8);  // row r % 4
      reinterpret_cast<uint16_t*>(&st.sa[mt >> 1][lane])[mt & 1] =
          (uint16_t)(((ea - 5u) << 8) | ((ea - 1u) & 0xFFu));
      bad |= rw.mask != 0 && ea - kSafeLo > kSafeHi - kSafeLo && ck < sc.count;
      if (++cs == iters) {
        if (bad) lds_unsafe[ck & 1] = 1;
        bad = false;
        cs = 0;
        ++ck;
      }
    };
    RawA ring[kU];
    if (t < 2) lds_unsafe[t] = 0;
#pragma unroll
    for (int i = 0; i < kU; ++i) load(ring[i]);
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // steps 0, 1 -> stages 0, 1
      stage(ring[i], lds_stage[i]);
      load(ring[i]);
    }
    __syncthreads();  // B0: steps 0 and 1 staged, flags clear
    // iteration u stages step u + 2 (ring slot (u + 2) % kU) into stage
    // (u + 2) % 3 and refills the slot with step u + 2 + kU (total is a
    // multiple of kU)
    for (uint32_t u0 = 0; u0 < total; u0 += kU) {
#pragma unroll
      for (int i = 0; i < kU; ++i) {
        stage(ring[(i + 2) % kU], lds_stage[(u0 + i + 2) % kStages]);
        load(ring[(i + 2) % kU]);
        __syncthreads();
      }
    }
    return;
  }

  // Consumer wave cw: panel cw of the tile, all 128 rows.  MFMA tile
  // j = mi * 2 + nj; output r of tile j of this lane is tile row
  // 32 mi + 4 (lane / 32) + 8 (r / 4) + r % 4, column 64 cw + 32 nj + lane % 32.
  const uint32_t tid = threadIdx.x - kP, lane = tid & 63;
  const uint32_t cw = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The lane's two scale bytes are bytes 2 (lane % 2), +1 of the aligned
  // dword at 2048 + 4 (lane / 2); a 16-bit load would be re-extended after
  // the ring's loop edge, which makes the compiler wait for it there.
  const uint32_t lane_codes = ((lane >> 5) * 64 + (lane & 31)) * 16;
  const uint32_t lane_scale = 2048 + 4 * (lane >> 1), scale_shift = 16 * (lane & 1);

  // W cursor: global step u; per tile, the panel's chunk 0.
  uint32_t wk = 0, ws = 0, wcached = ~0u;
  const uint8_t* wpanel = nullptr;
  auto wload = [&](RawW& rw) {
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t k = min(wk, sc.count - 1);
    if (k != wcached) {  // uniform
      wcached = k;
      const Tile tl = tile_of(k);
      const uint32_t panel = min(tl.col0 / kPanelCols + cw, n_panels - 1);
      wpanel = g.w[0] + tl.z * g.w_batch + (size_t)panel * steps * kPanelChunk;
    }
    const uint8_t* chunk = wpanel + min(ws, steps - 1) * kPanelChunk;
    rw.b[0] = *reinterpret_cast<const u32x4*>(chunk + lane_codes);
    rw.b[1] = *reinterpret_cast<const u32x4*>(chunk + lane_codes + 512);
    rw.sw = *reinterpret_cast<const uint32_t*>(chunk + lane_scale);
    if (++ws == iters) {
      ws = 0;
      ++wk;
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x16 acc[8];
  RawW wring[kU];
#pragma unroll
  for (int i = 0; i < kU; ++i) wload(wring[i]);
  __syncthreads();  // B0

  float* const xp = lds_xpose[cw];
  uint32_t u = 0;
  for (uint32_t k = 0; k < sc.count; ++k) {
    const Tile tl = tile_of(k);
    const uint8_t* a = g.a + tl.z * g.a_batch;
    const uint8_t* w0 = g.w[0] + tl.z * g.w_batch;
    uint32_t* c = g.c + tl.z * g.c_batch;
    const uint32_t colw = tl.col0 + cw * kPanelCols;  // this wave's first column
    auto trow = [&](uint32_t mi, uint32_t r) {
      return tl.row0 + mi * 32 + 4 * (lane >> 5) + 8 * (r / 4) + (r & 3);
    };
    bool init_unsafe = false;
    if (g.acc) {  // uniform: start from C
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t row = trow(j / 2, r), col = colw + (j % 2) * 32 + (lane & 31);
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
    uint32_t bad = 0;  // nonzero: a W scale byte of this tile left the window
    for (uint32_t s = 0; s < iters; s += kU) {
#pragma unroll
      for (int i = 0; i < kU; ++i, ++u) {
        const StageA& st = lds_stage[u % kStages];
        const RawW& w = wring[i];
        // The window check consumes the slot's scale bytes here, before the
        // slot is refilled: left to itself the compiler sinks it to the end
        // of the unrolled round and then has to copy the ring registers,
        // which makes it wait for every load in flight.
        const uint32_t sw = w.sw >> scale_shift;
        const uint32_t ew0 = sw & 0xFFu, ew1 = (sw >> 8) & 0xFFu;
        bad |= (uint32_t)(ew0 - kSafeLo > kSafeHi - kSafeLo) |
               (uint32_t)(ew1 - kSafeLo > kSafeHi - kSafeLo);
        asm volatile("" : "+v"(bad));
        const i32x8 b0 = {(int)w.b[0][0], (int)w.b[0][1], (int)w.b[0][2], (int)w.b[0][3], 0, 0, 0, 0};
        const i32x8 b1 = {(int)w.b[1][0], (int)w.b[1][1], (int)w.b[1][2], (int)w.b[1][3], 0, 0, 0, 0};
        const int sb = (int)sw;
        const int sa0 = (int)st.sa[0][lane], sa1 = (int)st.sa[1][lane];
        // A codes: dwords 0-7 of every m-tile first (the h plane and half of
        // the r plane), then dwords 8-11.  Plane h over all 8 accumulators,
        // then plane r: an accumulator's two updates are 8 MFMAs apart.
        uint4 v[4][3];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          v[mi][0] = st.a[mi][lane][0];
          v[mi][1] = st.a[mi][lane][1];
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) v[mi][2] = st.a[mi][lane][2];
        Unroll<4>([&](auto mi_c) {
          constexpr int kMi = decltype(mi_c)::value;
          const i32x8 ah = {(int)v[kMi][0].x, (int)v[kMi][0].y, (int)v[kMi][0].z, (int)v[kMi][0].w,
                            (int)v[kMi][1].x, (int)v[kMi][1].y, 0, 0};
          const int sa = kMi < 2 ? sa0 : sa1;
          constexpr int kSel = (kMi % 2) * 2;
          acc[kMi * 2] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              ah, b0, acc[kMi * 2], 2, 4, kSel, sa, 0, sb);
          acc[kMi * 2 + 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              ah, b1, acc[kMi * 2 + 1], 2, 4, kSel, sa, 1, sb);
        });
        Unroll<4>([&](auto mi_c) {
          constexpr int kMi = decltype(mi_c)::value;
          const i32x8 ar = {(int)v[kMi][1].z, (int)v[kMi][1].w, (int)v[kMi][2].x, (int)v[kMi][2].y,
                            (int)v[kMi][2].z, (int)v[kMi][2].w, 0, 0};
          const int sa = kMi < 2 ? sa0 : sa1;
          constexpr int kSel = (kMi % 2) * 2 + 1;
          acc[kMi * 2] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              ar, b0, acc[kMi * 2], 2, 4, kSel, sa, 0, sb);
          acc[kMi * 2 + 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              ar, b1, acc[kMi * 2 + 1], 2, 4, kSel, sa, 1, sb);
        });
        // refill this slot with step u + kU, once its MFMAs are issued
        wload(wring[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(acc[j]));
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(acc[j]));
      }
    }
    // Epilogue, this wave's 128 x 64 outputs.
    const bool slow = __builtin_amdgcn_readfirstlane(
        lds_unsafe[k & 1] != 0 ||
        __builtin_amdgcn_ballot_w64(init_unsafe || bad != 0) != 0);
    if (tid == 0) lds_unsafe[(k + 1) & 1] = 0;
    if (slow) {  // a scale byte or an initial C left the window: every output exactly
      for (uint32_t j = 0; j < 8; ++j)
        for (uint32_t r = 0; r < 16; ++r) {
          const uint32_t row = trow(j / 2, r), col = colw + (j % 2) * 32 + (lane & 31);
          if (row >= g.m || col >= g.n) continue;
          uint32_t* out = c + (size_t)row * g.n + col;
          *out = SlowLinear(g, a, w0, w0, g.acc ? *out : 0u, row, col);
        }
      continue;
    }
    // Each MFMA tile through the wave's LDS block, stored as 16-byte rows
    // of 4 columns (rows at row ^ ((row >> 2) & 1): conflict-free writes and
    // reads); +0 maps -0 (and a flushed denormal) to +0.  (The lane index is
    // read again here: held over the K loop, its addresses spilled.)
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
      const float4 v0 = rd[0], v1 = rd[64], v2 = rd[128], v3 = rd[192];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t col = colw + (kJ % 2) * 32 + 4 * (lane & 7);
      const uint32_t prow = lane >> 3;
      const uint32_t row = tl.row0 + (kJ / 2) * 32 + (prow ^ ((prow >> 2) & 1));
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

// One thread per 16-byte column-block (plus its scale byte) of the panels.
__global__ __launch_bounds__(256) void PackPanelsKernel(const uint8_t* w, uint32_t n,
                                                        uint32_t kb_total, uint8_t* out,
                                                        uint64_t pieces) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= pieces) return;
  const uint32_t steps = (kb_total + 1) / 2;
  const uint32_t c = (uint32_t)(i % kPanelCols), b = (uint32_t)((i / kPanelCols) % 2);
  const uint64_t chunk = i / (2 * kPanelCols);  // panel * steps + step
  const uint32_t step = (uint32_t)(chunk % steps), panel = (uint32_t)(chunk / steps);
  const uint32_t col = panel * kPanelCols + c, blk = 2 * step + b;
  uint8_t* dst = out + chunk * kPanelChunk;
  u32x4 codes = {0u, 0u, 0u, 0u};
  uint8_t scale = 127;
  if (col < n && blk < kb_total) {
    const uint8_t* word = w + ((uint64_t)(col / 8) * kb_total + blk) * kDdrWord;
    codes = *reinterpret_cast<const u32x4*>(word + (col % 8) * 16);
    scale = word[128 + col % 8];
  }
  *reinterpret_cast<u32x4*>(dst + (b * kPanelCols + c) * 16) = codes;
  dst[kPanelScales + 2 * (b * 32 + c % 32) + c / 32] = scale;
}

// One thread per 16-byte column-block of the DDR words; the thread of
// column 8g holds the word's scale bytes and padding too.
__global__ __launch_bounds__(256) void UnpackPanelsKernel(const uint8_t* in, uint32_t n,
                                                          uint32_t kb_total, uint8_t* w) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)n * kb_total) return;
  const uint32_t cl = (uint32_t)(i % 8), blk = (uint32_t)((i / 8) % kb_total);
  const uint32_t grp = (uint32_t)(i / (8ull * kb_total)), col = grp * 8 + cl;
  const uint32_t steps = (kb_total + 1) / 2, c = col % kPanelCols, b = blk % 2;
  const uint8_t* chunk = in + ((uint64_t)(col / kPanelCols) * steps + blk / 2) * kPanelChunk;
  uint8_t* word = w + ((uint64_t)grp * kb_total + blk) * kDdrWord;
  *reinterpret_cast<u32x4*>(word + cl * 16) =
      *reinterpret_cast<const u32x4*>(chunk + (b * kPanelCols + c) * 16);
  word[128 + cl] = chunk[kPanelScales + 2 * (b * 32 + c % 32) + c / 32];
  if (cl == 0) *reinterpret_cast<uint2*>(word + 136) = uint2{0u, 0u};
}

}  // namespace

bool PanelEligible(const GemmArgs& args) {
  // C is stored 16 bytes at a time; one piece over every block in order
  const bool aligned = reinterpret_cast<uintptr_t>(args.c) % 16 == 0 && args.c_batch % 4 == 0;
  return args.w_panels && args.n_planes == 1 && args.modes[0] == kModeFp4 && aligned &&
         args.n_ops == 0 && args.q_out == nullptr && args.n_pieces == 1 &&
         args.piece_off[0] == 0 && args.piece_kb[0] == args.kb_total && args.quads * 4 > 64;
}

hipError_t LaunchPanel(const GemmArgs& in, uint32_t batch, hipStream_t stream) {
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
  const dim3 grid(tiles < (uint32_t)cus[dev] ? tiles : (uint32_t)cus[dev]), block(512);
  hipLaunchKernelGGL(PanelKernel, grid, block, 0, stream, args);
  return hipGetLastError();
}

hipError_t LaunchPackPanels(const uint8_t* w, uint32_t n, uint32_t kb_total, uint8_t* out,
                            hipStream_t stream) {
  const uint64_t pieces = (uint64_t)((n + kPanelCols - 1) / kPanelCols) * ((kb_total + 1) / 2) *
                          2 * kPanelCols;
  hipLaunchKernelGGL(PackPanelsKernel, dim3((uint32_t)((pieces + 255) / 256)), dim3(256), 0,
                     stream, w, n, kb_total, out, pieces);
  return hipGetLastError();
}

hipError_t LaunchUnpackPanels(const uint8_t* in, uint32_t n, uint32_t kb_total, uint8_t* w,
                              hipStream_t stream) {
  const uint64_t pieces = (uint64_t)n * kb_total;
  hipLaunchKernelGGL(UnpackPanelsKernel, dim3((uint32_t)((pieces + 255) / 256)), dim3(256), 0,
                     stream, in, n, kb_total, w);
  return hipGetLastError();
}

}  // namespace hb

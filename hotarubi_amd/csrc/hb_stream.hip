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
// direct global-to-LDS loads (global_load_lds_dwordx4: lane l's 16 bytes
// land at M0 + 16 l), through a ring of kD steps.  A step is one table of
// 20 x 64 pieces of 16 bytes, 5 loads per wave:
//   A codes   [h][row][32 bytes]: row r's 32 codes of block 2s + h, the
//             two 16-byte halves of its 32 bytes in the 144-byte word;
//   A scales  [h][quad][16 bytes]: bytes 128..143 of quad's word of block
//             2s + h (the 4 rows' E8M0 bytes first);
//   W chunks  the tile's 5 panels' chunks of step s, 2176 bytes each;
// so each quad's A words of the step (288 contiguous bytes) and each W
// chunk are read whole, and the A layout in LDS is row-major: a lane's two
// 16-byte reads of its row are conflict-free.  The loads hold no registers
// while in flight, so kD - 2 = 5 steps (100 KB per CU) stream ahead of the
// matrix cores.
//   Wave w owns rows 32w..32w+31 of the tile (one m-tile) and all 10
// n-tiles: it converts only its own A rows (one (row, block) per lane per
// step), so converted A never passes through LDS; W is shared, read by each
// wave from the ring (its B operands, 1 KiB per n-tile).  The conversion of
// step u + 1 runs on the VALU while the matrix cores run step u.  C leaves
// through a 4 KiB LDS block per wave, as 16-byte stores.
//
// Synchronisation: one barrier per step, with the load counter counted by
// hand (the loads are issued from inline asm, which the compiler's own
// waits do not see).  Loads past the last step repeat a valid address, so
// every wave issues the same number of loads every step.
//
// MXFP8 activations (kA8, HB_LINEAR_A_FP8): the same ring and loads; the
// code bytes are the MFMA's FP8 A operand with scale byte ea.  8-bit A
// operands take K in 16-wide halves per lane (registers 0-3 of lane half h
// are K [16 h, 16 h + 16) of the step's first block, registers 4-7 the same
// of its second, each 32-wide K range scaled by its lane half's byte), so a
// lane reads bytes [16 h, 16 h + 16) of its row in both blocks.  Each step's
// codes go through two MFMAs per n-tile, split by exponent (fp8::Split).
#include <utility>

#include "hb_device.h"
#include "hb_internal.h"
#include "hb_ring.h"

namespace hb {
namespace {

using namespace ring;

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;                              // one per SIMD
constexpr int kBM = 32 * kWaves;                       // tile rows
constexpr int kTP = 5;                                 // panels per tile
constexpr int kBN = kTP * (int)kPanelCols;             // tile columns
constexpr int kNT = 2 * kTP;                           // 32-column n-tiles
constexpr int kD = 7;                                  // ring depth, steps
// the step's table of 16-byte pieces
constexpr uint32_t kChunkPieces = kPanelChunk / 16;    // 136 per W chunk
constexpr uint32_t kWPieces = kTP * kChunkPieces;      // 680
constexpr uint32_t kACodes = 2 * kBM * 32;             // 8192 bytes: [h][row][32]
constexpr uint32_t kAScales = 2 * (kBM / 4) * 16;      // 1024 bytes: [h][quad][16]
constexpr uint32_t kAPieces = (kACodes + kAScales) / 16;                  // 576
constexpr int kALoads = (int)(kAPieces / 64);                             // 9
constexpr int kWLoads = (int)((kWPieces + 63) / 64);                      // 11
constexpr int kOps = (kALoads + kWLoads) / kWaves;     // loads per wave per step
constexpr uint32_t kSlotW = kACodes + kAScales;        // W chunks' offset in a slot
constexpr uint32_t kSlot = kSlotW + kWLoads * 1024;
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;
static_assert(kAPieces % 64 == 0 && (kALoads + kWLoads) % kWaves == 0, "piece table");
static_assert(kD * kOps < 64, "load counter range");
static_assert(kSlot % 16 == 0, "16-byte slots");

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

// Operand set of parity p (steps v = p mod 2) for this lane: step v's B
// operands of the tile's 10 n-tiles (t: panel t / 2, columns 32 (t % 2) ..)
// and the panels' scale bytes (bytes 0, 1 of sw[q]: n-tiles 2q, 2q + 1);
// step v's A, converted: planes h and r/2 (FP6 E2M3 codes) with their scale
// bytes (ea - 1 | (ea - 5) << 8) and abad, the lane's A scale byte left the
// window; and the raw A codes and scale dword of a later step of the same
// parity, loaded ahead of their conversion.
// For MXFP8 (kA8) the converted A is the step's 8 code dwords with blocks
// past the layer zeroed (h holds dwords 0-5, r dwords 6-7), split into the
// exponent planes as the MFMAs issue.
struct Ops {
  u32x4 b[kNT];
  uint32_t sw[kTP];
  u32x6 h, r;
  int sa;
  uint32_t abad;
  u32x4 x0, x1;
  uint32_t sd;
};

template <bool kA8>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void StreamKernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_ring[kD * kSlot];
  __shared__ __attribute__((aligned(16))) float lds_xpose[kWaves][32 * 32];

  const Schedule sc = TilesOf(g.gx * g.gy * g.gz);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t steps = g.w_steps, nblocks = g.kb_total;
  const uint32_t esteps = steps + (steps & 1);  // an odd count gets one all-zero step
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

  // This lane's row r of the tile and block h of the step, in the MFMAs.
  const uint32_t r = w * 32 + (lane & 31), h = lane >> 5;
  // step s of a tile holds live A for this lane iff 2 s < nbh (kept in a
  // register: a reload of the argument inside the loop would wait for every
  // outstanding LDS read)
  uint32_t nbh = nblocks - h;
  asm volatile("" : "+v"(nbh));

  // The lane's pieces: load k of wave w is load i = kOps w + k of the table
  // (A for i < kALoads, else W), piece p = 64 i' + lane of its part.
  //   A: pcol = the piece's bytes in its quad's word, plus 144 h for block
  //      2s + h; pq = its quad (relative to the tile);
  //   W: pcol = its bytes in the tile's step-s chunks (panel-relative),
  //      pq = its panel; pieces past the last chunk repeat piece 0.
  uint32_t pcol[kOps], pq[kOps];
#pragma unroll
  for (int k = 0; k < kOps; ++k) {
    const uint32_t i = w * kOps + k;
    if (i < (uint32_t)kALoads) {
      const uint32_t pp = i * 64 + lane;
      if (pp < kACodes / 16) {  // [h][row][half]
        const uint32_t ph = pp / (kACodes / 32), row = (pp / 2) % kBM;
        pq[k] = row / 4;
        pcol[k] = ph * kDdrWord + (row % 4) * 32 + (pp % 2) * 16;
      } else {                  // [h][quad]
        const uint32_t q = pp - kACodes / 16;
        pq[k] = q % (kBM / 4);
        pcol[k] = (q / (kBM / 4)) * kDdrWord + 128;
      }
    } else {
      const uint32_t pp = (i - kALoads) * 64 + lane;
      pq[k] = pp < kWPieces ? pp / kChunkPieces : 0u;
      pcol[k] = pp < kWPieces ? (pp % kChunkPieces) * 16 : 0u;
    }
  }

  // Load cursor: the next global step to load (tile dk, step ds, slot
  // dslot), with the tile's bases cached.  The padding step and steps past
  // the last tile load the tile's last step again, so every wave issues
  // kOps loads per step, all in bounds.  A's block 2s + h is clamped to the
  // layer's last (a block past it is not live).
  uint32_t dk = 0, ds = 0, dslot = 0, dcached = ~0u;
  const uint8_t* da = nullptr;
  const uint8_t* dw = nullptr;
  uint32_t dbase[kOps], alim[kOps];
#pragma unroll
  for (int k = 0; k < kOps; ++k) alim[k] = (nblocks - 1) * kDdrWord + pcol[k] % kDdrWord;
  // issue_prepare: the step to load next (its source offsets, its slot);
  // issue_op(k2): the wave's load k2 of it; issue_advance: move the cursor.
  uint32_t is_s = 0, is_slot = 0;
  auto issue_prepare = [&]() __attribute__((always_inline)) {
    const uint32_t k = min(dk, sc.count - 1);
    if (k != dcached) {  // uniform: once per tile
      dcached = k;
      const Tile tl = tile_of(k);
      da = g.a + tl.z * g.a_batch;
      dw = g.w[0] + tl.z * g.w_batch;
#pragma unroll
      for (int k2 = 0; k2 < kOps; ++k2) {
        const bool is_a = w * kOps + k2 < (uint32_t)kALoads;
        dbase[k2] = is_a ? min(tl.row0 / 4 + pq[k2], g.quads - 1) * g.a_row * kDdrWord
                         : min(tl.p0 + pq[k2], n_panels - 1) * steps * kPanelChunk + pcol[k2];
      }
    }
    is_s = dk < sc.count ? min(ds, steps - 1) : steps - 1;
    is_slot = ring + dslot * kSlot;
  };
  auto issue_op = [&](int k2) __attribute__((always_inline)) {
    const uint32_t i = w * kOps + k2;
    const bool is_a = i < (uint32_t)kALoads;  // uniform
    const uint32_t off = is_a ? dbase[k2] + min(is_s * (2 * kDdrWord) + pcol[k2], alim[k2])
                              : dbase[k2] + is_s * kPanelChunk;
    const uint32_t lds = is_a ? is_slot + i * 1024 : is_slot + kSlotW + (i - kALoads) * 1024;
    Dma16(is_a ? da : dw, off, __builtin_amdgcn_readfirstlane(lds));
  };
  auto issue_advance = [&]() __attribute__((always_inline)) {
    if (++ds == esteps) {
      ds = 0;
      ++dk;
    }
    dslot = dslot + 1 == kD ? 0u : dslot + 1;
  };
  auto issue_next = [&]() __attribute__((always_inline)) {
    issue_prepare();
#pragma unroll
    for (int k2 = 0; k2 < kOps; ++k2) issue_op(k2);
    issue_advance();
  };

  // Reads from ring slot `slot`: the W chunks' B operands and scale dwords;
  // this lane's raw A.
  auto read_w = [&](Ops& o, uint32_t slot) __attribute__((always_inline)) {
    const uint8_t* wslot = lds_ring + slot * kSlot + kSlotW;
#pragma unroll
    for (int q = 0; q < kTP; ++q) {
      const uint8_t* chunk = wslot + q * kPanelChunk;
#pragma unroll
      for (int t = 0; t < 2; ++t)
        o.b[2 * q + t] = *reinterpret_cast<const u32x4*>(
            chunk + ((lane >> 5) * kPanelCols + t * 32 + (lane & 31)) * 16);
      o.sw[q] = *reinterpret_cast<const uint32_t*>(chunk + kPanelScales + 4 * (lane >> 1));
    }
  };
  auto read_a = [&](Ops& o, uint32_t slot) __attribute__((always_inline)) {
    const uint8_t* abuf = lds_ring + slot * kSlot;
    if constexpr (kA8) {  // bytes [16 h, 16 h + 16) of the row in both blocks
      o.x0 = *reinterpret_cast<const u32x4*>(abuf + r * 32 + 16 * h);
      o.x1 = *reinterpret_cast<const u32x4*>(abuf + (kBM + r) * 32 + 16 * h);
    } else {
      o.x0 = *reinterpret_cast<const u32x4*>(abuf + (h * kBM + r) * 32);
      o.x1 = *reinterpret_cast<const u32x4*>(abuf + (h * kBM + r) * 32 + 16);
    }
    o.sd = *reinterpret_cast<const uint32_t*>(abuf + kACodes + (h * (kBM / 4) + r / 4) * 16);
  };
  // Convert the raw A held in o, of step (k, s).
  auto convert = [&](Ops& o, uint32_t k, uint32_t s) __attribute__((always_inline)) {
    const bool live = k < sc.count && 2 * s < nbh;
    const uint32_t ea = __builtin_amdgcn_ubfe(o.sd, 8 * (r & 3), 8);
    o.abad = live && ea - kSafeLo > kSafeHi - kSafeLo ? 1u : 0u;
    if constexpr (kA8) {  // blocks 2 s (dwords 0-3) and 2 s + 1 (4-7) where they exist
      const uint32_t keep0 = k < sc.count && 2 * s < nblocks ? ~0u : 0u;
      const uint32_t keep1 = k < sc.count && 2 * s + 1 < nblocks ? ~0u : 0u;
      o.h = u32x6{o.x0[0] & keep0, o.x0[1] & keep0, o.x0[2] & keep0, o.x0[3] & keep0,
                  o.x1[0] & keep1, o.x1[1] & keep1};
      o.r = u32x6{o.x1[2] & keep1, o.x1[3] & keep1, 0u, 0u, 0u, 0u};
      o.sa = (int)ea;
      return;
    }
    const uint32_t x[8] = {o.x0[0], o.x0[1], o.x0[2], o.x0[3], o.x1[0], o.x1[1], o.x1[2], o.x1[3]};
    SplitA(x, live ? 0xFFFFFFFFu : 0u, o.h, o.r);
    o.sa = (int)(((ea - 5u) << 8) | ((ea - 1u) & 0xFFu));
  };

  float* const xp = lds_xpose[w];
  f32x16 acc[kNT];
  Tile tl{};
  uint32_t row_w = 0, live_nt = 0;
  bool init_unsafe = false;
  // Start tile k: its geometry and the accumulators (+0, or C).
  auto begin_tile = [&](uint32_t k) __attribute__((always_inline)) {
    tl = tile_of(k);
    row_w = tl.row0 + w * 32;
    live_nt = min((uint32_t)kNT, (g.n - min(tl.col0, g.n) + 31) / 32);
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
  // Finish the current tile: each n-tile's 32 x 32 values (the accumulators,
  // or the exact fold where a scale byte or an initial C left the window)
  // through the wave's LDS block, stored as 16-byte rows of 4 columns (rows
  // at row ^ ((row >> 2) & 1): conflict-free writes and reads); +0 maps -0
  // (and a flushed denormal) to +0.  A layer with ops or the requantize
  // takes each lane's 4 columns of 4 rows through the ops in FP32 hardware
  // arithmetic, C (when kept) and the MXINT8 requantize: a row's 32-column
  // block is 8 lanes, their largest exponent field by 3 swizzles, one
  // 4-byte store of codes per lane and row.
  auto end_tile = [&](uint32_t bad) __attribute__((always_inline)) {
    const uint32_t z = tl.z;
    const uint8_t* a = g.a + z * g.a_batch;
    const uint8_t* w0 = g.w[0] + z * g.w_batch;
    uint32_t* c = g.c != nullptr ? g.c + z * g.c_batch : nullptr;
    uint8_t* q = g.q_out != nullptr ? g.q_out + z * g.q_batch : nullptr;
    // (MXINT8 layers with ops or the requantize take the tile kernel, whose
    // epilogue runs on 16 waves; the fused path is compiled for MXFP8 only)
    const bool fused = kA8 && (g.n_ops != 0 || q != nullptr);  // uniform
    const bool slow = __builtin_amdgcn_readfirstlane(
        __builtin_amdgcn_ballot_w64(init_unsafe || bad != 0) != 0);
    if (slow && !fused) {  // every output exactly, straight to C
      WaitVm<0>();
      for (uint32_t j = 0; j < kNT; ++j)
        for (uint32_t e = 0; e < 16; ++e) {
          const uint32_t row = row_w + 4 * (lane >> 5) + 8 * (e / 4) + (e & 3);
          const uint32_t col = tl.col0 + j * 32 + (lane & 31);
          if (row >= g.m || col >= g.n) continue;
          uint32_t* out = c + (size_t)row * g.n + col;
          *out = kA8 ? SlowLinearFp8(g, a, w0, g.acc ? *out : 0u, row, col)
                     : SlowLinear(g, a, w0, w0, g.acc ? *out : 0u, row, col);
        }
      return;
    }
    if (slow) WaitVm<0>();
    const uint32_t rows4 = g.quads * 4, nb = g.n >> 5;
    Unroll<kNT>([&](auto jj) {
      constexpr int kJ = decltype(jj)::value;
      if ((uint32_t)kJ >= live_nt) return;
      if (slow) {  // the exact fold of each output (a layer with ops or requantize)
        for (uint32_t e = 0; e < 16; ++e) {
          const uint32_t rl = 8 * (e / 4) + 4 * (lane >> 5) + (e & 3);
          const uint32_t row = row_w + rl, col = tl.col0 + kJ * 32 + (lane & 31);
          uint32_t v = 0;
          if (row < rows4 && col < g.n) {
            const uint32_t init = g.acc && row < g.m ? c[(size_t)row * g.n + col] : 0u;
            v = kA8 ? SlowLinearFp8(g, a, w0, init, row, col)
                    : SlowLinear(g, a, w0, w0, init, row, col);
          }
          xp[(rl ^ ((rl >> 2) & 1)) * 32 + (lane & 31)] = __uint_as_float(v);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t row = 8 * (e / 4) + 4 * (lane >> 5) + (e & 3);
          xp[(row ^ ((row >> 2) & 1)) * 32 + (lane & 31)] = acc[kJ][e] + 0.0f;
        }
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
      if (!fused) {
        float4* out = reinterpret_cast<float4*>(c + (size_t)row * g.n + col);
        const size_t q_step = (size_t)2 * g.n;  // 8 rows, in float4 units
        if (col < g.n) {
          if (row < g.m) out[0] = v0;
          if (row + 8 < g.m) out[q_step] = v1;
          if (row + 16 < g.m) out[2 * q_step] = v2;
          if (row + 24 < g.m) out[3 * q_step] = v3;
        }
        return;
      }
      // rows row + 8 i, columns col .. col + 3 (n % 8 == 0: all four are
      // in the layer or none)
      f32x4_t y[4] = {f32x4_t{v0.x, v0.y, v0.z, v0.w}, f32x4_t{v1.x, v1.y, v1.z, v1.w},
                      f32x4_t{v2.x, v2.y, v2.z, v2.w}, f32x4_t{v3.x, v3.y, v3.z, v3.w}};
      const bool col_in = col < g.n;
      const uint32_t cc = col_in ? col : 0u;
      for (uint32_t o = 0; o < g.n_ops; ++o) {
        const uint32_t kind = g.op_kind[o];
        f32x4_t p = {};
        if (kind == kEpAddP || kind == kEpMulP) {
          const uint32_t* pv = g.op_vec[o] + z * g.op_vec_batch[o] + cc;
          p = f32x4_t{__uint_as_float(pv[0]), __uint_as_float(pv[1]), __uint_as_float(pv[2]),
                      __uint_as_float(pv[3])};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4_t x2 = {};
          if ((kind == kEpAdd || kind == kEpActMul) && row + 8 * i < g.m && col_in) {
            const uint32_t* xv = g.op_x2[o] + z * g.op_x2_batch[o] + (size_t)(row + 8 * i) * g.n + col;
            x2 = f32x4_t{__uint_as_float(xv[0]), __uint_as_float(xv[1]), __uint_as_float(xv[2]),
                         __uint_as_float(xv[3])};
          }
          EpApplyFastN<false>(kind, g.op_imm[o], y[i], x2, p, g.tbuf + 512);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = row + 8 * i;
        if (c != nullptr && col_in && r < g.m)
          *reinterpret_cast<float4*>(c + (size_t)r * g.n + col) =
              float4{y[i][0], y[i][1], y[i][2], y[i][3]};
        if (q == nullptr) continue;
        uint32_t e = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) e = max(e, ExpField(__float_as_uint(y[i][k])));
        // the row's 8 lanes (lanes 8 p .. 8 p + 7): xor 1, 2, 4
        e = max(e, (uint32_t)__builtin_amdgcn_ds_swizzle((int)e, 0x041F));
        e = max(e, (uint32_t)__builtin_amdgcn_ds_swizzle((int)e, 0x081F));
        e = max(e, (uint32_t)__builtin_amdgcn_ds_swizzle((int)e, 0x101F));
        if (r < rows4 && col_in) {
          uint8_t* word = q + ((size_t)(r >> 2) * nb + (col >> 5)) * kDdrWord;
          uint32_t codes = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            codes |= (uint32_t)QuantizeElementHw(__float_as_uint(y[i][k]), e) << (8 * k);
          *reinterpret_cast<uint32_t*>(word + (r & 3) * 32 + 4 * (lane & 7)) = codes;
          if ((lane & 7) == 0) word[128 + (r & 3)] = (uint8_t)ScaleByteOf(e);
          if ((lane & 7) == 1 && (r & 3) == 0) {
            uint32_t* pad = reinterpret_cast<uint32_t*>(word + 132);
            pad[0] = pad[1] = pad[2] = 0u;
          }
        }
      }
    });
  };

  // Prologue: steps 0 .. kD - 1 in flight (every slot); steps 0, 1 landed:
  // step 0's operands read and converted, step 1's raw A read.
#pragma unroll
  for (int v = 0; v < kD; ++v) issue_next();
  WaitVm<(kD - 2) * kOps>();
  __syncthreads();
  Ops o0, o1;
  read_w(o0, 0);
  read_a(o0, 0);
  read_a(o1, 1);
  convert(o0, 0, 0);

  // Step u = (tile k, step s), ring slot u mod kD, operands in `use` (the
  // set of u's parity): wait for this wave's loads of step u + 2, barrier
  // (every wave's loads of step u + 2 landed; every wave done reading slot
  // u: step u's W was read in step u - 1, its A in step u - 2), refill slot
  // u with step u + kD (the loads spread between the step's MFMAs); read
  // step u + 1's W into `oth` and step u + 2's raw
  // A into `use`; convert step u + 1's raw A (read in step u - 1, held in
  // `oth`) while the matrix cores run step u's 20 MFMAs.
  uint32_t slot = 0;
  auto iteration = [&](Ops& use, Ops& oth, uint32_t k, uint32_t s, uint32_t& bad)
      __attribute__((always_inline)) {
    WaitVm<(kD - 3) * kOps>();
    WaitLds();
    __syncthreads();
    issue_prepare();  // this step's loads go out between its MFMAs, below
    const uint32_t s1 = slot + 1 == kD ? 0u : slot + 1;
    const uint32_t s2 = s1 + 1 == kD ? 0u : s1 + 1;
    read_w(oth, s1);
    read_a(use, s2);
    const bool last = s + 1 == esteps;
    convert(oth, last ? k + 1 : k, last ? 0u : s + 1);
    slot = s1;
    // the window checks (a panel past the layer repeats the last one's bytes)
    uint32_t wb = use.abad;
#pragma unroll
    for (int q = 0; q < kTP; ++q) {
      const uint32_t sq = use.sw[q] >> (16 * (lane & 1));
      wb |= (uint32_t)((sq & 0xFFu) - kSafeLo > kSafeHi - kSafeLo) |
            (uint32_t)(((sq >> 8) & 0xFFu) - kSafeLo > kSafeHi - kSafeLo);
    }
    bad |= wb;
    i32x8 ah, ar;
    if constexpr (kA8) {  // the exponent planes: ah (exponents 0..7), then ar (8..15)
      const uint32_t x[8] = {use.h[0], use.h[1], use.h[2], use.h[3],
                             use.h[4], use.h[5], use.r[0], use.r[1]};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t lo, hi;
        fp8::Split(x[i], lo, hi);
        ah[i] = (int)lo;
        ar[i] = (int)hi;
      }
    } else {
      ah = i32x8{(int)use.h[0], (int)use.h[1], (int)use.h[2], (int)use.h[3],
                 (int)use.h[4], (int)use.h[5], 0, 0};
      ar = i32x8{(int)use.r[0], (int)use.r[1], (int)use.r[2], (int)use.r[3],
                 (int)use.r[4], (int)use.r[5], 0, 0};
    }
    // A's format (cbsz): FP6 E2M3 planes, or FP8 E4M3; its op_sel picks the
    // plane's scale byte in sa (FP6), or the one byte ea (FP8)
    constexpr int kAFmt = kA8 ? 0 : 2, kSelR = kA8 ? 0 : 1;
    // plane h over the n-tiles, then plane r (branch-free: n-tiles past the
    // layer compute outputs that are not stored)
    auto mfma = [&](auto t_c, const i32x8& av, auto sel_c) __attribute__((always_inline)) {
      constexpr int kT = decltype(t_c)::value, kSel = decltype(sel_c)::value;
      const i32x8 bt = {(int)use.b[kT][0], (int)use.b[kT][1], (int)use.b[kT][2],
                        (int)use.b[kT][3], 0, 0, 0, 0};
      const int sb = (int)(use.sw[kT / 2] >> (16 * (lane & 1)));
      acc[kT] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bt, acc[kT], kAFmt, 4, kSel,
                                                                use.sa, kT % 2, sb);
    };
    // The step's loads of step u + kD go out between the MFMAs (one after
    // every 2 kNT / kOps of them): a load waits to issue while the CU's
    // outstanding requests are at their limit, and the MFMAs issued before
    // it keep the matrix cores busy meanwhile, so the loads refill the
    // CU's request queue through the whole step.
    constexpr int kEvery = 2 * kNT / kOps;
    static_assert(2 * kNT % kOps == 0, "loads spread evenly over the MFMAs");
    Unroll<2 * kNT>([&](auto u_c) {
      constexpr int kU = decltype(u_c)::value;
      if constexpr (kU < kNT) mfma(std::integral_constant<int, kU>{}, ah, std::integral_constant<int, 0>{});
      else mfma(std::integral_constant<int, kU - kNT>{}, ar, std::integral_constant<int, kSelR>{});
      // Volatile asms keep their order, and the MFMA builtins (pure) would
      // otherwise move freely: an empty asm after each MFMA that takes the
      // previous MFMA's accumulators (complete by now, as this one runs)
      // holds every MFMA between its neighbours, and the loads in place.
      if constexpr (kU > 0) asm volatile("" ::"a"(acc[(kU - 1) % kNT]));
      if constexpr (kU % kEvery == kEvery - 1) issue_op(kU / kEvery);
    });
    issue_advance();
#pragma unroll
    for (int t = 0; t < kNT; ++t) asm volatile("" : "+a"(acc[t]));
    asm volatile("" : "+v"(oth.h), "+v"(oth.r), "+v"(oth.sa), "+v"(oth.abad));
  };

  for (uint32_t k = 0; k < sc.count; ++k) {
    begin_tile(k);
    uint32_t bad = 0;  // this wave's tile saw a scale byte outside the window
    for (uint32_t s = 0; s < esteps; s += 2) {
      iteration(o0, o1, k, s, bad);
      iteration(o1, o0, k, s + 1, bad);
    }
    end_tile(bad);
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
  // the requantized words are written 4 bytes at a time
  const bool q_aligned = args.q_out == nullptr ||
                         (reinterpret_cast<uintptr_t>(args.q_out) % 4 == 0 && args.q_batch % 4 == 0);
  // MXINT8 layers of up to 64 rows have the skinny and split kernels, and
  // with ops or the requantize the tile kernel; MXFP8 layers of any row
  // count, plain or not, stream here
  return args.w_panels && args.n_planes == 1 && args.modes[0] == kModeFp4 && aligned &&
         q_aligned && args.n_pieces == 1 && args.piece_off[0] == 0 &&
         args.piece_kb[0] == args.kb_total &&
         (args.a_fp8 || (args.quads * 4 > 64 && args.n_ops == 0 && args.q_out == nullptr));
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
  if (args.a_fp8) hipLaunchKernelGGL(StreamKernel<true>, grid, block, 0, stream, args);
  else hipLaunchKernelGGL(StreamKernel<false>, grid, block, 0, stream, args);
  return hipGetLastError();
}

}  // namespace hb

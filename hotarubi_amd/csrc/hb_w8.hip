// W8 layers over FP6 weight panels (HB_LINEAR_W8_PANELS): the packer that
// turns a W8 layer's two nibble planes into matrix-core operands once, and
// the streaming kernel that runs the layer from them.
//
// Arithmetic (tools/iss/gemm_array.cpp:84-110: a W8 weight is the hi plane's
// signed nibble with SBIAS -8 plus the lo plane's unsigned nibble with SBIAS
// -12, each plane with its own E8M0 byte ew).  A nibble value v is stored as
// the FP6 E2M3 code of v / 2 (exact for -8..15) with scale byte ew - 1 (hi)
// or ew - 5 (lo); A is split per block into the FP6 planes h = q / 32 at
// ea - 1 and (q - 32 h) / 2 at ea - 5 (SplitA), whose sum is q 2^(ea-133).
// Each of the four plane products of v_mfma_scale_f32_32x32x64_f8f6f4 then
// carries exactly the reference's weight:
//   hi: q 2^(ea-133) * v 2^(ew-129) = q v 2^((ea-127) + (ew-127) - 8),
//   lo: q 2^(ea-133) * v 2^(ew-133) = q v 2^((ea-127) + (ew-127) - 12).
// The matrix cores add the exact products in their own order, so fast-mode
// results are tolerance-equal, not bit-equal, to the NPU's ordered fold; a
// wave whose scale bytes leave [70, 179] (or whose initial C is near the top
// of the range) recomputes its outputs with the exact fold.  Exact mode
// folds every output exactly.
//
// Kernel.  Tiles of 128 rows x 64 kTP columns (kTP weight panels), 4 waves,
// one workgroup per CU.  Every operand byte of the K loop reaches LDS by
// direct global-to-LDS loads through a ring of kD steps; a step is A's 9216
// bytes ([h][row][32 codes], then [h][quad][16 bytes of scales], as in the
// MXFP4 streaming kernel) and the tile's kTP W8 chunks, read whole.  Wave w
// owns rows 32w..32w+31 and all 2 kTP n-tiles: it splits only its own A rows
// (one (row, block) per lane per step, in registers) and reads W's B operands
// from the ring (both planes of an n-tile: 16 + 8 bytes per lane each).  Per
// step a wave issues 8 kTP MFMAs (the four plane products of each n-tile,
// product by product so that consecutive MFMAs use different accumulators),
// the LDS reads of the next step and the conversion of the step after.
// After the K loop the ring is free: the outputs are staged there per wave,
// with the activation table, and the epilogue (ops, C, requantize) runs per
// 32-column tile.
#include <algorithm>
#include <utility>

#include "hb_device.h"
#include "hb_internal.h"
#include "hb_ring.h"

namespace hb {
namespace {

using namespace ring;

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;                              // one per SIMD
constexpr int kBM = 32 * kWaves;                       // tile rows
constexpr uint32_t kACodes = 2 * kBM * 32;             // [h][row][32 codes]: 8 loads
constexpr uint32_t kAScales = 2 * 1024;                // [h][lane]: 2 loads (32 quads used)
constexpr int kALoads = 3;                             // per wave: 12 = 8 + 2 + 2 repeats
constexpr uint32_t kSlotW = kWaves * kALoads * 1024;   // W chunks' offset in a ring slot
constexpr uint32_t kLds = 160u * 1024u;
constexpr uint32_t kStage = 8192;                      // epilogue: outputs after the table
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;
static_assert(kBM / 4 <= 32 && kACodes + 2 * kAScales == kSlotW, "A loads");

template <int kTP>
struct Cfg {
  static constexpr int kNT = 2 * kTP;                               // 32-column n-tiles
  static constexpr uint32_t kWPieces = kTP * (kW8Chunk / 16);       // 16-byte pieces
  static constexpr int kWOps = (int)((kWPieces + 64 * kWaves - 1) / (64 * kWaves));  // per wave
  static constexpr int kOps = kALoads + kWOps;                      // loads per wave per step
  static constexpr uint32_t kSlot = kSlotW + kWOps * kWaves * 1024; // the last W loads repeat
  static constexpr int kD = (int)(kLds / kSlot);                    // ring depth, steps
  static_assert(kD >= 4 && kD * kOps < 64, "ring depth and load counter range");
};

// One step's operands for this lane: the B operands of the tile's n-tiles
// (plane l of n-tile t in b[2 t + l]), each panel's scale dword (byte
// 2 (t % 2) + l for n-tile t, plane l); A's converted planes
// with their scale bytes (ea - 1 | (ea - 5) << 8) and window flag; and the
// raw A codes and scale dword of a later step, loaded ahead of conversion.
template <int kNT>
struct Ops {
  u32x6 b[2 * kNT];
  uint32_t sw[kNT / 2];
  u32x6 h, r;
  int sa;
  uint32_t abad;
  u32x4 x0, x1;
  uint32_t sd;
};

template <int kTP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void W8Kernel(GemmArgs g) {
  using C = Cfg<kTP>;
  constexpr int kNT = C::kNT, kOps = C::kOps, kD = C::kD;
  constexpr uint32_t kSlot = C::kSlot;
  __shared__ __attribute__((aligned(16))) uint8_t lds_ring[kD * kSlot];

  const TileId tile = BandTile(g.gx, g.gy, g.gz, g.band);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t steps = g.w_steps, nblocks = g.kb_total;
  const uint32_t n_panels = (g.n + kPanelCols - 1) / kPanelCols;
  const uint32_t row0 = tile.y * kBM, p0 = tile.x * kTP, col0 = p0 * kPanelCols;
  const uint8_t* a = g.a + tile.z * g.a_batch;
  const uint8_t* wp = g.w[0] + tile.z * g.w_batch;
  uint32_t* c = g.c + tile.z * g.c_batch;
  uint8_t* q_out = g.q_out ? g.q_out + tile.z * g.q_batch : nullptr;
  const uint32_t ring_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_ring));
  const bool fast = g.fast_ep != 0;

  // This lane's row r of the tile and block h of the step, in the MFMAs.
  const uint32_t r = w * 32 + (lane & 31), h = lane >> 5;
  const uint32_t row_w = row0 + w * 32;
  const uint32_t live_nt = min((uint32_t)kNT, (g.n - min(col0, g.n) + 31) / 32);

  // The packer's window flags of the tile's panels.
  const uint32_t* flags = reinterpret_cast<const uint32_t*>(
      wp + (size_t)n_panels * steps * kW8Chunk);
  uint32_t bad = 0;
#pragma unroll
  for (int q = 0; q < kTP; ++q) bad |= flags[min(p0 + q, n_panels - 1)];

  f32x16 acc[kNT];
  if (fast) {
    // Initial accumulators: +0, or C (before any load into LDS is issued:
    // the compiler's waits for these loads then count nothing else).
    if (g.acc) {
      const bool unsafe =
          AccFromC(acc, c, g.m, g.n, [&](uint32_t j, uint32_t e, uint32_t& row, uint32_t& col) {
            row = row_w + 4 * (lane >> 5) + 8 * (e / 4) + (e & 3);
            col = col0 + j * 32 + (lane & 31);
          });
      bad |= unsafe ? 1u : 0u;
    } else {
#pragma unroll
      for (int j = 0; j < kNT; ++j) acc[j] = f32x16{};
    }

    // The lane's pieces.  Loads k < 3 of wave w are A load i = 3w + k, the
    // others W load j = 4 (k - 3) + w; each covers 64 pieces of 16 bytes,
    // lane l the piece 64 i + l (64 j + l), landing at slot + 1024 i
    // (slot + kSlotW + 1024 j) + 16 l.  At step s a piece's address is a
    // wave-uniform base (scalar arithmetic) plus voff[k], its fixed offset:
    //   i < 8, A codes [h][row][half], h = i / 4; i >= 8, A scales [h][quad]
    //      (bytes 128..143 of the quad's word, lanes 32..63 repeating lanes
    //      0..31; loads 10 and 11 repeat 8 and 9 into unused space), h =
    //      i % 2: base a + min(2s + h, kb_total - 1) words (a block past the
    //      last is not live); rows past the layer read its last quad;
    //   W: piece pp of the tile's chunks, panel pp / 400, byte 16 (pp % 400):
    //      base wp + s chunks.  Pieces past the last chunk repeat piece 0
    //      into slot space no read uses; panels past the layer repeat its last.
    uint32_t voff[kOps];
#pragma unroll
    for (int k = 0; k < kOps; ++k) {
      if (k < kALoads) {
        const uint32_t i = kALoads * w + k;
        uint32_t quad, at;
        if (i < kACodes / 1024) {
          const uint32_t pp = i * 64 + lane, row = (pp / 2) % kBM;
          quad = row / 4;
          at = (row % 4) * 32 + (pp % 2) * 16;
        } else {
          quad = lane % 32;
          at = 128;
        }
        voff[k] = min(row0 / 4 + quad, g.quads - 1) * g.a_row * kDdrWord + at;
      } else {
        const uint32_t pp = (kWaves * (k - kALoads) + w) * 64 + lane;
        const uint32_t q = pp < C::kWPieces ? pp / (kW8Chunk / 16) : 0u;
        const uint32_t at = pp < C::kWPieces ? (pp % (kW8Chunk / 16)) * 16 : 0u;
        voff[k] = min(p0 + q, n_panels - 1) * steps * kW8Chunk + at;
      }
    }
    // Load cursor: the next step to load and its ring slot.  Steps past the
    // last load the last one again, so every wave issues kOps loads per
    // step, all in bounds.
    uint32_t ds = 0, dslot = 0;
    // load k of the step at s into the slot at LDS byte `slot`
    auto issue_op = [&](int k, uint32_t s, uint32_t slot) __attribute__((always_inline)) {
      if (k < kALoads) {
        const uint32_t i = kALoads * w + k;  // uniform
        const uint32_t h = i < kACodes / 1024 ? i / 4 : i % 2;
        Dma16(a + min(2 * s + h, nblocks - 1) * kDdrWord, voff[k], slot + i * 1024);
      } else {
        Dma16(wp + s * kW8Chunk, voff[k], slot + kSlotW + (kWaves * (k - kALoads) + w) * 1024);
      }
    };
    auto issue_advance = [&]() __attribute__((always_inline)) {
      ++ds;
      dslot = dslot + 1 == kD ? 0u : dslot + 1;
    };
    auto issue_next = [&]() __attribute__((always_inline)) {
      const uint32_t s = min(ds, steps - 1);
      const uint32_t slot = ring_base + dslot * kSlot;
#pragma unroll
      for (int k = 0; k < kOps; ++k) issue_op(k, s, slot);
      issue_advance();
    };

    // Reads from ring slot `slot`: W's B operands and scale dwords; this
    // lane's raw A codes and scale dword.
    auto read_w = [&](Ops<kNT>& o, uint32_t slot) __attribute__((always_inline)) {
      const uint8_t* wslot = lds_ring + slot * kSlot + kSlotW;
#pragma unroll
      for (int q = 0; q < kTP; ++q) {
        const uint8_t* chunk = wslot + q * kW8Chunk;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int l = 0; l < 2; ++l) {
            const uint32_t i = ((lane >> 5) * 2 + l) * kPanelCols + t * 32 + (lane & 31);
            const u32x4 v16 = *reinterpret_cast<const u32x4*>(chunk + i * 16);
            const u32x2 v8 = *reinterpret_cast<const u32x2*>(chunk + kW8Part8 + i * 8);
            o.b[2 * (2 * q + t) + l] = u32x6{v16[0], v16[1], v16[2], v16[3], v8[0], v8[1]};
          }
        o.sw[q] = *reinterpret_cast<const uint32_t*>(chunk + kW8Scales + lane * 4);
      }
    };
    auto read_a = [&](Ops<kNT>& o, uint32_t slot) __attribute__((always_inline)) {
      const uint8_t* abuf = lds_ring + slot * kSlot;
      o.x0 = *reinterpret_cast<const u32x4*>(abuf + (h * kBM + r) * 32);
      o.x1 = *reinterpret_cast<const u32x4*>(abuf + (h * kBM + r) * 32 + 16);
      o.sd = *reinterpret_cast<const uint32_t*>(abuf + kACodes + h * 1024 + (r / 4) * 16);
    };
    // A needs no mask: the one block past the last (block 2s + 1 of the
    // last step of an odd count, whose A is the last block again) meets zero
    // W codes in the chunk, and the loop has no step past the last.
    auto convert = [&](Ops<kNT>& o) __attribute__((always_inline)) {
      const uint32_t x[8] = {o.x0[0], o.x0[1], o.x0[2], o.x0[3],
                             o.x1[0], o.x1[1], o.x1[2], o.x1[3]};
      SplitA(x, 0xFFFFFFFFu, o.h, o.r);
      const uint32_t ea = __builtin_amdgcn_ubfe(o.sd, 8 * (r & 3), 8);
      o.sa = (int)(((ea - 5u) << 8) | ((ea - 1u) & 0xFFu));
      o.abad = ea - kSafeLo > kSafeHi - kSafeLo ? 1u : 0u;
    };

    // Prologue: steps 0 .. kD - 1 in flight (every slot); steps 0, 1 landed:
    // step 0's operands read and converted, step 1's raw A read.
#pragma unroll
    for (int v = 0; v < kD; ++v) issue_next();
    WaitVm<(kD - 2) * kOps>();
    __syncthreads();
    Ops<kNT> o0, o1;
    read_w(o0, 0);
    read_a(o0, 0);
    read_a(o1, 1);
    convert(o0);

    // Step u, ring slot u mod kD, operands in `use` (the set of u's parity):
    // wait for this wave's loads of step u + 2; barrier (every wave's loads
    // of step u + 2 landed; every wave done reading slot u: step u's W was
    // read in step u - 1, its A in step u - 2); refill slot u with step
    // u + kD; read step u + 1's W into `oth` and step u + 2's raw A into
    // `use`; convert step u + 1's raw A (held in `oth`) while the matrix
    // cores run step u.  (Reads and conversions past the last step work on
    // repeated data and go unused.)
    uint32_t slot = 0;
    auto iteration = [&](Ops<kNT>& use, Ops<kNT>& oth) __attribute__((always_inline)) {
      WaitVm<(kD - 3) * kOps>();
      WaitLds();
      __syncthreads();
      // the refill's loads go out between the step's MFMAs (one after every
      // kEvery), not in a burst ahead of them
      const uint32_t is_s = min(ds, steps - 1), is_slot = ring_base + dslot * kSlot;
      const uint32_t s1 = slot + 1 == kD ? 0u : slot + 1;
      const uint32_t s2 = s1 + 1 == kD ? 0u : s1 + 1;
      read_w(oth, s1);
      read_a(use, s2);
      convert(oth);
      slot = s1;
      bad |= use.abad;
      const i32x8 ah = {(int)use.h[0], (int)use.h[1], (int)use.h[2], (int)use.h[3],
                        (int)use.h[4], (int)use.h[5], 0, 0};
      const i32x8 ar = {(int)use.r[0], (int)use.r[1], (int)use.r[2], (int)use.r[3],
                        (int)use.r[4], (int)use.r[5], 0, 0};
      // product (A plane pa, W plane pl) over the n-tiles, for each of the
      // four products (n-tiles past the layer compute outputs not stored)
      constexpr int kM = 4 * kNT, kEvery = (kM + kOps - 1) / kOps;
      Unroll<4>([&](auto pc) {
        constexpr int kPa = decltype(pc)::value / 2, kPl = decltype(pc)::value % 2;
        Unroll<kNT>([&](auto tc) {
          constexpr int kT = decltype(tc)::value;
          constexpr int kI = decltype(pc)::value * kNT + kT;  // MFMA index in the step
          const u32x6& bv = use.b[2 * kT + kPl];
          const i32x8 bt = {(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3], (int)bv[4], (int)bv[5],
                            0, 0};
          acc[kT] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              kPa ? ar : ah, bt, acc[kT], 2, 2, kPa, use.sa, 2 * (kT % 2) + kPl,
              (int)use.sw[kT / 2]);
          if constexpr ((kI + 1) % kEvery == 0 && (kI + 1) / kEvery <= kOps) {
            // (the empty asm takes this MFMA's result: the MFMA issues first)
            asm volatile("" ::"a"(acc[kT]));
            issue_op((kI + 1) / kEvery - 1, is_s, is_slot);
          }
        });
      });
#pragma unroll
      for (int k = kM / kEvery; k < kOps; ++k) issue_op(k, is_s, is_slot);
      issue_advance();
#pragma unroll
      for (int t = 0; t < kNT; ++t) asm volatile("" : "+a"(acc[t]));
      asm volatile("" : "+v"(oth.h), "+v"(oth.r), "+v"(oth.sa), "+v"(oth.abad));
    };
    for (uint32_t s = 0; s + 1 < steps; s += 2) {
      iteration(o0, o1);
      iteration(o1, o0);
    }
    if (steps & 1) iteration(o0, o1);
    WaitVm<0>();  // no load into LDS outlives the K loop
  }
  __syncthreads();  // every wave's loads landed and reads done: the ring is free

  // Epilogue through the ring: the activation half of TBUF at byte 0; wave
  // w's 32 rows of outputs row-major, [32][kPitch] floats from kStage.
  // Lane l then finishes, per n-tile, columns 4 (l % 8) .. + 3 of the tile
  // in rows l / 8 + 8 i, i = 0..3 (a row's 32 columns on 8 lanes): C in
  // 16-byte stores, the requantize's block maximum over those 8 lanes and
  // its bytes in dword stores.
  // The tile's columns of each op's vector (ADDP, MULP) follow the outputs,
  // [op][kNT * 32] floats from kVec (loaded once, before any store).
  constexpr uint32_t kPitch = kNT * 32 + 4;
  constexpr uint32_t kVec = kStage + kWaves * 32 * kPitch * 4;
  static_assert(kVec + kMaxOps * kNT * 32 * 4 <= kD * kSlot, "epilogue staging");
  uint64_t* lds_act = reinterpret_cast<uint64_t*>(lds_ring);
  float* st = reinterpret_cast<float*>(lds_ring + kStage) + w * 32 * kPitch;
  float* lds_vec = reinterpret_cast<float*>(lds_ring + kVec);
  if (g.tbuf != nullptr)
    for (uint32_t i = threadIdx.x; i < 512; i += 256) lds_act[i] = g.tbuf[512 + i];
  if (fast)
    for (uint32_t i = threadIdx.x; i < g.n_ops * kNT * 32; i += 256) {
      const uint32_t o = i / (kNT * 32), kind = g.op_kind[o];
      if (kind == kEpAddP || kind == kEpMulP)
        lds_vec[i] = __uint_as_float(
            g.op_vec[o][tile.z * g.op_vec_batch[o] + min(col0 + i % (kNT * 32), g.n - 1)]);
    }
  const bool slow = !fast || __builtin_amdgcn_readfirstlane(
                                 __builtin_amdgcn_ballot_w64(bad != 0) != 0);
  // output (n-tile t, register e) of the MFMA layout: tile row
  // 4 (lane / 32) + 8 (e / 4) + e % 4, tile column 32 t + lane % 32
  if (!slow) {  // +0 maps -0 (and, flushed, a denormal sum) to +0
#pragma unroll
    for (int t = 0; t < kNT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st[(4 * (lane >> 5) + 8 * (e / 4) + (e & 3)) * kPitch + t * 32 + (lane & 31)] =
            acc[t][e] + 0.0f;
  } else {  // every output of the wave's rows by the exact fold
    for (uint32_t t = 0; t < live_nt; ++t)
      for (uint32_t e = 0; e < 16; ++e) {
        const uint32_t tr = 4 * (lane >> 5) + 8 * (e / 4) + (e & 3);
        const uint32_t row = row_w + tr, col = col0 + t * 32 + (lane & 31);
        uint32_t v = 0;
        if ((row >> 2) < g.quads && col < g.n) {
          const uint32_t init = (g.acc && row < g.m) ? c[(size_t)row * g.n + col] : 0u;
          v = SlowLinear<3>(g, a, wp, wp, init, row, col);
        }
        st[tr * kPitch + t * 32 + (lane & 31)] = __uint_as_float(v);
      }
  }
  __syncthreads();

  const uint32_t cg = lane & 7, rs = lane >> 3;
  if (!fast) {  // exact mode: the VEC lane formulas, element by element in LDS
    for (uint32_t t = 0; t < live_nt; ++t) {
      const uint32_t lc = t * 32 + 4 * cg, col = col0 + lc;
      for (uint32_t o = 0; o < g.n_ops; ++o) {
        const uint32_t kind = g.op_kind[o];
        const uint32_t* x2 = g.op_x2[o] ? g.op_x2[o] + tile.z * g.op_x2_batch[o] : nullptr;
        for (uint32_t e = 0; e < 16; ++e) {
          const uint32_t i = e / 4, j = e % 4, row = row_w + rs + 8 * i;
          const uint32_t p = (kind == kEpAddP || kind == kEpMulP) && col < g.n
                                 ? g.op_vec[o][tile.z * g.op_vec_batch[o] + col + j] : 0u;
          const uint32_t xv = (kind == kEpAdd || kind == kEpActMul) && row < g.m && col < g.n
                                  ? x2[(size_t)row * g.n + col + j] : 0u;
          float& y = st[(rs + 8 * i) * kPitch + lc + j];
          y = __uint_as_float(EpApply(kind, g.op_imm[o], __float_as_uint(y), xv, p, lds_act));
        }
      }
    }
  }

  // Fast-mode ops, one n-tile at a time (a rolled loop: the body stays in
  // the instruction cache), its 16 values per lane in registers and back
  // into the staging: y[4 i + j] is row rs + 8 i, column 32 t + 4 cg + j of
  // the wave's tile.  Every load of this pass precedes every store of the
  // next (loads and stores share one counter: a load behind a store waits
  // for it), and addresses are clamped into the layer instead of guarded,
  // so the loads are branch-free; values past the layer are not stored.
  auto load_y = [&](uint32_t t, f32x16& y) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = *reinterpret_cast<const float4*>(st + (rs + 8 * i) * kPitch + t * 32 + 4 * cg);
      y[4 * i] = v.x;
      y[4 * i + 1] = v.y;
      y[4 * i + 2] = v.z;
      y[4 * i + 3] = v.w;
    }
  };
  // One op over every n-tile, the op's kind a constant in each copy of the
  // tile loop (the switch is taken once per op, not per tile).
  auto apply = [&](uint32_t o, auto kind_c) __attribute__((always_inline)) {
    constexpr uint32_t kKind = decltype(kind_c)::value;
    const uint32_t imm = g.op_imm[o];
    const uint32_t* src = kKind == kEpAdd || kKind == kEpActMul
                              ? g.op_x2[o] + tile.z * g.op_x2_batch[o] : nullptr;
    const float* pv = lds_vec + o * kNT * 32;
    for (uint32_t t = 0; t < live_nt; ++t) {
      f32x16 y, x2 = {}, p = {};
      load_y(t, y);
      if (kKind == kEpAdd || kKind == kEpActMul) {
        const uint32_t colc = min(col0 + t * 32 + 4 * cg, g.n - 4);
#pragma unroll
        for (int e = 0; e < 16; ++e) {  // rows past the layer (its last quad's) take 0
          const uint32_t row = row_w + rs + 8 * (e / 4);
          const uint32_t v = src[(size_t)min(row, g.m - 1) * g.n + colc + e % 4];
          x2[e] = __uint_as_float(row < g.m ? v : 0u);
        }
      }
      if (kKind == kEpAddP || kKind == kEpMulP) {
        const float4 v = *reinterpret_cast<const float4*>(pv + t * 32 + 4 * cg);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[4 * i] = v.x;
          p[4 * i + 1] = v.y;
          p[4 * i + 2] = v.z;
          p[4 * i + 3] = v.w;
        }
      }
      EpApplyFast16<false>(kKind, imm, y, x2, p, lds_act);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(st + (rs + 8 * i) * kPitch + t * 32 + 4 * cg) =
            float4{y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]};
    }
  };
  for (uint32_t o = 0; fast && o < g.n_ops; ++o) {  // FP32 hardware arithmetic
    switch (g.op_kind[o]) {
      case kEpAddP: apply(o, std::integral_constant<uint32_t, kEpAddP>{}); break;
      case kEpMulP: apply(o, std::integral_constant<uint32_t, kEpMulP>{}); break;
      case kEpScale: apply(o, std::integral_constant<uint32_t, kEpScale>{}); break;
      case kEpCopy: apply(o, std::integral_constant<uint32_t, kEpCopy>{}); break;
      case kEpRelu: apply(o, std::integral_constant<uint32_t, kEpRelu>{}); break;
      case kEpAdd: apply(o, std::integral_constant<uint32_t, kEpAdd>{}); break;
      case kEpAct: apply(o, std::integral_constant<uint32_t, kEpAct>{}); break;
      case kEpActMul: apply(o, std::integral_constant<uint32_t, kEpActMul>{}); break;
      default: break;
    }
  }

  // C and requantize.
  const bool c_vec = (reinterpret_cast<uintptr_t>(c) & 15) == 0;
  const bool q_vec = (reinterpret_cast<uintptr_t>(q_out) & 3) == 0;
  for (uint32_t t = 0; t < live_nt; ++t) {
    const uint32_t col = col0 + t * 32 + 4 * cg;  // col < n: all 4 columns are (n % 8 == 0)
    f32x16 y;
    load_y(t, y);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = row_w + rs + 8 * i;
      if (row < g.m && col < g.n && g.c != nullptr) {
        uint32_t* out = c + (size_t)row * g.n + col;
        if (c_vec) {
          *reinterpret_cast<float4*>(out) = float4{y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]};
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) out[j] = __float_as_uint(y[4 * i + j]);
        }
      }
    }
    if (q_out == nullptr) continue;
    // MXINT8 requantize: a row's block is its 32 columns of the n-tile, on
    // the 8 lanes 8 rs .. 8 rs + 7.  Their largest exponent field by DPP
    // moves within the lane octet: swap neighbours, swap pairs, mirror.
    const uint32_t nb = g.n >> 5, blk = (col0 >> 5) + t;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = row_w + rs + 8 * i;
      uint32_t x = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) x = max(x, ExpField(__float_as_uint(y[4 * i + j])));
      x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));
      x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));
      x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false));
      uint32_t packed = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        packed |= (uint32_t)QuantizeElementHw(__float_as_uint(y[4 * i + j]), x) << (8 * j);
      if ((row >> 2) < g.quads && blk < nb) {
        uint8_t* word = q_out + ((size_t)(row >> 2) * nb + blk) * kDdrWord;
        uint8_t* dst = word + (row & 3) * 32 + 4 * cg;
        if (q_vec) {
          *reinterpret_cast<uint32_t*>(dst) = packed;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[j] = (uint8_t)(packed >> (8 * j));
        }
        if (cg == 0) word[128 + (row & 3)] = (uint8_t)ScaleByteOf(x);
        if ((row & 3) == 0 && cg >= 1 && cg <= 3) {
          uint8_t* pad = word + 132 + 4 * (cg - 1);
#pragma unroll
          for (int j = 0; j < 4; ++j) pad[j] = 0;
        }
      }
    }
  }
}

// Packer: one thread per 32-code column-block of one plane, in chunk order
// (the chunk's 256 column-blocks: b, then plane, then column).
__global__ __launch_bounds__(256) void PackW8Kernel(const uint8_t* hi, const uint8_t* lo,
                                                    uint32_t n, uint32_t kb_total, uint8_t* out,
                                                    uint32_t* flags, uint64_t count) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const uint32_t steps = (kb_total + 1) / 2;
  const uint32_t c = (uint32_t)(i % kPanelCols), l = (uint32_t)((i / kPanelCols) % 2);
  const uint32_t b = (uint32_t)((i / (2 * kPanelCols)) % 2);
  const uint64_t chunk = i / (4 * kPanelCols);  // panel * steps + step
  const uint32_t step = (uint32_t)(chunk % steps), panel = (uint32_t)(chunk / steps);
  const uint32_t col = panel * kPanelCols + c, blk = 2 * step + b;
  f16x32 v = {};
  uint32_t scale = 127;
  if (col < n && blk < kb_total) {
    const uint8_t* word = (l ? lo : hi) + ((uint64_t)(col / 8) * kb_total + blk) * kDdrWord;
    const u32x4 x = *reinterpret_cast<const u32x4*>(word + (col % 8) * 16);
#pragma unroll
    for (int k = 0; k < 32; ++k) {  // element k: nibble k % 2 of byte k / 2
      const uint32_t nib = (x[k / 8] >> (4 * (k % 8))) & 15u;
      const int val = l ? (int)nib : ((nib & 8u) ? (int)nib - 16 : (int)nib);
      v[k] = (_Float16)((float)val * 0.5f);
    }
    scale = word[128 + col % 8];
    if (scale - kSafeLo > kSafeHi - kSafeLo) flags[panel] = 1u;  // every writer stores 1
  }
  const u32x6 f6 = __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(v, 1.0f);
  uint8_t* dst = out + chunk * kW8Chunk;
  const uint32_t idx = (b * 2 + l) * kPanelCols + c;
  *reinterpret_cast<u32x4*>(dst + idx * 16) = u32x4{f6[0], f6[1], f6[2], f6[3]};
  *reinterpret_cast<u32x2*>(dst + kW8Part8 + idx * 8) = u32x2{f6[4], f6[5]};
  dst[kW8Scales + (b * 32 + c % 32) * 4 + 2 * (c / 32) + l] = (uint8_t)(scale - (l ? 5u : 1u));
}

__global__ __launch_bounds__(256) void ZeroFlagsKernel(uint32_t* flags, uint32_t count) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) flags[i] = 0;
}

// Unpacker: one thread per 16-byte column-block of one plane's DDR words;
// the thread of column 8g holds the word's padding too.
__global__ __launch_bounds__(256) void UnpackW8Kernel(const uint8_t* in, uint32_t n,
                                                      uint32_t kb_total, uint8_t* hi, uint8_t* lo) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= 2ull * n * kb_total) return;
  const uint32_t l = (uint32_t)(i / ((uint64_t)n * kb_total));
  const uint64_t j = i % ((uint64_t)n * kb_total);
  const uint32_t cl = (uint32_t)(j % 8), blk = (uint32_t)((j / 8) % kb_total);
  const uint32_t grp = (uint32_t)(j / (8ull * kb_total)), col = grp * 8 + cl;
  const uint32_t steps = (kb_total + 1) / 2, c = col % kPanelCols, b = blk % 2;
  const uint8_t* chunk = in + ((uint64_t)(col / kPanelCols) * steps + blk / 2) * kW8Chunk;
  const uint32_t idx = (b * 2 + l) * kPanelCols + c;
  const u32x4 d0 = *reinterpret_cast<const u32x4*>(chunk + idx * 16);
  const u32x2 d1 = *reinterpret_cast<const u32x2*>(chunk + kW8Part8 + idx * 8);
  const u32x6 f6 = {d0[0], d0[1], d0[2], d0[3], d1[0], d1[1]};
  const f16x32 v = __builtin_amdgcn_cvt_scalef32_pk32_f16_fp6(f6, 1.0f);
  u32x4 x = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint32_t nib = (uint32_t)(int)(float)(v[k] * (_Float16)2.0f) & 15u;
    x[k / 8] |= nib << (4 * (k % 8));
  }
  uint8_t* word = (l ? lo : hi) + ((uint64_t)grp * kb_total + blk) * kDdrWord;
  *reinterpret_cast<u32x4*>(word + cl * 16) = x;
  word[128 + cl] = (uint8_t)(chunk[kW8Scales + (b * 32 + c % 32) * 4 + 2 * (c / 32) + l] +
                             (l ? 5u : 1u));
  if (cl == 0) *reinterpret_cast<uint2*>(word + 136) = uint2{0u, 0u};
}

// Estimated cycles of one K step of a tile, by panels per tile (the
// matrix-core time of its 8 kTP MFMAs plus the LDS reads and the A split
// that do not overlap them).
uint32_t StepCycles(int tp) { return 420u * (uint32_t)tp + 300u; }


template <int kTP>
void Launch(const GemmArgs& args, hipStream_t stream) {
  hipLaunchKernelGGL(W8Kernel<kTP>, dim3(args.gx * args.gy * args.gz), dim3(256), 0, stream,
                     args);
}

}  // namespace

uint32_t BandFor(uint32_t gx, uint32_t gy, uint64_t a_tile, uint64_t w_tile) {
  const uint64_t run = std::max<uint64_t>(1, (uint64_t)gx * gy / kXcds);
  uint32_t best = gx;
  uint64_t best_bytes = ~0ull;
  for (uint32_t b = 1; b <= gx; ++b) {
    const uint64_t rows = std::min<uint64_t>(gy, (run + b - 1) / b);
    const uint64_t cols = std::min<uint64_t>(b, run);
    const uint64_t bytes = rows * a_tile + cols * w_tile;
    if (bytes < best_bytes) {
      best_bytes = bytes;
      best = b;
    }
  }
  return best;
}

int DeviceCus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

hipError_t LaunchW8Linear(const GemmArgs& in, uint32_t batch, bool fast, hipStream_t stream) {
  GemmArgs args = in;
  args.fast_ep = fast ? 1u : 0u;
  args.ws = nullptr;
  args.splits = 1;
  args.gy = (args.quads * 4 + kBM - 1) / kBM;
  args.gz = batch;
  // Panels per tile (1 to 4): the width whose rounds of workgroups over the
  // CUs take the fewest estimated cycles (wider tiles do more work per step,
  // narrower ones make more tiles).  Measured at M = 2048, K = 768 and 3072,
  // N = 768: 1 panel (192 tiles) 14.9 and 32.7 us against 18.7 and 43.3 us
  // at 2 panels (96 tiles).
  const uint64_t cus = (uint64_t)DeviceCus();
  const uint32_t n_panels = (args.n + kPanelCols - 1) / kPanelCols;
  int best = 4;
  uint64_t best_cost = ~0ull;
  for (int tp = 4; tp >= 1; --tp) {
    const uint64_t tiles = (uint64_t)((n_panels + tp - 1) / tp) * args.gy * batch;
    const uint64_t cost = (tiles + cus - 1) / cus * (uint64_t)StepCycles(tp);
    if (cost < best_cost) {
      best_cost = cost;
      best = tp;
    }
  }
  args.gx = (n_panels + best - 1) / best;
  if ((uint64_t)args.gx * args.gy * args.gz >= (1ull << 31)) return hipErrorInvalidValue;
  // A row tile: kBM rows x kb_total blocks of 36 bytes (32 codes, a scale);
  // a column tile: `best` panels of w_steps chunks
  args.band = BandFor(args.gx, args.gy, (uint64_t)kBM * args.kb_total * 36,
                      (uint64_t)best * args.w_steps * kW8Chunk);
  if (best == 4) Launch<4>(args, stream);
  else if (best == 3) Launch<3>(args, stream);
  else if (best == 2) Launch<2>(args, stream);
  else Launch<1>(args, stream);
  return hipGetLastError();
}

hipError_t LaunchPackW8(const uint8_t* hi, const uint8_t* lo, uint32_t n, uint32_t kb_total,
                        uint8_t* out, hipStream_t stream) {
  const uint32_t n_panels = (n + kPanelCols - 1) / kPanelCols;
  uint32_t* flags = reinterpret_cast<uint32_t*>(out + W8FlagsOffset(n, kb_total));
  hipLaunchKernelGGL(ZeroFlagsKernel, dim3((n_panels + 255) / 256), dim3(256), 0, stream, flags,
                     n_panels);
  const uint64_t count = (uint64_t)n_panels * ((kb_total + 1) / 2) * 4 * kPanelCols;
  hipLaunchKernelGGL(PackW8Kernel, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, stream,
                     hi, lo, n, kb_total, out, flags, count);
  return hipGetLastError();
}

hipError_t LaunchUnpackW8(const uint8_t* in, uint32_t n, uint32_t kb_total, uint8_t* hi,
                          uint8_t* lo, hipStream_t stream) {
  const uint64_t count = 2ull * n * kb_total;
  hipLaunchKernelGGL(UnpackW8Kernel, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, stream,
                     in, n, kb_total, hi, lo);
  return hipGetLastError();
}

}  // namespace hb

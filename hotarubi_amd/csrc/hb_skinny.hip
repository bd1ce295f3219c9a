// Skinny fast linear kernel for gfx950 (HB_LINEAR_FAST, a batch of layers of
// at most 16 rows each): MXFP4 or W8 weights streamed from HBM straight into
// the matrix cores.
//
// Matrix cores: v_mfma_scale_f32_16x16x128_f8f6f4.  One lane's A operand is
// 32 values of one row and one K-block (lane l: row l % 16, block l / 16 of
// a 4-block chunk), one lane's B operand 32 values of one column and block,
// each with its own E8M0 scale; the formats and scale bytes are those of the
// 128-row fast kernel (A as FP6 planes hi/2, lo/2 with ea-1, ea-5; MXFP4 W
// untouched; W8 W as FP6 planes with ew-1, ew-5, K in the W8 byte order).
//
// Work split: a workgroup holds every row (16 * kMT) and kCols
// columns; its 8 waves take contiguous ranges of 4-block K chunks (split-K).
// Each lane loads its own A bytes and W column-block (16 B per plane, the
// WBUF word layout) into registers, converts, and issues the chunk's MFMAs;
// the next chunk's loads are in flight meanwhile.  No LDS staging: no A or W
// byte is converted twice in a workgroup.  The waves' partial sums are then
// added in wave order through LDS, and the epilogue (ops in FP32 hardware
// arithmetic, C, requantize) runs over the workgroup's outputs.
#include <algorithm>
#include <utility>

#include "hb_device.h"
#include "hb_internal.h"

namespace hb {
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x6 __attribute__((ext_vector_type(6)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x32 __attribute__((ext_vector_type(32)));

constexpr int kWaves = 8;
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;

// Columns per workgroup: 16 * kNT, with the accumulators (kMT * kNT * 4) and
// two chunks of raw loads within the registers of a wave.  MXFP4 at 16 rows
// of one piece keeps to 128 registers (WavesPerSimd 4), so two workgroups
// share a CU and one's reduction and epilogue overlap the other's loads; the
// others take up to 256 (one workgroup per CU: several pieces' block lookup
// spilled to scratch at 128).
template <int kMT, bool kW8>
constexpr int NTiles() {
  return kW8 ? (kMT == 4 ? 2 : 4) : 4;
}
template <int kMT, bool kW8, bool kMulti>
constexpr int WavesPerSimd() {
  return kMT == 1 && !kW8 && !kMulti ? 4 : 2;
}

template <bool kMulti>
__device__ __forceinline__ uint32_t SkinnyBlockOf(const GemmArgs& g, uint32_t idx) {
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

// f16 pair {byte i, byte j of nb} minus bias (see the 128-row kernel).
__device__ __forceinline__ f16x2 PairS(uint32_t nb, uint32_t sel, f16x2 bias) {
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x60606060u, nb, sel)) - bias;
}
constexpr uint32_t SelS(uint32_t i, uint32_t j) { return 0x04000400u | i | (j << 16); }

// 32 int8 -> one FP6 plane (hi/2 or lo/2); kPermK: K in the W8 order.
template <bool kPermK>
__device__ __forceinline__ u32x6 APlane(const uint32_t* x, uint32_t nib, bool lo) {
  const uint32_t shift = lo ? 0u : 4u, flip = lo ? 0u : 0x08080808u;
  const _Float16 b = lo ? (_Float16)512.0f : (_Float16)516.0f;
  const f16x2 bias = {b, b};
  f16x32 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n0 = ((x[2 * i] >> shift) & nib) ^ flip;
    const uint32_t n1 = ((x[2 * i + 1] >> shift) & nib) ^ flip;
    f16x2 d[4];
    if (kPermK) {
      d[0] = PairS(n0, SelS(0, 2), bias);
      d[1] = PairS(n1, SelS(0, 2), bias);
      d[2] = PairS(n0, SelS(1, 3), bias);
      d[3] = PairS(n1, SelS(1, 3), bias);
    } else {
      d[0] = PairS(n0, SelS(0, 1), bias);
      d[1] = PairS(n0, SelS(2, 3), bias);
      d[2] = PairS(n1, SelS(0, 1), bias);
      d[3] = PairS(n1, SelS(2, 3), bias);
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      v[8 * i + 2 * p] = d[p][0];
      v[8 * i + 2 * p + 1] = d[p][1];
    }
  }
  return __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(v, 1.0f);
}

// One W8 plane's 16 bytes -> 32 FP6 codes, K in the W8 order.
__device__ __forceinline__ u32x6 WPlane(const uint32_t* x, bool lo) {
  const uint32_t flip = lo ? 0u : 0x88888888u;
  const _Float16 b = lo ? (_Float16)512.0f : (_Float16)516.0f;
  const f16x2 bias = {b, b};
  f16x32 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t y = x[j] ^ flip;
    const uint32_t ev = y & 0x0F0F0F0Fu, od = (y >> 4) & 0x0F0F0F0Fu;
    const f16x2 d[4] = {PairS(ev, SelS(0, 1), bias), PairS(ev, SelS(2, 3), bias),
                        PairS(od, SelS(0, 1), bias), PairS(od, SelS(2, 3), bias)};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      v[8 * j + 2 * p] = d[p][0];
      v[8 * j + 2 * p + 1] = d[p][1];
    }
  }
  return __builtin_amdgcn_cvt_scalef32_pk32_fp6_f16(v, 1.0f);
}

template <typename Fn, int... kI>
__device__ __forceinline__ void UnrollS(Fn&& f, std::integer_sequence<int, kI...>) {
  (f(std::integral_constant<int, kI>{}), ...);
}

// One chunk's raw registers: per m-tile 32 A bytes and the scale dword, per
// n-tile and plane 16 W bytes and the scale dword.
template <int kMT, int kNT, int kWP>
struct RawS {
  uint32_t a[kMT][8], sa[kMT];
  uint32_t w[kNT][kWP][4], sw[kNT][kWP];
  uint32_t nib;  // 0x0F0F0F0F, or 0 for a block past the end (adds zero)
};

// kA8 (MXFP8 activations, kMT 1, MXFP4 W): the code bytes are the MFMA's
// FP8 operand, which takes K in 16-wide chunks: lane group q = l / 16
// holds K [16 q, 16 q + 16) of the 128-deep chunk in registers 0-3 and K
// [64 + 16 q, + 16) in registers 4-7, i.e. bytes [16 (q % 2), + 16) of its
// row in blocks q / 2 and 2 + q / 2, while its scale byte is still block
// q's.  Each chunk's codes go through two MFMAs, split by exponent
// (fp8::Split), as in the other MXFP8 kernels.
template <int kMT, bool kW8, bool kMulti, bool kPanels, bool kA8 = false>
__global__ __launch_bounds__(kWaves * 64, (WavesPerSimd<kMT, kW8, kMulti>())) void SkinnyKernel(GemmArgs g) {
  static_assert(!kA8 || (kMT == 1 && !kW8), "MXFP8 activations: 16 rows, MXFP4 W");
  constexpr int kNT = NTiles<kMT, kW8>(), kCols = 16 * kNT, kWP = kW8 ? 2 : 1;
  constexpr int kRows = 16 * kMT, kOut = kRows * kCols;
  __shared__ float lds_part[kWaves][kOut];  // the waves' partial sums
  __shared__ uint64_t lds_act[512];
  __shared__ uint32_t lds_unsafe;

  const TileId tile = LogicalTile(g.gx, 1, g.gz);
  const uint32_t z = tile.z;
  const uint8_t* a = g.a + z * g.a_batch;
  const uint8_t* w0 = g.w[0] + z * g.w_batch;
  const uint8_t* w1 = kW8 ? g.w[1] + z * g.w_batch : w0;
  uint32_t* c = g.c + z * g.c_batch;
  uint8_t* q_out = g.q_out ? g.q_out + z * g.q_batch : nullptr;
  const uint32_t col0 = tile.x * kCols;
  const uint32_t t = threadIdx.x, lane = t & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t r16 = lane & 15, kq = lane >> 4;

  if (t == 0) lds_unsafe = 0;
  if (g.tbuf != nullptr)
    for (uint32_t i = t; i < 512; i += kWaves * 64) lds_act[i] = g.tbuf[512 + i];
  __syncthreads();

  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < g.n_pieces; ++p) nblocks += g.piece_kb[p];
  const uint32_t chunks = (nblocks + 3) / 4, per = (chunks + kWaves - 1) / kWaves;
  const uint32_t c_begin = wave * per, c_end = min(c_begin + per, chunks);
  const uint32_t word_row = g.kb_total * kDdrWord, a_row = g.a_row * kDdrWord;

  // Per-lane byte offsets within a block's words (fixed for the K loop).
  // The lane's row within a quad (r16 % 4) and column within a group (r16 %
  // 8) are the same in every tile, so the scale dword's offset from the data
  // and the scale byte's position are per lane, not per tile.
  // W in DDR words: the scale dword's offset from the codes and the scale
  // byte's position are per lane too (one register per column tile); in
  // panels (WLane) they differ between the lane's column tiles.  A column
  // past the layer reads the last group's column at the same position (its
  // outputs are not stored).
  const uint32_t ashift = 8 * (r16 & 3), as_delta = 128 - (r16 & 3) * 32;
  const uint32_t cl = r16 & 7, wshift_ddr = 8 * (cl & 3), ws_delta = 128 + (cl & 4) - cl * 16;
  uint32_t a_off[kMT], w_off[kNT];
#pragma unroll
  for (int mi = 0; mi < kMT; ++mi) {
    const uint32_t quad = min((mi * 16 + r16) >> 2, g.quads - 1);
    a_off[mi] = quad * a_row + (r16 & 3) * 32;
  }
  // Panels: the workgroup's 64 columns are one panel (col0 is a multiple of
  // 64; columns past n are zero codes there), column nj * 16 + r16 of it,
  // so column tile nj's offsets are column tile 0's plus constants: codes
  // + 256 nj, scale dword + 32 (nj % 2), scale byte shift + 8 (nj / 2).
  // Three registers per lane instead of three per column tile.
  static_assert(!kPanels || kCols == (int)kPanelCols, "one panel per workgroup");
  [[maybe_unused]] WLaneOff pw{};
  if constexpr (kPanels) {
    pw = WLane(g, col0 + r16, true);
  } else {
#pragma unroll
    for (int nj = 0; nj < kNT; ++nj) {
      const uint32_t grp = min((col0 + nj * 16 + r16) >> 3, g.groups - 1);
      w_off[nj] = grp * word_row + cl * 16;
    }
  }

  // Loads of chunk ch (its lane's block); a chunk at or past c_end, or a
  // block past the end, reloads a valid block and adds zero.
  auto load = [&](RawS<kMT, kNT, kWP>& rw, uint32_t ch) {
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t idx = 4 * ch + kq;
    rw.nib = (ch < c_end && idx < nblocks) ? 0x0F0F0F0Fu : 0u;
    const uint32_t ublk = SkinnyBlockOf<kMulti>(g, min(idx, nblocks - 1));
    const uint32_t blk = ublk * kDdrWord;
    const uint32_t wbc = kPanels ? WBlockCodes(g, ublk) : blk;
    const uint32_t wbs = kPanels ? WBlockScale(g, ublk) : blk;
    if constexpr (kA8) {  // the two 16-byte chunks (blocks 4 ch + q / 2 and + 2); nib bit i: chunk i live
      const uint32_t i0 = 4 * ch + (kq >> 1), i1 = i0 + 2;
      rw.nib = (ch < c_end && i0 < nblocks ? 1u : 0u) | (ch < c_end && i1 < nblocks ? 2u : 0u);
      const uint32_t b0 = SkinnyBlockOf<kMulti>(g, min(i0, nblocks - 1)) * kDdrWord;
      const uint32_t b1 = SkinnyBlockOf<kMulti>(g, min(i1, nblocks - 1)) * kDdrWord;
      const uint32_t at = a_off[0] + 16 * (kq & 1);  // the row's codes, this half
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(a + b0 + at);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(a + b1 + at);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[0][i] = v0[i];
        rw.a[0][4 + i] = v1[i];
      }
      rw.sa[0] = *reinterpret_cast<const uint32_t*>(a + blk + a_off[0] + as_delta);
    }
#pragma unroll
    for (int mi = 0; mi < (kA8 ? 0 : kMT); ++mi) {
      const uint8_t* p = a + blk + a_off[mi];
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[mi][i] = v0[i];
        rw.a[mi][4 + i] = v1[i];
      }
      rw.sa[mi] = *reinterpret_cast<const uint32_t*>(a + blk + a_off[mi] + as_delta);
    }
#pragma unroll
    for (int nj = 0; nj < kNT; ++nj)
#pragma unroll
      for (int pl = 0; pl < kWP; ++pl) {
        const uint8_t* wp = pl ? w1 : w0;
        const uint8_t* wc = wp + wbc + (kPanels ? pw.codes + 256u * nj : w_off[nj]);
        const u32x4 v = *reinterpret_cast<const u32x4*>(wc);
#pragma unroll
        for (int i = 0; i < 4; ++i) rw.w[nj][pl][i] = v[i];
        // (DDR words: the scale as an offset from the codes' address, so no
        // per-tile sum stays live across the K loop)
        rw.sw[nj][pl] = *reinterpret_cast<const uint32_t*>(
            kPanels ? wp + wbs + pw.scale + 32u * (nj % 2) : wc + ws_delta);
      }
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x4 acc[kMT][kNT];
#pragma unroll
  for (int mi = 0; mi < kMT; ++mi)
#pragma unroll
    for (int nj = 0; nj < kNT; ++nj) acc[mi][nj] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  bool unsafe = false;

  auto compute = [&](const RawS<kMT, kNT, kWP>& rw) {
    i32x8 b[kNT][kWP];
    uint32_t sb[kNT];
#pragma unroll
    for (int nj = 0; nj < kNT; ++nj) {
      const uint32_t sh = kPanels ? pw.shift + 8u * (nj / 2) : wshift_ddr;
      const uint32_t ewh = __builtin_amdgcn_ubfe(rw.sw[nj][0], sh, 8);
      unsafe |= ewh - kSafeLo > kSafeHi - kSafeLo;
      if constexpr (kW8) {
        const uint32_t ewl = __builtin_amdgcn_ubfe(rw.sw[nj][1], sh, 8);
        unsafe |= ewl - kSafeLo > kSafeHi - kSafeLo;
        sb[nj] = (ewh - 1u) | ((ewl - 5u) << 8);
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) {
          const u32x6 cw = WPlane(rw.w[nj][pl], pl != 0);
#pragma unroll
          for (int i = 0; i < 6; ++i) b[nj][pl][i] = (int)cw[i];
          b[nj][pl][6] = b[nj][pl][7] = 0;
        }
      } else {
        sb[nj] = ewh;
#pragma unroll
        for (int i = 0; i < 4; ++i) b[nj][0][i] = (int)rw.w[nj][0][i];
        b[nj][0][4] = b[nj][0][5] = b[nj][0][6] = b[nj][0][7] = 0;
      }
    }
    if constexpr (kA8) {
      const uint32_t ea = __builtin_amdgcn_ubfe(rw.sa[0], ashift, 8);
      unsafe |= ea - kSafeLo > kSafeHi - kSafeLo;
      const uint32_t keep0 = (rw.nib & 1u) ? ~0u : 0u, keep1 = (rw.nib & 2u) ? ~0u : 0u;
      i32x8 a_lo, a_hi;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t lo, hi;
        fp8::Split(rw.a[0][i] & (i < 4 ? keep0 : keep1), lo, hi);
        a_lo[i] = (int)lo;
        a_hi[i] = (int)hi;
      }
      UnrollS([&](auto nj_c) {
        constexpr int nj = decltype(nj_c)::value;
        acc[0][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a_lo, b[nj][0], acc[0][nj], 0, 4,
                                                                       0, (int)ea, 0, (int)sb[nj]);
      }, std::make_integer_sequence<int, kNT>{});
      UnrollS([&](auto nj_c) {
        constexpr int nj = decltype(nj_c)::value;
        acc[0][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a_hi, b[nj][0], acc[0][nj], 0, 4,
                                                                       0, (int)ea, 0, (int)sb[nj]);
      }, std::make_integer_sequence<int, kNT>{});
      return;
    }
#pragma unroll
    for (int mi = 0; mi < kMT; ++mi) {
      const uint32_t ea = __builtin_amdgcn_ubfe(rw.sa[mi], ashift, 8);
      unsafe |= ea - kSafeLo > kSafeHi - kSafeLo;
      const int sa = (int)((ea - 1u) | ((ea - 5u) << 8));
      i32x8 ap[2];
#pragma unroll
      for (int pa = 0; pa < 2; ++pa) {
        const u32x6 ca = APlane<kW8>(rw.a[mi], rw.nib, pa != 0);
#pragma unroll
        for (int i = 0; i < 6; ++i) ap[pa][i] = (int)ca[i];
        ap[pa][6] = ap[pa][7] = 0;
      }
      // plane products outer, column tiles inner: consecutive MFMAs update
      // different accumulators
      UnrollS([&](auto pa_c) {
        constexpr int pa = decltype(pa_c)::value;
        UnrollS([&](auto pb_c) {
          constexpr int pb = decltype(pb_c)::value;
          UnrollS([&](auto nj_c) {
            constexpr int nj = decltype(nj_c)::value;
            acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                ap[pa], b[nj][pb], acc[mi][nj], 2, kW8 ? 2 : 4, pa, sa, pb, (int)sb[nj]);
          }, std::make_integer_sequence<int, kNT>{});
        }, std::make_integer_sequence<int, kWP>{});
      }, std::make_integer_sequence<int, 2>{});
    }
  };

  if (c_begin < c_end) {
    // Two register sets: the next chunk's loads are in flight while this
    // one computes; a chunk past the end adds zero (branch-free loop).
    RawS<kMT, kNT, kWP> r0, r1;
    load(r0, c_begin);
    for (uint32_t ch = c_begin; ch < c_end; ch += 2) {
      load(r1, ch + 1);
      compute(r0);
      load(r0, ch + 2);
      compute(r1);
    }
  }
  if (unsafe) lds_unsafe = 1;

  // Partial sums to LDS: lane l holds rows 4*(l/16) + i of each 16x16 tile
  // (column l % 16).
#pragma unroll
  for (int mi = 0; mi < kMT; ++mi)
#pragma unroll
    for (int nj = 0; nj < kNT; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        lds_part[wave][(mi * 16 + 4 * kq + i) * kCols + nj * 16 + r16] = acc[mi][nj][i];
  __syncthreads();
  const bool slow = lds_unsafe != 0;

  // Epilogue: output o = t + 512 p is row o / kCols, column col0 + o % kCols;
  // 32 consecutive threads hold one row's 32-column block.
  for (uint32_t o = t; o < kOut; o += kWaves * 64) {
    const uint32_t row = o / kCols, col = col0 + o % kCols;
    const bool in = (row >> 2) < g.quads && col < g.n;
    uint32_t y = 0;
    if (in) {
      const uint32_t init = (g.acc && row < g.m) ? c[(size_t)row * g.n + col] : 0u;
      if (slow) {
        y = kA8 ? SlowLinearFp8(g, a, w0, init, row, col)
                : SlowLinear<kPanels ? 2 : 1>(g, a, w0, w1, init, row, col);
      } else {
        float s = __uint_as_float(init);
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) s += lds_part[wv][o];
        y = __float_as_uint(s + 0.0f);
      }
      for (uint32_t op = 0; op < g.n_ops; ++op) {
        const uint32_t kind = g.op_kind[op];
        const uint32_t x2 = (kind == kEpAdd || kind == kEpActMul) && row < g.m
                                ? g.op_x2[op][z * g.op_x2_batch[op] + (size_t)row * g.n + col] : 0u;
        const uint32_t pv = (kind == kEpAddP || kind == kEpMulP)
                                ? g.op_vec[op][z * g.op_vec_batch[op] + col] : 0u;
        y = __float_as_uint(EpApplyFast(kind, g.op_imm[op], __uint_as_float(y),
                                        __uint_as_float(x2), __uint_as_float(pv), lds_act));
      }
      if (row < g.m && g.c != nullptr) c[(size_t)row * g.n + col] = y;
    }
    if (q_out != nullptr) {
      const uint32_t e = HalfMax32(in ? ExpField(y) : 0u);
      if (in) {
        const uint32_t nb = g.n >> 5, c32 = col & 31;
        uint8_t* word = q_out + ((size_t)(row >> 2) * nb + (col >> 5)) * kDdrWord;
        word[(row & 3) * 32 + c32] = QuantizeElementHw(y, e);
        if (c32 == 0) word[128 + (row & 3)] = (uint8_t)ScaleByteOf(e);
        if (c32 < 12 && (row & 3) == 0) word[132 + c32] = 0;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// One small layer in one launch (HB_LINEAR_FAST, a single layer of at most
// kSplitMaxRows rows).  A workgroup computes a 32 x 32 output tile with
// v_mfma_scale_f32_32x32x64_f8f6f4 over K steps (64 K values: two blocks
// per step): lane l's A operand is 32 values of row l % 32 and block l / 32
// of the step, its B operand 32 values of column l % 32 and the same block
// (formats and scale bytes as above).  The K ranges ("splits") of a tile
// are the waves of its workgroup (up to kMaxSplitWaves; at least
// kSplitFinishWaves waves, the ones past the splits folding nothing): each
// wave folds its range, the partial sums meet in LDS, and each of 4
// finishers adds its row group's sums in split order, so the sum does not
// depend on which wave finishes first, then runs the epilogue and the
// requantize and stores C.  Per split about 3.4 KB of operands per step (MXFP4), so a workgroup
// moves a few 10 KB: small layers are latency-bound, and the splits put
// every tile's loads in flight at once with one round trip to memory,
// finishing in the same workgroup.
template <bool kW8>
struct RawSplit {
  uint32_t a[8], sa;
  uint32_t w[kW8 ? 2 : 1][4], sw[kW8 ? 2 : 1];
  uint32_t nib;  // 0x0F0F0F0F, or 0 for a block past the range (adds zero)
};

typedef float f32x16s __attribute__((ext_vector_type(16)));

// One layer's tile of a split launch, called by the waves of the workgroup
// that fold it (`split`: the wave's K range; a wave past the layer's splits
// folds nothing; nwaves: the layer's waves in the workgroup).  The
// partials meet in part / flag (LDS, [split][row group][lane] 16-byte
// slots) and up to 4 of the layer's waves finish the tile, 4 of each lane's
// 16 rows apiece.  A fused
// pair (`pair`) is two layers of one tile whose waves fold at the same
// time: the first layer's finishers leave its values in y_lds ([e][lane]),
// and after a second barrier the second layer's finishers read them from
// x2_lds as op x2_op's [m][n] operand.  Every wave of the workgroup calls
// this once (barriers).
// What a wave needs to issue its first operand loads.  The single-layer
// launch passes these as its leading kernel arguments, which the hardware
// preloads into SGPRs (this file is compiled with kernel-argument preload),
// so the loads go out before the argument block's round trip; a group
// launch takes them from its GemmArgs.
struct SplitHot {
  const uint8_t* a;
  const uint8_t* w0;
  const uint8_t* w1;
  uint32_t gy, quads, a_row, piece0, nblocks, split_steps, splits, w_row, groups, panels;
};
__device__ __forceinline__ SplitHot HotOf(const GemmArgs& g) {
  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < g.n_pieces; ++p) nblocks += g.piece_kb[p];
  return SplitHot{g.a, g.w[0], g.w[1], g.gy, g.quads, g.a_row, g.piece_off[0], nblocks,
                  g.split_steps, g.splits, g.w_panels ? g.w_steps : g.kb_total, g.groups,
                  g.w_panels};
}

// kSingle: the single-layer launch (its arguments untouched until its
// loads are out; the epilogue's scalars pinned in SGPRs), else a group's.
template <bool kW8, bool kMulti, bool kA8 = false, bool kSingle = false>
__device__ __forceinline__ void SplitTile(const GemmArgs& g, const SplitHot& h,
                                          uint32_t tile, uint32_t split,
                                          uint32_t nwaves, float (*lds_part)[16 * 64],
                                          uint32_t* lds_flag,
                                          bool pair, float* y_lds, const float* x2_lds,
                                          uint32_t x2_op) {
  constexpr int kWP = kW8 ? 2 : 1;
  typedef f32x16s f32x16;
  const uint32_t lane = threadIdx.x & 63;
  // logical tiles run row tiles fastest: the workgroups of one column tile
  // (which read the same weights) are neighbours, on one XCD
  const uint32_t col0 = (tile / h.gy) * 32, row0 = (tile % h.gy) * 32;
  const uint32_t r32 = lane & 31, hb = lane >> 5;
  const uint8_t* a = h.a;
  const uint8_t* w0 = h.w0;
  const uint8_t* w1 = kW8 ? h.w1 : w0;

  const uint32_t nblocks = h.nblocks;
  const uint32_t steps = (nblocks + 1) / 2;
  const uint32_t s_begin = split < h.splits ? split * h.split_steps : steps;
  const uint32_t s_end = min(s_begin + h.split_steps, steps);
  // a K block's word: one piece from piece0 on, or the piece list's
  auto block_of = [&](uint32_t idx) {
    return kMulti ? SkinnyBlockOf<true>(g, idx) : h.piece0 + idx;
  };

  // the lane's A row and W column (a row or column past the layer reads
  // the last one's bytes; its outputs are not stored)
  const uint32_t quad = min((row0 + r32) >> 2, h.quads - 1);
  const uint32_t a_off = quad * h.a_row * kDdrWord + (r32 & 3) * 32;
  const uint32_t ashift = 8 * (r32 & 3), as_delta = 128 - (r32 & 3) * 32;
  WLaneOff wo;
  {
    const uint32_t col = min((col0 + r32) >> 3, h.groups - 1) * 8 + (r32 & 7);
    if (h.panels) {  // (WLane with w_row = the panel's steps, or the DDR words' blocks)
      const uint32_t base = (col / kPanelCols) * h.w_row * kPanelChunk, c = col % kPanelCols;
      wo.codes = base + c * 16;
      wo.scale = base + kPanelScales + 4 * ((c % 32) / 2);
      wo.shift = 8 * (2 * (c % 2) + c / 32);
    } else {
      const uint32_t base = (col / 8) * h.w_row * kDdrWord, cl = col % 8;
      wo.codes = base + cl * 16;
      wo.scale = base + 128 + (cl & 4);
      wo.shift = 8 * (cl & 3);
    }
  }

  auto load = [&](RawSplit<kW8>& rw, uint32_t st) __attribute__((always_inline)) {
    const uint32_t idx = 2 * st + hb;
    const uint32_t ublk = block_of(min(idx, nblocks - 1));
    const uint8_t* p = a + (size_t)ublk * kDdrWord + a_off;
    if constexpr (kA8) {
      // 8-bit A operands take K in 16-wide halves per lane: registers 0-3
      // of lane half h are K [16 h, 16 h + 16), registers 4-7 K [32 + 16 h,
      // + 16), and each 32-wide K range is scaled by its lane half's byte.
      // So lane half h holds bytes [16 h, 16 h + 16) of both blocks of the
      // step (block 2 st in 0-3, 2 st + 1 in 4-7) and the scale of block
      // 2 st + h.  nib: bit 0 / 1 set when block 2 st / 2 st + 1 is in range.
      rw.nib = (st < s_end ? 1u : 0u) | ((st < s_end && 2 * st + 1 < nblocks) ? 2u : 0u);
      const uint32_t b0 = block_of(min(2 * st, nblocks - 1));
      const uint32_t b1 = block_of(min(2 * st + 1, nblocks - 1));
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(a + (size_t)b0 * kDdrWord + a_off + 16 * hb);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(a + (size_t)b1 * kDdrWord + a_off + 16 * hb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[i] = v0[i];
        rw.a[4 + i] = v1[i];
      }
    } else {
      rw.nib = (st < s_end && idx < nblocks) ? 0x0F0F0F0Fu : 0u;
      const u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
      const u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rw.a[i] = v0[i];
        rw.a[4 + i] = v1[i];
      }
    }
    rw.sa = *reinterpret_cast<const uint32_t*>(p + as_delta);
    const uint32_t wbc = WBlockCodes(g, ublk, h.panels != 0),
                   wbs = WBlockScale(g, ublk, h.panels != 0);
#pragma unroll
    for (int pl = 0; pl < kWP; ++pl) {
      const uint8_t* wp = pl ? w1 : w0;
      const u32x4 v = *reinterpret_cast<const u32x4*>(wp + wbc + wo.codes);
#pragma unroll
      for (int i = 0; i < 4; ++i) rw.w[pl][i] = v[i];
      rw.sw[pl] = *reinterpret_cast<const uint32_t*>(wp + wbs + wo.scale);
    }
  };

  f32x16 acc = {};
  bool unsafe = false;
  auto compute = [&](const RawSplit<kW8>& rw) __attribute__((always_inline)) {
    const uint32_t ewh = __builtin_amdgcn_ubfe(rw.sw[0], wo.shift, 8);
    unsafe |= ewh - kSafeLo > kSafeHi - kSafeLo;
    i32x8 b[kWP];
    uint32_t sb = ewh;
    if constexpr (kW8) {
      const uint32_t ewl = __builtin_amdgcn_ubfe(rw.sw[1], wo.shift, 8);
      unsafe |= ewl - kSafeLo > kSafeHi - kSafeLo;
      sb = (ewh - 1u) | ((ewl - 5u) << 8);
#pragma unroll
      for (int pl = 0; pl < 2; ++pl) {
        const u32x6 cw = WPlane(rw.w[pl], pl != 0);
#pragma unroll
        for (int i = 0; i < 6; ++i) b[pl][i] = (int)cw[i];
        b[pl][6] = b[pl][7] = 0;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) b[0][i] = (int)rw.w[0][i];
      b[0][4] = b[0][5] = b[0][6] = b[0][7] = 0;
    }
    const uint32_t ea = __builtin_amdgcn_ubfe(rw.sa, ashift, 8);
    unsafe |= ea - kSafeLo > kSafeHi - kSafeLo;
    if constexpr (kA8) {  // MXFP8: the code bytes are the FP8 operand (see load), scale ea
      const uint32_t keep0 = (rw.nib & 1u) ? ~0u : 0u, keep1 = (rw.nib & 2u) ? ~0u : 0u;
      // two planes by exponent (fp8::Split): each MFMA sums products of
      // at most 8 binades of A, which the matrix cores add without loss
      i32x8 a_lo, a_hi;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t lo, hi;
        fp8::Split(rw.a[i] & (i < 4 ? keep0 : keep1), lo, hi);
        a_lo[i] = (int)lo;
        a_hi[i] = (int)hi;
      }
      acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a_lo, b[0], acc, 0, 4, 0, (int)ea, 0,
                                                            (int)sb);
      acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a_hi, b[0], acc, 0, 4, 0, (int)ea, 0,
                                                            (int)sb);
      return;
    }
    const int sa = (int)((ea - 1u) | ((ea - 5u) << 8));
    i32x8 ap[2];
#pragma unroll
    for (int pa = 0; pa < 2; ++pa) {
      const u32x6 ca = APlane<kW8>(rw.a, rw.nib, pa != 0);
#pragma unroll
      for (int i = 0; i < 6; ++i) ap[pa][i] = (int)ca[i];
      ap[pa][6] = ap[pa][7] = 0;
    }
    UnrollS([&](auto pa_c) {
      constexpr int pa = decltype(pa_c)::value;
      UnrollS([&](auto pb_c) {
        constexpr int pb = decltype(pb_c)::value;
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ap[pa], b[pb], acc, 2, kW8 ? 2 : 4,
                                                              pa, sa, pb, (int)sb);
      }, std::make_integer_sequence<int, kWP>{});
    }, std::make_integer_sequence<int, 2>{});
  };

  // the lane's outputs: element e is row row0 + 8 (e / 4) + 4 hb + e % 4,
  // column col0 + r32
  const uint32_t col = col0 + r32;
  const bool col_in = col < g.n;
  auto row_of = [&](int e) { return row0 + 8 * (e / 4) + 4 * hb + (e & 3); };
  // K loop: kAhead steps' loads in flight (a split of a small layer has
  // about that many, so they all go out at once, first of all the wave's
  // loads); steps past the range are neither loaded nor computed.
  constexpr int kAhead = 4;
  RawSplit<kW8> ring[kAhead];
#pragma unroll
  for (int i = 0; i < kAhead; ++i)
    if (s_begin + i < s_end) load(ring[i], s_begin + i);
  // the rest of the arguments (one scalar load per 64-byte line, one wait)
  if constexpr (kSingle) TouchArgs(&g, sizeof g);
  // The epilogue's sizes and pointers.  A single layer reads them now and
  // holds them in SGPRs (the empty asm makes them opaque): read after the K
  // loop, they came one scalar round trip at a time.  (In the group kernel
  // the pinned values cost more registers than they save.)
  uint32_t p_m = 0, p_n = 0, p_quads = 0, p_ops = 0;
  uint32_t* p_c = nullptr;
  uint8_t* p_q = nullptr;
  const uint64_t* p_t = nullptr;
  if constexpr (kSingle) {
    p_m = g.m, p_n = g.n, p_quads = g.quads, p_ops = g.n_ops;
    p_c = g.c;
    p_q = g.q_out;
    p_t = g.tbuf;
    asm volatile("" : "+s"(p_m), "+s"(p_n), "+s"(p_quads), "+s"(p_ops), "+s"(p_c), "+s"(p_q),
                 "+s"(p_t));
  }

  // The epilogue is shared: the tile's 16 elements per lane form 4 groups
  // of 4 rows (e / 4), group j finished by the layer's wave j % min(4,
  // nwaves) (`own`: this wave's groups).  Each finisher loads its groups'
  // own operands (the initial C, and the first two ops' [m][n] operand or
  // column value) before the K loop, so it does not wait for them at the end.
  const uint32_t nfin = min(nwaves, 4u);
  uint32_t own = 0;
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) own |= j % nfin == split ? 1u << j : 0u;
  auto owns = [&](int e) { return ((own >> (e / 4)) & 1u) != 0; };
  // The loads are unconditional, at rows and columns clamped into the
  // layer (a guarded load would wait for its data at once); rows past m
  // select 0 in the epilogue.
  constexpr int kPreOps = 2;
  f32x16 pre_init = {}, pre_x2[kPreOps] = {};
  float pre_v[kPreOps] = {};
  const uint32_t ccol = min(col, g.n - 1);
  auto crow = [&](int e) { return (size_t)min(row_of(e), g.m - 1) * g.n + ccol; };
  if (own) {
    if (g.acc) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (owns(e)) pre_init[e] = __uint_as_float(g.c[crow(e)]);
    }
#pragma unroll
    for (int op = 0; op < kPreOps; ++op) {
      if ((uint32_t)op >= g.n_ops || (x2_lds && op == (int)x2_op)) continue;
      const uint32_t kind = g.op_kind[op];
      if (kind == kEpAddP || kind == kEpMulP) pre_v[op] = __uint_as_float(g.op_vec[op][ccol]);
      if (kind == kEpAdd || kind == kEpActMul) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (owns(e)) pre_x2[op][e] = __uint_as_float(g.op_x2[op][crow(e)]);
      }
    }
  }

  for (uint32_t st = s_begin; st < s_end; st += kAhead) {
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      if (st + i < s_end) compute(ring[i]);
      if (st + kAhead + i < s_end) load(ring[i], st + kAhead + i);
    }
  }
  // (read where used in a group's tile, as loads the compiler may repeat)
  auto e_m = [&] { return kSingle ? p_m : g.m; };
  auto e_n = [&] { return kSingle ? p_n : g.n; };
  auto e_quads = [&] { return kSingle ? p_quads : g.quads; };
  auto e_ops = [&] { return kSingle ? p_ops : g.n_ops; };
  auto e_c = [&] { return kSingle ? p_c : g.c; };
  auto e_q = [&] { return kSingle ? p_q : g.q_out; };
  auto e_t = [&] { return kSingle ? p_t : g.tbuf; };
  bool slow = __builtin_amdgcn_ballot_w64(unsafe) != 0;
  f32x16 sum = acc;
  if (blockDim.x > 64) {  // the partials meet in LDS; each finisher adds its groups' in split order
    // A split's partials as [group j][lane] 16-byte slots (values 4 j ..
    // 4 j + 3): one conflict-free access per group.  A finisher reads every
    // split's slot of its group at once (splits past the layer's read the
    // last one's, not added), then adds them in split order.
    f32x4_t* const part = reinterpret_cast<f32x4_t*>(&lds_part[0][0]);
    if (split < g.splits) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        part[(split * 4 + j) * 64 + lane] =
            f32x4_t{acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]};
      if (lane == 0) lds_flag[split] = slow ? 1u : 0u;
    }
    __syncthreads();
    if (own) {
      slow = false;
#pragma unroll
      for (uint32_t s = 0; s < kMaxSplitWaves; ++s)
        slow |= s < g.splits && lds_flag[min(s, g.splits - 1)] != 0;
      UnrollS([&](auto j_c) {
        constexpr int j = decltype(j_c)::value;
        if ((own >> j) & 1u) {  // uniform
          f32x4_t p[kMaxSplitWaves];
#pragma unroll
          for (uint32_t s = 0; s < kMaxSplitWaves; ++s)
            p[s] = part[(min(s, g.splits - 1) * 4 + j) * 64 + lane];
          f32x4_t t = p[0];
#pragma unroll
          for (uint32_t s = 1; s < kMaxSplitWaves; ++s)
            if (s < g.splits) t += p[s];
#pragma unroll
          for (int i = 0; i < 4; ++i) sum[4 * j + i] = t[i];
        }
      }, std::make_integer_sequence<int, 4>{});
    }
  }
  const uint64_t* act = e_t() != nullptr ? e_t() + 512 : nullptr;
  // group j's rows: ops, C, the requantize, and (a pair's first layer) the
  // values the second reads
  auto finish_group = [&](auto j_c) __attribute__((always_inline)) {
    constexpr int j = decltype(j_c)::value;
    f32x4_t y;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * j + i;
      const uint32_t row = row_of(e);
      const float init = row < e_m() ? pre_init[e] : 0.0f;
      y[i] = init + sum[e] + 0.0f;
      if (slow && col_in && (row >> 2) < e_quads()) {  // a scale byte left the window: exactly
        y[i] = __uint_as_float(kA8 ? SlowLinearFp8(g, a, w0, __float_as_uint(init), row, col)
                                   : SlowLinear(g, a, w0, w1, __float_as_uint(init), row, col));
      }
    }
    for (uint32_t op = 0; op < e_ops(); ++op) {
      const uint32_t kind = g.op_kind[op];
      float pv = 0.0f;
      f32x4_t x2 = {};
      if (x2_lds && op == x2_op) {  // rows past m read zeros, as from memory
#pragma unroll
        for (int i = 0; i < 4; ++i)
          x2[i] = row_of(4 * j + i) < e_m() && col_in ? x2_lds[(4 * j + i) * 64 + lane] : 0.0f;
      } else if (op < (uint32_t)kPreOps) {
#pragma unroll
        for (int o = 0; o < kPreOps; ++o)
          if (op == (uint32_t)o) {
            pv = pre_v[o];
#pragma unroll
            for (int i = 0; i < 4; ++i) x2[i] = row_of(4 * j + i) < e_m() ? pre_x2[o][4 * j + i] : 0.0f;
          }
      } else if (col_in) {
        if (kind == kEpAddP || kind == kEpMulP) pv = __uint_as_float(g.op_vec[op][col]);
        if (kind == kEpAdd || kind == kEpActMul) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (row_of(4 * j + i) < e_m())
              x2[i] = __uint_as_float(g.op_x2[op][(size_t)row_of(4 * j + i) * e_n() + col]);
        }
      }
      EpApplyFastN<false>(kind, g.op_imm[op], y, x2, pv, act);
    }
    if (col_in && e_c() != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t row = row_of(4 * j + i);
        if (row < e_m()) e_c()[(size_t)row * e_n() + col] = __float_as_uint(y[i]);
      }
    }
    if (e_q() != nullptr) {
      // one MXINT8 block: the row's 32 columns are the 32 lanes of this half
      uint32_t ex[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ex[i] = HalfMax32((row_of(4 * j + i) >> 2) < e_quads() && col_in
                              ? ExpField(__float_as_uint(y[i])) : 0u);
      // the 4 values are rows 0..3 of one quad: one DDR word; lanes 0..15
      // then write its bytes 128..143 (4 scale bytes, 12 zeros) in one store
      const uint32_t quad = row_of(4 * j) >> 2;
      if (quad < e_quads() && col_in) {
        uint8_t* word = e_q() + ((size_t)quad * (e_n() >> 5) + (col >> 5)) * kDdrWord;
#pragma unroll
        for (int i = 0; i < 4; ++i) word[i * 32 + r32] = QuantizeElementHw(__float_as_uint(y[i]), ex[i]);
        const uint32_t sb = ScaleByteOf(ex[0]) | ScaleByteOf(ex[1]) << 8 |
                           ScaleByteOf(ex[2]) << 16 | ScaleByteOf(ex[3]) << 24;
        if (r32 < 16) word[128 + r32] = r32 < 4 ? (uint8_t)(sb >> (8 * r32)) : 0;
      }
    }
    if (y_lds) {
#pragma unroll
      for (int i = 0; i < 4; ++i) y_lds[(4 * j + i) * 64 + lane] = y[i];
    }
  };
  // phase 0 finishes a lone layer or a pair's first; phase 1 a pair's second
  const uint32_t my_phase = x2_lds ? 1u : 0u;
#pragma clang loop unroll(disable)
  for (uint32_t phase = 0; phase < (pair ? 2u : 1u); ++phase) {
    if (phase == 1) __syncthreads();
    if (own && phase == my_phase) {
      UnrollS([&](auto j_c) {
        if ((own >> decltype(j_c)::value) & 1u) finish_group(j_c);
      }, std::make_integer_sequence<int, 4>{});
    }
  }
}

// The leading arguments (SplitHot's, 13 dwords, preloaded into SGPRs):
// gy_panels = gy | panels << 31, steps_splits = split_steps | splits << 24;
// w1 (W8 only) and the GemmArgs follow in memory.
template <bool kW8, bool kMulti, bool kA8 = false>
__global__ __launch_bounds__(64 * kMaxSplitWaves) void SplitKernel(
    const uint8_t* a, const uint8_t* w0, uint32_t tiles, uint32_t gy_panels, uint32_t quads,
    uint32_t a_row, uint32_t piece0, uint32_t nblocks, uint32_t steps_splits, uint32_t w_row,
    uint32_t groups, const uint8_t* w1, GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float lds_part[kMaxSplitWaves][16 * 64];
  __shared__ uint32_t lds_flag[kMaxSplitWaves];
  const SplitHot h{a, w0, w1, gy_panels & 0x7FFFFFFFu, quads, a_row, piece0, nblocks,
                   steps_splits & 0xFFFFFFu, steps_splits >> 24, w_row, groups, gy_panels >> 31};
  SplitTile<kW8, kMulti, kA8, true>(g, h, XcdLogical(blockIdx.x, tiles),
                         __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                         blockDim.x / 64, lds_part, lds_flag, false, nullptr, nullptr, 0);
}

// A group of layers in one launch: unit u owns workgroups [tile_end[u - 1],
// tile_end[u]) and is one layer, or a pair whose second layer's op x2_op
// reads the first's C.  A pair's layers fold at the same time, the first on
// waves [0, s1), the second on waves [s1, s1 + s2) (s = the layer's splits,
// s1 + s2 <= kMaxSplitWaves), their partials in rows of one LDS array; the
// first's values reach the second's finisher through LDS.
template <bool kW8, bool kMulti>
__global__ __launch_bounds__(64 * kMaxSplitWaves) void SplitGroupKernel(SplitGroup grp) {
  __shared__ __attribute__((aligned(16))) float lds_part[kMaxSplitWaves][16 * 64];
  __shared__ float lds_y[16 * 64];
  __shared__ uint32_t lds_flag[kMaxSplitWaves];
  TouchArgs(&grp.units, sizeof grp - offsetof(SplitGroup, units));
  const uint32_t l = XcdLogical(blockIdx.x, gridDim.x);
  uint32_t u = 0;
  while (u + 1 < grp.units && l >= grp.tile_end[u]) ++u;  // uniform
  const uint32_t tile = l - (u ? grp.tile_end[u - 1] : 0u);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t second = grp.second[u];
  const bool pair = second < kMaxGroup;
  const uint32_t s1 = pair ? grp.g[grp.first[u]].splits : kMaxSplitWaves;
  const bool in2 = wave >= s1;  // (a wave of the pair's second layer)
  const uint32_t base = in2 ? s1 : 0u;
  const uint32_t waves = blockDim.x / 64;
  const GemmArgs& g = grp.g[in2 ? second : grp.first[u]];
  TouchArgs(&g, sizeof g);
  SplitTile<kW8, kMulti>(g, HotOf(g), tile, wave - base,
                         in2 ? waves - s1 : min(s1, waves), lds_part + base, lds_flag + base, pair,
                         pair && !in2 ? lds_y : nullptr, in2 ? lds_y : nullptr, grp.x2_op[u]);
}

template <int kMT, bool kW8, bool kMulti, bool kA8 = false>
void LaunchS(const GemmArgs& in, uint32_t batch, hipStream_t stream) {
  constexpr int kCols = 16 * NTiles<kMT, kW8>();
  GemmArgs args = in;
  args.gx = (args.groups * 8 + kCols - 1) / kCols;
  args.gy = 1;
  args.gz = batch;
  if (args.w_panels)
    hipLaunchKernelGGL((SkinnyKernel<kMT, kW8, kMulti, true, kA8>), dim3(args.gx * args.gz),
                       dim3(kWaves * 64), 0, stream, args);
  else
    hipLaunchKernelGGL((SkinnyKernel<kMT, kW8, kMulti, false, kA8>), dim3(args.gx * args.gz),
                       dim3(kWaves * 64), 0, stream, args);
}

template <int kMT>
void LaunchRowsS(const GemmArgs& args, uint32_t batch, hipStream_t stream) {
  const bool multi = args.n_pieces > 1, w8 = args.n_planes == 2;
  if (w8) multi ? LaunchS<kMT, true, true>(args, batch, stream)
              : LaunchS<kMT, true, false>(args, batch, stream);
  else multi ? LaunchS<kMT, false, true>(args, batch, stream)
             : LaunchS<kMT, false, false>(args, batch, stream);
}

}  // namespace

bool SplitEligible(const GemmArgs& args, uint32_t batch) {
  return batch == 1 && args.quads * 4 <= kSplitMaxRows;
}

size_t SplitPlan(GemmArgs& args, uint32_t max_splits) {
  // splits (waves) of at least 2 steps, at most max_splits per tile: a
  // wave converts its A and issues its MFMAs one step after another once
  // its loads have landed, so shorter K ranges shorten the tile (measured,
  // B = 1 chains: 2 steps against 4, SmolVLA expert step 0.540 -> 0.495 ms,
  // SparseDrive-S head at one frame 0.588 -> 0.512 ms; 1 step: the head
  // 0.650 ms)
  constexpr uint32_t kMinSteps = 2;
  args.gx = (args.n + 31) / 32;
  args.gy = (args.quads * 4 + 31) / 32;
  args.gz = 1;
  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < args.n_pieces; ++p) nblocks += args.piece_kb[p];
  const uint32_t steps = (nblocks + 1) / 2;
  uint32_t per = (steps + max_splits - 1) / max_splits;
  per = per < kMinSteps ? kMinSteps : per;
  const uint32_t splits = (steps + per - 1) / per;
  args.splits = splits;
  args.split_steps = splits > 1 ? per : steps;
  return 0;  // the partials meet in LDS: no workspace
}

hipError_t LaunchSplitLinear(const GemmArgs& args, hipStream_t stream) {
  const uint32_t tiles = args.gx * args.gy;
  const dim3 grid(tiles), block(64 * std::max(args.splits, kSplitFinishWaves));
  const bool w8 = args.n_planes == 2, multi = args.n_pieces > 1;
  uint32_t nblocks = 0;
  for (uint32_t p = 0; p < args.n_pieces; ++p) nblocks += args.piece_kb[p];
  // the packed fields' ranges (steps below 2^24: W spans at most 4 GiB)
  if (args.gy >= (1u << 31) || args.split_steps >= (1u << 24) || args.splits > 255)
    return hipErrorInvalidValue;
  const uint32_t gy_panels = args.gy | (args.w_panels ? 1u << 31 : 0u);
  const uint32_t steps_splits = args.split_steps | args.splits << 24;
  const uint32_t w_row = args.w_panels ? args.w_steps : args.kb_total;
  const uint8_t* w1 = w8 ? args.w[1] : args.w[0];
#define HB_SPLIT_ARGS args.a, args.w[0], tiles, gy_panels, args.quads, args.a_row, \
    args.piece_off[0], nblocks, steps_splits, w_row, args.groups, w1, args
  if (w8) {
    if (multi) hipLaunchKernelGGL((SplitKernel<true, true>), grid, block, 0, stream, HB_SPLIT_ARGS);
    else hipLaunchKernelGGL((SplitKernel<true, false>), grid, block, 0, stream, HB_SPLIT_ARGS);
  } else if (args.a_fp8) {
    if (multi) hipLaunchKernelGGL((SplitKernel<false, true, true>), grid, block, 0, stream, HB_SPLIT_ARGS);
    else hipLaunchKernelGGL((SplitKernel<false, false, true>), grid, block, 0, stream, HB_SPLIT_ARGS);
  } else {
    if (multi) hipLaunchKernelGGL((SplitKernel<false, true>), grid, block, 0, stream, HB_SPLIT_ARGS);
    else hipLaunchKernelGGL((SplitKernel<false, false>), grid, block, 0, stream, HB_SPLIT_ARGS);
  }
#undef HB_SPLIT_ARGS
  return hipGetLastError();
}

hipError_t LaunchSplitGroup(const SplitGroup& grp, uint32_t waves, hipStream_t stream) {
  const dim3 grid(grp.tile_end[grp.units - 1]), block(64 * waves);
  const GemmArgs& g0 = grp.g[grp.first[0]];
  const bool w8 = g0.n_planes == 2, multi = g0.n_pieces > 1;
  if (w8) {
    if (multi) hipLaunchKernelGGL((SplitGroupKernel<true, true>), grid, block, 0, stream, grp);
    else hipLaunchKernelGGL((SplitGroupKernel<true, false>), grid, block, 0, stream, grp);
  } else {
    if (multi) hipLaunchKernelGGL((SplitGroupKernel<false, true>), grid, block, 0, stream, grp);
    else hipLaunchKernelGGL((SplitGroupKernel<false, false>), grid, block, 0, stream, grp);
  }
  return hipGetLastError();
}

hipError_t LaunchLinearSkinny(const GemmArgs& args, uint32_t batch, hipStream_t stream) {
  // (layers of up to 16 rows in a batch; one layer of up to kSplitMaxRows
  // rows runs as a split launch instead)
  if (args.quads * 4 > 16) return hipErrorInvalidValue;
  if (args.a_fp8) {  // one MXFP4 plane
    if (args.n_planes != 1 || args.modes[0] != kModeFp4) return hipErrorInvalidValue;
    if (args.n_pieces > 1) LaunchS<1, false, true, true>(args, batch, stream);
    else LaunchS<1, false, false, true>(args, batch, stream);
    return hipGetLastError();
  }
  LaunchRowsS<1>(args, batch, stream);
  return hipGetLastError();
}

}  // namespace hb
